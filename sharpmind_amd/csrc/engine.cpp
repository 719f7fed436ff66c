// engine.cpp — one training step of SharpMind's decoder on a single MI355X.
//
// Call order mirrors TrainLoop.ForwardBackward + BackpropEngine
// (SharpMind.Training/TrainLoop.cs:222-243; Autograd/BackpropEngine.cs:73-206,
// 517-657, 802-835) and then the optimizer (Gradients.ClipGlobalNorm,
// Gradients.cs:92-116; AdamW.Update, Optimizers/AdamW.cs:52-89).  Everything
// stays resident in HBM: weights, saved activations, gradients, AdamW state.
// No allocation happens inside a step.
//
// Two modes share the code:
//  * full-parameter (base_qtype = F32): every weight trains; precision fp32
//    (fp32 MFMA, the exactness configuration) or bf16 (bf16 weight shadows
//    with fp32 masters, bf16 MFMA);
//  * LoRA (lora_rank > 0, base Q8_0 / Q4_K): the base is frozen and stored as
//    repacked quantisation planes, dequantised in registers inside every GEMM;
//    only the adapters train.  Fused projections (q|k|v, gate|up) carry one
//    adapter of rank n*r whose B is block-diagonal; off-diagonal gradient
//    blocks are zeroed so they stay exactly zero under AdamW.
#include <hip/hip_runtime.h>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <ctime>
#include <filesystem>
#include <memory>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "common.hpp"
#include "gguf.hpp"
#include "kernels.hpp"

namespace smhip {

enum Proj { P_QKV = 0, P_O = 1, P_GU = 2, P_D = 3 };

struct DenseRef {  // trainable/frozen fp32 tensor inside an arena
  float* data = nullptr;
  float* grad = nullptr;  // null when frozen
  uint16_t* bf = nullptr; // bf16 shadow (full-param bf16 mode, weights only)
  int64_t n = 0;
};

struct LayerW {
  DenseRef norm1, norm2, qn, kn;
  DenseRef w[4], b[4];       // full-param weights [Out][In] and biases
  QuantPlanes q[4];          // LoRA mode frozen base
  void* qraw[4] = {};        // LoRA mode: planes storage
  QuantPlanes qt[4];         // LoRA bf16 mode: column planes (transposed copy) for dX
  void* qtraw[4] = {};
  Operand fq[4] = {}, fqt[4] = {};  // LoRA bf16 mode: fragment planes for y = x W^T and dX = dY W
  uint16_t* wb[4] = {};      // LoRA bf16 mode with the base workspace: bf16 [Out][In] and [In][Out]
  uint16_t* wbt[4] = {};
  DenseRef la[4], lb[4];     // LoRA A [In, nr], B [nr, Out]
  uint16_t* lat[4] = {};     // bf16 LoRA: A transposed, [nr][In] (k-contiguous operand of u = x A)
  int* lb_cols = nullptr;    // device: column start of each diagonal block
};

struct Saved {
  float *h_in, *rinv1, *rinv_qk, *lse, *probs, *h_mid, *rinv2;
  void *qkv;  // q|k|v projection output: bf16 when Engine::qkv_bf, fp32 otherwise
  void *xn1, *q, *k, *v, *o, *xn2, *gu, *act;
  void* u[4];  // LoRA x.A per projection
};

struct Engine {
  smhip_model_config c;
  int T, qd, kvd, nqkv, In[4], Out[4], nr[4], nblk[4];
  bool bf, lora;
  bool qkv_bf;  // bf16 engines with head_dim 64 / 128 keep the q|k|v projection output in bf16
  size_t esz;  // activation element size
  // arenas
  float* train = nullptr; float* grad = nullptr; float* m = nullptr; float* v = nullptr;
  uint16_t* train_bf = nullptr;
  int64_t n_train = 0, n_decay = 0;
  float* frozen = nullptr;
  int64_t n_frozen = 0;
  std::vector<void*> allocs;
  // tensors
  DenseRef emb, norm_f;
  QuantPlanes emb_q{}, emb_qt{};
  Operand emb_fq{}, emb_fqt{};  // fragment planes of the quantised embedding (head forward / dX)
  bool frag = false;            // bf16 LoRA: base GEMMs decode fragment planes in LDS
  // bf16 LoRA engines decode the frozen quantised base once per step into bf16 copies in both
  // layouts (row for y = x W^T, transposed for dX = dY W), so every base GEMM streams bf16
  // straight to LDS; without room for it the GEMMs decode the codes in their loaders
  bool base_ws = false;
  uint16_t *emb_b = nullptr, *emb_bt = nullptr;
  SkinnyBatch skb;                // deferred split reductions of a layer's adapter gradients
  SkinnyHold skh;                 // a projection's dB product waiting to share its launch with dA
  int lb_masked[4] = {};          // the last dB product of projection p applied the block-diagonal mask
  DequantJob* dq_jobs = nullptr;  // device table of the per-step decode (one launch)
  int dq_njobs = 0;
  int64_t dq_tiles = 0;
  BfTJob* lat_jobs = nullptr;  // device table of the per-step LoRA A transposes (one launch)
  int lat_njobs = 0;
  int64_t lat_max = 0;
  std::vector<LayerW> L;
  std::map<std::string, DenseRef*> dense_by_name;
  // activations
  std::vector<Saved> sv;
  float *h_fin, *rinv_f, *logits, *cosT, *sinT, *loss, *gnorm;
  // bf16 LoRA engines on fragment planes: the head GEMM's softmax row statistics ([T][V/64] pairs),
  // so cross-entropy reads the logits once (null: cross-entropy computes them itself)
  float* rowstat = nullptr;
  void *xnf, *dlogits;
  // backward work
  float *dh, *dx, *dq, *dk, *dv;
  void* dact;  // dL/d(SwiGLU output): bf16 in bf16 engines
  void *dh_ta, *dgu, *dO, *dqkv, *z;
  void* flash_ws = nullptr;
  int step = 0;
  // graph mode: forward_backward recorded once as a HIP graph on a private stream and replayed
  bool use_graph = false;
  hipStream_t cap = nullptr;
  hipGraphExec_t gexec = nullptr;
  int32_t *ids_in = nullptr, *labels_in = nullptr;  // engine-owned inputs the graph reads
};

static inline void* dalloc(Engine* e, size_t bytes) {
  void* p = nullptr;
  if (hipMalloc(&p, bytes < 256 ? 256 : bytes) != hipSuccess) return nullptr;
  e->allocs.push_back(p);
  return p;
}

static const char* kProjName[4] = {"qkv", "o", "gu", "d"};

// ------------------------------------------------------------------ layout
static int build(Engine* e) {
  const smhip_model_config& c = e->c;
  e->T = c.batch * c.seq;
  e->qd = c.n_heads * c.head_dim;
  e->kvd = c.n_kv_heads * c.head_dim;
  e->nqkv = e->qd + 2 * e->kvd;
  e->bf = c.precision == SMHIP_PREC_BF16;
  e->lora = c.lora_rank > 0;
  e->esz = e->bf ? 2 : 4;
  e->qkv_bf = e->bf && (c.head_dim == 64 || c.head_dim == 128);
  const int d = c.d_model, F = c.ffn_dim, V = c.vocab, r = c.lora_rank;
  e->In[P_QKV] = d; e->Out[P_QKV] = e->nqkv; e->nr[P_QKV] = 3 * r; e->nblk[P_QKV] = 3;
  e->In[P_O] = e->qd; e->Out[P_O] = d; e->nr[P_O] = r; e->nblk[P_O] = 1;
  e->In[P_GU] = d; e->Out[P_GU] = 2 * F; e->nr[P_GU] = 2 * r; e->nblk[P_GU] = 2;
  e->In[P_D] = F; e->Out[P_D] = d; e->nr[P_D] = r; e->nblk[P_D] = 1;
  e->L.resize(c.n_layers);

  // --- arena sizing: trainable tensors, weight-decayed ones first (AdamW.cs:25-41 no-decay names)
  struct Item { DenseRef* ref; int64_t n; bool decay; bool shadow; };
  std::vector<Item> tr, fr;
  auto add = [&](DenseRef* ref, int64_t n, bool trainable, bool decay, bool shadow) {
    (trainable ? tr : fr).push_back({ref, n, decay, shadow});
  };
  // AdamW skips weight decay for parameters whose reference name contains "bias", "norm.weight"
  // or "layernorm.weight" (AdamW.cs:38-41, 119-125).  The reference's parameter names are
  // EmbeddingTable.weight, q_proj.weight ... down_proj.weight, <proj>.bias, RmsNormLayer.weight
  // and lora.a / lora.b, so only the biases are exempt: "RmsNormLayer.weight" does not contain
  // "norm.weight".
  const bool full = !e->lora;
  add(&e->emb, (int64_t)V * d, full, true, true);  // LoRA mode keeps emb quantised (emb_q)
  add(&e->norm_f, d, full, true, false);
  for (int l = 0; l < c.n_layers; l++) {
    LayerW& w = e->L[l];
    add(&w.norm1, d, full, true, false);
    add(&w.norm2, d, full, true, false);
    if (c.qk_norm) { add(&w.qn, c.head_dim, full, true, false); add(&w.kn, c.head_dim, full, true, false); }
    for (int p = 0; p < 4; p++) {
      if (full) {
        add(&w.w[p], (int64_t)e->Out[p] * e->In[p], true, true, true);
        if (c.use_bias) add(&w.b[p], e->Out[p], true, false, false);
      } else {
        add(&w.la[p], (int64_t)e->In[p] * e->nr[p], true, true, true);
        add(&w.lb[p], (int64_t)e->nr[p] * e->Out[p], true, true, true);
      }
    }
  }
  if (e->lora) {  // emb is frozen and quantised: not part of the fp32 arenas
    for (size_t i = 0; i < fr.size(); i++)
      if (fr[i].ref == &e->emb) { fr.erase(fr.begin() + i); break; }
  }
  std::stable_partition(tr.begin(), tr.end(), [](const Item& it) { return it.decay; });
  for (auto& it : tr) { e->n_train += it.n; if (it.decay) e->n_decay += it.n; }
  for (auto& it : fr) e->n_frozen += it.n;
  const size_t tb = sizeof(float) * (size_t)std::max<int64_t>(e->n_train, 1);
  e->train = (float*)dalloc(e, tb);
  e->grad = (float*)dalloc(e, tb);
  e->m = (float*)dalloc(e, tb);
  e->v = (float*)dalloc(e, tb);
  if (!e->train || !e->grad || !e->m || !e->v) return fail(SMHIP_ENOMEM, "engine: parameter arena");
  if (e->bf) {  // bf16 GEMM operand copies of the trainable weights (full mode) or adapters (LoRA)
    e->train_bf = (uint16_t*)dalloc(e, sizeof(uint16_t) * (size_t)std::max<int64_t>(e->n_train, 1));
    if (!e->train_bf) return fail(SMHIP_ENOMEM, "engine: bf16 shadow");
  }
  if (e->n_frozen) {
    e->frozen = (float*)dalloc(e, sizeof(float) * (size_t)e->n_frozen);
    if (!e->frozen) return fail(SMHIP_ENOMEM, "engine: frozen arena");
  }
  // parameters start at zero (fused LoRA B off-diagonal blocks must stay exactly 0), AdamW m = v = 0
  for (float* a : {e->train, e->grad, e->m, e->v})
    if (int rc = zero_bytes(a, tb, nullptr)) return rc;
  if (e->frozen)
    if (int rc = zero_bytes(e->frozen, sizeof(float) * (size_t)e->n_frozen, nullptr)) return rc;
  SMHIP_CHECK_HIP(hipDeviceSynchronize());
  int64_t off = 0;
  for (auto& it : tr) {
    it.ref->data = e->train + off;
    it.ref->grad = e->grad + off;
    it.ref->bf = (e->train_bf && it.shadow) ? e->train_bf + off : nullptr;
    it.ref->n = it.n;
    off += it.n;
  }
  off = 0;
  for (auto& it : fr) {
    it.ref->data = e->frozen + off;
    it.ref->grad = nullptr;
    it.ref->n = it.n;
    off += it.n;
  }
  if (e->lora && e->bf) {  // transposed bf16 copies of the LoRA A shadows, refreshed each step
    std::vector<BfTJob> jobs;
    int64_t tot = 0;
    for (int l = 0; l < c.n_layers; l++)
      for (int p = 0; p < 4; p++) tot += (int64_t)e->In[p] * e->nr[p];
    uint16_t* at = (uint16_t*)dalloc(e, sizeof(uint16_t) * (size_t)std::max<int64_t>(tot, 1));
    if (!at) return fail(SMHIP_ENOMEM, "engine: transposed adapters");
    for (int l = 0; l < c.n_layers; l++)
      for (int p = 0; p < 4; p++) {
        LayerW& w = e->L[l];
        if (!w.la[p].bf) continue;
        w.lat[p] = at;
        jobs.push_back(BfTJob{w.la[p].bf, at, e->In[p], e->nr[p]});
        e->lat_max = std::max<int64_t>(e->lat_max, (int64_t)e->In[p] * e->nr[p]);
        at += (int64_t)e->In[p] * e->nr[p];
      }
    if (!jobs.empty()) {
      e->lat_njobs = (int)jobs.size();
      e->lat_jobs = (BfTJob*)dalloc(e, sizeof(BfTJob) * jobs.size());
      if (!e->lat_jobs) return fail(SMHIP_ENOMEM, "engine: transpose table");
      SMHIP_CHECK_HIP(hipMemcpy(e->lat_jobs, jobs.data(), sizeof(BfTJob) * jobs.size(), hipMemcpyHostToDevice));
    }
  }

  // --- LoRA: quantised base planes and block-diagonal column starts
  if (e->lora) {
    const int qt = c.base_qtype;
    SMHIP_REQUIRE(qt == SMHIP_QTYPE_Q8_0 || qt == SMHIP_QTYPE_Q4_K, "engine: LoRA base must be Q8_0 or Q4_K");
    auto mk = [&](QuantPlanes* q, void** store, int64_t n) -> int {
      size_t qb = 0;
      size_t bytes = planes_bytes(qt, n, &qb);
      *store = dalloc(e, bytes);
      if (!*store) return fail(SMHIP_ENOMEM, "engine: quantised base");
      q->kind = qt; q->n = n; q->qs = *store; q->sc = (float*)((char*)*store + qb);
      return SMHIP_OK;
    };
    void* emb_store = nullptr;
    if (int rc = mk(&e->emb_q, &emb_store, (int64_t)V * d)) return rc;
    for (int l = 0; l < c.n_layers; l++)
      for (int p = 0; p < 4; p++)
        if (int rc = mk(&e->L[l].q[p], &e->L[l].qraw[p], (int64_t)e->Out[p] * e->In[p])) return rc;
    if (e->bf) {  // bf16 base workspace when dims allow and it takes at most a quarter of free HBM
      int64_t n_all = (int64_t)V * d;
      bool dims_ok = d % 16 == 0 && V % 16 == 0;
      for (int p = 0; p < 4; p++) {
        n_all += (int64_t)c.n_layers * e->Out[p] * e->In[p];
        dims_ok = dims_ok && e->Out[p] % 16 == 0 && e->In[p] % 16 == 0;
      }
      size_t fr = 0, tot = 0;
      if (hipMemGetInfo(&fr, &tot) != hipSuccess) fr = 0;
      // a Q8_0 / Q4_K base is read as fragment planes by GEMMs that decode it in LDS, so it is never
      // expanded in HBM; SMHIP_BASE_WS=1 instead decodes the whole base into a bf16 workspace
      // every step (dims permitting, at most a quarter of free HBM), =0 forces the planes
      const char* ev = getenv("SMHIP_BASE_WS");
      bool frag_ok = V % 64 == 0 && d % 64 == 0;
      for (int p = 0; p < 4; p++) frag_ok = frag_ok && e->Out[p] % 64 == 0 && e->In[p] % 64 == 0;
      const bool want_ws = ev ? atoi(ev) != 0 : !frag_ok;
      e->base_ws = want_ws && dims_ok && (size_t)n_all * 4 <= fr / 4;
      e->frag = !e->base_ws && frag_ok;
    }
    if (e->base_ws) {
      auto bfbuf = [&](uint16_t** dst, int64_t n) -> int {
        *dst = (uint16_t*)dalloc(e, 2 * (size_t)n);
        return *dst ? SMHIP_OK : fail(SMHIP_ENOMEM, "engine: bf16 base workspace");
      };
      if (int rc = bfbuf(&e->emb_b, (int64_t)V * d)) return rc;
      if (int rc = bfbuf(&e->emb_bt, (int64_t)V * d)) return rc;
      for (int l = 0; l < c.n_layers; l++)
        for (int p = 0; p < 4; p++) {
          if (int rc = bfbuf(&e->L[l].wb[p], (int64_t)e->Out[p] * e->In[p])) return rc;
          if (int rc = bfbuf(&e->L[l].wbt[p], (int64_t)e->Out[p] * e->In[p])) return rc;
        }
      std::vector<DequantJob> jobs;
      auto job = [&](const QuantPlanes& q, int rows, int cols, uint16_t* w, uint16_t* wt) -> int {
        if (int rc = dequant_bf16_check(q, rows, cols, w, wt)) return rc;
        jobs.push_back({q, rows, cols, w, wt, e->dq_tiles});
        e->dq_tiles += (int64_t)ceil_div(rows, 64) * ceil_div(cols, 64);
        return SMHIP_OK;
      };
      if (int rc = job(e->emb_q, V, d, e->emb_b, e->emb_bt)) return rc;
      for (int l = 0; l < c.n_layers; l++)
        for (int p = 0; p < 4; p++)
          if (int rc = job(e->L[l].q[p], e->Out[p], e->In[p], e->L[l].wb[p], e->L[l].wbt[p])) return rc;
      e->dq_njobs = (int)jobs.size();
      e->dq_jobs = (DequantJob*)dalloc(e, sizeof(DequantJob) * jobs.size());
      if (!e->dq_jobs) return fail(SMHIP_ENOMEM, "engine: decode table");
      SMHIP_CHECK_HIP(hipMemcpy(e->dq_jobs, jobs.data(), sizeof(DequantJob) * jobs.size(), hipMemcpyHostToDevice));
    } else if (e->frag) {  // fragment planes, both orientations
      auto fr2 = [&](Operand* f, Operand* ft, int64_t n) -> int {
        const size_t b = frag_planes_bytes(n, qt);
        f->p = dalloc(e, b);
        ft->p = dalloc(e, b);
        return f->p && ft->p ? SMHIP_OK : fail(SMHIP_ENOMEM, "engine: fragment planes");
      };
      if (int rc = fr2(&e->emb_fq, &e->emb_fqt, (int64_t)V * d)) return rc;
      for (int l = 0; l < c.n_layers; l++)
        for (int p = 0; p < 4; p++)
          if (int rc = fr2(&e->L[l].fq[p], &e->L[l].fqt[p], (int64_t)e->Out[p] * e->In[p])) return rc;
    } else if (e->bf) {  // column planes for the bf16 dX GEMMs
      void* emb_t = nullptr;
      if (int rc = mk(&e->emb_qt, &emb_t, (int64_t)V * d)) return rc;
      for (int l = 0; l < c.n_layers; l++)
        for (int p = 0; p < 4; p++)
          if (int rc = mk(&e->L[l].qt[p], &e->L[l].qtraw[p], (int64_t)e->Out[p] * e->In[p])) return rc;
    }
    for (int l = 0; l < c.n_layers; l++) {
      // column start of each diagonal block of the fused B: q|k|v at [0..3), gate|up at [3..5)
      LayerW& w = e->L[l];
      w.lb_cols = (int*)dalloc(e, 8 * sizeof(int));
      if (!w.lb_cols) return fail(SMHIP_ENOMEM, "engine: LoRA block table");
      const int h_cols[5] = {0, e->qd, e->qd + e->kvd, 0, F};
      SMHIP_CHECK_HIP(hipMemcpy(w.lb_cols, h_cols, sizeof(h_cols), hipMemcpyHostToDevice));
    }
    // partials of one layer's dA / dB products (a full arena flushes early, which is only slower)
    e->skb.cap = (size_t)96 << 20;
    e->skb.arena = (float*)dalloc(e, e->skb.cap);
    if (!e->skb.arena) return fail(SMHIP_ENOMEM, "engine: adapter-gradient partials");
  }

  // --- activations
  const int T = e->T;
  const size_t ES = e->esz;
  e->sv.resize(c.n_layers);
  for (int l = 0; l < c.n_layers; l++) {
    Saved& s = e->sv[l];
    memset(&s, 0, sizeof(s));
    s.h_in = (float*)dalloc(e, sizeof(float) * (size_t)T * d);
    s.rinv1 = (float*)dalloc(e, sizeof(float) * T);
    s.xn1 = dalloc(e, ES * (size_t)T * d);
    s.qkv = dalloc(e, (e->qkv_bf ? 2 : 4) * (size_t)T * e->nqkv);
    s.rinv_qk = (float*)dalloc(e, sizeof(float) * (size_t)T * (c.n_heads + c.n_kv_heads));
    s.q = dalloc(e, ES * (size_t)T * e->qd);
    s.k = dalloc(e, ES * (size_t)T * e->kvd);
    s.v = dalloc(e, ES * (size_t)T * e->kvd);
    if (e->bf) s.lse = (float*)dalloc(e, sizeof(float) * (size_t)T * c.n_heads);
    else s.probs = (float*)dalloc(e, sizeof(float) * (size_t)c.batch * c.n_heads * c.seq * c.seq);
    s.o = dalloc(e, ES * (size_t)T * e->qd);
    s.h_mid = (float*)dalloc(e, sizeof(float) * (size_t)T * d);
    s.rinv2 = (float*)dalloc(e, sizeof(float) * T);
    s.xn2 = dalloc(e, ES * (size_t)T * d);
    s.gu = dalloc(e, ES * (size_t)T * 2 * F);
    s.act = dalloc(e, ES * (size_t)T * F);
    if (e->lora)
      for (int p = 0; p < 4; p++) s.u[p] = dalloc(e, ES * (size_t)T * e->nr[p]);
    if (!s.h_in || !s.act || !s.o || !s.gu) return fail(SMHIP_ENOMEM, "engine: activations");
  }
  e->h_fin = (float*)dalloc(e, sizeof(float) * (size_t)T * d);
  e->rinv_f = (float*)dalloc(e, sizeof(float) * T);
  e->xnf = dalloc(e, ES * (size_t)T * d);
  e->logits = (float*)dalloc(e, sizeof(float) * (size_t)T * V);
  e->dlogits = e->bf ? dalloc(e, 2 * (size_t)T * V) : (void*)e->logits;  // fp32 mode: in place
  if (e->bf && e->frag && T % 128 == 0 && V % 128 == 0 && (int64_t)(T / 128) * (V / 128) >= 4 * num_cus()) {
    e->rowstat = (float*)dalloc(e, sizeof(float) * 2 * (size_t)T * (V / 64));
    if (!e->rowstat) return fail(SMHIP_ENOMEM, "engine: row statistics");
  }
  e->cosT = (float*)dalloc(e, sizeof(float) * (size_t)c.seq * c.head_dim / 2);
  e->sinT = (float*)dalloc(e, sizeof(float) * (size_t)c.seq * c.head_dim / 2);
  e->loss = (float*)dalloc(e, 256);
  e->gnorm = e->loss + 4;
  const int wmax = std::max(std::max(d, F), std::max(e->nqkv, 2 * F));
  e->dh = (float*)dalloc(e, sizeof(float) * (size_t)T * d);
  e->dx = (float*)dalloc(e, sizeof(float) * (size_t)T * d);
  e->dact = dalloc(e, ES * (size_t)T * F);
  e->dq = (float*)dalloc(e, sizeof(float) * (size_t)T * e->qd);
  e->dk = (float*)dalloc(e, sizeof(float) * (size_t)T * e->kvd);
  e->dv = (float*)dalloc(e, sizeof(float) * (size_t)T * e->kvd);
  e->dh_ta = e->bf ? dalloc(e, 2 * (size_t)T * d) : (void*)e->dh;
  e->dgu = dalloc(e, ES * (size_t)T * 2 * F);
  e->dO = dalloc(e, ES * (size_t)T * e->qd);
  e->dqkv = dalloc(e, ES * (size_t)T * e->nqkv);
  e->z = dalloc(e, ES * (size_t)T * std::max(3 * r, 1));
  (void)wmax;
  if (e->bf) e->flash_ws = dalloc(e, flash_backward_workspace(c.batch, c.seq, c.n_heads, c.head_dim));
  e->ids_in = (int32_t*)dalloc(e, sizeof(int32_t) * (size_t)T);
  e->labels_in = (int32_t*)dalloc(e, sizeof(int32_t) * (size_t)T);
  if (!e->ids_in || !e->labels_in || !e->dh || !e->dgu || !e->dqkv || !e->logits || !e->dlogits || (e->bf && !e->flash_ws))
    return fail(SMHIP_ENOMEM, "engine: work buffers");

  // RoPE tables (host, RoPE.cs:99-148)
  std::vector<float> ct((size_t)c.seq * c.head_dim / 2), st((size_t)c.seq * c.head_dim / 2);
  if (int rc = smhip_rope_tables(c.rope_theta, c.head_dim, c.seq, ct.data(), st.data())) return rc;
  SMHIP_CHECK_HIP(hipMemcpy(e->cosT, ct.data(), sizeof(float) * ct.size(), hipMemcpyHostToDevice));
  SMHIP_CHECK_HIP(hipMemcpy(e->sinT, st.data(), sizeof(float) * st.size(), hipMemcpyHostToDevice));

  // names
  e->dense_by_name["emb"] = &e->emb;
  e->dense_by_name["norm_f"] = &e->norm_f;
  for (int l = 0; l < c.n_layers; l++) {
    LayerW& w = e->L[l];
    std::string p = "l" + std::to_string(l) + ".";
    e->dense_by_name[p + "norm1"] = &w.norm1;
    e->dense_by_name[p + "norm2"] = &w.norm2;
    if (c.qk_norm) { e->dense_by_name[p + "q_norm"] = &w.qn; e->dense_by_name[p + "k_norm"] = &w.kn; }
    if (!e->lora) {
      const char* wn[4] = {"wqkv", "wo", "wgu", "wd"};
      const char* bn[4] = {"bqkv", "bo", "bgu", "bd"};
      for (int q = 0; q < 4; q++) {
        e->dense_by_name[p + wn[q]] = &w.w[q];
        if (c.use_bias) e->dense_by_name[p + bn[q]] = &w.b[q];
      }
    }
  }
  return SMHIP_OK;
}

// ------------------------------------------------------------------ operand helpers
static Operand act_k(const Engine* e, const void* p, int64_t ld) {
  return Operand{e->bf ? SRC_BF16_K : SRC_F32_K, p, nullptr, ld};
}
static Operand act_r(const Engine* e, const void* p, int64_t ld) {
  return Operand{e->bf ? SRC_BF16_R : SRC_F32_R, p, nullptr, ld};
}
// weight W[Out][In] as the B operand of  y = x W^T (k = In contiguous)
static Operand w_fwd(const Engine* e, const LayerW& w, int p) {
  if (e->base_ws) return Operand{SRC_BF16_K, w.wb[p], nullptr, e->In[p]};
  if (e->frag) return w.fq[p];
  if (e->lora) {
    const QuantPlanes& q = w.q[p];
    return Operand{q.kind == SMHIP_QTYPE_Q8_0 ? SRC_Q8_K : SRC_Q4K_K, q.qs, q.sc, e->In[p]};
  }
  return w.w[p].bf ? Operand{SRC_BF16_K, w.w[p].bf, nullptr, e->In[p]} : Operand{SRC_F32_K, w.w[p].data, nullptr, e->In[p]};
}
// weight as the B operand of  dX = dY W  (n = In, k = Out)
static Operand w_bwd(const Engine* e, const LayerW& w, int p) {
  if (e->base_ws) return Operand{SRC_BF16_K, w.wbt[p], nullptr, e->Out[p]};
  if (e->frag) return w.fqt[p];
  if (e->lora && e->bf) {
    const QuantPlanes& q = w.qt[p];
    return Operand{q.kind == SMHIP_QTYPE_Q8_0 ? SRC_Q8T : SRC_Q4KT, q.qs, q.sc, e->Out[p]};
  }
  if (e->lora) {
    const QuantPlanes& q = w.q[p];
    return Operand{q.kind == SMHIP_QTYPE_Q8_0 ? SRC_Q8_R : SRC_Q4K_R, q.qs, q.sc, e->In[p]};
  }
  return w.w[p].bf ? Operand{SRC_BF16_R, w.w[p].bf, nullptr, e->In[p]} : Operand{SRC_F32_R, w.w[p].data, nullptr, e->In[p]};
}
static int prec(const Engine* e) { return e->bf ? SMHIP_PREC_BF16 : SMHIP_PREC_FP32; }
static float lora_scale(const Engine* e) { return e->c.lora_alpha / (float)e->c.lora_rank; }

// split-K factor: enough workgroups (2 per CU, the occupancy of the 128x128 tile) for GEMMs
// whose output has few 128x128 tiles, keeping >= 8 K tiles of 64 per split
static int split_for(int M, int N, int K) {
  const int tiles = ceil_div(M, 128) * ceil_div(N, 128);
  const int kt = K / 64;
  if (tiles >= 2 * num_cus() || kt < 16) return 1;
  int s = ceil_div(2 * num_cus(), tiles);
  s = std::min(s, kt / 8);
  return std::max(1, std::min(s, 32));
}

// bf16 engines let the GEMM choose the split (0 = automatic); fp32 (exactness) engines use split_for
static int split_arg(const Engine* e, int M, int N, int K) { return e->bf ? 0 : split_for(M, N, K); }

// LoRA operand: bf16 shadow in bf16 mode, fp32 master otherwise
static Operand lora_op(const Engine* e, const DenseRef& t, bool kmode, int64_t ld) {
  if (e->bf && t.bf) return Operand{kmode ? SRC_BF16_K : SRC_BF16_R, t.bf, nullptr, ld};
  return Operand{kmode ? SRC_F32_K : SRC_F32_R, t.data, nullptr, ld};
}

// y (fp32 or TA) = x W^T [+ s (x A) B] [+ bias] [+ R]
static int proj_forward(Engine* e, int l, int p, const void* x, void* y, int y_bf16, const float* R, hipStream_t s,
                        bool u_ready = false) {
  LayerW& w = e->L[l];
  const int T = e->T, In = e->In[p], Out = e->Out[p];
  GemmArgs g{};
  g.precision = prec(e);
  g.alpha = 1.f;
  g.split_k = 1;
  if (e->lora) {  // u = x A  (saved for dB; u_ready: the RMSNorm producing x computed it)
    const int nr = e->nr[p];
    GemmArgs u{};
    u.precision = prec(e);
    u.alpha = 1.f;
    u.M = T; u.N = nr; u.K = In;
    u.A = act_k(e, x, In);
    u.B = w.lat[p] ? Operand{SRC_BF16_K, w.lat[p], nullptr, In} : lora_op(e, w.la[p], false, nr);
    u.C = e->sv[l].u[p]; u.ldc = nr; u.c_bf16 = e->bf;
    u.split_k = split_arg(e, T, nr, In);
    if (!u_ready)
      if (int rc = gemm(u, s)) return rc;
    g.K2 = nr;
    g.A2 = act_k(e, e->sv[l].u[p], nr);
    g.B2 = lora_op(e, w.lb[p], false, Out);
    g.alpha2 = lora_scale(e);
  }
  g.M = T; g.N = Out; g.K = In;
  g.split_k = split_arg(e, T, Out, In);
  g.A = act_k(e, x, In);
  g.B = w_fwd(e, w, p);
  g.C = y; g.ldc = Out; g.c_bf16 = y_bf16;
  g.bias = (!e->lora && e->c.use_bias) ? w.b[p].data : nullptr;
  g.R = R; g.ldr = Out;
  return gemm(g, s);
}

// dX (fp32 [T, In]) = dY W [+ s z A^T];  grads: dW += dY^T x (full), db, dA, dB (LoRA)
static int proj_backward(Engine* e, int l, int p, const void* dY, const float* dY_f32, const void* x, float* dX,
                         int dX_bf16, void* dX_out, hipStream_t s) {
  LayerW& w = e->L[l];
  const int T = e->T, In = e->In[p], Out = e->Out[p];
  GemmArgs g{};
  g.precision = prec(e);
  g.alpha = 1.f;
  g.split_k = 1;
  if (e->lora) {
    const int nr = e->nr[p];
    const float sc = lora_scale(e);
    // z = dY B^T   [T, nr]
    GemmArgs z{};
    z.precision = prec(e); z.alpha = 1.f;
    z.M = T; z.N = nr; z.K = Out;
    z.A = act_k(e, dY, Out);
    z.B = lora_op(e, w.lb[p], true, Out);
    z.C = e->z; z.ldc = nr; z.c_bf16 = e->bf;
    z.split_k = split_arg(e, T, nr, Out);
    if (int rc = gemm(z, s)) return rc;
    // dB += s u^T dY   [nr, Out]
    GemmArgs gb{};
    gb.precision = prec(e); gb.alpha = sc; gb.beta = 1.f;
    gb.M = nr; gb.N = Out; gb.K = T;
    gb.A = act_r(e, e->sv[l].u[p], nr);
    gb.B = act_r(e, dY, Out);
    gb.C = w.lb[p].grad; gb.ldc = Out;
    gb.split_k = split_arg(e, nr, Out, T);
    gb.defer = &e->skb;
    gb.hold = &e->skh;
    if (e->nblk[p] > 1) {  // fused q|k|v or gate|up: only the diagonal blocks of dB are gradients
      gb.mask_cols = p == P_QKV ? w.lb_cols : w.lb_cols + 3;
      gb.mask_rank = e->c.lora_rank;
      gb.mask_nblk = e->nblk[p];
      gb.masked = &e->lb_masked[p];
    }
    if (int rc = gemm(gb, s)) return rc;
    // dA += s x^T z   [In, nr]
    GemmArgs ga{};
    ga.precision = prec(e); ga.alpha = sc; ga.beta = 1.f;
    ga.M = In; ga.N = nr; ga.K = T;
    ga.A = act_r(e, x, In);
    ga.B = act_r(e, e->z, nr);
    ga.C = w.la[p].grad; ga.ldc = nr;
    ga.split_k = split_arg(e, In, nr, T);
    ga.defer = &e->skb;
    ga.hold = &e->skh;
    if (int rc = gemm(ga, s)) return rc;
    if (int rc = skinny_release(&e->skh, s)) return rc;  // when the two did not pair
    g.K2 = nr;
    g.A2 = act_k(e, e->z, nr);
    g.B2 = lora_op(e, w.la[p], true, nr);
    g.alpha2 = sc;
  } else {
    // dW += dY^T x   [Out, In]
    GemmArgs gw{};
    gw.precision = prec(e); gw.alpha = 1.f; gw.beta = 1.f;
    gw.M = Out; gw.N = In; gw.K = T;
    gw.A = act_r(e, dY, Out);
    gw.B = act_r(e, x, In);
    gw.C = w.w[p].grad; gw.ldc = In;
    gw.split_k = split_arg(e, Out, In, T);
    if (int rc = gemm(gw, s)) return rc;
    if (e->c.use_bias) {
      SMHIP_REQUIRE(dY_f32, "engine: bias gradients need fp32 activations");
      if (int rc = colsum_add(dY_f32, w.b[p].grad, T, Out, s)) return rc;
    }
  }
  g.M = T; g.N = In; g.K = Out;
  g.split_k = split_arg(e, T, In, Out);
  g.A = act_k(e, dY, Out);
  g.B = w_bwd(e, w, p);
  if (e->lora) g.prof_cat = PROF_GEMM_DX;
  g.C = dX_out ? dX_out : (void*)dX; g.ldc = In; g.c_bf16 = dX_bf16;
  return gemm(g, s);
}

// attention's V: in place inside the bf16 q|k|v projection output (row pitch nqkv), else the
// separate copy the QK-norm/RoPE pass writes
static const uint16_t* vsrc(const Engine* e, const Saved& sv) {
  return e->qkv_bf ? (const uint16_t*)sv.qkv + e->qd + e->kvd : (const uint16_t*)sv.v;
}
static int64_t vld(const Engine* e) { return e->qkv_bf ? e->nqkv : e->kvd; }

// ------------------------------------------------------------------ step
static int forward_backward(Engine* e, const int32_t* ids, const int32_t* labels, hipStream_t s) {
  const smhip_model_config& c = e->c;
  const int T = e->T, d = c.d_model, F = c.ffn_dim, V = c.vocab, Hq = c.n_heads, Hkv = c.n_kv_heads, D = c.head_dim;
  int rc;
#define R_(x) do { if ((rc = (x))) return rc; } while (0)
  // gradients accumulate (+=) into the arena; the caller zeroes it at the start of an
  // accumulation window (optimizer.ZeroGrad, TrainLoop.cs:108-109)

  // decode the frozen base into the bf16 workspace (both layouts), all matrices in one launch
  if (e->base_ws) R_(dequant_bf16_many(e->dq_jobs, e->dq_njobs, e->dq_tiles, s));
  // the adapters' A shadows (rewritten by every optimizer step and parameter load) transposed
  if (e->lat_jobs) R_(transpose_bf16_jobs(e->lat_jobs, e->lat_njobs, e->lat_max, s));

  // ---------------- forward
  if (e->lora) {
    // embedding rows are gathered from the frozen quantised table: dequantise the needed rows
    // (row t of E lives at flat elements ids[t]*d ...): gather via GEMM-free dequant path
    R_(dequant_rows(e->emb_q, ids, e->sv[0].h_in, T, d, s));
  } else {
    R_(embedding_forward(e->emb.data, ids, e->sv[0].h_in, T, d, s));
  }
  for (int l = 0; l < c.n_layers; l++) {
    Saved& sv = e->sv[l];
    LayerW& w = e->L[l];
    float* h_out = (l + 1 < c.n_layers) ? e->sv[l + 1].h_in : e->h_fin;
    // bf16 LoRA: the RMSNorm also computes the qkv adapters' u = xn A (rows already in registers)
    int fused = 0;
    if (e->lora && e->bf && w.lat[P_QKV]) {
      fused = rmsnorm_lora_u(sv.h_in, w.norm1.data, c.norm_eps, (uint16_t*)sv.xn1, sv.rinv1, w.lat[P_QKV],
                             e->nr[P_QKV], (uint16_t*)sv.u[P_QKV], T, d, s);
      if (fused < 0) return fused;
    }
    if (!fused)
      R_(rmsnorm_forward(sv.h_in, w.norm1.data, e->bf ? nullptr : (float*)sv.xn1, e->bf ? (uint16_t*)sv.xn1 : nullptr,
                         sv.rinv1, T, d, c.norm_eps, s));
    R_(proj_forward(e, l, P_QKV, sv.xn1, sv.qkv, e->qkv_bf, nullptr, s, fused == 1));
    // bf16 q|k|v projections: attention reads V in place (row pitch nqkv), no copy
    R_(qkv_prep_forward(sv.qkv, e->qkv_bf, sv.q, sv.k, e->qkv_bf ? nullptr : sv.v, sv.rinv_qk, c.qk_norm ? w.qn.data : nullptr,
                        c.qk_norm ? w.kn.data : nullptr, e->cosT, e->sinT, T, c.seq, Hq, Hkv, D, c.qk_norm,
                        c.rope_neox, c.norm_eps, e->bf, s));
    if (e->bf) {
      R_(flash_forward((const uint16_t*)sv.q, (const uint16_t*)sv.k, vsrc(e, sv), (uint16_t*)sv.o, sv.lse, c.batch,
                       c.seq, Hq, Hkv, D, e->qd, e->kvd, vld(e), e->qd, s));
    } else {
      R_(attention_forward_probs((const float*)sv.q, (const float*)sv.k, (const float*)sv.v, sv.probs, (float*)sv.o,
                                 c.batch, c.seq, Hq, Hkv, D, s));
    }
    R_(proj_forward(e, l, P_O, sv.o, sv.h_mid, 0, sv.h_in, s));  // h_mid = h_in + attn
    fused = 0;
    if (e->lora && e->bf && w.lat[P_GU]) {
      fused = rmsnorm_lora_u(sv.h_mid, w.norm2.data, c.norm_eps, (uint16_t*)sv.xn2, sv.rinv2, w.lat[P_GU],
                             e->nr[P_GU], (uint16_t*)sv.u[P_GU], T, d, s);
      if (fused < 0) return fused;
    }
    if (!fused)
      R_(rmsnorm_forward(sv.h_mid, w.norm2.data, e->bf ? nullptr : (float*)sv.xn2, e->bf ? (uint16_t*)sv.xn2 : nullptr,
                         sv.rinv2, T, d, c.norm_eps, s));
    R_(proj_forward(e, l, P_GU, sv.xn2, sv.gu, e->bf, nullptr, s, fused == 1));
    // bf16 LoRA: the SwiGLU also computes the down adapter's u = act A
    fused = 0;
    if (e->lora && e->bf && w.lat[P_D]) {
      fused = swiglu_lora_u((const uint16_t*)sv.gu, (uint16_t*)sv.act, w.lat[P_D], e->nr[P_D], (uint16_t*)sv.u[P_D], T,
                            F, s);
      if (fused < 0) return fused;
    }
    if (!fused) R_(swiglu_fused_forward(sv.gu, sv.act, T, F, e->bf, s));
    R_(proj_forward(e, l, P_D, sv.act, h_out, 0, sv.h_mid, s, fused == 1));  // h_out = h_mid + ffn
  }
  R_(rmsnorm_forward(e->h_fin, e->norm_f.data, e->bf ? nullptr : (float*)e->xnf, e->bf ? (uint16_t*)e->xnf : nullptr,
                     e->rinv_f, T, d, c.norm_eps, s));
  {  // tied LM head (BackpropEngine.cs:889-907)
    GemmArgs g{};
    g.precision = prec(e); g.alpha = 1.f; g.split_k = 1;
    g.M = T; g.N = V; g.K = d;
    g.A = act_k(e, e->xnf, d);
    if (e->base_ws) g.B = Operand{SRC_BF16_K, e->emb_b, nullptr, d};
    else if (e->frag) g.B = e->emb_fq;
    else if (e->lora) g.B = Operand{e->emb_q.kind == SMHIP_QTYPE_Q8_0 ? SRC_Q8_K : SRC_Q4K_K, e->emb_q.qs, e->emb_q.sc, d};
    else g.B = e->emb.bf ? Operand{SRC_BF16_K, e->emb.bf, nullptr, d} : Operand{SRC_F32_K, e->emb.data, nullptr, d};
    g.C = e->logits; g.ldc = V;
    g.rowstat = e->rowstat;
    R_(gemm(g, s));
  }
  // loss + dLogits (CrossEntropyLoss.Compute / Backward, TrainLoop.cs:233-237)
  if (e->rowstat) R_(ce_softmax_grad_bf16_stats(e->logits, e->rowstat, V / 64, labels, (uint16_t*)e->dlogits, e->loss, T, V, -100, s));
  else if (e->bf) R_(ce_softmax_grad_bf16(e->logits, labels, (uint16_t*)e->dlogits, e->loss, T, V, -100, 0.f, s));
  else R_(ce_softmax_grad(e->logits, labels, (float*)e->dlogits, e->loss, T, V, -100, 0.f, s));

  // ---------------- backward
  {  // head: dxnf = dLogits E ; dE += dLogits^T xnf (full)
    GemmArgs g{};
    g.precision = prec(e); g.alpha = 1.f; g.split_k = 1;
    g.M = T; g.N = d; g.K = V;
    g.A = act_k(e, e->dlogits, V);
    if (e->base_ws) g.B = Operand{SRC_BF16_K, e->emb_bt, nullptr, V};
    else if (e->frag) g.B = e->emb_fqt;
    else if (e->lora && e->bf) g.B = Operand{e->emb_qt.kind == SMHIP_QTYPE_Q8_0 ? SRC_Q8T : SRC_Q4KT, e->emb_qt.qs, e->emb_qt.sc, V};
    else if (e->lora) g.B = Operand{e->emb_q.kind == SMHIP_QTYPE_Q8_0 ? SRC_Q8_R : SRC_Q4K_R, e->emb_q.qs, e->emb_q.sc, d};
    else g.B = e->emb.bf ? Operand{SRC_BF16_R, e->emb.bf, nullptr, d} : Operand{SRC_F32_R, e->emb.data, nullptr, d};
    g.C = e->dx; g.ldc = d;
    g.split_k = split_arg(e, T, d, V);
    if (e->lora) g.prof_cat = PROF_GEMM_DX;
    R_(gemm(g, s));
    if (!e->lora) {
      GemmArgs gw{};
      gw.precision = prec(e); gw.alpha = 1.f; gw.beta = 1.f;
      gw.M = V; gw.N = d; gw.K = T;
      gw.A = act_r(e, e->dlogits, V);
      gw.B = act_r(e, e->xnf, d);
      gw.C = e->emb.grad; gw.ldc = d;
      gw.split_k = split_arg(e, V, d, T);
      R_(gemm(gw, s));
    }
  }
  // final norm (BackpropEngine.cs:168)
  R_(rmsnorm_backward(e->dx, e->h_fin, 1, e->rinv_f, e->norm_f.data, e->norm_f.grad, e->dh, T, d, 0,
                      e->bf ? (uint16_t*)e->dh_ta : nullptr, s));
  for (int l = c.n_layers - 1; l >= 0; l--) {
    Saved& sv = e->sv[l];
    LayerW& w = e->L[l];
    // FfnBackward (BackpropEngine.cs:623-657)
    if (e->bf) R_(proj_backward(e, l, P_D, e->dh_ta, e->dh, sv.act, nullptr, 1, e->dact, s));
    else R_(proj_backward(e, l, P_D, e->dh_ta, e->dh, sv.act, (float*)e->dact, 0, nullptr, s));
    R_(swiglu_fused_backward(e->dact, sv.gu, e->dgu, T, F, e->bf, s));
    R_(proj_backward(e, l, P_GU, e->dgu, e->bf ? nullptr : (float*)e->dgu, sv.xn2, e->dx, 0, nullptr, s));
    // norm2 backward, residual add into dh (BackpropEngine.cs:521-526)
    R_(rmsnorm_backward(e->dx, sv.h_mid, 1, sv.rinv2, w.norm2.data, w.norm2.grad, e->dh, T, d, 1,
                        e->bf ? (uint16_t*)e->dh_ta : nullptr, s));
    // AttentionBackward (BackpropEngine.cs:539-602)
    R_(proj_backward(e, l, P_O, e->dh_ta, e->dh, sv.o, nullptr, e->bf, e->dO, s));
    const void *dk = e->dk, *dv = e->dv;
    int kv_grp = 0;
    if (e->bf) {
      // dK / dV stay per query head; the QK-norm / RoPE backward sums each GQA group as it reads
      // them.  dQ and the partials are bf16: their one consumer rounds its output to bf16.
      R_(flash_backward((const uint16_t*)sv.q, (const uint16_t*)sv.k, vsrc(e, sv), (const uint16_t*)sv.o,
                        (const uint16_t*)e->dO, sv.lse, e->dq, nullptr, nullptr, c.batch, c.seq, Hq, Hkv, D, e->qd,
                        e->kvd, vld(e), e->qd, e->qd, e->qd, e->kvd, e->kvd, e->flash_ws, s, 1));
      flash_backward_partials(e->flash_ws, c.batch, c.seq, Hq, D, &dk, &dv);
      kv_grp = Hq / Hkv;
    } else {
      R_(attention_probs_backward((const float*)e->dO, (const float*)sv.q, (const float*)sv.k, (const float*)sv.v,
                                  sv.probs, e->dq, e->dk, e->dv, c.batch, c.seq, Hq, Hkv, D, s));
    }
    R_(qkv_prep_backward(e->dq, dk, dv, e->bf, sv.qkv, e->qkv_bf, sv.rinv_qk, c.qk_norm ? w.qn.data : nullptr,
                         c.qk_norm ? w.kn.data : nullptr, c.qk_norm ? w.qn.grad : nullptr,
                         c.qk_norm ? w.kn.grad : nullptr, e->cosT, e->sinT, e->dqkv, T, c.seq, Hq, Hkv, D,
                         c.qk_norm, c.rope_neox, e->bf, kv_grp, s));
    R_(proj_backward(e, l, P_QKV, e->dqkv, e->bf ? nullptr : (float*)e->dqkv, sv.xn1, e->dx, 0, nullptr, s));
    R_(rmsnorm_backward(e->dx, sv.h_in, 1, sv.rinv1, w.norm1.data, w.norm1.grad, e->dh, T, d, 1,
                        e->bf ? (uint16_t*)e->dh_ta : nullptr, s));
    if (e->lora) {
      // the layer's adapter gradients: queued split reductions, then the off-diagonal blocks
      // of the fused B gradients back to zero
      R_(skinny_flush(&e->skb, s));
      const int nrq = e->nr[P_QKV], nrg = e->nr[P_GU];
      // (skipped where the rank-sized dB product already left those blocks untouched)
      if (!e->lb_masked[P_QKV]) R_(lora_mask(w.lb[P_QKV].grad, nrq, c.lora_rank, e->Out[P_QKV], w.lb_cols, 3, s));
      if (!e->lb_masked[P_GU]) R_(lora_mask(w.lb[P_GU].grad, nrg, c.lora_rank, e->Out[P_GU], w.lb_cols + 3, 2, s));
    }
  }
  if (!e->lora) R_(embedding_backward(e->dh, ids, e->emb.grad, T, d, V, s));  // BackpropEngine.cs:203-205
#undef R_
  return SMHIP_OK;
}

static int optimizer_step(Engine* e, hipStream_t s) {
  const smhip_model_config& c = e->c;
  int rc;
  e->step++;
  // TrainLoop.cs:125-127 -> Gradients.ClipGlobalNorm: the norm here, the scaling inside the AdamW
  // pass (which also refreshes the bf16 shadows of bf16 engines)
  const bool clip = c.max_grad_norm > 0.f;
  if (clip && (rc = l2normsq(e->grad, e->n_train, e->gnorm, 0, s))) return rc;
  const float* nsq = clip ? e->gnorm : nullptr;
  // AdamW.Update (AdamW.cs:52-89): bc_i = 1 - beta_i^t ; decayed tensors first, then no-decay
  const float bc1 = 1.f - powf(c.beta1, (float)e->step), bc2 = 1.f - powf(c.beta2, (float)e->step);
  if ((rc = adamw_update(e->train, e->grad, e->m, e->v, e->n_decay, c.beta1, c.beta2, bc1, bc2, c.lr, c.adam_eps,
                         c.weight_decay, s, e->train_bf, nsq, c.max_grad_norm)))
    return rc;
  if (e->n_train > e->n_decay)
    if ((rc = adamw_update(e->train + e->n_decay, e->grad + e->n_decay, e->m + e->n_decay, e->v + e->n_decay,
                           e->n_train - e->n_decay, c.beta1, c.beta2, bc1, bc2, c.lr, c.adam_eps, 0.f, s,
                           e->train_bf ? e->train_bf + e->n_decay : nullptr, nsq, c.max_grad_norm)))
      return rc;
  return SMHIP_OK;
}

}  // namespace smhip


// ------------------------------------------------------------------ checkpoint files
// Checkpoint.Save / Load / ReadMeta / FindLatest (SharpMind.Training/Checkpoint.cs:27-82,
// 90-237) and AdamW.SaveState / LoadState (Optimizers/AdamW.cs:96-117), byte-compatible:
//   model.bin      int32 count; per tensor: int32 name length, UTF-8 name, int32 rank,
//                  int32 dims[rank], fp32 data (little endian, the reference's row-major
//                  [In, Out] layout for linear weights)
//   optimizer.bin  int32 AdamW step, fp32 lr; per tensor, in the same order: m, then v
//   meta.json      {"step", "loss" (null when NaN), "note", "savedUtc", "paramCount"}
// The tensor list is the reference's trainable parameter list:
//   full-parameter: Transformer.Parameters (Transformer.cs:239-260): EmbeddingTable.weight,
//     then per block (TransformerBlock.cs:52-66) attention q_proj, k_proj, v_proj, o_proj
//     (.weight [In, Out], .bias [Out] when biased; AttentionLayer.cs:425-433), the QK-norm
//     weights (RmsNormLayer.weight [head_dim]), wgated_proj and down_proj (FFnLayer.cs:317-327),
//     norm1, norm2 (RmsNormLayer.weight [d]), and last the final RmsNormLayer.weight;
//   LoRA: per block, the adapters of q, k, v, o, gate, up, down, each lora.a [In, r] then
//     lora.b [r, Out] (LoRALayer.cs:94-98, in LoRAAttention / LoRAFFN order).  The reference's
//     LoRAModel holds one such set for the whole model; the engine has one per block.
// Repeated names (RmsNormLayer.weight, lora.a, lora.b) are matched in order, as Load does.
namespace smhip {

// geometry of block blk of fused projection p: (In, Out, column offset in the fused output)
static void block_geom(const Engine* e, int p, int blk, int* In, int* Out, int* coff) {
  *In = e->In[p];
  if (p == P_QKV) { const int o[3] = {0, e->qd, e->qd + e->kvd}, n[3] = {e->qd, e->kvd, e->kvd}; *Out = n[blk]; *coff = o[blk]; }
  else if (p == P_GU) { *Out = e->c.ffn_dim; *coff = blk * e->c.ffn_dim; }
  else { *Out = e->Out[p]; *coff = 0; }
}

struct RefParam {
  std::string name;
  std::vector<int> dims;
  const DenseRef* d;
  // element (i, j) of the reference [R][C] tensor is storage[base + i * si + j * sj]
  int64_t base, si, sj;
  int R, C;
};

static std::vector<RefParam> ref_params(const Engine* e) {
  std::vector<RefParam> v;
  const smhip_model_config& c = e->c;
  const int d = c.d_model, F = c.ffn_dim, r = c.lora_rank;
  auto vec = [&](const char* name, const DenseRef* t, int64_t base, int n) {
    v.push_back({name, {n}, t, base, 0, 1, 1, n});
  };
  // reference [In, Out] weight = rows [off, off + Out) of an engine [Out_all][In] matrix
  auto lin = [&](const char* name, const DenseRef* t, int In, int Out, int off) {
    v.push_back({name, {In, Out}, t, (int64_t)off * In, 1, In, In, Out});
  };
  if (!e->lora) {
    v.push_back({"EmbeddingTable.weight", {c.vocab, d}, &e->emb, 0, d, 1, c.vocab, d});
    for (const LayerW& w : e->L) {
      const char* qkv[3] = {"q_proj", "k_proj", "v_proj"};
      const int off[3] = {0, e->qd, e->qd + e->kvd}, outs[3] = {e->qd, e->kvd, e->kvd};
      for (int j = 0; j < 3; j++) {
        lin((std::string(qkv[j]) + ".weight").c_str(), &w.w[P_QKV], d, outs[j], off[j]);
        if (c.use_bias) vec((std::string(qkv[j]) + ".bias").c_str(), &w.b[P_QKV], off[j], outs[j]);
      }
      lin("o_proj.weight", &w.w[P_O], e->qd, d, 0);
      if (c.use_bias) vec("o_proj.bias", &w.b[P_O], 0, d);
      if (c.qk_norm) {
        vec("RmsNormLayer.weight", &w.qn, 0, c.head_dim);
        vec("RmsNormLayer.weight", &w.kn, 0, c.head_dim);
      }
      lin("wgated_proj.weight", &w.w[P_GU], d, 2 * F, 0);
      if (c.use_bias) vec("wgated_proj.bias", &w.b[P_GU], 0, 2 * F);
      lin("down_proj.weight", &w.w[P_D], F, d, 0);
      if (c.use_bias) vec("down_proj.bias", &w.b[P_D], 0, d);
      vec("RmsNormLayer.weight", &w.norm1, 0, d);
      vec("RmsNormLayer.weight", &w.norm2, 0, d);
    }
    vec("RmsNormLayer.weight", &e->norm_f, 0, d);
    return v;
  }
  static const int proj[7] = {P_QKV, P_QKV, P_QKV, P_O, P_GU, P_GU, P_D};
  static const int blk[7] = {0, 1, 2, 0, 0, 1, 0};
  for (const LayerW& w : e->L)
    for (int t = 0; t < 7; t++) {
      const int p = proj[t];
      int In, Out, coff;
      block_geom(e, p, blk[t], &In, &Out, &coff);
      const int nr = e->nr[p], OutF = e->Out[p];
      // A [In][nr] fused by columns; B [nr][Out_fused] block-diagonal
      v.push_back({"lora.a", {In, r}, &w.la[p], (int64_t)blk[t] * r, nr, 1, In, r});
      v.push_back({"lora.b", {r, Out}, &w.lb[p], (int64_t)blk[t] * r * OutF + coff, OutF, 1, r, Out});
    }
  return v;
}

// host copies of the parameter, m and v arenas
struct ArenaCopy {
  std::vector<float> a[3];
  int get(const Engine* e) {
    for (int k = 0; k < 3; k++) {
      a[k].resize((size_t)std::max<int64_t>(e->n_train, 1));
      const float* src = k == 0 ? e->train : (k == 1 ? e->m : e->v);
      SMHIP_CHECK_HIP(hipMemcpy(a[k].data(), src, sizeof(float) * (size_t)e->n_train, hipMemcpyDeviceToHost));
    }
    return SMHIP_OK;
  }
  int put(Engine* e) const {
    for (int k = 0; k < 3; k++) {
      float* dst = k == 0 ? e->train : (k == 1 ? e->m : e->v);
      SMHIP_CHECK_HIP(hipMemcpy(dst, a[k].data(), sizeof(float) * (size_t)e->n_train, hipMemcpyHostToDevice));
    }
    return SMHIP_OK;
  }
};

static void gather(const Engine* e, const ArenaCopy& ac, int k, const RefParam& p, float* out) {
  const float* st = ac.a[k].data() + (p.d->data - e->train);
  for (int i = 0; i < p.R; i++)
    for (int j = 0; j < p.C; j++) out[(int64_t)i * p.C + j] = st[p.base + i * p.si + j * p.sj];
}
static void scatter(const Engine* e, ArenaCopy& ac, int k, const RefParam& p, const float* in) {
  float* st = ac.a[k].data() + (p.d->data - e->train);
  for (int i = 0; i < p.R; i++)
    for (int j = 0; j < p.C; j++) st[p.base + i * p.si + j * p.sj] = in[(int64_t)i * p.C + j];
}

static std::string json_escape(const std::string& x) {
  std::string o;
  for (unsigned char ch : x) {
    if (ch == '"') o += "\\\"";
    else if (ch == '\\') o += "\\\\";
    else if (ch == '\n') o += "\\n";
    else if (ch == '\r') o += "\\r";
    else if (ch == '\t') o += "\\t";
    else if (ch < 0x20) { char b[8]; snprintf(b, sizeof b, "\\u%04x", ch); o += b; }
    else o += (char)ch;
  }
  return o;
}
// shortest decimal that reads back as the same float
static std::string float_repr(float f) {
  char b[64];
  for (int prec = 1; prec <= 9; prec++) {
    snprintf(b, sizeof b, "%.*g", prec, (double)f);
    if (strtof(b, nullptr) == f) break;
  }
  return b;
}

struct FileCloser { void operator()(FILE* f) const { if (f) fclose(f); } };
using File = std::unique_ptr<FILE, FileCloser>;

static int save_checkpoint(Engine* e, const std::string& dir, int step, float loss, const char* note, bool with_opt) {
  std::error_code ec;
  std::filesystem::create_directories(dir, ec);
  if (ec) return fail(SMHIP_EINVAL, "checkpoint: cannot create directory " + dir + ": " + ec.message());
  SMHIP_CHECK_HIP(hipDeviceSynchronize());
  const std::vector<RefParam> ps = ref_params(e);
  ArenaCopy ac;
  if (int rc = ac.get(e)) return rc;
  std::vector<float> buf;
  {
    File f(fopen((dir + "/model.bin").c_str(), "wb"));
    if (!f) return fail(SMHIP_EINVAL, "checkpoint: cannot write " + dir + "/model.bin");
    bool ok = true;
    auto w32 = [&](int32_t x) { ok = ok && fwrite(&x, 4, 1, f.get()) == 1; };
    w32((int32_t)ps.size());
    for (const RefParam& p : ps) {
      w32((int32_t)p.name.size());
      ok = ok && fwrite(p.name.data(), 1, p.name.size(), f.get()) == p.name.size();
      w32((int32_t)p.dims.size());
      for (int dd : p.dims) w32(dd);
      buf.resize((size_t)p.R * p.C);
      gather(e, ac, 0, p, buf.data());
      ok = ok && fwrite(buf.data(), 4, buf.size(), f.get()) == buf.size();
    }
    if (!ok) return fail(SMHIP_EINVAL, "checkpoint: short write to model.bin");
  }
  if (with_opt) {
    File f(fopen((dir + "/optimizer.bin").c_str(), "wb"));
    if (!f) return fail(SMHIP_EINVAL, "checkpoint: cannot write " + dir + "/optimizer.bin");
    const int32_t st = e->step;
    const float lr = e->c.lr;
    bool ok = fwrite(&st, 4, 1, f.get()) == 1 && fwrite(&lr, 4, 1, f.get()) == 1;
    for (const RefParam& p : ps)
      for (int k = 1; k <= 2; k++) {
        buf.resize((size_t)p.R * p.C);
        gather(e, ac, k, p, buf.data());
        ok = ok && fwrite(buf.data(), 4, buf.size(), f.get()) == buf.size();
      }
    if (!ok) return fail(SMHIP_EINVAL, "checkpoint: short write to optimizer.bin");
  }
  {
    // DateTime.UtcNow.ToString("o"): yyyy-MM-ddTHH:mm:ss.fffffffZ
    const auto now = std::chrono::system_clock::now();
    const auto us = std::chrono::duration_cast<std::chrono::microseconds>(now.time_since_epoch()).count();
    const time_t secs = (time_t)(us / 1000000);
    struct tm tmv;
    gmtime_r(&secs, &tmv);
    char ts[64];
    snprintf(ts, sizeof ts, "%04d-%02d-%02dT%02d:%02d:%02d.%07lldZ", tmv.tm_year + 1900, tmv.tm_mon + 1, tmv.tm_mday,
             tmv.tm_hour, tmv.tm_min, tmv.tm_sec, (long long)(us % 1000000) * 10);
    std::string js = "{\n";
    js += "  \"step\": " + std::to_string(step) + ",\n";
    js += "  \"loss\": " + (std::isnan(loss) ? std::string("null") : float_repr(loss)) + ",\n";
    js += "  \"note\": " + (note ? "\"" + json_escape(note) + "\"" : std::string("null")) + ",\n";
    js += std::string("  \"savedUtc\": \"") + ts + "\",\n";
    js += "  \"paramCount\": " + std::to_string(ps.size()) + "\n}";
    File f(fopen((dir + "/meta.json").c_str(), "wb"));
    if (!f || fwrite(js.data(), 1, js.size(), f.get()) != js.size())
      return fail(SMHIP_EINVAL, "checkpoint: cannot write " + dir + "/meta.json");
  }
  return SMHIP_OK;
}

// the "step" and "loss" members of meta.json (ReadMeta: absent file -> step 0, loss NaN)
static void read_meta(const std::string& dir, int* step, float* loss) {
  *step = 0;
  *loss = NAN;
  File f(fopen((dir + "/meta.json").c_str(), "rb"));
  if (!f) return;
  std::string js;
  char b[4096];
  size_t n;
  while ((n = fread(b, 1, sizeof b, f.get())) > 0) js.append(b, n);
  auto member = [&](const char* key) -> const char* {
    const std::string k = std::string("\"") + key + "\"";
    size_t at = js.find(k);
    if (at == std::string::npos) return nullptr;
    at = js.find(':', at + k.size());
    if (at == std::string::npos) return nullptr;
    const char* p = js.c_str() + at + 1;
    while (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t') p++;
    return p;
  };
  if (const char* p = member("step")) *step = (int)strtol(p, nullptr, 10);
  if (const char* p = member("loss")) {
    if (strncmp(p, "null", 4) != 0) *loss = strtof(p, nullptr);
  }
}

// A tensor whose element count differs from the parameter's fails the load before anything
// reaches the device (the reference has by then overwritten the earlier parameters in place).
static int load_checkpoint(Engine* e, const std::string& dir, bool with_opt, int* step_out, float* loss_out) {
  std::error_code ec;
  if (!std::filesystem::is_directory(dir, ec))
    return fail(SMHIP_EINVAL, "checkpoint: directory not found: " + dir);
  File f(fopen((dir + "/model.bin").c_str(), "rb"));
  if (!f) return fail(SMHIP_EINVAL, "checkpoint: model.bin not found in " + dir);
  SMHIP_CHECK_HIP(hipDeviceSynchronize());
  const std::vector<RefParam> ps = ref_params(e);
  std::map<std::string, std::vector<int>> queue;  // name -> FIFO of parameter indices
  for (int i = (int)ps.size() - 1; i >= 0; i--) queue[ps[i].name].push_back(i);
  ArenaCopy ac;
  if (int rc = ac.get(e)) return rc;
  auto r32 = [&](int32_t* x) { return fread(x, 4, 1, f.get()) == 1; };
  int32_t count = 0;
  if (!r32(&count) || count < 0) return fail(SMHIP_EINVAL, "checkpoint: truncated model.bin");
  std::vector<float> buf;
  for (int32_t t = 0; t < count; t++) {
    int32_t len = 0, rank = 0;
    if (!r32(&len) || len < 0 || len > (1 << 20)) return fail(SMHIP_EINVAL, "checkpoint: bad tensor name in model.bin");
    std::string name((size_t)len, '\0');
    if (fread(name.data(), 1, (size_t)len, f.get()) != (size_t)len || !r32(&rank) || rank < 0 || rank > 16)
      return fail(SMHIP_EINVAL, "checkpoint: truncated model.bin");
    int64_t elems = 1;
    for (int k = 0; k < rank; k++) {
      int32_t dd = 0;
      if (!r32(&dd)) return fail(SMHIP_EINVAL, "checkpoint: truncated model.bin");
      elems *= dd;
    }
    auto it = queue.find(name);
    if (it == queue.end() || it->second.empty()) {  // not a parameter of this model: skip
      if (fseeko(f.get(), (off_t)elems * 4, SEEK_CUR) != 0) return fail(SMHIP_EINVAL, "checkpoint: truncated model.bin");
      continue;
    }
    const RefParam& p = ps[it->second.back()];
    it->second.pop_back();
    const int64_t have = (int64_t)p.R * p.C;
    if (elems != have)
      return fail(SMHIP_EINVAL, "Checkpoint tensor '" + name + "' has " + std::to_string(elems) +
                                    " elements but the model parameter '" + p.name + "' has " + std::to_string(have) + ".");
    buf.resize((size_t)have);
    if (fread(buf.data(), 4, buf.size(), f.get()) != buf.size()) return fail(SMHIP_EINVAL, "checkpoint: truncated model.bin");
    scatter(e, ac, 0, p, buf.data());
  }
  int step = 0;
  float loss = NAN;
  read_meta(dir, &step, &loss);
  File fo(with_opt ? fopen((dir + "/optimizer.bin").c_str(), "rb") : nullptr);
  if (fo) {  // LoadState: stored step skipped, the meta step is authoritative
    int32_t st;
    float lr;
    if (fread(&st, 4, 1, fo.get()) != 1 || fread(&lr, 4, 1, fo.get()) != 1)
      return fail(SMHIP_EINVAL, "checkpoint: truncated optimizer.bin");
    for (const RefParam& p : ps)
      for (int k = 1; k <= 2; k++) {
        buf.resize((size_t)p.R * p.C);
        if (fread(buf.data(), 4, buf.size(), fo.get()) != buf.size())
          return fail(SMHIP_EINVAL, "checkpoint: truncated optimizer.bin");
        scatter(e, ac, k, p, buf.data());
      }
    e->c.lr = lr;
    e->step = step;
  }
  if (int rc = ac.put(e)) return rc;
  if (e->train_bf)
    if (int rc = cast_bf16(e->train, e->train_bf, e->n_train, nullptr)) return rc;
  SMHIP_CHECK_HIP(hipDeviceSynchronize());
  if (step_out) *step_out = step;
  if (loss_out) *loss_out = loss;
  return SMHIP_OK;
}

}  // namespace smhip

using namespace smhip;

extern "C" {

int smhip_engine_create(const smhip_model_config* cfg, void** out) {
  SMHIP_REQUIRE(cfg && out, "engine_create: null argument");
  const smhip_model_config& c = *cfg;
  SMHIP_REQUIRE(c.n_layers > 0 && c.d_model > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.head_dim > 0 &&
                    c.ffn_dim > 0 && c.vocab > 0 && c.batch > 0 && c.seq > 0,
                "engine_create: non-positive dimension");
  SMHIP_REQUIRE(c.n_heads % c.n_kv_heads == 0, "engine_create: n_heads must be a multiple of n_kv_heads");
  SMHIP_REQUIRE(c.head_dim % 2 == 0 && c.head_dim <= 128, "engine_create: head_dim must be even and <= 128");
  SMHIP_REQUIRE(c.precision == SMHIP_PREC_FP32 || c.precision == SMHIP_PREC_BF16, "engine_create: bad precision");
  if (c.precision == SMHIP_PREC_BF16) {
    SMHIP_REQUIRE(c.seq % 128 == 0 && (c.head_dim == 64 || c.head_dim == 128),
                  "engine_create: bf16 mode needs seq % 128 == 0 and head_dim 64 or 128 (flash attention)");
    SMHIP_REQUIRE(!c.use_bias, "engine_create: biases are supported in fp32 mode only");
  }
  if (c.lora_rank > 0) {
    SMHIP_REQUIRE(c.base_qtype == SMHIP_QTYPE_Q8_0 || c.base_qtype == SMHIP_QTYPE_Q4_K,
                  "engine_create: LoRA needs a Q8_0 or Q4_K base");
    SMHIP_REQUIRE(!c.use_bias, "engine_create: LoRA bases are bias-free");
    SMHIP_REQUIRE(c.d_model % 256 == 0 && c.ffn_dim % 256 == 0 && (c.n_heads * c.head_dim) % 256 == 0,
                  "engine_create: quantised base needs dimensions that are multiples of 256");
  } else {
    SMHIP_REQUIRE(c.base_qtype == SMHIP_QTYPE_F32, "engine_create: full-parameter training needs an F32 base");
  }
  Engine* e = new Engine();
  e->c = c;
  int rc = build(e);
  if (rc) {
    for (void* p : e->allocs) hipFree(p);
    delete e;
    return rc;
  }
  *out = e;
  return SMHIP_OK;
}

int smhip_engine_destroy(void* engine) {
  if (!engine) return SMHIP_OK;
  Engine* e = (Engine*)engine;
  hipDeviceSynchronize();
  if (e->gexec) hipGraphExecDestroy(e->gexec);
  if (e->cap) hipStreamDestroy(e->cap);
  for (void* p : e->allocs) hipFree(p);
  delete e;
  return SMHIP_OK;
}

int smhip_engine_param_count(void* engine, int64_t* trainable, int64_t* frozen) {
  SMHIP_REQUIRE(engine, "engine: null handle");
  Engine* e = (Engine*)engine;
  int64_t tr = e->n_train, fr = e->n_frozen;
  if (e->lora) {  // only diagonal blocks of fused B train
    tr = 0;
    for (int l = 0; l < e->c.n_layers; l++)
      for (int p = 0; p < 4; p++) tr += (int64_t)e->In[p] * e->nr[p] + (int64_t)e->c.lora_rank * e->Out[p];
    fr += (int64_t)e->c.vocab * e->c.d_model;
    for (int p = 0; p < 4; p++) fr += (int64_t)e->c.n_layers * e->In[p] * e->Out[p];
  }
  if (trainable) *trainable = tr;
  if (frozen) *frozen = fr;
  return SMHIP_OK;
}

// storage of a trainable tensor: 0 parameter, 1 gradient, 2 AdamW m, 3 AdamW v (m and v
// arenas are laid out like the parameter arena)
static float* arena_view(const Engine* e, const DenseRef& d, int which) {
  if (which == 0) return d.data;
  if (which == 1) return d.grad;
  if (!d.grad) return nullptr;
  return (which == 2 ? e->m : e->v) + (d.data - e->train);
}

// rebuild the column planes of row planes q (bf16 LoRA engines keep both)
static int refresh_cols(Engine* e, const QuantPlanes* q, hipStream_t s) {
  if (!e->bf || !e->lora || e->base_ws) return SMHIP_OK;
  if (e->frag) {
    auto two = [&](Operand* f, Operand* ft, int rows, int cols) -> int {
      if (int rc = make_frag_planes(*q, rows, cols, 0, const_cast<void*>(f->p), f, s)) return rc;
      return make_frag_planes(*q, rows, cols, 1, const_cast<void*>(ft->p), ft, s);
    };
    if (q == &e->emb_q) return two(&e->emb_fq, &e->emb_fqt, e->c.vocab, e->c.d_model);
    for (auto& w : e->L)
      for (int p = 0; p < 4; p++)
        if (q == &w.q[p]) return two(&w.fq[p], &w.fqt[p], e->Out[p], e->In[p]);
    return fail(SMHIP_EINVAL, "engine: unknown quantised tensor");
  }
  QuantPlanes out;
  if (q == &e->emb_q) return make_col_planes(*q, e->c.vocab, e->c.d_model, e->emb_qt.qs, &out, s);
  for (auto& w : e->L)
    for (int p = 0; p < 4; p++)
      if (q == &w.q[p]) return make_col_planes(*q, e->Out[p], e->In[p], w.qt[p].qs, &out, s);
  return fail(SMHIP_EINVAL, "engine: unknown quantised tensor");
}

static int parse_layer(const char* name, int* layer, std::string* rest) {
  if (name[0] != 'l' || !isdigit((unsigned char)name[1])) return 0;
  const char* dot = strchr(name, '.');
  if (!dot) return 0;
  *layer = atoi(name + 1);
  *rest = dot + 1;
  return 1;
}

// LoRA tensor -> (fused projection, block index)
static int lora_target(const std::string& rest, int* p, int* blk, int* isB) {
  static const char* t[7] = {"q", "k", "v", "o", "gate", "up", "down"};
  static const int proj[7] = {P_QKV, P_QKV, P_QKV, P_O, P_GU, P_GU, P_D};
  static const int bl[7] = {0, 1, 2, 0, 0, 1, 0};
  if (rest.rfind("lora.", 0) != 0) return 0;
  for (int i = 0; i < 7; i++) {
    std::string a = std::string("lora.") + t[i] + ".A", b = std::string("lora.") + t[i] + ".B";
    if (rest == a || rest == b) { *p = proj[i]; *blk = bl[i]; *isB = rest == b; return 1; }
  }
  return 0;
}


int smhip_engine_set_tensor(void* engine, const char* name, const void* host, int64_t nbytes) {
  SMHIP_REQUIRE(engine && name && host, "engine_set_tensor: null argument");
  Engine* e = (Engine*)engine;
  const int r = e->c.lora_rank;
  int layer;
  std::string rest;
  // quantised base (LoRA mode): reference byte layout, repacked once
  if (e->lora) {
    static const char* wn[4] = {"wqkv", "wo", "wgu", "wd"};
    QuantPlanes* q = nullptr;
    if (!strcmp(name, "emb")) q = &e->emb_q;
    else if (parse_layer(name, &layer, &rest) && layer < e->c.n_layers)
      for (int p = 0; p < 4; p++) if (rest == wn[p]) q = &e->L[layer].q[p];
    if (q) {
      const int64_t bpb = q->kind == SMHIP_QTYPE_Q8_0 ? 34 : 144, epb = q->kind == SMHIP_QTYPE_Q8_0 ? 32 : 256;
      SMHIP_REQUIRE(nbytes == q->n / epb * bpb, "engine_set_tensor: quantised byte count does not match the shape");
      void* tmp = nullptr;
      SMHIP_CHECK_HIP(hipMalloc(&tmp, nbytes));
      hipMemcpy(tmp, host, nbytes, hipMemcpyHostToDevice);
      QuantPlanes out;
      int rc = repack_planes(q->kind, tmp, q->n, q->qs, &out, nullptr);
      if (!rc) rc = refresh_cols(e, q, nullptr);
      hipDeviceSynchronize();
      hipFree(tmp);
      return rc;
    }
    int p, blk, isB;
    if (parse_layer(name, &layer, &rest) && layer < e->c.n_layers && lora_target(rest, &p, &blk, &isB)) {
      int In, Out, coff;
      block_geom(e, p, blk, &In, &Out, &coff);
      LayerW& w = e->L[layer];
      if (!isB) {  // A_blk [In, r] -> columns blk*r.. of A [In, nr]
        SMHIP_REQUIRE(nbytes == (int64_t)In * r * 4, "engine_set_tensor: LoRA A size mismatch");
        SMHIP_CHECK_HIP(hipMemcpy2D(w.la[p].data + blk * r, sizeof(float) * e->nr[p], host, sizeof(float) * r,
                                    sizeof(float) * r, In, hipMemcpyHostToDevice));
      } else {  // B_blk [r, Out] -> rows blk*r.., columns coff.. of B [nr, OutF]
        SMHIP_REQUIRE(nbytes == (int64_t)r * Out * 4, "engine_set_tensor: LoRA B size mismatch");
        SMHIP_CHECK_HIP(hipMemcpy2D(w.lb[p].data + (int64_t)blk * r * e->Out[p] + coff, sizeof(float) * e->Out[p], host,
                                    sizeof(float) * Out, sizeof(float) * Out, r, hipMemcpyHostToDevice));
      }
      const DenseRef& t = isB ? w.lb[p] : w.la[p];
      if (t.bf) return cast_bf16(t.data, t.bf, t.n, nullptr);
      return SMHIP_OK;
    }
  }
  auto it = e->dense_by_name.find(name);
  SMHIP_REQUIRE(it != e->dense_by_name.end(), std::string("engine_set_tensor: unknown tensor ") + name);
  DenseRef* d = it->second;
  SMHIP_REQUIRE(nbytes == d->n * 4, std::string("engine_set_tensor: size mismatch for ") + name);
  SMHIP_CHECK_HIP(hipMemcpy(d->data, host, nbytes, hipMemcpyHostToDevice));
  if (d->bf) return cast_bf16(d->data, d->bf, d->n, nullptr);
  return SMHIP_OK;
}

int smhip_engine_get_tensor(void* engine, const char* name, int which, void* host, int64_t nbytes) {
  SMHIP_REQUIRE(engine && name && host, "engine_get_tensor: null argument");
  SMHIP_REQUIRE(which >= 0 && which <= 3, "engine_get_tensor: which must be 0 (parameter), 1 (gradient), 2 (AdamW m), 3 (AdamW v)");
  Engine* e = (Engine*)engine;
  SMHIP_CHECK_HIP(hipDeviceSynchronize());
  const int r = e->c.lora_rank;
  int layer, p, blk, isB;
  std::string rest;
  if (e->lora && parse_layer(name, &layer, &rest) && layer < e->c.n_layers && lora_target(rest, &p, &blk, &isB)) {
    int In, Out, coff;
    block_geom(e, p, blk, &In, &Out, &coff);
    LayerW& w = e->L[layer];
    const DenseRef& dr = isB ? w.lb[p] : w.la[p];
    const float* base = arena_view(e, dr, which);
    if (!isB) {
      SMHIP_REQUIRE(nbytes == (int64_t)In * r * 4, "engine_get_tensor: LoRA A size mismatch");
      SMHIP_CHECK_HIP(hipMemcpy2D(host, sizeof(float) * r, base + blk * r, sizeof(float) * e->nr[p], sizeof(float) * r,
                                  In, hipMemcpyDeviceToHost));
    } else {
      SMHIP_REQUIRE(nbytes == (int64_t)r * Out * 4, "engine_get_tensor: LoRA B size mismatch");
      SMHIP_CHECK_HIP(hipMemcpy2D(host, sizeof(float) * Out, base + (int64_t)blk * r * e->Out[p] + coff,
                                  sizeof(float) * e->Out[p], sizeof(float) * Out, r, hipMemcpyDeviceToHost));
    }
    return SMHIP_OK;
  }
  auto it = e->dense_by_name.find(name);
  SMHIP_REQUIRE(it != e->dense_by_name.end(), std::string("engine_get_tensor: unknown tensor ") + name);
  DenseRef* d = it->second;
  SMHIP_REQUIRE(nbytes == d->n * 4, std::string("engine_get_tensor: size mismatch for ") + name);
  SMHIP_REQUIRE(which == 0 || d->grad, std::string("engine_get_tensor: no gradient or optimizer state for frozen tensor ") + name);
  const float* src = arena_view(e, *d, which);
  SMHIP_CHECK_HIP(hipMemcpy(host, src, nbytes, hipMemcpyDeviceToHost));
  return SMHIP_OK;
}

int smhip_engine_init_synthetic(void* engine, uint64_t seed) {
  SMHIP_REQUIRE(engine, "engine: null handle");
  Engine* e = (Engine*)engine;
  const smhip_model_config& c = e->c;
  hipStream_t s = nullptr;
  int rc;
  uint64_t sd = seed * 1000003ull;
  auto next = [&]() { return ++sd; };
  // norms = 1 (ModelFactory.cs:178-181), biases = 0
  auto ones = [&](DenseRef& d) { return d.n ? fill_normal(d.data, d.n, next(), 1.f, 0.f, s) : 0; };
  if ((rc = ones(e->norm_f))) return rc;
  for (auto& w : e->L) {
    if ((rc = ones(w.norm1)) || (rc = ones(w.norm2))) return rc;
    if (c.qk_norm && ((rc = ones(w.qn)) || (rc = ones(w.kn)))) return rc;
  }
  if (!e->lora) {  // WeightInitializer.InitializeRandomly: N(0, 0.02) (WeightInitializer.cs:23-45)
    if ((rc = fill_normal(e->emb.data, e->emb.n, next(), 0.f, 0.02f, s))) return rc;
    for (auto& w : e->L)
      for (int p = 0; p < 4; p++) {
        if ((rc = fill_normal(w.w[p].data, w.w[p].n, next(), 0.f, 0.02f, s))) return rc;
        if (c.use_bias && (rc = zero_bytes(w.b[p].data, sizeof(float) * w.b[p].n, s))) return rc;
      }
    if (e->train_bf) rc = cast_bf16(e->train, e->train_bf, e->n_train, s);
    return rc ? rc : (hipDeviceSynchronize() == hipSuccess ? SMHIP_OK : fail(SMHIP_EHIP, "init_synthetic"));
  }
  // LoRA: base N(0, 0.02) quantised with the TensorQuantizer encoders, repacked to planes
  int64_t maxn = (int64_t)c.vocab * c.d_model;
  for (int p = 0; p < 4; p++) maxn = std::max<int64_t>(maxn, (int64_t)e->In[p] * e->Out[p]);
  float* tmpf = nullptr;
  void* tmpq = nullptr;
  SMHIP_CHECK_HIP(hipMalloc(&tmpf, sizeof(float) * maxn));
  SMHIP_CHECK_HIP(hipMalloc(&tmpq, (size_t)maxn / 32 * 34 + 256));
  auto quant = [&](QuantPlanes& q) -> int {
    int r2;
    if ((r2 = fill_normal(tmpf, q.n, next(), 0.f, 0.02f, s))) return r2;
    if ((r2 = encode_quant(q.kind, tmpf, q.n, tmpq, s))) return r2;
    QuantPlanes o;
    if ((r2 = repack_planes(q.kind, tmpq, q.n, q.qs, &o, s))) return r2;
    return refresh_cols(e, &q, s);
  };
  rc = quant(e->emb_q);
  for (int l = 0; l < c.n_layers && !rc; l++)
    for (int p = 0; p < 4 && !rc; p++) rc = quant(e->L[l].q[p]);
  hipDeviceSynchronize();
  hipFree(tmpf);
  hipFree(tmpq);
  if (rc) return rc;
  // adapters: A ~ Kaiming-uniform U(-1/sqrt(In), 1/sqrt(In)), B = 0 then + N(0, 1e-3), off-diagonal blocks 0
  for (auto& w : e->L)
    for (int p = 0; p < 4; p++) {
      const float bound = 1.f / sqrtf((float)e->In[p]);
      if ((rc = fill_uniform(w.la[p].data, w.la[p].n, next(), -bound, bound, s))) return rc;
      if ((rc = fill_normal(w.lb[p].data, w.lb[p].n, next(), 0.f, 1e-3f, s))) return rc;
      if (e->nblk[p] > 1)
        if ((rc = lora_mask(w.lb[p].data, e->nr[p], c.lora_rank, e->Out[p], p == P_QKV ? w.lb_cols : w.lb_cols + 3,
                            p == P_QKV ? 3 : 2, s)))
          return rc;
    }
  if (e->train_bf && (rc = cast_bf16(e->train, e->train_bf, e->n_train, s))) return rc;
  return hipDeviceSynchronize() == hipSuccess ? SMHIP_OK : fail(SMHIP_EHIP, "init_synthetic");
}

int smhip_engine_use_graph(void* engine, int on) {
  SMHIP_REQUIRE(engine, "engine: null handle");
  Engine* e = (Engine*)engine;
  e->use_graph = on != 0;
  return SMHIP_OK;
}

// Graph mode.  The first call runs forward_backward eagerly on the engine's private stream
// (so every workspace the step needs is allocated, keyed to that stream), then records the
// same sequence as a graph; later calls copy the inputs into engine buffers and launch the
// graph on the caller's stream.  Every kernel is deterministic, so a replay produces the same
// bits as the eager step.  The live profiler (smhip_profile_begin) needs eager launches, so a
// call while it is active runs eagerly.
static int forward_backward_graph(Engine* e, const int32_t* ids, const int32_t* labels, hipStream_t s) {
  const size_t bytes = sizeof(int32_t) * (size_t)e->T;
  SMHIP_CHECK_HIP(hipMemcpyAsync(e->ids_in, ids, bytes, hipMemcpyDeviceToDevice, s));
  SMHIP_CHECK_HIP(hipMemcpyAsync(e->labels_in, labels, bytes, hipMemcpyDeviceToDevice, s));
  if (e->gexec) {
    SMHIP_CHECK_HIP(hipGraphLaunch(e->gexec, s));
    return SMHIP_OK;
  }
  if (!e->cap) SMHIP_CHECK_HIP(hipStreamCreateWithFlags(&e->cap, hipStreamNonBlocking));
  SMHIP_CHECK_HIP(hipStreamSynchronize(s));
  int rc = forward_backward(e, e->ids_in, e->labels_in, e->cap);  // this step's result + workspaces
  if (rc) return rc;
  SMHIP_CHECK_HIP(hipStreamSynchronize(e->cap));
  SMHIP_CHECK_HIP(hipStreamBeginCapture(e->cap, hipStreamCaptureModeThreadLocal));
  rc = forward_backward(e, e->ids_in, e->labels_in, e->cap);
  hipGraph_t g = nullptr;
  const hipError_t ec = hipStreamEndCapture(e->cap, &g);
  if (rc) {
    if (g) hipGraphDestroy(g);
    return rc;
  }
  if (ec != hipSuccess || !g) return fail(SMHIP_EHIP, "engine: graph capture failed");
  const hipError_t ei = hipGraphInstantiate(&e->gexec, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (ei != hipSuccess) {
    e->gexec = nullptr;
    return fail(SMHIP_EHIP, "engine: graph instantiation failed");
  }
  return SMHIP_OK;
}

int smhip_engine_zero_grad(void* engine, smhip_stream_t stream) {
  SMHIP_REQUIRE(engine, "engine: null handle");
  Engine* e = (Engine*)engine;
  return zero_bytes(e->grad, sizeof(float) * (size_t)e->n_train, (hipStream_t)stream);
}

int smhip_engine_set_lr(void* engine, float lr) {
  SMHIP_REQUIRE(engine, "engine: null handle");
  SMHIP_REQUIRE(std::isfinite(lr) && lr >= 0.f, "engine_set_lr: learning rate must be finite and >= 0");
  ((Engine*)engine)->c.lr = lr;
  return SMHIP_OK;
}

int smhip_engine_get_lr(void* engine, float* lr) {
  SMHIP_REQUIRE(engine && lr, "engine_get_lr: null argument");
  *lr = ((Engine*)engine)->c.lr;
  return SMHIP_OK;
}

int smhip_engine_forward_backward(void* engine, const int32_t* ids, const int32_t* labels, float* loss,
                                  smhip_stream_t stream) {
  return smhip_engine_forward_backward_accum(engine, ids, labels, loss, 0, stream);
}

int smhip_engine_forward_backward_accum(void* engine, const int32_t* ids, const int32_t* labels, float* loss,
                                        int accumulate, smhip_stream_t stream) {
  SMHIP_REQUIRE(engine && ids && labels, "engine_forward_backward: null argument");
  Engine* e = (Engine*)engine;
  int rc;
  if (!accumulate && (rc = smhip_engine_zero_grad(engine, stream))) return rc;
  if (e->use_graph && !profiling_active()) rc = forward_backward_graph(e, ids, labels, (hipStream_t)stream);
  else rc = forward_backward(e, ids, labels, (hipStream_t)stream);
  if (rc) return rc;
  if (loss) SMHIP_CHECK_HIP(hipMemcpyAsync(loss, e->loss, sizeof(float), hipMemcpyDeviceToDevice, (hipStream_t)stream));
  return SMHIP_OK;
}

int smhip_engine_optimizer_step(void* engine, float* grad_norm_sq, smhip_stream_t stream) {
  SMHIP_REQUIRE(engine, "engine: null handle");
  Engine* e = (Engine*)engine;
  int rc = optimizer_step(e, (hipStream_t)stream);
  if (rc) return rc;
  if (grad_norm_sq)
    SMHIP_CHECK_HIP(hipMemcpyAsync(grad_norm_sq, e->gnorm, sizeof(float), hipMemcpyDeviceToDevice, (hipStream_t)stream));
  return SMHIP_OK;
}

int smhip_engine_step(void* engine, const int32_t* ids, const int32_t* labels, float* loss, smhip_stream_t stream) {
  int rc = smhip_engine_forward_backward(engine, ids, labels, loss, stream);
  if (rc) return rc;
  return smhip_engine_optimizer_step(engine, nullptr, stream);
}

int smhip_engine_read_activation(void* engine, const char* what, int layer, void* host, int64_t nbytes) {
  SMHIP_REQUIRE(engine && what && host, "engine_read_activation: null argument");
  Engine* e = (Engine*)engine;
  SMHIP_REQUIRE(layer >= 0 && layer < e->c.n_layers, "engine_read_activation: bad layer");
  const Saved& s = e->sv[layer];
  const int64_t T = e->T, d = e->c.d_model, F = e->c.ffn_dim;
  const void* src = nullptr;
  int64_t bytes = 0;
  const int64_t es = (int64_t)e->esz;
  std::string w(what);
  if (w == "h_in") { src = s.h_in; bytes = T * d * 4; }
  else if (w == "h_mid") { src = s.h_mid; bytes = T * d * 4; }
  else if (w == "xn1") { src = s.xn1; bytes = T * d * es; }
  else if (w == "qkv") { src = s.qkv; bytes = T * e->nqkv * (e->qkv_bf ? 2 : 4); }
  else if (w == "q") { src = s.q; bytes = T * e->qd * es; }
  else if (w == "k") { src = s.k; bytes = T * e->kvd * es; }
  else if (w == "v") { src = s.v; bytes = T * e->kvd * es; }
  else if (w == "o") { src = s.o; bytes = T * e->qd * es; }
  else if (w == "gu") { src = s.gu; bytes = T * 2 * F * es; }
  else if (w == "act") { src = s.act; bytes = T * F * es; }
  else if (w == "h_fin") { src = e->h_fin; bytes = T * d * 4; }
  else if (w == "logits") { src = e->logits; bytes = T * e->c.vocab * 4; }
  else return fail(SMHIP_EINVAL, "engine_read_activation: unknown activation " + w);
  SMHIP_REQUIRE(nbytes == bytes, "engine_read_activation: size mismatch for " + w);
  SMHIP_CHECK_HIP(hipDeviceSynchronize());
  SMHIP_CHECK_HIP(hipMemcpy(host, src, bytes, hipMemcpyDeviceToHost));
  return SMHIP_OK;
}

int smhip_fill_token_ids(int32_t* ids, int64_t n, uint64_t seed, int vocab, smhip_stream_t stream) {
  SMHIP_REQUIRE(ids && n >= 0 && vocab > 0, "fill_token_ids: bad arguments");
  return fill_ids(ids, n, seed, vocab, (hipStream_t)stream);
}

int smhip_quantize(int qtype, const float* x, int64_t n, void* out, smhip_stream_t stream) {
  SMHIP_REQUIRE(x && out && n >= 0, "quantize: bad arguments");
  return encode_quant(qtype, x, n, out, (hipStream_t)stream);
}


int smhip_engine_save_checkpoint(void* engine, const char* dir, int with_optimizer, int step, float loss,
                                 const char* note) {
  SMHIP_REQUIRE(engine && dir && *dir, "engine_save_checkpoint: null argument");
  return save_checkpoint((Engine*)engine, dir, step, loss, note, with_optimizer != 0);
}

int smhip_engine_load_checkpoint(void* engine, const char* dir, int with_optimizer, int* step, float* loss) {
  SMHIP_REQUIRE(engine && dir && *dir, "engine_load_checkpoint: null argument");
  return load_checkpoint((Engine*)engine, dir, with_optimizer != 0, step, loss);
}

int smhip_checkpoint_find_latest(const char* dir, char* out, int64_t cap) {
  SMHIP_REQUIRE(out && cap > 0, "checkpoint_find_latest: null output");
  out[0] = '\0';
  if (!dir || !*dir) return 0;
  std::error_code ec;
  if (!std::filesystem::is_directory(dir, ec)) return 0;
  // Checkpoint.FindLatest compares parsed steps (Checkpoint.cs:117-134), but its ParseStep
  // returns 0 for every name that starts with "step-" (Checkpoint.cs:138-145), so every candidate ties and the
  // ordinal-greatest directory name wins; that is the behaviour reproduced here (for the
  // zero-padded names TrainLoop writes it is also the highest step)
  std::string best;
  for (const auto& ent : std::filesystem::directory_iterator(dir, ec)) {
    std::error_code ec2;
    if (!ent.is_directory(ec2)) continue;
    const std::string name = ent.path().filename().string();
    if (name.rfind("step-", 0) != 0) continue;
    if (best.empty() || name.compare(best) > 0) best = name;
  }
  if (best.empty()) return 0;
  const std::string path = (std::filesystem::path(dir) / best).string();
  SMHIP_REQUIRE((int64_t)path.size() < cap, "checkpoint_find_latest: output buffer too small");
  memcpy(out, path.c_str(), path.size() + 1);
  return 1;
}


// GgufLoader.LoadAllWeights / LoadSingleTensor (SharpMind.Model/Format/GgufLoader.cs:435-600) for
// the frozen base of a LoRA engine: the standard llama.cpp tensor names, raw quantised bytes
// handed to set_tensor unchanged (q|k|v and gate|up rows concatenated: each row is whole
// blocks, so the fused matrix is the byte concatenation), norms from F32 or F16.
int smhip_engine_load_gguf(void* engine, const char* path) {
  SMHIP_REQUIRE(engine && path, "engine_load_gguf: null argument");
  Engine* e = (Engine*)engine;
  SMHIP_REQUIRE(e->lora, "engine_load_gguf: GGUF supplies the frozen quantised base of a LoRA engine (base_qtype Q8_0 or Q4_K)");
  GgufFile g;
  if (int rc = gguf_parse(path, &g)) return rc;
  const smhip_model_config& c = e->c;
  const int d = c.d_model, F = c.ffn_dim, D = c.head_dim;
  const uint32_t qt = (uint32_t)c.base_qtype;
  if (const std::string* arch = g.string_value("general.architecture")) {
    int64_t blocks;
    if (g.int_value(*arch + ".block_count", &blocks))
      SMHIP_REQUIRE(blocks == c.n_layers, "engine_load_gguf: file has " + std::to_string(blocks) +
                                              " blocks, the engine " + std::to_string(c.n_layers));
  }
  SMHIP_REQUIRE(!g.find("output.weight"),
                "engine_load_gguf: the file has an untied output.weight; the engine's LM head is tied to token_embd");
  struct Closer { void operator()(FILE* f) const { if (f) fclose(f); } };
  std::unique_ptr<FILE, Closer> f(fopen(path, "rb"));
  SMHIP_REQUIRE(f, std::string("engine_load_gguf: cannot open ") + path);
  auto tname = [](const char* fmt, int l) {
    char b[128];
    snprintf(b, sizeof b, fmt, l);
    return std::string(b);
  };
  // appends the raw bytes of tensor `name` (type `type`, dims innermost first) to buf
  auto read = [&](const std::string& name, uint32_t type, std::vector<int64_t> dims, std::vector<uint8_t>* buf) -> int {
    const GgufTensor* t = g.find(name);
    SMHIP_REQUIRE(t, "engine_load_gguf: missing tensor " + name);
    SMHIP_REQUIRE(t->type == type, "engine_load_gguf: " + name + " has ggml type " + std::to_string(t->type) +
                                       ", expected " + std::to_string(type));
    SMHIP_REQUIRE(t->dims == dims, "engine_load_gguf: " + name + " has an unexpected shape");
    const int64_t bytes = gguf_tensor_bytes(type, dims);
    SMHIP_REQUIRE(bytes > 0, "engine_load_gguf: unsupported layout for " + name);
    const size_t at = buf->size();
    buf->resize(at + (size_t)bytes);
    if (fseeko(f.get(), (off_t)(g.data_offset + t->offset), SEEK_SET) != 0 ||
        fread(buf->data() + at, 1, (size_t)bytes, f.get()) != (size_t)bytes)
      return fail(SMHIP_EINVAL, "engine_load_gguf: truncated data for " + name);
    return SMHIP_OK;
  };
  auto set = [&](const std::string& name, const std::vector<uint8_t>& buf) {
    return smhip_engine_set_tensor(engine, name.c_str(), buf.data(), (int64_t)buf.size());
  };
  auto norm = [&](const std::string& gname, int n, const std::string& ename) -> int {
    const GgufTensor* t = g.find(gname);
    SMHIP_REQUIRE(t, "engine_load_gguf: missing tensor " + gname);
    SMHIP_REQUIRE(t->type == 0 || t->type == 1, "engine_load_gguf: " + gname + " must be F32 or F16");
    std::vector<uint8_t> raw;
    if (int rc = read(gname, t->type, {n}, &raw)) return rc;
    std::vector<float> w((size_t)n);
    for (int i = 0; i < n; i++) {
      if (t->type == 0) memcpy(&w[i], raw.data() + 4 * i, 4);
      else w[i] = half_bits_to_float((uint16_t)(raw[2 * i] | (raw[2 * i + 1] << 8)));
    }
    return smhip_engine_set_tensor(engine, ename.c_str(), w.data(), (int64_t)n * 4);
  };
  std::vector<uint8_t> buf;
  int rc;
  if ((rc = read("token_embd.weight", qt, {d, c.vocab}, &buf)) || (rc = set("emb", buf))) return rc;
  if ((rc = norm("output_norm.weight", d, "norm_f"))) return rc;
  for (int l = 0; l < c.n_layers; l++) {
    for (const char* b : {"blk.%d.attn_q.bias", "blk.%d.attn_k.bias", "blk.%d.attn_v.bias", "blk.%d.attn_output.bias"})
      SMHIP_REQUIRE(!g.find(tname(b, l)), "engine_load_gguf: linear biases are not supported by LoRA engines (" +
                                              tname(b, l) + ")");
    buf.clear();
    if ((rc = read(tname("blk.%d.attn_q.weight", l), qt, {d, e->qd}, &buf)) ||
        (rc = read(tname("blk.%d.attn_k.weight", l), qt, {d, e->kvd}, &buf)) ||
        (rc = read(tname("blk.%d.attn_v.weight", l), qt, {d, e->kvd}, &buf)) || (rc = set(tname("l%d.wqkv", l), buf)))
      return rc;
    buf.clear();
    if ((rc = read(tname("blk.%d.attn_output.weight", l), qt, {e->qd, d}, &buf)) || (rc = set(tname("l%d.wo", l), buf)))
      return rc;
    buf.clear();
    if ((rc = read(tname("blk.%d.ffn_gate.weight", l), qt, {d, F}, &buf)) ||
        (rc = read(tname("blk.%d.ffn_up.weight", l), qt, {d, F}, &buf)) || (rc = set(tname("l%d.wgu", l), buf)))
      return rc;
    buf.clear();
    if ((rc = read(tname("blk.%d.ffn_down.weight", l), qt, {F, d}, &buf)) || (rc = set(tname("l%d.wd", l), buf)))
      return rc;
    if ((rc = norm(tname("blk.%d.attn_norm.weight", l), d, tname("l%d.norm1", l))) ||
        (rc = norm(tname("blk.%d.ffn_norm.weight", l), d, tname("l%d.norm2", l))))
      return rc;
    if (c.qk_norm && ((rc = norm(tname("blk.%d.attn_q_norm.weight", l), D, tname("l%d.q_norm", l))) ||
                      (rc = norm(tname("blk.%d.attn_k_norm.weight", l), D, tname("l%d.k_norm", l)))))
      return rc;
  }
  return SMHIP_OK;
}

}  // extern "C"
