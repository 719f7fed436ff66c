// capi.cpp — extern "C" entry points of libsharpmind_hip.
//
// Device entries validate shapes on the host, then launch on the caller's
// stream.  Host entries (smhip_host_*) mirror the reference's JigSaw slot
// signatures on host memory: copy in, run the device entry, copy out.
#include <hip/hip_runtime.h>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace smhip {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

struct WsKey {
  hipStream_t s;
  int slot;
  int dev;
  bool operator==(const WsKey& o) const { return s == o.s && slot == o.slot && dev == o.dev; }
};
struct WsHash {
  size_t operator()(const WsKey& k) const {
    return std::hash<void*>()((void*)k.s) ^ ((size_t)k.slot * 0x9E3779B97F4A7C15ull) ^ ((size_t)k.dev << 20);
  }
};
struct WsBuf {
  void* p = nullptr;
  size_t n = 0;
};
static std::mutex g_ws_mu;
static std::unordered_map<WsKey, WsBuf, WsHash> g_ws;

void* workspace(hipStream_t s, size_t bytes, int slot) {
  int dev = 0;
  hipGetDevice(&dev);
  std::lock_guard<std::mutex> lk(g_ws_mu);
  WsBuf& b = g_ws[WsKey{s, slot, dev}];
  if (b.n >= bytes && b.p) return b.p;
  if (b.p) {
    // the old buffer may still be read by queued work on this stream
    hipStreamSynchronize(s);
    hipFree(b.p);
    b.p = nullptr;
    b.n = 0;
  }
  size_t want = bytes < 256 ? 256 : bytes;
  want = (want + 4095) & ~(size_t)4095;
  if (hipMalloc(&b.p, want) != hipSuccess) {
    b.p = nullptr;
    return nullptr;
  }
  b.n = want;
  return b.p;
}

void workspace_release(hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_ws_mu);
  for (auto it = g_ws.begin(); it != g_ws.end();) {
    if (it->first.s == s) {
      if (it->second.p) hipFree(it->second.p);
      it = g_ws.erase(it);
    } else {
      ++it;
    }
  }
}

struct Profiler {
  std::vector<hipEvent_t> ev;
  size_t used = 0;
  struct Rec { int cat, i0, i1; double flops; int M, N, K; };
  std::vector<Rec> recs;
};
static thread_local Profiler* g_prof = nullptr;

int prof_mark(hipStream_t s) {
  Profiler* p = g_prof;
  if (!p || p->used >= p->ev.size()) return -1;
  hipEventRecord(p->ev[p->used], s);
  return (int)p->used++;
}
bool profiling_active() { return g_prof != nullptr; }
bool prof_reserve(int* i0, int* i1, hipEvent_t* e0, hipEvent_t* e1) {
  Profiler* p = g_prof;
  if (!p || p->used + 2 > p->ev.size()) return false;
  *i0 = (int)p->used;
  *e0 = p->ev[p->used++];
  *i1 = (int)p->used;
  *e1 = p->ev[p->used++];
  return true;
}
void prof_add(int cat, int i0, int i1, double flops, int M, int N, int K) {
  if (g_prof && i0 >= 0 && i1 >= 0) g_prof->recs.push_back({cat, i0, i1, flops, M, N, K});
}

}  // namespace smhip

using namespace smhip;

extern "C" int smhip_profile_begin(int max_events) {
  SMHIP_REQUIRE(max_events > 0, "profile_begin: max_events must be positive");
  if (g_prof) return fail(SMHIP_EINVAL, "profile_begin: profiling already active on this thread");
  Profiler* p = new Profiler();
  p->ev.resize(max_events);
  for (auto& e : p->ev) {
    if (hipEventCreate(&e) != hipSuccess) { delete p; return fail(SMHIP_EHIP, "profile_begin: hipEventCreate"); }
  }
  g_prof = p;
  return SMHIP_OK;
}

extern "C" int smhip_profile_end(double* out, int ncat) {
  Profiler* p = g_prof;
  SMHIP_REQUIRE(p, "profile_end: profiling not active");
  g_prof = nullptr;
  int rc = SMHIP_OK;
  if (hipDeviceSynchronize() != hipSuccess) rc = fail(SMHIP_EHIP, "profile_end: synchronize failed");
  if (!rc && out) {
    for (int i = 0; i < 3 * ncat; i++) out[i] = 0.0;
    for (auto& r : p->recs) {
      if (r.cat >= ncat) continue;
      float ms = 0.f;
      hipEventElapsedTime(&ms, p->ev[r.i0], p->ev[r.i1]);
      out[3 * r.cat] += ms;
      out[3 * r.cat + 1] += 1.0;
      out[3 * r.cat + 2] += r.flops;
    }
  }
  if (!rc) {
    // optional per-launch listing for offline analysis: SMHIP_PROFILE_DUMP=<path>
    const char* path = getenv("SMHIP_PROFILE_DUMP");
    if (path && *path) {
      FILE* f = fopen(path, "w");
      if (f) {
        for (auto& r : p->recs) {
          float ms = 0.f;
          hipEventElapsedTime(&ms, p->ev[r.i0], p->ev[r.i1]);
          fprintf(f, "%d %d %d %d %.6f %.0f\n", r.cat, r.M, r.N, r.K, ms, r.flops);
        }
        fclose(f);
      }
    }
  }
  for (auto& e : p->ev) hipEventDestroy(e);
  delete p;
  return rc;
}

#define STREAM(s) ((hipStream_t)(s))

extern "C" {

const char* smhip_last_error(void) { return g_last_error.c_str(); }
int smhip_version(void) { return 100; }
int smhip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

// ---------------------------------------------------------------- GradientMapping
int smhip_grad_linear(const float* dY, const float* X, const float* W, float* dW, float* db,
                      float* dX, int M, int In, int Out, int precision, smhip_stream_t stream) {
  SMHIP_REQUIRE(M >= 0 && In > 0 && Out > 0, "grad_linear: bad shape");
  SMHIP_REQUIRE(dY && (!dX || W) && (!dW || X), "grad_linear: null operand");
  hipStream_t s = STREAM(stream);
  GemmArgs g{};
  g.precision = precision;
  g.split_k = 1;
  g.alpha = 1.f;
  if (dX) {  // dX[M,In] = dY[M,Out] W[Out,In]
    g.M = M; g.N = In; g.K = Out;
    g.A = {SRC_F32_K, dY, nullptr, Out};
    g.B = {SRC_F32_R, W, nullptr, In};
    g.beta = 0.f;
    g.C = dX; g.ldc = In;
    int rc = gemm(g, s);
    if (rc) return rc;
  }
  if (dW) {  // dW[Out,In] += dY^T X
    g.M = Out; g.N = In; g.K = M;
    g.A = {SRC_F32_R, dY, nullptr, Out};
    g.B = {SRC_F32_R, X, nullptr, In};
    g.beta = 1.f;
    g.C = dW; g.ldc = In;
    // long reductions over tokens with few output tiles: split K
    int tiles = ceil_div(Out, 128) * ceil_div(In, 128);
    int ksteps = ceil_div(M, 32);
    g.split_k = (tiles < num_cus() && ksteps >= 16) ? std::min(std::max(num_cus() / tiles, 1), ksteps / 8) : 1;
    int rc = gemm(g, s);
    if (rc) return rc;
  }
  if (db) return colsum_add(dY, db, M, Out, s);
  return SMHIP_OK;
}

int smhip_grad_rmsnorm(const float* dY, const float* xNorm, const float* rmsInv, const float* w,
                       float* dw, float* dX, int T, int D, smhip_stream_t stream) {
  SMHIP_REQUIRE(T >= 0 && D > 0, "grad_rmsnorm: bad shape");
  SMHIP_REQUIRE(dY && xNorm && rmsInv && w && dX, "grad_rmsnorm: null operand");
  return rmsnorm_backward(dY, xNorm, 0, rmsInv, w, dw, dX, T, D, 0, nullptr, STREAM(stream));
}

int smhip_grad_layernorm(const float* dY, const float* x, const float* w, float* dw, float* db,
                         float* dX, int T, int D, float eps, smhip_stream_t stream) {
  SMHIP_REQUIRE(T >= 0 && D > 0, "grad_layernorm: bad shape");
  SMHIP_REQUIRE(dY && x && w && dX, "grad_layernorm: null operand");
  return layernorm_backward(dY, x, w, dw, db, dX, T, D, eps, STREAM(stream));
}

int smhip_grad_attention(const float* dO, const float* q, const float* k, const float* v,
                         const float* probs, float* dQ, float* dK, float* dV, int S, int D,
                         float scale, smhip_stream_t stream) {
  SMHIP_REQUIRE(S >= 0 && D > 0, "grad_attention: bad shape");
  SMHIP_REQUIRE(dO && q && k && v && probs && dQ && dK && dV, "grad_attention: null operand");
  return attention_slot_backward(dO, q, k, v, probs, dQ, dK, dV, S, D, scale, STREAM(stream));
}

int smhip_grad_embedding(const float* dY, const int32_t* ids, float* dE, int T, int D, int V,
                         smhip_stream_t stream) {
  SMHIP_REQUIRE(T >= 0 && D > 0 && V > 0, "grad_embedding: bad shape");
  SMHIP_REQUIRE(dY && ids && dE, "grad_embedding: null operand");
  return embedding_backward(dY, ids, dE, T, D, V, STREAM(stream));
}

int smhip_grad_silu(const float* dY, const float* x, float* dX, int64_t n, smhip_stream_t stream) {
  SMHIP_REQUIRE(n >= 0 && (n == 0 || (dY && x && dX)), "grad_silu: bad arguments");
  return silu_backward(dY, x, dX, n, STREAM(stream));
}
int smhip_grad_gelu(const float* dY, const float* x, float* dX, int64_t n, smhip_stream_t stream) {
  SMHIP_REQUIRE(n >= 0 && (n == 0 || (dY && x && dX)), "grad_gelu: bad arguments");
  return gelu_backward(dY, x, dX, n, STREAM(stream));
}

// ---------------------------------------------------------------- TrainingOps
int smhip_adamw_update(float* data, const float* grad, float* m, float* v, int64_t n, float beta1,
                       float beta2, float bc1, float bc2, float lr, float eps, float decay,
                       smhip_stream_t stream) {
  SMHIP_REQUIRE(n >= 0 && (n == 0 || (data && grad && m && v)), "adamw_update: bad arguments");
  return adamw_update(data, grad, m, v, n, beta1, beta2, bc1, bc2, lr, eps, decay, STREAM(stream));
}
int smhip_l2normsq(const float* data, int64_t n, float* out, smhip_stream_t stream) {
  SMHIP_REQUIRE(n >= 0 && out && (n == 0 || data), "l2normsq: bad arguments");
  return l2normsq(data, n, out, 0, STREAM(stream));
}
int smhip_scale_inplace(float* x, int64_t n, float scale, smhip_stream_t stream) {
  SMHIP_REQUIRE(n >= 0 && (n == 0 || x), "scale_inplace: bad arguments");
  return scale_inplace(x, n, scale, STREAM(stream));
}

// ---------------------------------------------------------------- QuantizationOps
int smhip_qmatmul(int qtype, const float* in, const void* rawW, float* out, int M, int K, int N,
                  int precision, smhip_stream_t stream) {
  SMHIP_REQUIRE(M >= 0 && K > 0 && N > 0, "qmatmul: bad shape");
  SMHIP_REQUIRE(in && rawW && out, "qmatmul: null operand");
  hipStream_t s = STREAM(stream);
  GemmArgs g{};
  g.precision = precision;
  g.split_k = 1;
  g.alpha = 1.f;
  g.beta = 0.f;
  g.M = M; g.N = N; g.K = K;
  g.A = {SRC_F32_K, in, nullptr, K};
  g.C = out; g.ldc = N;
  if (qtype == SMHIP_QTYPE_F32) {
    g.B = {SRC_F32_K, rawW, nullptr, K};
    return gemm(g, s);
  }
  SMHIP_REQUIRE(qtype == SMHIP_QTYPE_Q8_0 || qtype == SMHIP_QTYPE_Q4_K, "qmatmul: qtype must be 0 (F32), 8 (Q8_0) or 12 (Q4_K)");
  SMHIP_REQUIRE(K % 32 == 0, "qmatmul: K must be a multiple of 32 for block formats");
  const int64_t n = (int64_t)N * K;
  if (qtype == SMHIP_QTYPE_Q4_K) SMHIP_REQUIRE(n % 256 == 0, "qmatmul: Q4_K needs N*K multiple of 256");
  void* planes = workspace(s, planes_bytes(qtype, n, nullptr), 5);
  if (!planes) return fail(SMHIP_ENOMEM, "qmatmul: workspace");
  QuantPlanes qp;
  int rc = repack_planes(qtype, rawW, n, planes, &qp, s);
  if (rc) return rc;
  g.B = {qtype == SMHIP_QTYPE_Q8_0 ? SRC_Q8_K : SRC_Q4K_K, qp.qs, qp.sc, K};
  return gemm(g, s);
}

int smhip_qgemm_bf16(int qtype, int trans_w, int M, int N, int K, const void* A, int64_t lda, const void* rawW,
                     float* C, int64_t ldc, smhip_stream_t stream) {
  SMHIP_REQUIRE(M >= 0 && N > 0 && K > 0 && A && rawW && C, "qgemm_bf16: bad arguments");
  SMHIP_REQUIRE(qtype == SMHIP_QTYPE_Q8_0 || qtype == SMHIP_QTYPE_Q4_K, "qgemm_bf16: qtype must be 8 (Q8_0) or 12 (Q4_K)");
  SMHIP_REQUIRE(K % 64 == 0 && N % 32 == 0, "qgemm_bf16: K must be a multiple of 64 and N of 32");
  hipStream_t s = STREAM(stream);
  const int64_t n = (int64_t)N * K;
  // W rows: [N][K] (trans_w = 0) or [K][N] (trans_w = 1); the row length must hold whole blocks
  const int64_t row = trans_w ? N : K;
  if (qtype == SMHIP_QTYPE_Q4_K) SMHIP_REQUIRE(row % 256 == 0, "qgemm_bf16: Q4_K rows must hold whole 256-element super-blocks");
  void* planes = workspace(s, planes_bytes(qtype, n, nullptr), 5);
  if (!planes) return fail(SMHIP_ENOMEM, "qgemm_bf16: workspace");
  QuantPlanes qp;
  if (int rc = repack_planes(qtype, rawW, n, planes, &qp, s)) return rc;
  GemmArgs g{};
  g.precision = SMHIP_PREC_BF16;
  g.split_k = 1;
  g.alpha = 1.f;
  g.M = M; g.N = N; g.K = K;
  g.A = {SRC_BF16_K, A, nullptr, lda};
  g.C = C; g.ldc = ldc;
  if (K % 64 == 0 && N % 32 == 0) {
    // fragment planes: the GEMM copies codes and scales to LDS and decodes there
    void* fr = workspace(s, frag_planes_bytes(n, qtype), 8);
    if (!fr) return fail(SMHIP_ENOMEM, "qgemm_bf16: workspace");
    if (int rc = make_frag_planes(qp, trans_w ? K : N, trans_w ? N : K, trans_w, fr, &g.B, s)) return rc;
  } else if (!trans_w) {
    g.B = {qtype == SMHIP_QTYPE_Q8_0 ? SRC_Q8_K : SRC_Q4K_K, qp.qs, qp.sc, K};
  } else {
    void* cols = workspace(s, planes_bytes(qtype, n, nullptr), 8);
    if (!cols) return fail(SMHIP_ENOMEM, "qgemm_bf16: workspace");
    QuantPlanes qc;
    if (int rc = make_col_planes(qp, K, N, cols, &qc, s)) return rc;
    g.B = {qtype == SMHIP_QTYPE_Q8_0 ? SRC_Q8T : SRC_Q4KT, qc.qs, qc.sc, K};
  }
  const int rc = gemm(g, s);
  return rc;
}

int smhip_qgemm_bf16_lora(int qtype, int trans_w, int M, int N, int K, const void* A, int64_t lda, const void* rawW,
                          int K2, const void* A2, int64_t lda2, int b2_mode, const void* B2, int64_t ldb2,
                          float alpha2, float* C, int64_t ldc, smhip_stream_t stream) {
  SMHIP_REQUIRE(M >= 0 && N > 0 && K > 0 && A && rawW && C, "qgemm_bf16_lora: bad arguments");
  SMHIP_REQUIRE(qtype == SMHIP_QTYPE_Q8_0 || qtype == SMHIP_QTYPE_Q4_K, "qgemm_bf16_lora: qtype must be 8 (Q8_0) or 12 (Q4_K)");
  SMHIP_REQUIRE(K % 64 == 0 && N % 32 == 0, "qgemm_bf16_lora: K must be a multiple of 64 and N of 32");
  SMHIP_REQUIRE(K2 > 0 && A2 && B2 && (b2_mode == 2 || b2_mode == 3), "qgemm_bf16_lora: bad rank operands");
  hipStream_t s = STREAM(stream);
  const int64_t n = (int64_t)N * K;
  const int64_t row = trans_w ? N : K;
  if (qtype == SMHIP_QTYPE_Q4_K) SMHIP_REQUIRE(row % 256 == 0, "qgemm_bf16_lora: Q4_K rows must hold whole 256-element super-blocks");
  void* planes = workspace(s, planes_bytes(qtype, n, nullptr), 5);
  if (!planes) return fail(SMHIP_ENOMEM, "qgemm_bf16_lora: workspace");
  QuantPlanes qp;
  if (int rc = repack_planes(qtype, rawW, n, planes, &qp, s)) return rc;
  void* fr = workspace(s, frag_planes_bytes(n, qtype), 8);
  if (!fr) return fail(SMHIP_ENOMEM, "qgemm_bf16_lora: workspace");
  GemmArgs g{};
  g.precision = SMHIP_PREC_BF16;
  g.split_k = 1;
  g.alpha = 1.f;
  g.M = M; g.N = N; g.K = K;
  g.A = {SRC_BF16_K, A, nullptr, lda};
  if (int rc = make_frag_planes(qp, trans_w ? K : N, trans_w ? N : K, trans_w, fr, &g.B, s)) return rc;
  g.K2 = K2;
  g.A2 = {SRC_BF16_K, A2, nullptr, lda2};
  g.B2 = {b2_mode == 2 ? SRC_BF16_K : SRC_BF16_R, B2, nullptr, ldb2};
  g.alpha2 = alpha2;
  g.C = C; g.ldc = ldc;
  return gemm(g, s);
}

int smhip_lm_head_ce_bf16(int qtype, int T, int V, int d, const void* x, const void* rawE, const int32_t* labels,
                          float* logits, void* dlogits, float* loss, smhip_stream_t stream) {
  SMHIP_REQUIRE(T > 0 && V > 0 && d > 0 && x && rawE && labels && logits && dlogits, "lm_head_ce_bf16: bad arguments");
  SMHIP_REQUIRE(qtype == SMHIP_QTYPE_Q8_0 || qtype == SMHIP_QTYPE_Q4_K, "lm_head_ce_bf16: qtype must be 8 (Q8_0) or 12 (Q4_K)");
  SMHIP_REQUIRE(d % 64 == 0 && V % 64 == 0, "lm_head_ce_bf16: d and V must be multiples of 64");
  if (qtype == SMHIP_QTYPE_Q4_K) SMHIP_REQUIRE(d % 256 == 0, "lm_head_ce_bf16: Q4_K rows must hold whole super-blocks");
  hipStream_t s = STREAM(stream);
  const int64_t n = (int64_t)V * d;
  void* planes = workspace(s, planes_bytes(qtype, n, nullptr), 5);
  void* fr = workspace(s, frag_planes_bytes(n, qtype), 8);
  if (!planes || !fr) return fail(SMHIP_ENOMEM, "lm_head_ce_bf16: workspace");
  QuantPlanes qp;
  if (int rc = repack_planes(qtype, rawE, n, planes, &qp, s)) return rc;
  GemmArgs g{};
  g.precision = SMHIP_PREC_BF16;
  g.split_k = 1;
  g.alpha = 1.f;
  g.M = T; g.N = V; g.K = d;
  g.A = {SRC_BF16_K, x, nullptr, d};
  if (int rc = make_frag_planes(qp, V, d, 0, fr, &g.B, s)) return rc;
  g.C = logits; g.ldc = V;
  // the head GEMM's softmax row statistics when its persistent form applies
  const bool stats = T % 128 == 0 && V % 128 == 0 && (int64_t)(T / 128) * (V / 128) >= 4 * num_cus() &&
                     ((uintptr_t)logits % 16 == 0) && ((uintptr_t)dlogits % 16 == 0);
  if (stats) {
    g.rowstat = (float*)workspace(s, sizeof(float) * 2 * (size_t)T * (V / 64), 9);
    if (!g.rowstat) return fail(SMHIP_ENOMEM, "lm_head_ce_bf16: workspace");
  }
  if (int rc = gemm(g, s)) return rc;
  if (stats) return ce_softmax_grad_bf16_stats(logits, g.rowstat, V / 64, labels, (uint16_t*)dlogits, loss, T, V, -100, s);
  return ce_softmax_grad_bf16(logits, labels, (uint16_t*)dlogits, loss, T, V, -100, 0.f, s);
}

int smhip_dequant(int qtype, const void* raw, float* out, int64_t n, smhip_stream_t stream) {
  SMHIP_REQUIRE(n >= 0 && (n == 0 || (raw && out)), "dequant: bad arguments");
  return dequant_raw(qtype, raw, out, n, STREAM(stream));
}

// ---------------------------------------------------------------- BackpropEngine inline math
int smhip_grad_swiglu(const float* dAct, const float* gate, const float* up, float* dFused, int T,
                      int F, smhip_stream_t stream) {
  SMHIP_REQUIRE(T >= 0 && F > 0, "grad_swiglu: bad shape");
  SMHIP_REQUIRE(dAct && gate && up && dFused, "grad_swiglu: null operand");
  return swiglu_backward_f32(dAct, gate, up, dFused, T, F, STREAM(stream));
}
int smhip_swiglu_forward(const float* gate, const float* up, float* act, int64_t n,
                         smhip_stream_t stream) {
  SMHIP_REQUIRE(n >= 0 && (n == 0 || (gate && up && act)), "swiglu_forward: bad arguments");
  return swiglu_forward_f32(gate, up, act, n, STREAM(stream));
}

int smhip_rope_tables(float theta, int ropeDim, int maxSeq, float* cosT, float* sinT) {
  SMHIP_REQUIRE(ropeDim > 0 && ropeDim % 2 == 0 && maxSeq > 0 && cosT && sinT, "rope_tables: bad arguments");
  const int half = ropeDim / 2;
  std::vector<float> freqs(half);
  // RoPE.cs:124-126: freqs[i] = 1 / theta^(2i/ropeDim), float arithmetic
  for (int i = 0; i < half; i++) freqs[i] = 1.f / powf(theta, 2.f * (float)i / (float)ropeDim);
  for (int pos = 0; pos < maxSeq; pos++)
    for (int i = 0; i < half; i++) {
      float angle = (float)pos * freqs[i];
      cosT[(int64_t)pos * half + i] = cosf(angle);
      sinT[(int64_t)pos * half + i] = sinf(angle);
    }
  return SMHIP_OK;
}
int smhip_rope_forward(float* x, const float* cosT, const float* sinT, int B, int S, int H, int D,
                       int neox, smhip_stream_t stream) {
  SMHIP_REQUIRE(B >= 0 && S >= 0 && H >= 0 && D > 0 && D % 2 == 0, "rope_forward: bad shape");
  return rope_apply(x, cosT, sinT, B, S, H, D, neox, 0, STREAM(stream));
}
int smhip_rope_backward(float* dx, const float* cosT, const float* sinT, int B, int S, int H, int D,
                        int neox, smhip_stream_t stream) {
  SMHIP_REQUIRE(B >= 0 && S >= 0 && H >= 0 && D > 0 && D % 2 == 0, "rope_backward: bad shape");
  return rope_apply(dx, cosT, sinT, B, S, H, D, neox, 1, STREAM(stream));
}

int smhip_rmsnorm_forward(const float* x, const float* w, float* y, float* rmsInv, int T, int D,
                          float eps, smhip_stream_t stream) {
  SMHIP_REQUIRE(T >= 0 && D > 0 && x && w && y && rmsInv, "rmsnorm_forward: bad arguments");
  return rmsnorm_forward(x, w, y, nullptr, rmsInv, T, D, eps, STREAM(stream));
}

int smhip_ce_softmax_grad(const float* logits, const int32_t* labels, float* dLogits, float* loss,
                          int T, int V, int ignoreId, float smoothing, smhip_stream_t stream) {
  SMHIP_REQUIRE(T >= 0 && V > 0 && logits && labels && dLogits, "ce_softmax_grad: bad arguments");
  SMHIP_REQUIRE(smoothing >= 0.f && smoothing < 1.f, "ce_softmax_grad: label smoothing must be in [0,1)");
  return ce_softmax_grad(logits, labels, dLogits, loss, T, V, ignoreId, smoothing, STREAM(stream));
}

int smhip_attention_forward_probs(const float* q, const float* k, const float* v, float* probs,
                                  float* out, int B, int S, int Hq, int Hkv, int D,
                                  smhip_stream_t stream) {
  SMHIP_REQUIRE(B >= 0 && S >= 0 && Hq > 0 && Hkv > 0 && D > 0, "attention_forward_probs: bad shape");
  return attention_forward_probs(q, k, v, probs, out, B, S, Hq, Hkv, D, STREAM(stream));
}

}  // extern "C"

// ---------------------------------------------------------------- host-pointer slot entries
// The reference calls its slots concurrently from Parallel.For bodies (_mapping.Attention per
// batch row, BackpropEngine.cs:563-582), so every host entry runs on a stream owned by the
// calling thread (one per device).  Internal scratch is keyed by stream, so two threads never
// share a split-K partial or a dP buffer, and a thread's grow-only device buffers are reused
// from call to call instead of being allocated and freed each time.
namespace {

struct HostCtx {
  hipStream_t s = nullptr;
  std::vector<std::pair<void*, size_t>> bufs;  // argument slot -> device buffer
  ~HostCtx() {
    if (s) {
      hipStreamSynchronize(s);
      workspace_release(s);
      hipStreamDestroy(s);
    }
    for (auto& b : bufs)
      if (b.first) hipFree(b.first);
  }
};
thread_local std::unordered_map<int, HostCtx> t_host;

struct DevArena {
  HostCtx* ctx = nullptr;
  hipStream_t s = nullptr;
  int rc = SMHIP_OK;
  int next = 0;  // argument slot of the next buffer
  DevArena() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) { rc = fail(SMHIP_EHIP, "host entry: no HIP device"); return; }
    ctx = &t_host[dev];
    // default priority, non-blocking: the calling thread's private queue
    if (!ctx->s && hipStreamCreateWithFlags(&ctx->s, hipStreamNonBlocking) != hipSuccess) {
      ctx->s = nullptr;
      rc = fail(SMHIP_EHIP, "host entry: hipStreamCreate failed");
      return;
    }
    s = ctx->s;
  }
  void* slot(size_t bytes) {
    if (rc) return nullptr;
    const int k = next++;
    if ((int)ctx->bufs.size() <= k) ctx->bufs.resize(k + 1, {nullptr, 0});
    auto& b = ctx->bufs[k];
    if (b.second < bytes || !b.first) {
      if (b.first) {
        hipStreamSynchronize(s);  // an earlier call that failed part-way may still be queued
        hipFree(b.first);
        b = {nullptr, 0};
      }
      size_t want = ((bytes < 256 ? 256 : bytes) + 4095) & ~(size_t)4095;
      if (hipMalloc(&b.first, want) != hipSuccess) { b = {nullptr, 0}; rc = fail(SMHIP_ENOMEM, "host entry: hipMalloc failed"); return nullptr; }
      b.second = want;
    }
    return b.first;
  }
  template <typename T>
  T* up(const T* h, size_t n) {  // device copy of n host elements
    const size_t bytes = n * sizeof(T);
    void* d = slot(bytes);
    if (!d) return nullptr;
    if (h && bytes && hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, s) != hipSuccess) { rc = fail(SMHIP_EHIP, "host entry: H2D copy failed"); return nullptr; }
    return (T*)d;
  }
  template <typename T>
  T* zeros(size_t n) {
    T* d = up<T>(nullptr, n);
    if (d && n && hipMemsetAsync(d, 0, n * sizeof(T), s) != hipSuccess) rc = fail(SMHIP_EHIP, "host entry: memset failed");
    return d;
  }
  template <typename T>
  void down(T* h, const T* d, size_t n) {
    if (rc || !h || !n) return;
    if (hipMemcpyAsync(h, d, n * sizeof(T), hipMemcpyDeviceToHost, s) != hipSuccess) { rc = fail(SMHIP_EHIP, "host entry: D2H copy failed"); return; }
    if (hipStreamSynchronize(s) != hipSuccess) rc = fail(SMHIP_EHIP, "host entry: synchronize failed");
  }
  int sync() {
    if (rc) return rc;
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) rc = fail(SMHIP_EHIP, std::string("host entry: ") + hipGetErrorString(e));
    return rc;
  }
};

}  // namespace

extern "C" {

int smhip_host_grad_linear(const float* dY, const float* X, const float* W, float* dW, float* db,
                           float* dX, int M, int In, int Out, int precision) {
  DevArena a;
  float* ddY = a.up(dY, (size_t)M * Out);
  float* dXin = a.up(X, (size_t)M * In);
  float* dWt = a.up(W, (size_t)Out * In);
  float* ddW = dW ? a.up(dW, (size_t)Out * In) : nullptr;
  float* ddb = db ? a.up(db, (size_t)Out) : nullptr;
  float* ddX = dX ? a.zeros<float>((size_t)M * In) : nullptr;
  if (a.rc) return a.rc;
  int rc = smhip_grad_linear(ddY, dXin, dWt, ddW, ddb, ddX, M, In, Out, precision, a.s);
  if (rc) return rc;
  if (a.sync()) return a.rc;
  a.down(dX, ddX, (size_t)M * In);
  a.down(dW, ddW, (size_t)Out * In);
  a.down(db, ddb, (size_t)Out);
  return a.rc;
}

int smhip_host_grad_rmsnorm(const float* dY, const float* xNorm, const float* rmsInv,
                            const float* w, float* dw, float* dX, int T, int D) {
  DevArena a;
  float *p1 = a.up(dY, (size_t)T * D), *p2 = a.up(xNorm, (size_t)T * D), *p3 = a.up(rmsInv, (size_t)T);
  float *p4 = a.up(w, (size_t)D), *p5 = dw ? a.up(dw, (size_t)D) : nullptr, *p6 = a.zeros<float>((size_t)T * D);
  if (a.rc) return a.rc;
  int rc = smhip_grad_rmsnorm(p1, p2, p3, p4, p5, p6, T, D, a.s);
  if (rc) return rc;
  if (a.sync()) return a.rc;
  a.down(dX, p6, (size_t)T * D);
  a.down(dw, p5, (size_t)D);
  return a.rc;
}

int smhip_host_grad_layernorm(const float* dY, const float* x, const float* w, float* dw,
                              float* db, float* dX, int T, int D, float eps) {
  DevArena a;
  float *p1 = a.up(dY, (size_t)T * D), *p2 = a.up(x, (size_t)T * D), *p3 = a.up(w, (size_t)D);
  float *p4 = dw ? a.up(dw, (size_t)D) : nullptr, *p5 = db ? a.up(db, (size_t)D) : nullptr;
  float* p6 = a.zeros<float>((size_t)T * D);
  if (a.rc) return a.rc;
  int rc = smhip_grad_layernorm(p1, p2, p3, p4, p5, p6, T, D, eps, a.s);
  if (rc) return rc;
  if (a.sync()) return a.rc;
  a.down(dX, p6, (size_t)T * D);
  a.down(dw, p4, (size_t)D);
  a.down(db, p5, (size_t)D);
  return a.rc;
}

int smhip_host_grad_attention(const float* dO, const float* q, const float* k, const float* v,
                              const float* probs, float* dQ, float* dK, float* dV, int S, int D,
                              float scale) {
  DevArena a;
  size_t sd = (size_t)S * D;
  float *p1 = a.up(dO, sd), *p2 = a.up(q, sd), *p3 = a.up(k, sd), *p4 = a.up(v, sd), *p5 = a.up(probs, (size_t)S * S);
  float *o1 = a.zeros<float>(sd), *o2 = a.zeros<float>(sd), *o3 = a.zeros<float>(sd);
  if (a.rc) return a.rc;
  int rc = smhip_grad_attention(p1, p2, p3, p4, p5, o1, o2, o3, S, D, scale, a.s);
  if (rc) return rc;
  if (a.sync()) return a.rc;
  a.down(dQ, o1, sd);
  a.down(dK, o2, sd);
  a.down(dV, o3, sd);
  return a.rc;
}

int smhip_host_grad_embedding(const float* dY, const int32_t* ids, float* dE, int T, int D, int V) {
  DevArena a;
  float* p1 = a.up(dY, (size_t)T * D);
  int32_t* p2 = a.up(ids, (size_t)T);
  float* p3 = a.up(dE, (size_t)V * D);
  if (a.rc) return a.rc;
  int rc = smhip_grad_embedding(p1, p2, p3, T, D, V, a.s);
  if (rc) return rc;
  if (a.sync()) return a.rc;
  a.down(dE, p3, (size_t)V * D);
  return a.rc;
}

int smhip_host_grad_silu(const float* dY, const float* x, float* dX, int64_t n) {
  DevArena a;
  float *p1 = a.up(dY, (size_t)n), *p2 = a.up(x, (size_t)n), *p3 = a.zeros<float>((size_t)n);
  if (a.rc) return a.rc;
  int rc = smhip_grad_silu(p1, p2, p3, n, a.s);
  if (rc) return rc;
  if (a.sync()) return a.rc;
  a.down(dX, p3, (size_t)n);
  return a.rc;
}

int smhip_host_grad_gelu(const float* dY, const float* x, float* dX, int64_t n) {
  DevArena a;
  float *p1 = a.up(dY, (size_t)n), *p2 = a.up(x, (size_t)n), *p3 = a.zeros<float>((size_t)n);
  if (a.rc) return a.rc;
  int rc = smhip_grad_gelu(p1, p2, p3, n, a.s);
  if (rc) return rc;
  if (a.sync()) return a.rc;
  a.down(dX, p3, (size_t)n);
  return a.rc;
}

int smhip_host_adamw_update(float* data, const float* grad, float* m, float* v, int64_t n,
                            float beta1, float beta2, float bc1, float bc2, float lr, float eps,
                            float decay) {
  DevArena a;
  float *p1 = a.up(data, (size_t)n), *p2 = a.up(grad, (size_t)n), *p3 = a.up(m, (size_t)n), *p4 = a.up(v, (size_t)n);
  if (a.rc) return a.rc;
  int rc = smhip_adamw_update(p1, p2, p3, p4, n, beta1, beta2, bc1, bc2, lr, eps, decay, a.s);
  if (rc) return rc;
  if (a.sync()) return a.rc;
  a.down(data, p1, (size_t)n);
  a.down(m, p3, (size_t)n);
  a.down(v, p4, (size_t)n);
  return a.rc;
}

int smhip_host_l2normsq(const float* data, int64_t n, float* out) {
  DevArena a;
  float* p1 = a.up(data, (size_t)n);
  float* p2 = a.zeros<float>(1);
  if (a.rc) return a.rc;
  int rc = smhip_l2normsq(p1, n, p2, a.s);
  if (rc) return rc;
  if (a.sync()) return a.rc;
  a.down(out, p2, 1);
  return a.rc;
}

int smhip_host_qmatmul(int qtype, const float* in, const void* rawW, float* out, int M, int K, int N) {
  size_t wbytes;
  if (qtype == SMHIP_QTYPE_F32) wbytes = (size_t)N * K * 4;
  else if (qtype == SMHIP_QTYPE_Q8_0) wbytes = (size_t)N * K / 32 * 34;
  else if (qtype == SMHIP_QTYPE_Q4_K) wbytes = (size_t)N * K / 256 * 144;
  else return fail(SMHIP_EUNSUPPORTED, "host_qmatmul: qtype must be 0, 8 or 12");
  DevArena a;
  float* p1 = a.up(in, (size_t)M * K);
  uint8_t* p2 = a.up((const uint8_t*)rawW, wbytes);
  float* p3 = a.zeros<float>((size_t)M * N);
  if (a.rc) return a.rc;
  int rc = smhip_qmatmul(qtype, p1, p2, p3, M, K, N, SMHIP_PREC_FP32, a.s);
  if (rc) return rc;
  if (a.sync()) return a.rc;
  a.down(out, p3, (size_t)M * N);
  return a.rc;
}

}  // extern "C"

extern "C" {

int smhip_gemm(int M, int N, int K, int a_mode, const void* A, int64_t lda, int b_mode, const void* B, int64_t ldb,
               float alpha, float beta, void* C, int64_t ldc, int c_bf16, int split_k, int precision,
               smhip_stream_t stream) {
  SMHIP_REQUIRE(M >= 0 && N >= 0 && K > 0 && A && B && C, "gemm: bad arguments");
  SMHIP_REQUIRE(a_mode >= 0 && a_mode <= 3 && b_mode >= 0 && b_mode <= 3, "gemm: operand modes must be 0..3");
  SMHIP_REQUIRE(beta == 0.f || beta == 1.f, "gemm: beta must be 0 or 1");
  GemmArgs g{};
  g.M = M; g.N = N; g.K = K;
  g.A = {a_mode, A, nullptr, lda};
  g.B = {b_mode, B, nullptr, ldb};
  g.alpha = alpha; g.beta = beta;
  g.C = C; g.ldc = ldc; g.c_bf16 = c_bf16;
  g.precision = precision;
  // split_k 0: the bf16 path picks the tile, ring depth and split itself (the engine's choice)
  g.split_k = split_k > 0 ? split_k : (precision == SMHIP_PREC_BF16 ? 0 : 1);
  return gemm(g, STREAM(stream));
}

int smhip_flash_attention_forward(const void* q, const void* k, const void* v, void* o, float* lse, int B, int S,
                                  int Hq, int Hkv, int D, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo,
                                  smhip_stream_t stream) {
  SMHIP_REQUIRE(q && k && v && o && lse && B > 0 && S > 0, "flash_attention_forward: bad arguments");
  return flash_forward((const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, lse, B, S, Hq, Hkv,
                       D, ldq, ldk, ldv, ldo, STREAM(stream));
}

int smhip_flash_attention_backward(const void* q, const void* k, const void* v, const void* o, const void* dO,
                                   const float* lse, float* dq, float* dk, float* dv, int B, int S, int Hq, int Hkv,
                                   int D, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo, int64_t lddo,
                                   int64_t lddq, int64_t lddk, int64_t lddv, smhip_stream_t stream) {
  SMHIP_REQUIRE(q && k && v && o && dO && lse && dq && dk && dv && B > 0 && S > 0, "flash_attention_backward: bad arguments");
  hipStream_t s = STREAM(stream);
  void* ws = workspace(s, flash_backward_workspace(B, S, Hq, D), 6);
  if (!ws) return fail(SMHIP_ENOMEM, "flash_attention_backward: workspace");
  return flash_backward((const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)o,
                        (const uint16_t*)dO, lse, dq, dk, dv, B, S, Hq, Hkv, D, ldq, ldk, ldv, ldo, lddo, lddq, lddk,
                        lddv, ws, s);
}

}  // extern "C"

// ---------------------------------------------------------------- allocation-free flash backward
// For callers that cannot allocate device memory (code under HIP graph capture, tight serving
// loops): the backward's scratch (row terms D_i and the per-query-head dK/dV partials) lives in a
// file-scope device array instead of the workspace pool.  Each device holds its own copy; its
// address is looked up once per device with the device current.  Calls on one device share the
// array, so calls that overlap on one device race.
namespace {
constexpr size_t kNoAllocScratchBytes = (size_t)80 << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(void** out) {
  int dev = 0;
  SMHIP_CHECK_HIP(hipGetDevice(&dev));
  SMHIP_REQUIRE(dev >= 0 && dev < kMaxDevices, "flash_attention_backward_noalloc: device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    SMHIP_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    SMHIP_REQUIRE(p, "flash_attention_backward_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SMHIP_OK;
}
}  // namespace

extern "C" {

int smhip_flash_attention_backward_noalloc_limit(int64_t* bytes) {
  SMHIP_REQUIRE(bytes, "flash_attention_backward_noalloc_limit: null argument");
  *bytes = (int64_t)kNoAllocScratchBytes;
  return SMHIP_OK;
}

int smhip_flash_attention_backward_noalloc(const void* q, const void* k, const void* v, const void* o, const void* dO,
                                           const float* lse, float* dq, float* dk, float* dv, int B, int S, int Hq,
                                           int Hkv, int D, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo,
                                           int64_t lddo, int64_t lddq, int64_t lddk, int64_t lddv,
                                           smhip_stream_t stream) {
  SMHIP_REQUIRE(q && k && v && o && dO && lse && dq && dk && dv && B > 0 && S > 0 && Hq > 0 && D > 0,
                "flash_attention_backward_noalloc: bad arguments");
  const size_t need = flash_backward_workspace(B, S, Hq, D);
  if (need > kNoAllocScratchBytes)
    return fail(SMHIP_EINVAL, "flash_attention_backward_noalloc: B*Hq*S*(2*D+1)*4 bytes of scratch (" +
                                  std::to_string(need) + ") exceed the fixed " + std::to_string(kNoAllocScratchBytes) +
                                  "-byte array; use smhip_flash_attention_backward");
  void* ws = nullptr;
  if (int rc = scratch_for_current_device(&ws)) return rc;
  return flash_backward((const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)o,
                        (const uint16_t*)dO, lse, dq, dk, dv, B, S, Hq, Hkv, D, ldq, ldk, ldv, ldo, lddo, lddq, lddk,
                        lddv, ws, STREAM(stream));
}

}  // extern "C"

