/*
 * engine.c — CPU restatement of one training step of SharpMind's autograd
 * engine, used as the end-to-end checker of the GPU engine.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Follows BackpropEngine.ForwardAndRecord / Backward
 * (SharpMind.Training/Autograd/BackpropEngine.cs:73-206) for a decoder of
 * RMSNorm -> attention (RoPE, causal softmax with materialised probs, GQA) ->
 * residual -> RMSNorm -> gated SwiGLU FFN -> residual, final RMSNorm and a tied
 * LM head, plus the two extensions the reference's training path lacks and
 * this backend needs: per-head QK-norm before RoPE (the inference forward,
 * AttentionLayer.cs:284) and LoRA adapters y += s (x A) B on the seven block
 * projections (LoRALayer.cs:52-80 math).  Every kernel call is one of the
 * pinned restatements in oracle.c.  Linear weights are [Out][In].
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

typedef struct {
  int L, d, Hq, Hkv, D, F, V, B, S;
  float eps, theta;
  int neox, qk_norm;
  int lora_rank;
  float lora_alpha;
} orc_cfg;

#define PL 26
enum { T_NORM1 = 0, T_WQKV, T_BQKV, T_QN, T_KN, T_WO, T_BO, T_NORM2, T_WGU, T_BGU, T_WD, T_BD, T_LORA };
#define GIDX(l, k) (2 + (l) * PL + (k))

static float* zalloc(int64_t n) { return (float*)calloc((size_t)(n > 0 ? n : 1), sizeof(float)); }

/* y[T,Out] = x[T,In] W^T (+ b), double accumulation (VecDotF32 semantics) */
static void linear_fwd(const float* x, const float* W, const float* b, float* y, int T, int In, int Out) {
  orc_qmatmul_f32(x, W, y, T, In, Out);
  if (b)
    for (int t = 0; t < T; t++)
      for (int o = 0; o < Out; o++) y[(int64_t)t * Out + o] += b[o];
}

/* LoRA projection p of a layer: In/Out and the column offset inside the fused output */
static void lora_geom(const orc_cfg* c, int p, int* In, int* Out, int* off, int* fusedOut) {
  int qd = c->Hq * c->D, kvd = c->Hkv * c->D;
  switch (p) {
    case 0: *In = c->d; *Out = qd; *off = 0; *fusedOut = qd + 2 * kvd; break;
    case 1: *In = c->d; *Out = kvd; *off = qd; *fusedOut = qd + 2 * kvd; break;
    case 2: *In = c->d; *Out = kvd; *off = qd + kvd; *fusedOut = qd + 2 * kvd; break;
    case 3: *In = qd; *Out = c->d; *off = 0; *fusedOut = c->d; break;
    case 4: *In = c->d; *Out = c->F; *off = 0; *fusedOut = 2 * c->F; break;
    case 5: *In = c->d; *Out = c->F; *off = c->F; *fusedOut = 2 * c->F; break;
    default: *In = c->F; *Out = c->d; *off = 0; *fusedOut = c->d; break;
  }
}

/* y[:, off:off+Out] += s (x A) B */
static void lora_fwd_add(const orc_cfg* c, float** P, int l, int p, const float* x, float* y, int T) {
  int In, Out, off, fo;
  lora_geom(c, p, &In, &Out, &off, &fo);
  const float* A = P[GIDX(l, T_LORA + 2 * p)];
  const float* Bm = P[GIDX(l, T_LORA + 2 * p + 1)];
  if (!A || !Bm) return;
  int r = c->lora_rank;
  float s = c->lora_alpha / (float)r;
  if (r > 256) abort(); /* the per-thread u below holds at most 256 ranks */
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; t++) {
    double u[256];
    for (int j = 0; j < r; j++) {
      double a = 0;
      for (int i = 0; i < In; i++) a += (double)x[(int64_t)t * In + i] * A[(int64_t)i * r + j];
      u[j] = a;
    }
    for (int o = 0; o < Out; o++) {
      double a = 0;
      for (int j = 0; j < r; j++) a += u[j] * Bm[(int64_t)j * Out + o];
      y[(int64_t)t * fo + off + o] += (float)((double)s * a);
    }
  }
}

/* LoRA backward of projection p: dA, dB += ; dX[T,In] += s (dY B^T) A^T */
static void lora_bwd_add(const orc_cfg* c, float** P, float** G, int l, int p, const float* x,
                         const float* dYf, float* dX, int T) {
  int In, Out, off, fo;
  lora_geom(c, p, &In, &Out, &off, &fo);
  const float* A = P[GIDX(l, T_LORA + 2 * p)];
  const float* Bm = P[GIDX(l, T_LORA + 2 * p + 1)];
  if (!A || !Bm) return;
  float* dA = G[GIDX(l, T_LORA + 2 * p)];
  float* dB = G[GIDX(l, T_LORA + 2 * p + 1)];
  int r = c->lora_rank;
  double s = (double)(c->lora_alpha / (float)r);
  double* u = (double*)calloc((size_t)T * r, sizeof(double));
  double* z = (double*)calloc((size_t)T * r, sizeof(double));
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; t++)
    for (int j = 0; j < r; j++) {
      double a = 0, b = 0;
      for (int i = 0; i < In; i++) a += (double)x[(int64_t)t * In + i] * A[(int64_t)i * r + j];
      for (int o = 0; o < Out; o++) b += (double)dYf[(int64_t)t * fo + off + o] * Bm[(int64_t)j * Out + o];
      u[(int64_t)t * r + j] = a;
      z[(int64_t)t * r + j] = b;
    }
  if (dB)
#pragma omp parallel for schedule(static)
    for (int j = 0; j < r; j++)
      for (int o = 0; o < Out; o++) {
        double a = 0;
        for (int t = 0; t < T; t++) a += u[(int64_t)t * r + j] * dYf[(int64_t)t * fo + off + o];
        dB[(int64_t)j * Out + o] += (float)(s * a);
      }
  if (dA)
#pragma omp parallel for schedule(static)
    for (int i = 0; i < In; i++)
      for (int j = 0; j < r; j++) {
        double a = 0;
        for (int t = 0; t < T; t++) a += (double)x[(int64_t)t * In + i] * z[(int64_t)t * r + j];
        dA[(int64_t)i * r + j] += (float)(s * a);
      }
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; t++)
    for (int i = 0; i < In; i++) {
      double a = 0;
      for (int j = 0; j < r; j++) a += z[(int64_t)t * r + j] * A[(int64_t)i * r + j];
      dX[(int64_t)t * In + i] += (float)(s * a);
    }
  free(u);
  free(z);
}

/* xn[T,D] = x*rinv (NormBackward rebuilds it the same way, BackpropEngine.cs:807-822) */
static void make_xhat(const float* x, const float* rinv, float* xh, int T, int D) {
  for (int t = 0; t < T; t++)
    for (int i = 0; i < D; i++) xh[(int64_t)t * D + i] = x[(int64_t)t * D + i] * rinv[t];
}

typedef struct {
  float *h_in, *xn1, *rinv1, *qkv_raw, *rq, *rk, *q, *k, *v, *probs, *o, *h_mid, *xn2, *rinv2, *gu, *act;
} orc_saved;

int orc_engine_step(const orc_cfg* c, float** P, float** G, const int32_t* ids, const int32_t* labels,
                    float* loss_out, float* logits_out) {
  const int T = c->B * c->S, d = c->d, D = c->D, Hq = c->Hq, Hkv = c->Hkv, F = c->F, V = c->V;
  const int qd = Hq * D, kvd = Hkv * D, nqkv = qd + 2 * kvd;
  const float scale = 1.f / sqrtf((float)D);
  float* cosT = zalloc((int64_t)c->S * D / 2);
  float* sinT = zalloc((int64_t)c->S * D / 2);
  orc_rope_tables(c->theta, D, c->S, cosT, sinT);
  orc_saved* sv = (orc_saved*)calloc((size_t)c->L, sizeof(orc_saved));
  const float* emb = P[0];

  /* ---------------- forward (BackpropEngine.cs:73-139) ---------------- */
  float* h = zalloc((int64_t)T * d);
  for (int t = 0; t < T; t++) memcpy(h + (int64_t)t * d, emb + (int64_t)ids[t] * d, sizeof(float) * d);
  for (int l = 0; l < c->L; l++) {
    orc_saved* s = &sv[l];
    s->h_in = zalloc((int64_t)T * d);
    memcpy(s->h_in, h, sizeof(float) * (size_t)T * d);
    s->xn1 = zalloc((int64_t)T * d);
    s->rinv1 = zalloc(T);
    orc_rmsnorm_fwd(h, P[GIDX(l, T_NORM1)], s->xn1, s->rinv1, T, d, c->eps);
    s->qkv_raw = zalloc((int64_t)T * nqkv);
    linear_fwd(s->xn1, P[GIDX(l, T_WQKV)], P[GIDX(l, T_BQKV)], s->qkv_raw, T, d, nqkv);
    for (int p = 0; p < 3; p++) lora_fwd_add(c, P, l, p, s->xn1, s->qkv_raw, T);
    s->q = zalloc((int64_t)T * qd);
    s->k = zalloc((int64_t)T * kvd);
    s->v = zalloc((int64_t)T * kvd);
    for (int t = 0; t < T; t++) {
      memcpy(s->q + (int64_t)t * qd, s->qkv_raw + (int64_t)t * nqkv, sizeof(float) * qd);
      memcpy(s->k + (int64_t)t * kvd, s->qkv_raw + (int64_t)t * nqkv + qd, sizeof(float) * kvd);
      memcpy(s->v + (int64_t)t * kvd, s->qkv_raw + (int64_t)t * nqkv + qd + kvd, sizeof(float) * kvd);
    }
    if (c->qk_norm) { /* per-head RMSNorm (AttentionLayer.cs:284) */
      s->rq = zalloc((int64_t)T * Hq);
      s->rk = zalloc((int64_t)T * Hkv);
      float* tq = zalloc((int64_t)T * qd);
      float* tk = zalloc((int64_t)T * kvd);
      orc_rmsnorm_fwd(s->q, P[GIDX(l, T_QN)], tq, s->rq, T * Hq, D, c->eps);
      orc_rmsnorm_fwd(s->k, P[GIDX(l, T_KN)], tk, s->rk, T * Hkv, D, c->eps);
      memcpy(s->q, tq, sizeof(float) * (size_t)T * qd);
      memcpy(s->k, tk, sizeof(float) * (size_t)T * kvd);
      free(tq);
      free(tk);
    }
    for (int b = 0; b < c->B; b++) {
      orc_rope_fwd(s->q + (int64_t)b * c->S * qd, cosT, sinT, c->S, Hq, D, c->neox);
      orc_rope_fwd(s->k + (int64_t)b * c->S * kvd, cosT, sinT, c->S, Hkv, D, c->neox);
    }
    s->probs = zalloc((int64_t)c->B * Hq * c->S * c->S);
    s->o = zalloc((int64_t)T * qd);
    orc_attention_fwd(s->q, s->k, s->v, s->probs, s->o, c->B, c->S, Hq, Hkv, D);
    float* attn = zalloc((int64_t)T * d);
    linear_fwd(s->o, P[GIDX(l, T_WO)], P[GIDX(l, T_BO)], attn, T, qd, d);
    lora_fwd_add(c, P, l, 3, s->o, attn, T);
    for (int64_t i = 0; i < (int64_t)T * d; i++) h[i] += attn[i];
    free(attn);
    s->h_mid = zalloc((int64_t)T * d);
    memcpy(s->h_mid, h, sizeof(float) * (size_t)T * d);
    s->xn2 = zalloc((int64_t)T * d);
    s->rinv2 = zalloc(T);
    orc_rmsnorm_fwd(h, P[GIDX(l, T_NORM2)], s->xn2, s->rinv2, T, d, c->eps);
    s->gu = zalloc((int64_t)T * 2 * F);
    linear_fwd(s->xn2, P[GIDX(l, T_WGU)], P[GIDX(l, T_BGU)], s->gu, T, d, 2 * F);
    lora_fwd_add(c, P, l, 4, s->xn2, s->gu, T);
    lora_fwd_add(c, P, l, 5, s->xn2, s->gu, T);
    s->act = zalloc((int64_t)T * F);
    for (int t = 0; t < T; t++)
      orc_swiglu_fwd(s->gu + (int64_t)t * 2 * F, s->gu + (int64_t)t * 2 * F + F, s->act + (int64_t)t * F, F);
    float* ffn = zalloc((int64_t)T * d);
    linear_fwd(s->act, P[GIDX(l, T_WD)], P[GIDX(l, T_BD)], ffn, T, F, d);
    lora_fwd_add(c, P, l, 6, s->act, ffn, T);
    for (int64_t i = 0; i < (int64_t)T * d; i++) h[i] += ffn[i];
    free(ffn);
  }
  float* xnf = zalloc((int64_t)T * d);
  float* rinvf = zalloc(T);
  orc_rmsnorm_fwd(h, P[1], xnf, rinvf, T, d, c->eps);
  float* logits = zalloc((int64_t)T * V);
  orc_qmatmul_f32(xnf, emb, logits, T, d, V); /* ProjectHead (BackpropEngine.cs:889-907) */
  if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t)T * V);
  *loss_out = orc_ce_loss(logits, labels, T, V, -100, 0.f);
  float* dlog = zalloc((int64_t)T * V);
  orc_ce_softmax_grad(logits, labels, dlog, T, V, -100, 0.f);

  /* ---------------- backward (BackpropEngine.cs:146-206) ---------------- */
  float* dxn = zalloc((int64_t)T * d);
  orc_grad_linear(dlog, xnf, emb, G[0], NULL, dxn, T, d, V); /* head, tied */
  float* dh = zalloc((int64_t)T * d);
  float* xh = zalloc((int64_t)T * d);
  float* tmp = zalloc((int64_t)T * d);
  float dummy_d[1];
  (void)dummy_d;
  make_xhat(h, rinvf, xh, T, d);
  float* gnf = G[1] ? G[1] : zalloc(d);
  orc_grad_rmsnorm(dxn, xh, rinvf, P[1], gnf, dh, T, d);
  if (!G[1]) free(gnf);
  for (int l = c->L - 1; l >= 0; l--) {
    orc_saved* s = &sv[l];
    /* FfnBackward, gated (BackpropEngine.cs:623-657) */
    float* dact = zalloc((int64_t)T * F);
    orc_grad_linear(dh, s->act, P[GIDX(l, T_WD)], G[GIDX(l, T_WD)], G[GIDX(l, T_BD)], dact, T, F, d);
    lora_bwd_add(c, P, G, l, 6, s->act, dh, dact, T);
    float* dgu = zalloc((int64_t)T * 2 * F);
    for (int t = 0; t < T; t++)
      orc_grad_swiglu(dact + (int64_t)t * F, s->gu + (int64_t)t * 2 * F, s->gu + (int64_t)t * 2 * F + F,
                      dgu + (int64_t)t * 2 * F, 1, F);
    float* dxn2 = zalloc((int64_t)T * d);
    orc_grad_linear(dgu, s->xn2, P[GIDX(l, T_WGU)], G[GIDX(l, T_WGU)], G[GIDX(l, T_BGU)], dxn2, T, d, 2 * F);
    lora_bwd_add(c, P, G, l, 4, s->xn2, dgu, dxn2, T);
    lora_bwd_add(c, P, G, l, 5, s->xn2, dgu, dxn2, T);
    /* NormBackward(norm2) then residual (BackpropEngine.cs:521-526) */
    make_xhat(s->h_mid, s->rinv2, xh, T, d);
    float* gn2 = G[GIDX(l, T_NORM2)] ? G[GIDX(l, T_NORM2)] : zalloc(d);
    orc_grad_rmsnorm(dxn2, xh, s->rinv2, P[GIDX(l, T_NORM2)], gn2, tmp, T, d);
    if (!G[GIDX(l, T_NORM2)]) free(gn2);
    for (int64_t i = 0; i < (int64_t)T * d; i++) dh[i] += tmp[i];
    free(dact);
    free(dgu);
    free(dxn2);
    /* AttentionBackward (BackpropEngine.cs:539-602) */
    float* dO = zalloc((int64_t)T * qd);
    orc_grad_linear(dh, s->o, P[GIDX(l, T_WO)], G[GIDX(l, T_WO)], G[GIDX(l, T_BO)], dO, T, qd, d);
    lora_bwd_add(c, P, G, l, 3, s->o, dh, dO, T);
    float* dq = zalloc((int64_t)T * qd);
    float* dk = zalloc((int64_t)T * kvd);
    float* dv = zalloc((int64_t)T * kvd);
    const int S = c->S, grp = Hq / Hkv;
    float *hO = zalloc((int64_t)S * D), *hQ = zalloc((int64_t)S * D), *hK = zalloc((int64_t)S * D), *hV = zalloc((int64_t)S * D);
    float *gQ = zalloc((int64_t)S * D), *gK = zalloc((int64_t)S * D), *gV = zalloc((int64_t)S * D);
    for (int b = 0; b < c->B; b++)
      for (int hh = 0; hh < Hq; hh++) {
        int kvh = hh / grp;
        for (int i = 0; i < S; i++) { /* SliceHead (BackpropEngine.cs:928-939) */
          int64_t tt = (int64_t)b * S + i;
          memcpy(hO + (int64_t)i * D, dO + tt * qd + hh * D, sizeof(float) * D);
          memcpy(hQ + (int64_t)i * D, s->q + tt * qd + hh * D, sizeof(float) * D);
          memcpy(hK + (int64_t)i * D, s->k + tt * kvd + kvh * D, sizeof(float) * D);
          memcpy(hV + (int64_t)i * D, s->v + tt * kvd + kvh * D, sizeof(float) * D);
        }
        const float* pr = s->probs + ((int64_t)b * Hq + hh) * S * S;
        orc_grad_attention(hO, hQ, hK, hV, pr, gQ, gK, gV, S, D, scale);
        for (int i = 0; i < S; i++) { /* AddHead (BackpropEngine.cs:954-966) */
          int64_t tt = (int64_t)b * S + i;
          for (int j = 0; j < D; j++) {
            dq[tt * qd + hh * D + j] += gQ[(int64_t)i * D + j];
            dk[tt * kvd + kvh * D + j] += gK[(int64_t)i * D + j];
            dv[tt * kvd + kvh * D + j] += gV[(int64_t)i * D + j];
          }
        }
      }
    free(hO); free(hQ); free(hK); free(hV); free(gQ); free(gK); free(gV);
    for (int b = 0; b < c->B; b++) { /* RoPE backward (BackpropEngine.cs:587-590) */
      orc_rope_bwd(dq + (int64_t)b * S * qd, cosT, sinT, S, Hq, D, c->neox);
      orc_rope_bwd(dk + (int64_t)b * S * kvd, cosT, sinT, S, Hkv, D, c->neox);
    }
    if (c->qk_norm) { /* per-head RMSNorm backward, same slot math as a7 */
      float* rq = s->rq;
      float* rk = s->rk;
      float* raw_q = zalloc((int64_t)T * qd);
      float* raw_k = zalloc((int64_t)T * kvd);
      for (int t = 0; t < T; t++) {
        memcpy(raw_q + (int64_t)t * qd, s->qkv_raw + (int64_t)t * nqkv, sizeof(float) * qd);
        memcpy(raw_k + (int64_t)t * kvd, s->qkv_raw + (int64_t)t * nqkv + qd, sizeof(float) * kvd);
      }
      float* xq = zalloc((int64_t)T * qd);
      float* xk = zalloc((int64_t)T * kvd);
      make_xhat(raw_q, rq, xq, T * Hq, D);
      make_xhat(raw_k, rk, xk, T * Hkv, D);
      float* gq = G[GIDX(l, T_QN)] ? G[GIDX(l, T_QN)] : zalloc(D);
      float* gk = G[GIDX(l, T_KN)] ? G[GIDX(l, T_KN)] : zalloc(D);
      float* oq = zalloc((int64_t)T * qd);
      float* ok = zalloc((int64_t)T * kvd);
      orc_grad_rmsnorm(dq, xq, rq, P[GIDX(l, T_QN)], gq, oq, T * Hq, D);
      orc_grad_rmsnorm(dk, xk, rk, P[GIDX(l, T_KN)], gk, ok, T * Hkv, D);
      memcpy(dq, oq, sizeof(float) * (size_t)T * qd);
      memcpy(dk, ok, sizeof(float) * (size_t)T * kvd);
      if (!G[GIDX(l, T_QN)]) free(gq);
      if (!G[GIDX(l, T_KN)]) free(gk);
      free(raw_q); free(raw_k); free(xq); free(xk); free(oq); free(ok);
    }
    /* fused q|k|v linear backward == the three LinearBackward calls summed (BackpropEngine.cs:593-600) */
    float* dqkv = zalloc((int64_t)T * nqkv);
    for (int t = 0; t < T; t++) {
      memcpy(dqkv + (int64_t)t * nqkv, dq + (int64_t)t * qd, sizeof(float) * qd);
      memcpy(dqkv + (int64_t)t * nqkv + qd, dk + (int64_t)t * kvd, sizeof(float) * kvd);
      memcpy(dqkv + (int64_t)t * nqkv + qd + kvd, dv + (int64_t)t * kvd, sizeof(float) * kvd);
    }
    float* dxn1 = zalloc((int64_t)T * d);
    orc_grad_linear(dqkv, s->xn1, P[GIDX(l, T_WQKV)], G[GIDX(l, T_WQKV)], G[GIDX(l, T_BQKV)], dxn1, T, d, nqkv);
    for (int p = 0; p < 3; p++) lora_bwd_add(c, P, G, l, p, s->xn1, dqkv, dxn1, T);
    make_xhat(s->h_in, s->rinv1, xh, T, d);
    float* gn1 = G[GIDX(l, T_NORM1)] ? G[GIDX(l, T_NORM1)] : zalloc(d);
    orc_grad_rmsnorm(dxn1, xh, s->rinv1, P[GIDX(l, T_NORM1)], gn1, tmp, T, d);
    if (!G[GIDX(l, T_NORM1)]) free(gn1);
    for (int64_t i = 0; i < (int64_t)T * d; i++) dh[i] += tmp[i];
    free(dO); free(dq); free(dk); free(dv); free(dqkv); free(dxn1);
  }
  if (G[0]) orc_grad_embedding(dh, ids, G[0], T, d); /* BackpropEngine.cs:203-205 */

  for (int l = 0; l < c->L; l++) {
    orc_saved* s = &sv[l];
    free(s->h_in); free(s->xn1); free(s->rinv1); free(s->qkv_raw); free(s->rq); free(s->rk);
    free(s->q); free(s->k); free(s->v); free(s->probs); free(s->o); free(s->h_mid); free(s->xn2);
    free(s->rinv2); free(s->gu); free(s->act);
  }
  free(sv); free(h); free(xnf); free(rinvf); free(logits); free(dlog); free(dxn); free(dh); free(xh);
  free(tmp); free(cosT); free(sinT);
  return 0;
}
