/*
 * cpu_twin.c — timing twin of the reference's AVX2/FMA CPU training path.
 *
 * TEST AND MEASUREMENT INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg runs it to time
 * what the reference's own CPU tiers would take for one block and the LM head of the
 * benchmark's LoRA step.  It is a C restatement of those tiers' loop structure, vector
 * width and thread partitioning (OpenMP standing in for Parallel.For), not a checker:
 * parity is established by oracle.c / engine.c.
 *
 *   forward linear through the Q8_0 base  QuantizedMatMulQ8_0_Parallel_FMA: rows in
 *                                         parallel, VecDotQ8_0_FMA per output column
 *                                         (QuantizationKernels.Q8.cs:69-106, 556-573)
 *   linear backward (dX, and dW for the   GradientKernels.Linear_FMA: dX rows in parallel,
 *   adapters)                             dW output rows in parallel, 8-wide FMA axpys
 *                                         (GradientKernels.cs:210-291)
 *   RMSNorm forward / backward            RMSNormParamAVX2 / RMSNormRowAVX2 rows
 *                                         (NormKernels.cs:13-60), RMSNorm_Scalar backward
 *                                         (GradientKernels.cs:303-337), serial
 *   attention forward                     BackpropEngine.ForwardAttention: (batch, head) in
 *                                         parallel, 8-wide dots (BackpropEngine.cs:237-388)
 *   attention backward                    Parallel.For over batch rows, heads serial,
 *                                         Attention_Scalar per head over the full S x S
 *                                         (BackpropEngine.cs:563-582, GradientKernels.cs:408-481)
 *   SwiGLU, RoPE, CE                      the serial scalar loops (BackpropEngine.cs:623-657,
 *                                         RoPE.cs:286-347, Gradients.cs:33-84)
 *   AdamW                                 AdamWUpdate_AVX2 (TrainingKernels.cs:19-70)
 *
 * The reference has no backward through a quantised base; the twin takes the base's dX
 * with Linear_FMA's dX loop on the dequantised fp32 weight (decoded inside the timed
 * region, as ReadQ8_0_Scalar would).  Built -O3 -mavx2 -mfma -fopenmp.
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

typedef struct {
  int d, Hq, Hkv, D, F, V, B, S, r;
  int head_tokens; /* tokens the head is timed on (its cost is linear in tokens) */
  int full;        /* full-parameter step: base weight gradients too (Linear_FMA dW), no adapters */
} twin_cfg;

static double now(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec + 1e-9 * ts.tv_nsec;
}

static float half_to_float(uint16_t h) { return _cvtsh_ss(h); }

static float hsum256(__m256 v) {
  __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
  lo = _mm_add_ps(lo, hi);
  lo = _mm_hadd_ps(lo, lo);
  lo = _mm_hadd_ps(lo, lo);
  return _mm_cvtss_f32(lo);
}

/* VecDotQ8_0_FMA (QuantizationKernels.Q8.cs:69-106) */
static float vecdot_q8_0_fma(const float* in, const uint8_t* raw, int col, int K) {
  const int nb = K / 32;
  __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
  for (int b = 0; b < nb; b++) {
    const uint8_t* blk = raw + ((int64_t)col * nb + b) * 34;
    __m256 vd = _mm256_set1_ps(half_to_float((uint16_t)(blk[0] | blk[1] << 8)));
    const int8_t* q = (const int8_t*)(blk + 2);
    const float* x = in + b * 32;
    for (int i = 0; i < 32; i += 16) {
      __m256 w0 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(q + i))));
      __m256 w1 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(q + i + 8))));
      a0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i), _mm256_mul_ps(w0, vd), a0);
      a1 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i + 8), _mm256_mul_ps(w1, vd), a1);
    }
  }
  return (float)(double)hsum256(_mm256_add_ps(a0, a1));
}

/* QuantizedMatMulQ8_0_Parallel_FMA: out[M,N] = in[M,K] . W^T (QuantizationKernels.Q8.cs:556-573) */
static void qmatmul_q8_0(const float* in, const uint8_t* raw, float* out, int M, int K, int N) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) out[(int64_t)m * N + n] = vecdot_q8_0_fma(in + (int64_t)m * K, raw, n, K);
}

static void axpy8(float* y, const float* x, float a, int n) {
  __m256 va = _mm256_set1_ps(a);
  int i = 0;
  for (; i <= n - 8; i += 8) _mm256_storeu_ps(y + i, _mm256_fmadd_ps(va, _mm256_loadu_ps(x + i), _mm256_loadu_ps(y + i)));
  for (; i < n; i++) y[i] += a * x[i];
}

/* Linear_FMA (GradientKernels.cs:210-291): dX[B,In] = dY W (W [Out,In]); dW += dY^T X */
static void linear_bwd_fma(const float* dY, const float* X, const float* W, float* dW, float* dX, int Bn, int In, int Out) {
  if (dX) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < Bn; b++) {
      float* row = dX + (int64_t)b * In;
      memset(row, 0, sizeof(float) * In);
      for (int o = 0; o < Out; o++) axpy8(row, W + (int64_t)o * In, dY[(int64_t)b * Out + o], In);
    }
  }
  if (dW) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int o = 0; o < Out; o++)
      for (int b = 0; b < Bn; b++) axpy8(dW + (int64_t)o * In, X + (int64_t)b * In, dY[(int64_t)b * Out + o], In);
  }
}

/* y[T,N] (+)= x[T,K] Wt where Wt is [K][N] (the adapters' x A and u B products), rows in parallel */
static void matmul_rows(const float* x, const float* Wt, float* y, int T, int K, int N, float alpha, int accumulate) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; t++) {
    float acc[8192];
    memset(acc, 0, sizeof(float) * N);
    for (int k = 0; k < K; k++) axpy8(acc, Wt + (int64_t)k * N, x[(int64_t)t * K + k], N);
    float* yr = y + (int64_t)t * N;
    for (int n = 0; n < N; n++) yr[n] = (accumulate ? yr[n] : 0.f) + alpha * acc[n];
  }
}

static void dequant_q8_0(const uint8_t* raw, float* out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < n / 32; b++) {
    const uint8_t* blk = raw + b * 34;
    float d = half_to_float((uint16_t)(blk[0] | blk[1] << 8));
    for (int j = 0; j < 32; j++) out[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
  }
}

/* RMSNormParamAVX2 + RMSNormRowAVX2 (NormKernels.cs:13-60), rows serial */
static void rmsnorm_fwd(const float* x, const float* w, float* y, float* rinv, int T, int D) {
  for (int t = 0; t < T; t++) {
    const float* r = x + (int64_t)t * D;
    __m256 s = _mm256_setzero_ps();
    int i = 0;
    for (; i <= D - 8; i += 8) { __m256 v = _mm256_loadu_ps(r + i); s = _mm256_add_ps(s, _mm256_mul_ps(v, v)); }
    float ss = hsum256(s);
    for (; i < D; i++) ss += r[i] * r[i];
    float ri = 1.f / sqrtf(ss / D + 1e-6f);
    rinv[t] = ri;
    for (i = 0; i < D; i++) y[(int64_t)t * D + i] = r[i] * ri * w[i];
  }
}

/* RMSNorm_Scalar backward (GradientKernels.cs:303-337) */
static void rmsnorm_bwd(const float* dY, const float* xn, const float* rinv, const float* w, float* dw, float* dX, int T, int D) {
  for (int t = 0; t < T; t++) {
    const float *dy = dY + (int64_t)t * D, *x = xn + (int64_t)t * D;
    float* dx = dX + (int64_t)t * D;
    for (int i = 0; i < D; i++) dw[i] += dy[i] * x[i];
    float dot = 0.f;
    for (int i = 0; i < D; i++) dot += dy[i] * w[i] * x[i];
    dot /= (float)D;
    for (int i = 0; i < D; i++) dx[i] = rinv[t] * (dy[i] * w[i] - x[i] * dot);
  }
}

/* RoPE (RoPE.cs:168-347), NeoX pairing, serial */
static void rope(float* x, const float* cs, const float* sn, int Bn, int S, int H, int D, int inverse) {
  const int half = D / 2;
  for (int b = 0; b < Bn; b++)
    for (int s = 0; s < S; s++)
      for (int h = 0; h < H; h++) {
        float* v = x + (((int64_t)b * S + s) * H + h) * D;
        for (int i = 0; i < half; i++) {
          float c = cs[s * half + i], si = inverse ? -sn[s * half + i] : sn[s * half + i];
          float a = v[i], bb = v[i + half];
          v[i] = a * c - bb * si;
          v[i + half] = bb * c + a * si;
        }
      }
}

/* ForwardAttention (BackpropEngine.cs:237-388): (b, h) in parallel, causal rows, 8-wide dots */
static void attention_fwd(const float* q, const float* k, const float* v, float* probs, float* out, int Bn, int S, int Hq,
                          int Hkv, int D) {
  const float scale = 1.f / sqrtf((float)D);
  const int grp = Hq / Hkv;
#pragma omp parallel for schedule(dynamic, 1)
  for (int bh = 0; bh < Bn * Hq; bh++) {
    const int b = bh / Hq, h = bh % Hq, kvh = h / grp;
    for (int i = 0; i < S; i++) {
      float* p = probs + ((int64_t)bh * S + i) * S;
      const float* qi = q + (((int64_t)b * S + i) * Hq + h) * D;
      float mx = -INFINITY;
      for (int j = 0; j <= i; j++) {
        const float* kj = k + (((int64_t)b * S + j) * Hkv + kvh) * D;
        __m256 acc = _mm256_setzero_ps();
        for (int d = 0; d < D; d += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(qi + d), _mm256_loadu_ps(kj + d), acc);
        float s = hsum256(acc) * scale;
        p[j] = s;
        if (s > mx) mx = s;
      }
      float sum = 0.f;
      for (int j = 0; j <= i; j++) { p[j] = expf(p[j] - mx); sum += p[j]; }
      const float inv = 1.f / sum;
      for (int j = 0; j <= i; j++) p[j] *= inv;
      float* o = out + ((int64_t)b * S + i) * Hq * D + h * D;
      memset(o, 0, sizeof(float) * D);
      for (int j = 0; j <= i; j++) axpy8(o, v + (((int64_t)b * S + j) * Hkv + kvh) * D, p[j], D);
    }
  }
}

/* Attention_Scalar (GradientKernels.cs:408-481) on one head, full S x S */
static void attention_bwd_head(const float* dO, const float* q, const float* k, const float* v, const float* P,
                               float* dQ, float* dK, float* dV, float* dP, int S, int D, float scale) {
  for (int j = 0; j < S; j++)
    for (int d = 0; d < D; d++) {
      float s = 0.f;
      for (int i = 0; i < S; i++) s += P[(int64_t)i * S + j] * dO[i * D + d];
      dV[j * D + d] = s;
    }
  for (int i = 0; i < S; i++)
    for (int j = 0; j < S; j++) {
      float s = 0.f;
      for (int d = 0; d < D; d++) s += dO[i * D + d] * v[j * D + d];
      dP[(int64_t)i * S + j] = s;
    }
  for (int i = 0; i < S; i++) {
    float dot = 0.f;
    for (int j = 0; j < S; j++) dot += P[(int64_t)i * S + j] * dP[(int64_t)i * S + j];
    for (int j = 0; j < S; j++) dP[(int64_t)i * S + j] = P[(int64_t)i * S + j] * (dP[(int64_t)i * S + j] - dot);
  }
  for (int i = 0; i < S; i++)
    for (int d = 0; d < D; d++) {
      float sq = 0.f, sk = 0.f;
      for (int j = 0; j < S; j++) {
        sq += dP[(int64_t)i * S + j] * k[j * D + d];
        sk += dP[(int64_t)j * S + i] * q[j * D + d];
      }
      dQ[i * D + d] = sq * scale;
      dK[i * D + d] = sk * scale;
    }
}

/* AttentionBackward driver: Parallel.For over batch rows, heads serial (BackpropEngine.cs:563-582) */
static void attention_bwd(const float* dO, const float* q, const float* k, const float* v, const float* probs, float* dq,
                          float* dk, float* dv, int Bn, int S, int Hq, int Hkv, int D) {
  const int grp = Hq / Hkv;
  const float scale = 1.f / sqrtf((float)D);
  memset(dq, 0, sizeof(float) * (size_t)Bn * S * Hq * D);
  memset(dk, 0, sizeof(float) * (size_t)Bn * S * Hkv * D);
  memset(dv, 0, sizeof(float) * (size_t)Bn * S * Hkv * D);
#pragma omp parallel for schedule(dynamic, 1)
  for (int b = 0; b < Bn; b++) {
    float* buf = (float*)malloc(sizeof(float) * ((size_t)7 * S * D + (size_t)S * S));
    float *hO = buf, *hQ = hO + S * D, *hK = hQ + S * D, *hV = hK + S * D, *gQ = hV + S * D, *gK = gQ + S * D,
          *gV = gK + S * D, *dP = gV + S * D;
    for (int h = 0; h < Hq; h++) {
      const int kvh = h / grp;
      for (int i = 0; i < S; i++) { /* SliceHead */
        const int64_t t = (int64_t)b * S + i;
        memcpy(hO + i * D, dO + (t * Hq + h) * D, sizeof(float) * D);
        memcpy(hQ + i * D, q + (t * Hq + h) * D, sizeof(float) * D);
        memcpy(hK + i * D, k + (t * Hkv + kvh) * D, sizeof(float) * D);
        memcpy(hV + i * D, v + (t * Hkv + kvh) * D, sizeof(float) * D);
      }
      attention_bwd_head(hO, hQ, hK, hV, probs + ((int64_t)b * Hq + h) * S * S, gQ, gK, gV, dP, S, D, scale);
      for (int i = 0; i < S; i++) { /* AddHead */
        const int64_t t = (int64_t)b * S + i;
        for (int d = 0; d < D; d++) {
          dq[(t * Hq + h) * D + d] += gQ[i * D + d];
          dk[(t * Hkv + kvh) * D + d] += gK[i * D + d];
          dv[(t * Hkv + kvh) * D + d] += gV[i * D + d];
        }
      }
    }
    free(buf);
  }
}

/* CrossEntropySoftmax (Gradients.cs:33-84), serial rows, exact exp */
static void ce_grad(const float* z, const int32_t* lab, float* dz, int T, int V) {
  const float scale = 1.f / (float)T;
  for (int t = 0; t < T; t++) {
    const float* r = z + (int64_t)t * V;
    float* d = dz + (int64_t)t * V;
    float mx = r[0];
    for (int v = 1; v < V; v++) if (r[v] > mx) mx = r[v];
    float sum = 0.f;
    for (int v = 0; v < V; v++) { d[v] = expf(r[v] - mx); sum += d[v]; }
    const float inv = 1.f / sum;
    for (int v = 0; v < V; v++) d[v] *= inv;
    d[lab[t]] -= 1.f;
    for (int v = 0; v < V; v++) d[v] *= scale;
  }
}

/* AdamWUpdate_AVX2 (TrainingKernels.cs:19-70) */
static void adamw_avx2(float* p, const float* g, float* m, float* v, int64_t n, float lr) {
  const float b1 = 0.9f, b2 = 0.95f, bc1 = 0.1f, bc2 = 0.05f, eps = 1e-8f, wd = 0.1f;
  const __m256 vb1 = _mm256_set1_ps(b1), vb2 = _mm256_set1_ps(b2), v1b1 = _mm256_set1_ps(1 - b1),
               v1b2 = _mm256_set1_ps(1 - b2), vlr = _mm256_set1_ps(lr), veps = _mm256_set1_ps(eps),
               vwd = _mm256_set1_ps(wd), vc1 = _mm256_set1_ps(bc1), vc2 = _mm256_set1_ps(bc2);
  int64_t i = 0;
  for (; i <= n - 8; i += 8) {
    __m256 vg = _mm256_loadu_ps(g + i);
    __m256 vm = _mm256_add_ps(_mm256_mul_ps(vb1, _mm256_loadu_ps(m + i)), _mm256_mul_ps(v1b1, vg));
    __m256 vv = _mm256_add_ps(_mm256_mul_ps(vb2, _mm256_loadu_ps(v + i)), _mm256_mul_ps(v1b2, _mm256_mul_ps(vg, vg)));
    _mm256_storeu_ps(m + i, vm);
    _mm256_storeu_ps(v + i, vv);
    __m256 vd = _mm256_loadu_ps(p + i);
    __m256 upd = _mm256_mul_ps(vlr, _mm256_add_ps(_mm256_div_ps(_mm256_div_ps(vm, vc1), _mm256_add_ps(_mm256_sqrt_ps(_mm256_div_ps(vv, vc2)), veps)),
                                                  _mm256_mul_ps(vwd, vd)));
    _mm256_storeu_ps(p + i, _mm256_sub_ps(vd, upd));
  }
}

static float* fill(int64_t n, float sd, uint64_t* st) {
  float* a = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
  for (int64_t i = 0; i < n; i++) {
    *st = *st * 6364136223846793005ull + 1442695040888963407ull;
    a[i] = sd * ((float)((*st >> 40) & 0xFFFFFF) / 8388608.f - 1.f);
  }
  return a;
}

static uint8_t* quant_q8(const float* w, int64_t n) {
  uint8_t* raw = (uint8_t*)malloc((size_t)n / 32 * 34);
  for (int64_t b = 0; b < n / 32; b++) {
    float amax = 0.f;
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(w[b * 32 + j]));
    float d = amax / 127.f;
    uint16_t h = _cvtss_sh(d, 0);
    raw[b * 34] = (uint8_t)h;
    raw[b * 34 + 1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 32; j++) raw[b * 34 + 2 + j] = (uint8_t)(int8_t)(d > 0 ? roundf(w[b * 32 + j] / d) : 0);
  }
  return raw;
}

/* One LoRA projection y = x W^T + s (x A) B forward: W Q8_0 [Out][In] */
typedef struct { int In, Out; uint8_t* W; float *A, *Bm, *dA, *dB, *mA, *vA, *mB, *vB; } proj_t;

static void proj_make(proj_t* p, int In, int Out, int r, uint64_t* st) {
  p->In = In; p->Out = Out;
  float* w = fill((int64_t)In * Out, 0.035f, st);
  p->W = quant_q8(w, (int64_t)In * Out);
  free(w);
  p->A = fill((int64_t)In * r, 1.f / sqrtf((float)In), st);
  p->Bm = fill((int64_t)r * Out, 1e-3f, st);
  p->dA = calloc((size_t)In * r, 4); p->dB = calloc((size_t)r * Out, 4);
  p->mA = calloc((size_t)In * r, 4); p->vA = calloc((size_t)In * r, 4);
  p->mB = calloc((size_t)r * Out, 4); p->vB = calloc((size_t)r * Out, 4);
}

/* VecDotF32 FMA tier (QuantizationKernels.Float.cs:11-55): out[M,N] = in[M,K] . W^T, fp32 rows [N][K] */
static void matmul_f32(const float* in, const float* W, float* out, int M, int K, int N) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      __m256 a = _mm256_setzero_ps();
      for (int k = 0; k < K; k += 8)
        a = _mm256_fmadd_ps(_mm256_loadu_ps(in + (int64_t)m * K + k), _mm256_loadu_ps(W + (int64_t)n * K + k), a);
      out[(int64_t)m * N + n] = hsum256(a);
    }
}

/* r == 0: the full-parameter step's fp32 weight (held here as its Q8_0 bytes, decoded to wtmp) */
static void proj_fwd(const proj_t* p, const float* x, float* u, float* y, int T, int r, float s, float* wtmp) {
  if (r == 0) {
    dequant_q8_0(p->W, wtmp, (int64_t)p->In * p->Out);
    matmul_f32(x, wtmp, y, T, p->In, p->Out);
    return;
  }
  qmatmul_q8_0(x, p->W, y, T, p->In, p->Out);
  matmul_rows(x, p->A, u, T, p->In, r, 1.f, 0);
  matmul_rows(u, p->Bm, y, T, r, p->Out, s, 1);
}

/* dX = dY W + s (dY B^T) A^T; dB += s u^T dY; dA += s x^T z */
static void proj_bwd(proj_t* p, const float* dY, const float* x, const float* u, float* dX, float* z, float* wtmp, int T,
                     int r, float s, float* dWfull) {
  dequant_q8_0(p->W, wtmp, (int64_t)p->In * p->Out);
  linear_bwd_fma(dY, x, wtmp, dWfull, dX, T, p->In, p->Out);
  if (dWfull) return; /* full-parameter step: no adapters */
  linear_bwd_fma(dY, u, p->Bm, p->dB, z, T, r, p->Out); /* z = dY B^T (B as an [r][Out] weight), dB += dY^T u */
#pragma omp parallel for schedule(static)
  for (int i = 0; i < p->In; i++) /* dA[i][j] += s sum_t x[t][i] z[t][j] */
    for (int t = 0; t < T; t++) axpy8(p->dA + (int64_t)i * r, z + (int64_t)t * r, s * x[(int64_t)t * p->In + i], r);
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; t++) /* dX[t] += s sum_j z[t][j] A[:, j] */
    for (int i = 0; i < p->In; i++) {
      float a = 0.f;
      for (int j = 0; j < r; j++) a += z[(int64_t)t * r + j] * p->A[(int64_t)i * r + j];
      dX[(int64_t)t * p->In + i] += s * a;
    }
}

/*
 * Times one decoder block (forward + backward + AdamW of its adapters) at the given shape
 * and the head (final norm, LM-head forward through the Q8_0 table, CE, head dX) on the
 * first head_tokens tokens.  out[0] = block seconds, out[1] = head seconds, out[2] = threads.
 */
int twin_time_step(const twin_cfg* c, double* out) {
  const int T = c->B * c->S, d = c->d, Hq = c->Hq, Hkv = c->Hkv, D = c->D, F = c->F, V = c->V, r = c->r;
  const int qd = Hq * D, kvd = Hkv * D;
  const float s = 2.f;
  const int rr = c->full ? 0 : r;
  uint64_t st = 12345;
  proj_t P[7];
  const int ins[7] = {d, d, d, qd, d, d, F}, outs[7] = {qd, kvd, kvd, d, F, F, d};
  for (int i = 0; i < 7; i++) proj_make(&P[i], ins[i], outs[i], r, &st);
  float* h = fill((int64_t)T * d, 1.f, &st);
  float* w1 = fill(d, 1.f, &st);
  float *xn = calloc((size_t)T * d, 4), *rinv = calloc(T, 4), *q = calloc((size_t)T * qd, 4), *k = calloc((size_t)T * kvd, 4),
        *v = calloc((size_t)T * kvd, 4), *o = calloc((size_t)T * qd, 4), *attn = calloc((size_t)T * d, 4);
  float* probs = calloc((size_t)c->B * Hq * c->S * c->S, 4);
  float *gate = calloc((size_t)T * F, 4), *up = calloc((size_t)T * F, 4), *act = calloc((size_t)T * F, 4);
  float* u[7];
  for (int i = 0; i < 7; i++) u[i] = calloc((size_t)T * r, 4);
  float *cs = calloc((size_t)c->S * D / 2, 4), *sn = calloc((size_t)c->S * D / 2, 4);
  for (int p = 0; p < c->S; p++)
    for (int i = 0; i < D / 2; i++) {
      float a = p * (1.f / powf(1e6f, 2.f * i / D));
      cs[p * D / 2 + i] = cosf(a);
      sn[p * D / 2 + i] = sinf(a);
    }
  float *dh = fill((int64_t)T * d, 1e-3f, &st), *dx = calloc((size_t)T * qd > (size_t)T * F ? (size_t)T * qd : (size_t)T * F, 4);
  float *dq = calloc((size_t)T * qd, 4), *dk = calloc((size_t)T * kvd, 4), *dv = calloc((size_t)T * kvd, 4);
  float *dg = calloc((size_t)T * F, 4), *du = calloc((size_t)T * F, 4), *z = calloc((size_t)T * r, 4);
  float *dw = calloc(d, 4), *tmp = calloc((size_t)T * d, 4);
  size_t wmax = (size_t)F * d > (size_t)qd * d ? (size_t)F * d : (size_t)qd * d;
  float* wtmp = malloc(sizeof(float) * wmax);
  float* dWf = c->full ? calloc(wmax, 4) : NULL;

  double t0 = now();
  /* ---- forward of one block (BackpropEngine.ForwardAndRecord) */
  rmsnorm_fwd(h, w1, xn, rinv, T, d);
  proj_fwd(&P[0], xn, u[0], q, T, rr, s, wtmp);
  proj_fwd(&P[1], xn, u[1], k, T, rr, s, wtmp);
  proj_fwd(&P[2], xn, u[2], v, T, rr, s, wtmp);
  rope(q, cs, sn, c->B, c->S, Hq, D, 0);
  rope(k, cs, sn, c->B, c->S, Hkv, D, 0);
  attention_fwd(q, k, v, probs, o, c->B, c->S, Hq, Hkv, D);
  proj_fwd(&P[3], o, u[3], attn, T, rr, s, wtmp);
  for (int64_t i = 0; i < (int64_t)T * d; i++) attn[i] += h[i];
  rmsnorm_fwd(attn, w1, xn, rinv, T, d);
  proj_fwd(&P[4], xn, u[4], gate, T, rr, s, wtmp);
  proj_fwd(&P[5], xn, u[5], up, T, rr, s, wtmp);
  for (int64_t i = 0; i < (int64_t)T * F; i++) act[i] = gate[i] / (1.f + expf(-gate[i])) * up[i];
  proj_fwd(&P[6], act, u[6], tmp, T, rr, s, wtmp);
  /* ---- backward (BackpropEngine.Backward: FfnBackward, NormBackward, AttentionBackward) */
  proj_bwd(&P[6], dh, act, u[6], dx, z, wtmp, T, r, s, dWf);
  for (int64_t i = 0; i < (int64_t)T * F; i++) { /* SwiGLU backward (BackpropEngine.cs:623-657) */
    float g = gate[i], sg = 1.f / (1.f + expf(-g));
    du[i] = dx[i] * g * sg;
    dg[i] = dx[i] * up[i] * sg * (1.f + g * (1.f - sg));
  }
  proj_bwd(&P[4], dg, xn, u[4], tmp, z, wtmp, T, r, s, dWf);
  proj_bwd(&P[5], du, xn, u[5], dx, z, wtmp, T, r, s, dWf);
  for (int64_t i = 0; i < (int64_t)T * d; i++) tmp[i] += dx[i];
  rmsnorm_bwd(tmp, xn, rinv, w1, dw, dx, T, d);
  proj_bwd(&P[3], dh, o, u[3], dx, z, wtmp, T, r, s, dWf);
  attention_bwd(dx, q, k, v, probs, dq, dk, dv, c->B, c->S, Hq, Hkv, D);
  rope(dq, cs, sn, c->B, c->S, Hq, D, 1);
  rope(dk, cs, sn, c->B, c->S, Hkv, D, 1);
  proj_bwd(&P[0], dq, xn, u[0], dx, z, wtmp, T, r, s, dWf);
  proj_bwd(&P[1], dk, xn, u[1], tmp, z, wtmp, T, r, s, dWf);
  proj_bwd(&P[2], dv, xn, u[2], tmp, z, wtmp, T, r, s, dWf);
  rmsnorm_bwd(dx, xn, rinv, w1, dw, tmp, T, d);
  for (int i = 0; i < 7 && !c->full; i++) {
    adamw_avx2(P[i].A, P[i].dA, P[i].mA, P[i].vA, (int64_t)P[i].In * r, 1e-3f);
    adamw_avx2(P[i].Bm, P[i].dB, P[i].mB, P[i].vB, (int64_t)r * P[i].Out, 1e-3f);
  }
  if (c->full) { /* AdamW over the block's weights (the 7 projections' element count) */
    float *mm = calloc(wmax, 4), *vv = calloc(wmax, 4);
    for (int i = 0; i < 7; i++) adamw_avx2(wtmp, dWf, mm, vv, (int64_t)P[i].In * P[i].Out, 1e-4f);
    free(mm);
    free(vv);
  }
  double t1 = now();

  /* ---- head: final norm, logits through the Q8_0 table, CE, head dX */
  float* E = fill((int64_t)V * d, 0.035f, &st);
  uint8_t* Eq = quant_q8(E, (int64_t)V * d);
  const int Th = c->head_tokens > 0 && c->head_tokens < T ? c->head_tokens : T;
  float *logits = malloc(sizeof(float) * (size_t)Th * V), *dlog = malloc(sizeof(float) * (size_t)Th * V);
  int32_t* lab = malloc(sizeof(int32_t) * Th);
  for (int t = 0; t < Th; t++) lab[t] = (int32_t)((t * 2654435761u) % (uint32_t)V);
  double t2 = now();
  rmsnorm_fwd(h, w1, xn, rinv, Th, d);
  qmatmul_q8_0(xn, Eq, logits, Th, d, V);
  ce_grad(logits, lab, dlog, Th, V);
  dequant_q8_0(Eq, E, (int64_t)V * d);
  linear_bwd_fma(dlog, NULL, E, NULL, tmp, Th, d, V);
  rmsnorm_bwd(tmp, xn, rinv, w1, dw, dx, Th, d);
  double t3 = now();

  out[0] = t1 - t0;
  out[1] = t3 - t2;
  out[2] = omp_get_max_threads();
  for (int i = 0; i < 7; i++) {
    free(P[i].W); free(P[i].A); free(P[i].Bm); free(P[i].dA); free(P[i].dB);
    free(P[i].mA); free(P[i].vA); free(P[i].mB); free(P[i].vB); free(u[i]);
  }
  free(h); free(w1); free(xn); free(rinv); free(q); free(k); free(v); free(o); free(attn); free(probs);
  free(gate); free(up); free(act); free(cs); free(sn); free(dh); free(dx); free(dq); free(dk); free(dv);
  free(dg); free(du); free(z); free(dw); free(tmp); free(wtmp); free(dWf); free(E); free(Eq); free(logits); free(dlog); free(lab);
  return 0;
}
