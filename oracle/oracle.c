/*
 * oracle.c — CPU restatement of SharpMind's training-path kernels.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Citations are relative to the
 * SharpMind repository root.  Compiled with -O2 -ffp-contract=off so that
 * float expressions round exactly as the C# scalar tiers do (RyuJIT does not
 * contract a*b+c into an FMA).
 *
 * Parity pins (tests/test_oracle_*.py): every function below is checked
 * against reference golden data, a reference known-answer test, the
 * reference's own C tool (oracle/_ref), or an independent mathematical check
 * (closed form in float64, finite differences, IEEE conversion identities).
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* .NET System.Random(int seed): the legacy seeded generator (Knuth's        */
/* subtractive method, "Numerical Recipes" ran3 with MBIG = int.MaxValue,    */
/* MSEED = 161803398).  Seeded Random instances in .NET 6+ keep this         */
/* algorithm for compatibility; the reference seeds its golden data with it  */
/* (SharpMind.Tests/Quantization/VecDotTests.cs:524-590,                     */
/* tools/ReferenceDataGenerator/vecdot_ref.cs:1620-1629) and its weight init  */
/* (SharpMind.Training/WeightInitializer.cs:27-45).                          */
/* ------------------------------------------------------------------------ */
#define NET_MBIG 2147483647
#define NET_MSEED 161803398

void orc_rng_init(orc_rng* r, int32_t seed) {
  int32_t subtraction = (seed == INT32_MIN) ? NET_MBIG : (seed < 0 ? -seed : seed);
  int32_t mj = NET_MSEED - subtraction;
  r->seed[55] = mj;
  int32_t mk = 1;
  int ii = 0;
  for (int i = 1; i < 55; i++) {
    ii += 21;
    if (ii >= 55) ii -= 55;
    r->seed[ii] = mk;
    mk = mj - mk;
    if (mk < 0) mk += NET_MBIG;
    mj = r->seed[ii];
  }
  for (int k = 1; k < 5; k++) {
    for (int i = 1; i < 56; i++) {
      int n = i + 30;
      if (n >= 55) n -= 55;
      r->seed[i] -= r->seed[1 + n];
      if (r->seed[i] < 0) r->seed[i] += NET_MBIG;
    }
  }
  r->inext = 0;
  r->inextp = 21;
}

int32_t orc_rng_sample(orc_rng* r) {
  int a = r->inext + 1;
  if (a >= 56) a = 1;
  int b = r->inextp + 1;
  if (b >= 56) b = 1;
  int32_t ret = r->seed[a] - r->seed[b];
  if (ret == NET_MBIG) ret--;
  if (ret < 0) ret += NET_MBIG;
  r->seed[a] = ret;
  r->inext = a;
  r->inextp = b;
  return ret;
}

double orc_rng_next_double(orc_rng* r) { return orc_rng_sample(r) * (1.0 / NET_MBIG); }

void orc_rng_next_bytes(orc_rng* r, uint8_t* buf, int64_t n) {
  for (int64_t i = 0; i < n; i++) buf[i] = (uint8_t)orc_rng_sample(r);
}

void orc_fill_normal(orc_rng* r, float* data, int64_t n, float std) {
  /* WeightInitializer.FillNormal: Box-Muller, double precision, one draw per pair of samples */
  for (int64_t i = 0; i < n; i++) {
    double u1 = 1.0 - orc_rng_next_double(r);
    double u2 = orc_rng_next_double(r);
    data[i] = (float)((double)std * sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u2));
  }
}

void orc_fill_uniform_pm1(orc_rng* r, float* data, int64_t n) {
  for (int64_t i = 0; i < n; i++) data[i] = (float)(orc_rng_next_double(r) * 2 - 1);
}

/* ------------------------------------------------------------------------ */
/* half <-> float                                                            */
/* ------------------------------------------------------------------------ */
static float bits_to_float(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t float_to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

float orc_half_to_float(uint16_t half) {
  /* HalfToFloat_Scalar, QuantizationKernels.cs:117-146 */
  int exp5 = (half >> 10) & 0x1F;
  if (exp5 == 0) {
    uint32_t mant10 = half & 0x3FFu;
    if (mant10 == 0) return (half & 0x8000) ? -0.0f : 0.0f;
    int k = 31 - __builtin_clz(mant10);
    uint32_t e = (uint32_t)(k + 103);
    uint32_t m = (mant10 - (1u << k)) << (23 - k);
    return bits_to_float(((uint32_t)(half & 0x8000) << 16) | (e << 23) | m);
  }
  if (exp5 == 31) {
    if ((half & 0x3FF) == 0) return (half & 0x8000) ? -INFINITY : INFINITY;
    return NAN;
  }
  uint32_t eb = (uint32_t)(exp5 + 112);
  uint32_t mm = (uint32_t)(half & 0x3FF) << 13;
  return bits_to_float(((uint32_t)(half & 0x8000) << 16) | (eb << 23) | mm);
}

uint16_t orc_float_to_half_rne(float f) {
  /* (Half)f: IEEE 754 binary32 -> binary16, round to nearest even,
   * overflow to infinity, NaN stays NaN (quiet). */
  uint32_t x = float_to_bits(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t absx = x & 0x7FFFFFFFu;
  if (absx >= 0x7F800000u) { /* inf or nan */
    if (absx == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | 0x7E00u | ((absx >> 13) & 0x3FFu));
  }
  if (absx >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
  if (absx >= 0x38800000u) { /* normal half range */
    uint32_t mant = absx & 0x7FFFFFu;
    uint32_t exp = (absx >> 23) - 127 + 15;
    uint32_t h = (exp << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  /* subnormal or zero: value = absx as float; half ulp = 2^-24 */
  if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25 -> 0 (2^-25 exactly ties to even 0) */
  {
    uint32_t mant = (absx & 0x7FFFFFu) | 0x800000u;
    int e = (int)(absx >> 23) - 127; /* -25 .. -15 */
    int shift = -e - 14 + 13;        /* bits to drop to reach units of 2^-24 */
    uint32_t h = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
}

/* ------------------------------------------------------------------------ */
/* Q8_0 / Q4_K                                                               */
/* ------------------------------------------------------------------------ */
static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

void orc_dequant_q8_0(const uint8_t* raw, float* out, int64_t n) {
  /* ReadQ8_0_Scalar, QuantizationKernels.Q8.cs:412-433 */
  int64_t nb = (n + 31) / 32;
  for (int64_t b = 0; b < nb; b++) {
    const uint8_t* blk = raw + b * 34;
    float d = orc_half_to_float(rd16(blk));
    int64_t valid = n - b * 32 < 32 ? n - b * 32 : 32;
    for (int j = 0; j < valid; j++) out[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
  }
}

static int k4_scale(int j, const uint8_t* s) {
  /* GetScaleMinK4_Scale_Scalar, QuantizationKernels.cs:177-182 */
  return j < 4 ? (s[j] & 0x3F) : ((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
}
static int k4_min(int j, const uint8_t* s) {
  /* GetScaleMinK4_Min_Scalar, QuantizationKernels.cs:184-189 */
  return j < 4 ? (s[j + 4] & 0x3F) : ((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
}

void orc_dequant_q4k(const uint8_t* raw, float* out, int64_t n) {
  /* ReadQ4K_Scalar, QuantizationKernels.Q4.cs:951-981 */
  int64_t nb = (n + 255) / 256;
  for (int64_t b = 0; b < nb; b++) {
    const uint8_t* blk = raw + b * 144;
    float dS = orc_half_to_float(rd16(blk));
    float mS = orc_half_to_float(rd16(blk + 2));
    const uint8_t* sc = blk + 4;
    const uint8_t* qs = blk + 16;
    for (int i = 0; i < 256 && b * 256 + i < n; i++) {
      int sub = i / 32;
      float s = (float)k4_scale(sub, sc);
      float m = (float)k4_min(sub, sc);
      int qb = (i / 64) * 32 + (i % 32);
      int sh = ((i % 64) / 32) * 4;
      int v = (qs[qb] >> sh) & 0x0F;
      float t1 = s * (float)v;
      t1 = t1 * dS;
      float t2 = m * mS;
      out[b * 256 + i] = t1 - t2;
    }
  }
}

float orc_vecdot_q8_0(const float* in, const uint8_t* raw, int col, int K) {
  /* VecDotQ8_0_Scalar, QuantizationKernels.Q8.cs:11-26 (double accumulation) */
  int nb = (K + 31) / 32;
  double sum = 0;
  for (int b = 0; b < nb; b++) {
    const uint8_t* blk = raw + ((int64_t)col * nb + b) * 34;
    float d = orc_half_to_float(rd16(blk));
    int end = K - b * 32 < 32 ? K - b * 32 : 32;
    for (int i = 0; i < end; i++) {
      float w = (float)(int8_t)blk[2 + i] * d;
      float p = in[b * 32 + i] * w;
      sum += p;
    }
  }
  return (float)sum;
}

float orc_vecdot_q4k(const float* in, const uint8_t* raw, int col, int K) {
  /* VecDotQ4K_Scalar, QuantizationKernels.Q4.cs:586-624 */
  int startBlock = (int)(((int64_t)col * K) / 256);
  int colBlockStart = (int)(((int64_t)col * K) % 256);
  int nb = (K + 255) / 256;
  double sum = 0;
  for (int b = 0; b < nb; b++) {
    const uint8_t* blk = raw + (int64_t)(startBlock + b) * 144;
    float dS = orc_half_to_float(rd16(blk));
    float mS = orc_half_to_float(rd16(blk + 2));
    const uint8_t* sc = blk + 4;
    const uint8_t* qs = blk + 16;
    int cur = b == 0 ? colBlockStart : 0;
    int end = K + colBlockStart - b * 256;
    if (end > 256) end = 256;
    for (int n16 = cur; n16 < end; n16 += 128) {
      for (int j = 0; j < 4 && n16 + j * 32 < end; j++) {
        int basePos = n16 + j * 32;
        int isc = (n16 / 128) * 4 + j;
        float s = (float)k4_scale(isc, sc);
        float m = (float)k4_min(isc, sc);
        for (int l = 0; l < 32 && basePos + l < end; l++) {
          int idx = basePos + l;
          int qb = (idx / 64) * 32 + (idx % 32);
          int sh = ((idx % 64) / 32) * 4;
          int v = (qs[qb] >> sh) & 0x0F;
          float t1 = s * (float)v;
          t1 = t1 * dS;
          float w = t1 - m * mS;
          float p = in[b * 256 + idx - colBlockStart] * w;
          sum += p;
        }
      }
    }
  }
  return (float)sum;
}

void orc_qmatmul_q8_0(const float* in, const uint8_t* raw, float* out, int M, int K, int N) {
  #pragma omp parallel for schedule(static)
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) out[(int64_t)m * N + n] = orc_vecdot_q8_0(in + (int64_t)m * K, raw, n, K);
}
void orc_qmatmul_q4k(const float* in, const uint8_t* raw, float* out, int M, int K, int N) {
  #pragma omp parallel for schedule(static)
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) out[(int64_t)m * N + n] = orc_vecdot_q4k(in + (int64_t)m * K, raw, n, K);
}
void orc_qmatmul_f32(const float* in, const float* w, float* out, int M, int K, int N) {
  /* VecDotF32 semantics: W rows [N][K]; double accumulation (QuantizationKernels.Float.cs:11-55) */
  #pragma omp parallel for schedule(static)
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      double s = 0;
      for (int k = 0; k < K; k++) s += (double)(in[(int64_t)m * K + k] * w[(int64_t)n * K + k]);
      out[(int64_t)m * N + n] = (float)s;
    }
}

static void write_half(uint8_t* p, float v) {
  uint16_t h = orc_float_to_half_rne(v);
  p[0] = (uint8_t)h;
  p[1] = (uint8_t)(h >> 8);
}
static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
static int round_away(float x) { return (int)roundf(x); } /* MathF.Round(x, AwayFromZero) */

int orc_quantize_q8_0(const float* x, int64_t n, uint8_t* out) {
  /* TensorQuantizer.WriteBlock(isQ4: false), TensorQuantizer.cs:80-144 */
  if (n % 32) return -1;
  int64_t nb = n / 32;
  memset(out, 0, (size_t)nb * 34);
  for (int64_t b = 0; b < nb; b++) {
    const float* v = x + b * 32;
    float amax = 0.f;
    for (int j = 0; j < 32; j++) {
      float a = fabsf(v[j]);
      if (a > amax) amax = a;
    }
    uint8_t* o = out + b * 34;
    if (amax == 0.f) { write_half(o, 0.f); continue; }
    float d = amax / 127.f;
    write_half(o, d);
    for (int j = 0; j < 32; j++) {
      float scaled = v[j] / d;
      int q = round_away(scaled);
      q = clampi(q, -128, 127);
      o[2 + j] = (uint8_t)(int8_t)q;
    }
  }
  return 0;
}

int orc_quantize_q4k(const float* x, int64_t n, uint8_t* out) {
  /* TensorQuantizer.WriteKQ4, TensorQuantizer.KQuant.cs:173-225; PackScaleMinK4 :451-459 */
  if (n % 256) return -1;
  int64_t nb = n / 256;
  memset(out, 0, (size_t)nb * 144);
  for (int64_t b = 0; b < nb; b++) {
    const float* v = x + b * 256;
    uint8_t* o = out + b * 144;
    float amax = 0.f;
    for (int j = 0; j < 256; j++) {
      float a = fabsf(v[j]);
      if (a > amax) amax = a;
    }
    if (amax == 0.f) continue;
    float step = amax / 63.f;
    write_half(o, step);
    write_half(o + 2, step);
    int sc[8], mn[8];
    for (int sub = 0; sub < 8; sub++) {
      const float* g = v + sub * 32;
      float gmn = 3.40282347e+38f, gmx = -3.40282347e+38f;
      for (int j = 0; j < 32; j++) {
        if (g[j] < gmn) gmn = g[j];
        if (g[j] > gmx) gmx = g[j];
      }
      float range = gmx - gmn;
      if (range <= 0.f) {
        sc[sub] = 0;
        mn[sub] = clampi(round_away(-gmn / step), 0, 63);
        continue;
      }
      sc[sub] = clampi(round_away(range / (15.f * step)), 1, 63);
      mn[sub] = clampi(round_away(-gmn / step), 0, 63);
      float scF = (float)sc[sub] * step;
      for (int j = 0; j < 32; j++) {
        float num = g[j] + (float)mn[sub] * step;
        int code = clampi(round_away(num / scF), 0, 15);
        int i = sub * 32 + j;
        int qb = (i / 64) * 32 + (i % 32);
        int sh = ((i % 64) / 32) * 4;
        o[16 + qb] |= (uint8_t)(code << sh);
      }
    }
    for (int j = 0; j < 4; j++) {
      o[4 + j] = (uint8_t)((sc[j] & 0x3F) | ((sc[4 + j] >> 4) << 6));
      o[4 + 4 + j] = (uint8_t)((mn[j] & 0x3F) | ((mn[4 + j] >> 4) << 6));
      o[4 + 8 + j] = (uint8_t)((sc[4 + j] & 0x0F) | ((mn[4 + j] & 0x0F) << 4));
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* GradientMapping slots                                                     */
/* ------------------------------------------------------------------------ */
void orc_grad_linear(const float* dY, const float* X, const float* W, float* dW, float* db,
                     float* dX, int B, int In, int Out) {
  /* Linear_Scalar, GradientKernels.cs:50-112 */
  memset(dX, 0, sizeof(float) * (size_t)B * In);
  #pragma omp parallel for schedule(static)
  for (int b = 0; b < B; b++)
    for (int o = 0; o < Out; o++) {
      float g = dY[(int64_t)b * Out + o];
      const float* w = W + (int64_t)o * In;
      float* d = dX + (int64_t)b * In;
      for (int i = 0; i < In; i++) d[i] += g * w[i];
    }
  if (dW) {
#pragma omp parallel for schedule(static)
  for (int o = 0; o < Out; o++) {
    float* dw = dW + (int64_t)o * In;
    for (int b = 0; b < B; b++) {
      float g = dY[(int64_t)b * Out + o];
      const float* x = X + (int64_t)b * In;
      for (int i = 0; i < In; i++) dw[i] += g * x[i];
    }
  }
  }
  if (db)
    for (int o = 0; o < Out; o++) {
      float acc = 0.f;
      for (int b = 0; b < B; b++) acc += dY[(int64_t)b * Out + o];
      db[o] += acc;
    }
}

void orc_grad_rmsnorm(const float* dY, const float* xn, const float* rmsInv, const float* w,
                      float* dw, float* dX, int T, int D) {
  /* RMSNorm_Scalar, GradientKernels.cs:303-337 */
  for (int t = 0; t < T; t++) {
    const float* dy = dY + (int64_t)t * D;
    const float* x = xn + (int64_t)t * D;
    float* dx = dX + (int64_t)t * D;
    float ri = rmsInv[t];
    for (int d = 0; d < D; d++) dw[d] += dy[d] * x[d];
    float dot = 0.f;
    for (int d = 0; d < D; d++) dot += dy[d] * w[d] * x[d];
    dot /= (float)D;
    for (int d = 0; d < D; d++) dx[d] = ri * (dy[d] * w[d] - x[d] * dot);
  }
}

void orc_grad_layernorm(const float* dY, const float* X, const float* w, float* dw, float* db,
                        float* dX, int T, int D, float eps) {
  /* LayerNorm_Scalar, GradientKernels.cs:345-398 */
  for (int t = 0; t < T; t++) {
    const float* x = X + (int64_t)t * D;
    const float* dy = dY + (int64_t)t * D;
    float* dx = dX + (int64_t)t * D;
    float mean = 0.f;
    for (int d = 0; d < D; d++) mean += x[d];
    mean /= (float)D;
    float var = 0.f;
    for (int d = 0; d < D; d++) { float q = x[d] - mean; var += q * q; }
    var /= (float)D;
    float invStd = 1.f / sqrtf(var + eps);
    float dyDotXhat = 0.f, dySum = 0.f;
    for (int d = 0; d < D; d++) {
      float xhat = (x[d] - mean) * invStd;
      dw[d] += dy[d] * xhat;
      db[d] += dy[d];
      dyDotXhat += dy[d] * w[d] * xhat;
      dySum += dy[d] * w[d];
    }
    for (int d = 0; d < D; d++) {
      float xhat = (x[d] - mean) * invStd;
      dx[d] = invStd * (dy[d] * w[d] - (dySum + xhat * dyDotXhat) / (float)D);
    }
  }
}

void orc_grad_attention(const float* dO, const float* q, const float* k, const float* v,
                        const float* P, float* dQ, float* dK, float* dV, int S, int D, float scale) {
  /* Attention_Scalar, GradientKernels.cs:408-481 */
  float* dP = (float*)malloc(sizeof(float) * (size_t)S * S);
  memset(dQ, 0, sizeof(float) * (size_t)S * D);
  memset(dK, 0, sizeof(float) * (size_t)S * D);
  memset(dV, 0, sizeof(float) * (size_t)S * D);
  #pragma omp parallel for schedule(static)
  for (int j = 0; j < S; j++)
    for (int d = 0; d < D; d++) {
      float sum = 0.f;
      for (int i = 0; i < S; i++) sum += P[(int64_t)i * S + j] * dO[(int64_t)i * D + d];
      dV[(int64_t)j * D + d] += sum;
    }
  #pragma omp parallel for schedule(static)
  for (int i = 0; i < S; i++)
    for (int j = 0; j < S; j++) {
      float sum = 0.f;
      for (int d = 0; d < D; d++) sum += dO[(int64_t)i * D + d] * v[(int64_t)j * D + d];
      dP[(int64_t)i * S + j] = sum;
    }
  for (int i = 0; i < S; i++) {
    const float* p = P + (int64_t)i * S;
    float* dp = dP + (int64_t)i * S;
    float dot = 0.f;
    for (int j = 0; j < S; j++) dot += p[j] * dp[j];
    for (int j = 0; j < S; j++) dp[j] = p[j] * (dp[j] - dot); /* dScores in place */
  }
  #pragma omp parallel for schedule(static)
  for (int i = 0; i < S; i++)
    for (int d = 0; d < D; d++) {
      float sq = 0.f, sk = 0.f;
      for (int j = 0; j < S; j++) {
        sq += dP[(int64_t)i * S + j] * k[(int64_t)j * D + d];
        sk += dP[(int64_t)j * S + i] * q[(int64_t)j * D + d];
      }
      dQ[(int64_t)i * D + d] += sq * scale;
      dK[(int64_t)i * D + d] += sk * scale;
    }
  free(dP);
}

void orc_grad_embedding(const float* dY, const int32_t* ids, float* dE, int T, int D) {
  /* Embedding_Scalar, GradientKernels.cs:490-506 */
  for (int t = 0; t < T; t++) {
    float* row = dE + (int64_t)ids[t] * D;
    const float* g = dY + (int64_t)t * D;
    for (int d = 0; d < D; d++) row[d] += g[d];
  }
}

void orc_grad_silu(const float* dY, const float* X, float* dX, int64_t n) {
  /* ActivationSiLU_Scalar, GradientKernels.cs:559-573 */
  for (int64_t i = 0; i < n; i++) {
    float x = X[i];
    float sig = 1.f / (1.f + expf(-x));
    dX[i] = dY[i] * (sig + x * sig * (1.f - sig));
  }
}

void orc_grad_gelu(const float* dY, const float* X, float* dX, int64_t n) {
  /* ActivationGELU_Scalar, GradientKernels.cs:612-630 */
  const float c0 = 0.7978845608f, c1 = 0.044715f;
  for (int64_t i = 0; i < n; i++) {
    float x = X[i];
    float x3 = x * x * x;
    float inner = c0 * (x + c1 * x3);
    float th = tanhf(inner);
    float dth = 1.f - th * th;
    float dinner = c0 * (1.f + 3.f * c1 * x * x);
    dX[i] = dY[i] * (0.5f * (1.f + th) + 0.5f * x * dth * dinner);
  }
}

/* ------------------------------------------------------------------------ */
/* BackpropEngine inline pieces                                              */
/* ------------------------------------------------------------------------ */
void orc_grad_swiglu(const float* dAct, const float* gate, const float* up, float* dFused, int T, int F) {
  /* BackpropEngine.cs:623-657; GateValue/GateDerivative (SiLU) :859-875 */
  for (int t = 0; t < T; t++)
    for (int d = 0; d < F; d++) {
      float g = gate[(int64_t)t * F + d], u = up[(int64_t)t * F + d], da = dAct[(int64_t)t * F + d];
      float sig = 1.f / (1.f + expf(-g));
      float gv = g * sig;
      float sig2 = 1.f / (1.f + expf(-g));
      float gd = sig2 * (1.f + g * (1.f - sig2));
      dFused[(int64_t)t * 2 * F + F + d] = da * gv;
      dFused[(int64_t)t * 2 * F + d] = da * gd * u;
    }
}

void orc_swiglu_fwd(const float* gate, const float* up, float* act, int64_t n) {
  /* SwiGLUScalar, ActivationKernels.cs:194-205 */
  for (int64_t i = 0; i < n; i++) {
    float g = gate[i];
    act[i] = (g / (1.f + expf(-g))) * up[i];
  }
}

void orc_rope_tables(float theta, int ropeDim, int maxSeq, float* cosT, float* sinT) {
  /* RoPE constructor, RoPE.cs:99-148 (no scaling) */
  int half = ropeDim / 2;
  float* freqs = (float*)malloc(sizeof(float) * (size_t)half);
  for (int i = 0; i < half; i++) freqs[i] = 1.f / powf(theta, 2.f * (float)i / (float)ropeDim);
  for (int pos = 0; pos < maxSeq; pos++)
    for (int i = 0; i < half; i++) {
      float angle = (float)pos * freqs[i];
      cosT[(int64_t)pos * half + i] = cosf(angle);
      sinT[(int64_t)pos * half + i] = sinf(angle);
    }
  free(freqs);
}

void orc_rope_fwd(float* x, const float* cosT, const float* sinT, int S, int H, int D, int neox) {
  /* RoPE.Apply, RoPE.cs:168-259 (scalar form of both pairings) */
  int pairs = D / 2;
  for (int s = 0; s < S; s++)
    for (int h = 0; h < H; h++) {
      float* p = x + ((int64_t)s * H + h) * D;
      const float* c = cosT + (int64_t)s * pairs;
      const float* sn = sinT + (int64_t)s * pairs;
      for (int i = 0; i < pairs; i++) {
        int i0 = neox ? i : 2 * i, i1 = neox ? i + pairs : 2 * i + 1;
        float a = p[i0], b = p[i1];
        p[i0] = a * c[i] - b * sn[i];
        p[i1] = b * c[i] + a * sn[i];
      }
    }
}

void orc_rope_bwd(float* dx, const float* cosT, const float* sinT, int S, int H, int D, int neox) {
  /* RoPE.ApplyBackward, RoPE.cs:300-347 */
  int pairs = D / 2;
  for (int s = 0; s < S; s++)
    for (int h = 0; h < H; h++) {
      float* p = dx + ((int64_t)s * H + h) * D;
      const float* c = cosT + (int64_t)s * pairs;
      const float* sn = sinT + (int64_t)s * pairs;
      for (int i = 0; i < pairs; i++) {
        int i0 = neox ? i : 2 * i, i1 = neox ? i + pairs : 2 * i + 1;
        float g0 = p[i0], g1 = p[i1];
        p[i0] = c[i] * g0 + sn[i] * g1;
        p[i1] = -sn[i] * g0 + c[i] * g1;
      }
    }
}

float orc_rmsnorm_param(const float* row, int n, float eps) {
  /* RMSNormParamAVX2, NormKernels.cs:40-60: 8 lane partial sums, horizontal add, scalar tail */
  float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int i = 0;
  for (; i <= n - 8; i += 8)
    for (int l = 0; l < 8; l++) lane[l] = lane[l] + row[i + l] * row[i + l];
  /* HSum256_Avx (MathHelpers.cs:10-17): add high/low 128-bit halves, then pairwise */
  float a0 = lane[0] + lane[4], a1 = lane[1] + lane[5], a2 = lane[2] + lane[6], a3 = lane[3] + lane[7];
  float ss = (a0 + a2) + (a1 + a3);
  for (; i < n; i++) ss += row[i] * row[i];
  return 1.f / sqrtf(ss / (float)n + eps);
}

void orc_rmsnorm_fwd(const float* x, const float* w, float* y, float* rmsInv, int T, int D, float eps) {
  /* NormLayer.ForwardWithState (NormLayer.cs:72-89) with RmsNormLayer (RmsNormLayer.cs:7-20) */
  for (int t = 0; t < T; t++) {
    const float* r = x + (int64_t)t * D;
    float ri = orc_rmsnorm_param(r, D, eps);
    rmsInv[t] = ri;
    for (int d = 0; d < D; d++) y[(int64_t)t * D + d] = r[d] * ri * w[d];
  }
}

void orc_ce_softmax_grad(const float* logits, const int32_t* labels, float* dL, int T, int V,
                         int ignoreId, float smoothing) {
  /* Gradients.CrossEntropySoftmax, Gradients.cs:33-84 */
  int real = 0;
  for (int t = 0; t < T; t++) if (labels[t] != ignoreId) real++;
  float scale = real > 0 ? 1.f / (float)real : 0.f;
  float epsOverV = smoothing / (float)V, oneMinusE = 1.f - smoothing;
  memset(dL, 0, sizeof(float) * (size_t)T * V);
  for (int t = 0; t < T; t++) {
    if (labels[t] == ignoreId) continue;
    const float* z = logits + (int64_t)t * V;
    float* d = dL + (int64_t)t * V;
    float mx = z[0];
    for (int v = 1; v < V; v++) if (z[v] > mx) mx = z[v];
    float sum = 0.f;
    for (int v = 0; v < V; v++) { d[v] = expf(z[v] - mx); sum += d[v]; }
    float inv = 1.f / sum;
    for (int v = 0; v < V; v++) d[v] *= inv;
    if (smoothing > 0.f) {
      for (int v = 0; v < V; v++) d[v] -= epsOverV;
      d[labels[t]] -= oneMinusE;
    } else {
      d[labels[t]] -= 1.f;
    }
    for (int v = 0; v < V; v++) d[v] *= scale;
  }
}

float orc_ce_loss(const float* logits, const int32_t* labels, int T, int V, int ignoreId, float smoothing) {
  /* CrossEntropyLoss.Compute, CrossEntropyLoss.cs:44-104 */
  double total = 0.0;
  int real = 0;
  for (int t = 0; t < T; t++) {
    if (labels[t] == ignoreId) continue;
    real++;
    const float* z = logits + (int64_t)t * V;
    float mx = z[0], sumRow = z[0];
    for (int v = 1; v < V; v++) { if (z[v] > mx) mx = z[v]; sumRow += z[v]; }
    float se = 0.f;
    for (int v = 0; v < V; v++) se += expf(z[v] - mx);
    float lp = (z[labels[t]] - mx) - logf(se);
    if (smoothing <= 0.f) {
      total -= lp;
    } else {
      float epsOverV = smoothing / (float)V;
      float slp = sumRow - (float)V * mx - (float)V * logf(se);
      total -= (1.f - smoothing) * lp + epsOverV * slp;
    }
  }
  return real > 0 ? (float)(total / real) : 0.f;
}

void orc_adamw(float* data, const float* grad, float* m, float* v, int64_t n, float beta1, float beta2,
               float bc1, float bc2, float lr, float eps, float decay) {
  /* AdamWUpdate_Scalar, TrainingKernels.cs:75-89 (the AVX2 tier, :19-70, performs the same
   * IEEE operations per element in the same order) */
  for (int64_t i = 0; i < n; i++) {
    float g = grad[i];
    m[i] = beta1 * m[i] + (1.f - beta1) * g;
    v[i] = beta2 * v[i] + (1.f - beta2) * (g * g);
    float mhat = m[i] / bc1;
    float vhat = v[i] / bc2;
    data[i] -= lr * (mhat / (sqrtf(vhat) + eps) + decay * data[i]);
  }
}

float orc_l2normsq(const float* data, int64_t n) {
  /* L2NormSq_Scalar, TrainingKernels.cs:129-134 */
  float s = 0.f;
  for (int64_t i = 0; i < n; i++) s += data[i] * data[i];
  return s;
}

void orc_attention_fwd(const float* q, const float* k, const float* v, float* probs, float* out,
                       int B, int S, int Hq, int Hkv, int D) {
  /* BackpropEngine.ForwardAttention, exact-exp (non-AVX2) branch, BackpropEngine.cs:237-388 */
  float scale = 1.f / sqrtf((float)D);
  int group = Hq / Hkv;
  memset(probs, 0, sizeof(float) * (size_t)B * Hq * S * S);
  #pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; b++)
    for (int h = 0; h < Hq; h++) {
      int kvh = h / group;
      for (int i = 0; i < S; i++) {
        float* p = probs + (((int64_t)b * Hq + h) * S + i) * S;
        const float* qi = q + (((int64_t)b * S + i) * Hq + h) * D;
        float mx = -INFINITY;
        for (int j = 0; j <= i; j++) {
          const float* kj = k + (((int64_t)b * S + j) * Hkv + kvh) * D;
          float s = 0.f;
          for (int d = 0; d < D; d++) s += qi[d] * kj[d];
          s *= scale;
          p[j] = s;
          if (s > mx) mx = s;
        }
        float sum = 0.f;
        for (int j = 0; j <= i; j++) { float e = expf(p[j] - mx); p[j] = e; sum += e; }
        float inv = 1.f / sum;
        for (int j = 0; j <= i; j++) p[j] *= inv;
        float* o = out + ((int64_t)b * S + i) * (Hq * D) + h * D;
        for (int d = 0; d < D; d++) {
          float acc = 0.f;
          for (int j = 0; j <= i; j++) acc += p[j] * v[(((int64_t)b * S + j) * Hkv + kvh) * D + d];
          o[d] = acc;
        }
      }
    }
}

void orc_lora_fwd(const float* x, const float* W, const float* A, const float* Bm, float* y,
                  int T, int In, int Out, int r, float s) {
  double* u = (double*)malloc(sizeof(double) * (size_t)r);
  for (int t = 0; t < T; t++) {
    const float* xt = x + (int64_t)t * In;
    for (int j = 0; j < r; j++) {
      double a = 0;
      for (int i = 0; i < In; i++) a += (double)xt[i] * A[(int64_t)i * r + j];
      u[j] = a;
    }
    for (int o = 0; o < Out; o++) {
      double a = 0;
      for (int i = 0; i < In; i++) a += (double)xt[i] * W[(int64_t)o * In + i];
      double l = 0;
      for (int j = 0; j < r; j++) l += u[j] * Bm[(int64_t)j * Out + o];
      y[(int64_t)t * Out + o] = (float)(a + (double)s * l);
    }
  }
  free(u);
}

void orc_lora_bwd(const float* dY, const float* x, const float* W, const float* A, const float* Bm,
                  float* dA, float* dB, float* dX, int T, int In, int Out, int r, float s) {
  double* u = (double*)malloc(sizeof(double) * (size_t)T * r); /* x A   */
  double* z = (double*)malloc(sizeof(double) * (size_t)T * r); /* dY B^T */
  for (int t = 0; t < T; t++)
    for (int j = 0; j < r; j++) {
      double a = 0, c = 0;
      for (int i = 0; i < In; i++) a += (double)x[(int64_t)t * In + i] * A[(int64_t)i * r + j];
      for (int o = 0; o < Out; o++) c += (double)dY[(int64_t)t * Out + o] * Bm[(int64_t)j * Out + o];
      u[(int64_t)t * r + j] = a;
      z[(int64_t)t * r + j] = c;
    }
  for (int j = 0; j < r; j++)
    for (int o = 0; o < Out; o++) {
      double a = 0;
      for (int t = 0; t < T; t++) a += u[(int64_t)t * r + j] * dY[(int64_t)t * Out + o];
      dB[(int64_t)j * Out + o] += (float)((double)s * a);
    }
  for (int i = 0; i < In; i++)
    for (int j = 0; j < r; j++) {
      double a = 0;
      for (int t = 0; t < T; t++) a += (double)x[(int64_t)t * In + i] * z[(int64_t)t * r + j];
      dA[(int64_t)i * r + j] += (float)((double)s * a);
    }
  for (int t = 0; t < T; t++)
    for (int i = 0; i < In; i++) {
      double a = 0, l = 0;
      for (int o = 0; o < Out; o++) a += (double)dY[(int64_t)t * Out + o] * W[(int64_t)o * In + i];
      for (int j = 0; j < r; j++) l += z[(int64_t)t * r + j] * A[(int64_t)i * r + j];
      dX[(int64_t)t * In + i] = (float)(a + (double)s * l);
    }
  free(u);
  free(z);
}
