// gemm.hip — MFMA GEMM for gfx950 with fused operand decode.
//
//   C[M,N] = alpha * sum_k A(m,k) B(n,k)  [+ alpha2 * sum_k A2(m,k) B2(n,k)]  [+ C]
//
// One kernel serves every linear of the training step.  Each operand is read
// through a descriptor (SrcMode) so that:
//   * k-contiguous and row-contiguous fp32/bf16 matrices (dY.W, dY^T.X, x.W^T)
//     need no transposed copies — the transposition happens while staging the
//     tile into LDS;
//   * frozen Q8_0 / Q4_K weights are dequantised in registers from their
//     repacked planes (bit-exact fp32 values) and never exist dequantised in HBM;
//   * a rank-r LoRA term rides along as a second, short K loop (A2, B2).
//
// Tiling: 256 threads = 4 wave64s in a 2x2 grid, block tile 128x128, each wave
// owns 64x64.  bf16 mode: K-tile 32, v_mfma_f32_32x32x16_bf16 (fp32 accumulate).
// fp32 mode: K-tile 16, v_mfma_f32_32x32x2_f32 (exact fp32 products and sums).
// LDS holds [row][k] tiles (k contiguous, 8-element pad) double-buffered; the
// next tile's global loads are issued before the current tile's MFMAs.
#include "common.hpp"
#include "kernels.hpp"

namespace smhip {

static constexpr int BM = 128, BN = 128, NT = 256;

template <int PREC> struct TileCfg;
template <> struct TileCfg<SMHIP_PREC_BF16> { static constexpr int BK = 32, PK = 40, EPT = 16; using T = uint16_t; };
template <> struct TileCfg<SMHIP_PREC_FP32> { static constexpr int BK = 16, PK = 20, EPT = 8; using T = float; };

struct OpDev {
  int mode;
  const void* p;
  const float* s;
  int64_t ld;
  int R, K;     // logical extent (rows = M or N, reduction length)
  float mult;   // applied to every loaded value (1 for the main pair)
  int vec;      // wide loads allowed
};

// ---------------------------------------------------------------- element fetch (scalar path)
__device__ inline float elem(const OpDev& o, int r, int k) {
  if (r >= o.R || k >= o.K) return 0.f;
  switch (o.mode) {
    case SRC_F32_K: return ((const float*)o.p)[(int64_t)r * o.ld + k];
    case SRC_F32_R: return ((const float*)o.p)[(int64_t)k * o.ld + r];
    case SRC_BF16_K: return bf2f(((const uint16_t*)o.p)[(int64_t)r * o.ld + k]);
    case SRC_BF16_R: return bf2f(((const uint16_t*)o.p)[(int64_t)k * o.ld + r]);
    case SRC_Q8_K:
    case SRC_Q8_R: {
      int64_t e = o.mode == SRC_Q8_K ? (int64_t)r * o.ld + k : (int64_t)k * o.ld + r;
      return (float)((const int8_t*)o.p)[e] * o.s[e >> 5];
    }
    default: {  // Q4_K
      int64_t e = o.mode == SRC_Q4K_K ? (int64_t)r * o.ld + k : (int64_t)k * o.ld + r;
      int w = (int)(e & 255);
      uint8_t byte = ((const uint8_t*)o.p)[(e >> 8) * 128 + (w >> 6) * 32 + (w & 31)];
      int v = (byte >> (((w & 63) >> 5) * 4)) & 0xF;
      float sd = o.s[2 * (e >> 5)], md = o.s[2 * (e >> 5) + 1];
      return sd * (float)v - md;
    }
  }
}

// ---------------------------------------------------------------- vector fetch helpers
__device__ inline void unpack_i8x4(uint32_t w, float d, float* out) {
  out[0] = (float)(int8_t)(w & 0xFF) * d;
  out[1] = (float)(int8_t)((w >> 8) & 0xFF) * d;
  out[2] = (float)(int8_t)((w >> 16) & 0xFF) * d;
  out[3] = (float)(int8_t)(w >> 24) * d;
}
__device__ inline void unpack_nib4(uint32_t w, int sh, float sd, float md, float* out) {
  out[0] = sd * (float)((w >> sh) & 0xF) - md;
  out[1] = sd * (float)((w >> (8 + sh)) & 0xF) - md;
  out[2] = sd * (float)((w >> (16 + sh)) & 0xF) - md;
  out[3] = sd * (float)((w >> (24 + sh)) & 0xF) - md;
}

// n (8 or 16) consecutive elements along k of row r, starting at k (k-contiguous modes).
template <int N>
__device__ inline void fetch_krun(const OpDev& o, int r, int k, float* v) {
  if (o.vec && r < o.R && k + N <= o.K) {
    switch (o.mode) {
      case SRC_F32_K: {
        const float4* p = reinterpret_cast<const float4*>((const float*)o.p + (int64_t)r * o.ld + k);
#pragma unroll
        for (int j = 0; j < N / 4; j++) { float4 a = p[j]; v[4 * j] = a.x; v[4 * j + 1] = a.y; v[4 * j + 2] = a.z; v[4 * j + 3] = a.w; }
        return;
      }
      case SRC_BF16_K: {
        const uint4* p = reinterpret_cast<const uint4*>((const uint16_t*)o.p + (int64_t)r * o.ld + k);
#pragma unroll
        for (int j = 0; j < N / 8; j++) {
          uint4 a = p[j];
          uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
          for (int q = 0; q < 4; q++) { v[8 * j + 2 * q] = bf2f(w[q] & 0xFFFF); v[8 * j + 2 * q + 1] = bf2f(w[q] >> 16); }
        }
        return;
      }
      case SRC_Q8_K: {
        const int64_t e = (int64_t)r * o.ld + k;
        const float d = o.s[e >> 5];
        if constexpr (N == 16) {
          uint4 a = *reinterpret_cast<const uint4*>((const int8_t*)o.p + e);
          unpack_i8x4(a.x, d, v); unpack_i8x4(a.y, d, v + 4); unpack_i8x4(a.z, d, v + 8); unpack_i8x4(a.w, d, v + 12);
        } else {
          uint2 a = *reinterpret_cast<const uint2*>((const int8_t*)o.p + e);
          unpack_i8x4(a.x, d, v); unpack_i8x4(a.y, d, v + 4);
        }
        return;
      }
      case SRC_Q4K_K: {
        const int64_t e = (int64_t)r * o.ld + k;
        const int w = (int)(e & 255);
        const uint8_t* qb = (const uint8_t*)o.p + (e >> 8) * 128 + (w >> 6) * 32 + (w & 31);
        const int sh = ((w & 63) >> 5) * 4;
        const float sd = o.s[2 * (e >> 5)], md = o.s[2 * (e >> 5) + 1];
        if constexpr (N == 16) {
          uint4 a = *reinterpret_cast<const uint4*>(qb);
          unpack_nib4(a.x, sh, sd, md, v); unpack_nib4(a.y, sh, sd, md, v + 4);
          unpack_nib4(a.z, sh, sd, md, v + 8); unpack_nib4(a.w, sh, sd, md, v + 12);
        } else {
          uint2 a = *reinterpret_cast<const uint2*>(qb);
          unpack_nib4(a.x, sh, sd, md, v); unpack_nib4(a.y, sh, sd, md, v + 4);
        }
        return;
      }
      default: break;
    }
  }
#pragma unroll
  for (int j = 0; j < N; j++) v[j] = elem(o, r, k + j);
}

// 8 consecutive rows r0..r0+7 at one k (row-contiguous modes).
__device__ inline void fetch_rrun8(const OpDev& o, int r0, int k, float* v) {
  if (o.vec && r0 + 8 <= o.R && k < o.K) {
    switch (o.mode) {
      case SRC_F32_R: {
        const float4* p = reinterpret_cast<const float4*>((const float*)o.p + (int64_t)k * o.ld + r0);
        float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        return;
      }
      case SRC_BF16_R: {
        uint4 a = *reinterpret_cast<const uint4*>((const uint16_t*)o.p + (int64_t)k * o.ld + r0);
        uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int q = 0; q < 4; q++) { v[2 * q] = bf2f(w[q] & 0xFFFF); v[2 * q + 1] = bf2f(w[q] >> 16); }
        return;
      }
      case SRC_Q8_R: {
        const int64_t e = (int64_t)k * o.ld + r0;
        const float d = o.s[e >> 5];
        uint2 a = *reinterpret_cast<const uint2*>((const int8_t*)o.p + e);
        unpack_i8x4(a.x, d, v); unpack_i8x4(a.y, d, v + 4);
        return;
      }
      case SRC_Q4K_R: {
        const int64_t e = (int64_t)k * o.ld + r0;
        const int w = (int)(e & 255);
        const uint8_t* qb = (const uint8_t*)o.p + (e >> 8) * 128 + (w >> 6) * 32 + (w & 31);
        const int sh = ((w & 63) >> 5) * 4;
        const float sd = o.s[2 * (e >> 5)], md = o.s[2 * (e >> 5) + 1];
        uint2 a = *reinterpret_cast<const uint2*>(qb);
        unpack_nib4(a.x, sh, sd, md, v); unpack_nib4(a.y, sh, sd, md, v + 4);
        return;
      }
      default: break;
    }
  }
#pragma unroll
  for (int j = 0; j < 8; j++) v[j] = elem(o, r0 + j, k);
}

__device__ inline bool is_krow(int mode) { return (mode & 1) == 0; }

// Load this thread's share of a 128 x BK tile into registers.
template <int PREC>
__device__ inline void load_tile(const OpDev& o, int base_r, int k0, float* v) {
  using C = TileCfg<PREC>;
  const int t = threadIdx.x;
  if (is_krow(o.mode)) {
    fetch_krun<C::EPT>(o, base_r + (t >> 1), k0 + (t & 1) * C::EPT, v);
  } else if constexpr (PREC == SMHIP_PREC_BF16) {
    const int kp = t >> 4, r0 = base_r + (t & 15) * 8;
    float a[8], b[8];
    fetch_rrun8(o, r0, k0 + 2 * kp, a);
    fetch_rrun8(o, r0, k0 + 2 * kp + 1, b);
#pragma unroll
    for (int j = 0; j < 8; j++) { v[2 * j] = a[j]; v[2 * j + 1] = b[j]; }
  } else {
    fetch_rrun8(o, base_r + (t & 15) * 8, k0 + (t >> 4), v);
  }
  if (o.mult != 1.f) {
#pragma unroll
    for (int j = 0; j < C::EPT; j++) v[j] *= o.mult;
  }
}

// Store the registers into the LDS tile [row][k] (pitch PK elements).
template <int PREC>
__device__ inline void store_tile(int mode, typename TileCfg<PREC>::T* lds, const float* v) {
  using C = TileCfg<PREC>;
  const int t = threadIdx.x;
  if constexpr (PREC == SMHIP_PREC_BF16) {
    if (is_krow(mode)) {
      uint32_t w[8];
#pragma unroll
      for (int j = 0; j < 8; j++) w[j] = pack_bf2(v[2 * j], v[2 * j + 1]);
      uint4* dst = reinterpret_cast<uint4*>(lds + (t >> 1) * C::PK + (t & 1) * 16);
      dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
      dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    } else {
      const int kp = t >> 4, r0 = (t & 15) * 8;
#pragma unroll
      for (int j = 0; j < 8; j++)
        *reinterpret_cast<uint32_t*>(lds + (r0 + j) * C::PK + 2 * kp) = pack_bf2(v[2 * j], v[2 * j + 1]);
    }
  } else {
    if (is_krow(mode)) {
      float4* dst = reinterpret_cast<float4*>(lds + (t >> 1) * C::PK + (t & 1) * 8);
      dst[0] = make_float4(v[0], v[1], v[2], v[3]);
      dst[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      const int k = t >> 4, r0 = (t & 15) * 8;
#pragma unroll
      for (int j = 0; j < 8; j++) lds[(r0 + j) * C::PK + k] = v[j];
    }
  }
}

template <int PREC, bool C_BF16>
__global__ __launch_bounds__(NT) void gemm_kernel(OpDev A, OpDev B, OpDev A2, OpDev B2, int M, int N,
                                                  int nk1, int nk2, float alpha, float beta,
                                                  void* __restrict__ Cp, int64_t ldc, int tiles_per_split,
                                                  float* __restrict__ partial, const float* __restrict__ bias,
                                                  const float* __restrict__ R, int64_t ldr) {
  using C = TileCfg<PREC>;
  using T = typename C::T;
  __shared__ __attribute__((aligned(16))) T lds[2][2][BM * C::PK];  // [buf][A/B]

  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wm = wv >> 1, wn = wv & 1;

  const int nt_total = nk1 + nk2;
  const int t_begin = blockIdx.z * tiles_per_split;
  const int t_end = min(nt_total, t_begin + tiles_per_split);

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  float ra[C::EPT], rb[C::EPT];
  auto load = [&](int t) {
    if (t < nk1) {
      load_tile<PREC>(A, m0, t * C::BK, ra);
      load_tile<PREC>(B, n0, t * C::BK, rb);
    } else {
      load_tile<PREC>(A2, m0, (t - nk1) * C::BK, ra);
      load_tile<PREC>(B2, n0, (t - nk1) * C::BK, rb);
    }
  };
  auto store = [&](int t, int buf) {
    const int ma = t < nk1 ? A.mode : A2.mode, mb = t < nk1 ? B.mode : B2.mode;
    store_tile<PREC>(ma, lds[buf][0], ra);
    store_tile<PREC>(mb, lds[buf][1], rb);
  };

  if (t_begin < t_end) {
    load(t_begin);
    store(t_begin, 0);
    __syncthreads();
    for (int t = t_begin; t < t_end; t++) {
      const int buf = (t - t_begin) & 1;
      if (t + 1 < t_end) load(t + 1);
      const T* la = lds[buf][0];
      const T* lb = lds[buf][1];
      if constexpr (PREC == SMHIP_PREC_BF16) {
#pragma unroll
        for (int kk = 0; kk < C::BK; kk += 16) {
          bf16x8 fa[2], fb[2];
#pragma unroll
          for (int i = 0; i < 2; i++)
            fa[i] = *reinterpret_cast<const bf16x8*>(la + (wm * 64 + i * 32 + (lane & 31)) * C::PK + kk + (lane >> 5) * 8);
#pragma unroll
          for (int j = 0; j < 2; j++)
            fb[j] = *reinterpret_cast<const bf16x8*>(lb + (wn * 64 + j * 32 + (lane & 31)) * C::PK + kk + (lane >> 5) * 8);
#pragma unroll
          for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int kk = 0; kk < C::BK; kk += 2) {
          float fa[2], fb[2];
#pragma unroll
          for (int i = 0; i < 2; i++) fa[i] = la[(wm * 64 + i * 32 + (lane & 31)) * C::PK + kk + (lane >> 5)];
#pragma unroll
          for (int j = 0; j < 2; j++) fb[j] = lb[(wn * 64 + j * 32 + (lane & 31)) * C::PK + kk + (lane >> 5)];
#pragma unroll
          for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
      }
      if (t + 1 < t_end) store(t + 1, buf ^ 1);
      __syncthreads();
    }
  }

  // epilogue: lane holds column (lane&31), rows (e/4)*8 + (lane>>5)*4 + e%4 of each 32x32 block
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int col = n0 + wn * 64 + j * 32 + (lane & 31);
      if (col >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int row = m0 + wm * 64 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        if (row >= M) continue;
        float val = acc[i][j][e];
        if (partial) {
          partial[((int64_t)blockIdx.z * M + row) * N + col] = val;
        } else if constexpr (C_BF16) {
          uint16_t* Cb = (uint16_t*)Cp + (int64_t)row * ldc + col;
          float o = alpha * val;
          if (bias) o = o + bias[col];
          if (beta != 0.f) o = o + beta * bf2f(*Cb);
          *Cb = f2bf(o);
        } else {
          float* Cf = (float*)Cp + (int64_t)row * ldc + col;
          float o = alpha * val;
          if (bias) o = o + bias[col];
          if (R) o = o + R[(int64_t)row * ldr + col];
          if (beta != 0.f) o = o + beta * *Cf;
          *Cf = o;
        }
      }
    }
}

// split-K: C = alpha * sum_s partial[s] + beta * C, splits summed in order.
__global__ void splitk_reduce_kernel(const float* __restrict__ partial, int splits, int M, int N,
                                     float alpha, float beta, void* __restrict__ Cp, int64_t ldc,
                                     int c_bf16, const float* __restrict__ bias, const float* __restrict__ R,
                                     int64_t ldr) {
  const int64_t n = (int64_t)M * N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int k = 0; k < splits; k++) s += partial[(int64_t)k * n + i];
    const int64_t row = i / N, col = i - row * N;
    float o = alpha * s;
    if (bias) o = o + bias[col];
    if (R && !c_bf16) o = o + R[row * ldr + col];
    if (c_bf16) {
      uint16_t* c = (uint16_t*)Cp + row * ldc + col;
      if (beta != 0.f) o = o + beta * bf2f(*c);
      *c = f2bf(o);
    } else {
      float* c = (float*)Cp + row * ldc + col;
      if (beta != 0.f) o = o + beta * *c;
      *c = o;
    }
  }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static OpDev make_op(const Operand& o, int R, int K, float mult) {
  OpDev d;
  d.mode = o.mode;
  d.p = o.p;
  d.s = o.s;
  d.ld = o.ld;
  d.R = R;
  d.K = K;
  d.mult = mult;
  int esz = (o.mode == SRC_F32_K || o.mode == SRC_F32_R) ? 4 : (o.mode == SRC_BF16_K || o.mode == SRC_BF16_R) ? 2 : 1;
  // wide loads need 16-byte aligned base and rows whose length keeps every chunk aligned
  bool v = aligned16(o.p);
  if (o.mode <= SRC_BF16_R) v = v && ((o.ld * esz) % 16 == 0);
  else v = v && (o.ld % 32 == 0);
  d.vec = v ? 1 : 0;
  return d;
}

int gemm(const GemmArgs& g, hipStream_t s) {
  if (g.masked) *g.masked = 0;  // set by the rank-sized path when it applies the mask
  if (g.M <= 0 || g.N <= 0) return SMHIP_OK;
  if (!g.R || !g.c_bf16) {
    const int fast = gemm_bf16_fast(g, s);
    if (fast < 0) return fast;
    if (fast > 0) return SMHIP_OK;
  }
  SMHIP_REQUIRE(!g.rowstat, "gemm: softmax row statistics need the persistent fragment-plane path");
  SMHIP_REQUIRE(g.A.mode < SRC_Q8T && g.B.mode < SRC_Q8T,
                "gemm: column-plane operands need the bf16 MFMA path (bf16 precision, K a multiple of 64)");
  SMHIP_REQUIRE(!(g.R && g.c_bf16), "gemm: residual input needs fp32 output");
  SMHIP_REQUIRE(g.precision == SMHIP_PREC_FP32 || g.precision == SMHIP_PREC_BF16, "gemm: bad precision");
  const int BK = g.precision == SMHIP_PREC_BF16 ? TileCfg<SMHIP_PREC_BF16>::BK : TileCfg<SMHIP_PREC_FP32>::BK;
  for (const Operand* o : {&g.A, &g.B}) {
    if (o->mode >= SRC_Q8_K) SMHIP_REQUIRE(g.K % 32 == 0 && o->ld % 32 == 0, "gemm: quantised operand needs K and row length multiples of 32");
  }
  OpDev A = make_op(g.A, g.M, g.K, 1.f), B = make_op(g.B, g.N, g.K, 1.f);
  OpDev A2 = A, B2 = B;
  int nk2 = 0;
  if (g.K2 > 0) {
    float mult = g.alpha != 0.f ? g.alpha2 / g.alpha : 0.f;
    A2 = make_op(g.A2, g.M, g.K2, mult);
    B2 = make_op(g.B2, g.N, g.K2, 1.f);
    nk2 = ceil_div(g.K2, BK);
  }
  const int nk1 = ceil_div(g.K, BK);
  const int nt = nk1 + nk2;
  int splits = g.split_k > 1 ? g.split_k : 1;
  if (splits > nt) splits = nt > 0 ? nt : 1;
  const int per = ceil_div(nt, splits);
  splits = ceil_div(nt, per);
  float* partial = nullptr;
  if (splits > 1) {
    partial = (float*)workspace(s, sizeof(float) * (size_t)splits * g.M * g.N, 3);
    if (!partial) return fail(SMHIP_ENOMEM, "gemm: split-K workspace");
  }
  dim3 grid(ceil_div(g.N, BN), ceil_div(g.M, BM), splits);
  const int ev0 = prof_mark(s);
  if (g.precision == SMHIP_PREC_BF16) {
    if (g.c_bf16)
      hipLaunchKernelGGL((gemm_kernel<SMHIP_PREC_BF16, true>), grid, dim3(NT), 0, s, A, B, A2, B2, g.M, g.N, nk1, nk2, g.alpha, g.beta, g.C, g.ldc, per, partial, g.bias, g.R, g.ldr);
    else
      hipLaunchKernelGGL((gemm_kernel<SMHIP_PREC_BF16, false>), grid, dim3(NT), 0, s, A, B, A2, B2, g.M, g.N, nk1, nk2, g.alpha, g.beta, g.C, g.ldc, per, partial, g.bias, g.R, g.ldr);
  } else {
    SMHIP_REQUIRE(!g.c_bf16, "gemm: fp32 mode writes fp32 output");
    hipLaunchKernelGGL((gemm_kernel<SMHIP_PREC_FP32, false>), grid, dim3(NT), 0, s, A, B, A2, B2, g.M, g.N, nk1, nk2, g.alpha, g.beta, g.C, g.ldc, per, partial, g.bias, g.R, g.ldr);
  }
  SMHIP_CHECK_LAUNCH();
  prof_add(PROF_GEMM, ev0, prof_mark(s), 2.0 * g.M * g.N * ((double)g.K + g.K2), g.M, g.N, g.K + g.K2);
  if (splits > 1) {
    int blocks = (int)std::min<int64_t>(((int64_t)g.M * g.N + 255) / 256, (int64_t)num_cus() * 8);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, s, partial, splits, g.M, g.N, g.alpha, g.beta, g.C, g.ldc, g.c_bf16, g.bias, g.R, g.ldr);
    SMHIP_CHECK_LAUNCH();
  }
  return SMHIP_OK;
}

}  // namespace smhip
