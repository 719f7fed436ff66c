// flash.hip — causal GQA attention on bf16 MFMA for gfx950, forward and backward.
//
// Same mathematics as the reference's recorded-probabilities path
// (BackpropEngine.cs:237-388 forward, GradientKernels.Attention_Scalar
// GradientKernels.cs:408-481 backward), restructured so that S x S
// probabilities are never stored: the forward keeps a running (max, sum) per
// query and saves only log-sum-exp; the backward recomputes P from it.
//
// All products use v_mfma_f32_32x32x16_bf16 (fp32 accumulate).  Each wave64
// owns 32 query (or key) columns.  Scores are computed transposed where that
// puts one query per lane, so row statistics are lane-local plus one
// xor-32 shuffle, and the probability tile feeds the next MFMA straight from
// registers: a lane's 16 accumulator rows are exactly the 8+8 keys it must
// supply as the k-slice of the next product, and the matching V/K/Q/dO
// operand is read from a transposed LDS tile with two 8-byte loads.
//
// Backward is deterministic: dK/dV are accumulated per (key block, query head)
// by one workgroup and summed over the GQA group in a fixed order; dQ is a
// separate pass over key blocks (no atomics).
#include "common.hpp"
#include "kernels.hpp"

namespace smhip {

static constexpr float kLog2e = 1.4426950408889634f;

// 2^x by the hardware v_exp_f32 (no denormal range handling: softmax weights below 2^-126
// flush to zero, which is below the bf16 resolution of the products they feed)
__device__ inline float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline floatx16 mfma16(const bf16x8& a, const bf16x8& b, const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ inline void zero16(floatx16& a) {
#pragma unroll
  for (int e = 0; e < 16; e++) a[e] = 0.f;
}
__device__ inline bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }
// gradient outputs: fp32, or bf16 (the training engine, whose next consumer rounds to bf16)
__device__ inline void stg(float* p, float v) { *p = v; }
__device__ inline void stg(uint16_t* p, float v) { *p = f2bf(v); }
// accumulator row of element e for this lane (32x32 MFMA output layout)
__device__ inline int acc_row(int e, int lane) { return (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3); }

// 8 accumulator values (e0..e0+7) -> bf16x8 operand (keys/queries in the lane's k-slice order)
__device__ inline bf16x8 pack8(const floatx16& a, int e0) {
  uint4 u;
  u.x = pack_bf2(a[e0 + 0], a[e0 + 1]);
  u.y = pack_bf2(a[e0 + 2], a[e0 + 3]);
  u.z = pack_bf2(a[e0 + 4], a[e0 + 5]);
  u.w = pack_bf2(a[e0 + 6], a[e0 + 7]);
  return as_bf16x8(u);
}
// operand from a transposed LDS tile [D][NR + 4]: row d = 32 i + lane % 32, keys
// c16 + half*4 + {0..3} and c16 + 8 + half*4 + {0..3} (half = lane / 32)
template <int NR>
__device__ inline bf16x8 tload(const uint16_t* tile, int i, int c16, int lane) {
  const uint16_t* p = tile + (i * 32 + (lane & 31)) * (NR + 4) + c16 + (lane >> 5) * 4;
  uint2 lo = *reinterpret_cast<const uint2*>(p);
  uint2 hi = *reinterpret_cast<const uint2*>(p + 8);
  return as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
}

// Register-prefetched staging: load() issues the global reads of a [NR][D] row tile (pairs
// of rows per 16-byte column chunk) into registers, store() writes them to LDS as [NR][D+8]
// and/or transposed [D][NR+4].  Loading tile t+1 before the MFMAs of tile t hides the
// global latency behind the compute.
template <int D, int NR, int NT = 256>
struct Pref {
  static constexpr int U = (NR / 2) * (D / 8);  // (row pair, chunk) units
  static constexpr int PER = (U + NT - 1) / NT;
  static_assert(PER <= 2, "Pref holds at most two units per thread");
  uint4 a0, b0, a1, b1;  // named registers: no dynamically indexed (scratch) arrays
  // unit c = (row pair rp, 8-column chunk dc): consecutive units walk the row pairs of a chunk
  __device__ static inline void unit(int c, int& rp, int& dc) {
    rp = c % (NR / 2);
    dc = (c / (NR / 2)) * 8;
  }
  // unit c's two rows; units past U (only when U is not a multiple of NT) read row pair 0
  __device__ static inline uint4 ld1(const uint16_t* __restrict__ g, int64_t ld, int r0, int c, int odd) {
    if constexpr (U % NT != 0) c = c < U ? c : 0;
    int rp, dc;
    unit(c, rp, dc);
    return *reinterpret_cast<const uint4*>(g + (int64_t)(r0 + 2 * rp + odd) * ld + dc);
  }
  __device__ inline void load(const uint16_t* __restrict__ g, int64_t ld, int r0) {
    a0 = ld1(g, ld, r0, threadIdx.x, 0);
    b0 = ld1(g, ld, r0, threadIdx.x, 1);
    if constexpr (PER > 1) {
      a1 = ld1(g, ld, r0, NT + threadIdx.x, 0);
      b1 = ld1(g, ld, r0, NT + threadIdx.x, 1);
    }
  }
  template <bool ROWS, bool TRANS>
  __device__ inline void store1(uint16_t* sRow, uint16_t* sT, int c, const uint4& a, const uint4& b) const {
    constexpr int RP = D + 8, TP = NR + 4;
    if (c >= U) return;
    int rp, dc;
    unit(c, rp, dc);
    if constexpr (ROWS) {
      *reinterpret_cast<uint4*>(sRow + (2 * rp) * RP + dc) = a;
      *reinterpret_cast<uint4*>(sRow + (2 * rp + 1) * RP + dc) = b;
    }
    if constexpr (TRANS) {
      const uint32_t av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const uint32_t lo = (j & 1) ? (av[j >> 1] >> 16) : (av[j >> 1] & 0xFFFFu);
        const uint32_t hi = (j & 1) ? (bv[j >> 1] >> 16) : (bv[j >> 1] & 0xFFFFu);
        *reinterpret_cast<uint32_t*>(sT + (dc + j) * TP + 2 * rp) = lo | (hi << 16);
      }
    }
  }
  template <bool ROWS, bool TRANS>
  __device__ inline void store(uint16_t* sRow, uint16_t* sT) const {
    store1<ROWS, TRANS>(sRow, sT, threadIdx.x, a0, b0);
    if constexpr (PER > 1) store1<ROWS, TRANS>(sRow, sT, NT + threadIdx.x, a1, b1);
  }
};

// ---------------------------------------------------------------- D = 128: DMA-staged tiles
// A [64][128] bf16 tile in LDS is four 4 KiB sub-tiles, one per 32 columns; a sub-tile row is
// 64 bytes, and 16-byte chunk c (0..3) of row r sits at slot c ^ ((r / 4) % 4).  Tiles are
// filled by buffer_load ... lds (global straight to LDS: no staging registers, no store
// instructions) and read as MFMA operands either row-wise (16-byte reads, 16 consecutive rows
// per quarter-wave) or column-wise with ds_read_b64_tr_b16, which hands each lane four rows of
// one column.  Both patterns touch 64 distinct banks per 32 lanes, and in both the per-lane
// part of the address is one of two values: the sub-tile, row block and k-step of a read are
// compile-time offsets.
typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void fa_lds_void;
typedef __attribute__((address_space(3))) short4v fa_lds_s4;
// byte offset of 16-byte chunk c (0..15) of row r
__device__ inline int toff(int r, int c) { return (c >> 2) * 4096 + r * 64 + (((c & 3) ^ ((r >> 2) & 3)) << 4); }
__device__ inline __amdgpu_buffer_rsrc_t fa_rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}
__device__ inline void fa_wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// global -> LDS copy of one [64][128] tile: 16 wave instructions of 64 x 16 bytes; instruction
// blk fills sub-tile blk / 4, rows 16 (blk % 4) .. +15 (lane l: row 16 (blk % 4) + l / 4,
// slot l % 4).  Rows are ld elements apart; the tile's first row is passed as a byte offset in
// the scalar operand.
template <int NT>
struct Dma128 {
  static constexpr int NW = NT / 64, NI = 16 / NW;
  uint32_t off[NI];
  __device__ inline void init(int64_t ld) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < NI; j++) {
      const int blk = j * NW + w, r = (blk & 3) * 16 + (l >> 2);
      const int c = (l & 3) ^ ((r >> 2) & 3);
      off[j] = (uint32_t)(r * ld * 2 + ((blk >> 2) * 32 + c * 8) * 2);
    }
  }
  __device__ inline void fetch(__amdgpu_buffer_rsrc_t rs, uint8_t* tile, int soff) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < NI; j++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (fa_lds_void*)(tile + (j * NW + w) * 1024), 16, off[j], soff, 0, 0);
#endif
  }
};
// 64 fp32 row statistics (one wave instruction of 4-byte copies)
__device__ inline void fa_dma_row64(__amdgpu_buffer_rsrc_t rs, float* dst, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (fa_lds_void*)dst, 4, (threadIdx.x & 63) * 4, soff, 0, 0);
#endif
}
// row operand: row r, 16-byte chunk c
__device__ inline bf16x8 rrow(const uint8_t* tile, int r, int c) {
  return as_bf16x8(*reinterpret_cast<const uint4*>(tile + toff(r, c)));
}
// column operand: column i*32 + lane%32, rows r0 + 4 half + {0..3} and r0 + 8 + 4 half + {0..3}
// (r0 a multiple of 16, half = lane / 32), i.e. the lane's k-slice order of a 32x32x16 operand.
// ds_read_b64_tr_b16 over 16 lanes: source lane s reads 4 elements of row s/4 at columns
// 4 (s%4) .. +3; destination lane s receives element s of rows 0..3.
__device__ inline bf16x8 rtr(const uint8_t* tile, int r0, int i, int lane) {
  const int s = lane & 15;
  const int c = 2 * ((lane >> 4) & 1) + ((s & 3) >> 1), hb = (s & 1) * 8;  // chunk in sub-tile, half
  const int ra = r0 + (lane >> 5) * 4 + (s >> 2), rb = ra + 8;
  const uint8_t* st = tile + i * 4096 + hb;
  short4v lo, hi;
#if defined(__HIP_DEVICE_COMPILE__)
  lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((fa_lds_s4*)(st + ra * 64 + ((c ^ ((ra >> 2) & 3)) << 4)));
  hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((fa_lds_s4*)(st + rb * 64 + ((c ^ ((rb >> 2) & 3)) << 4)));
#else
  lo = hi = short4v{};
#endif
  const uint2 a = __builtin_bit_cast(uint2, lo), b = __builtin_bit_cast(uint2, hi);
  return as_bf16x8(make_uint4(a.x, a.y, b.x, b.y));
}

// ============================================================================
// forward: grid (S/128, Hq, B), 4 waves x 32 queries, key tiles of 64 (the next one loaded into
// registers while the current one is multiplied).
// PAIR (S/128 even): grid (S/256, Hq, B) of 8 waves; waves 0-3 take query block nb-1-x and
// waves 4-7 block x, so every workgroup (and every SIMD, which hosts wave s and wave s+4)
// carries the same causal work and the two blocks share the staged K/V tiles.  Without it
// the query-block index, the fastest grid dimension, lands each block on one XCD (blocks
// are dispatched round-robin over the 8 XCDs): the XCD of the longest rows bounded the kernel.
// ============================================================================
template <int D, bool PAIR>
__global__ __launch_bounds__(PAIR ? 512 : 256) void fa_fwd_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                     const uint16_t* __restrict__ v, uint16_t* __restrict__ o,
                                                     float* __restrict__ lse, int S, int Hq, int Hkv, int64_t ldq,
                                                     int64_t ldk, int64_t ldv, int64_t ldo, float sl2) {
  constexpr int KB = 64, KP = D + 8, VP = KB + 4, NT = PAIR ? 512 : 256;
  __shared__ __attribute__((aligned(16))) uint16_t sK[KB * KP];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[D * VP];
  const int nb = PAIR ? 2 * (int)gridDim.x : (int)gridDim.x;
  const int half = PAIR ? (int)(threadIdx.x >> 8) : 0;
  const int qb = half == 0 ? nb - 1 - (int)blockIdx.x : (int)blockIdx.x;  // longest causal rows first
  const int h = blockIdx.y, b = blockIdx.z, kvh = h / (Hq / Hkv);
  const int lane = threadIdx.x & 63, w = (threadIdx.x >> 6) & 3;
  const int qi = qb * 128 + w * 32 + (lane & 31);
  const uint16_t* kb = k + (int64_t)b * S * ldk + kvh * D;
  const uint16_t* vb = v + (int64_t)b * S * ldv + kvh * D;

  bf16x8 qf[D / 16];
  {
    const uint16_t* qrow = q + ((int64_t)b * S + qi) * ldq + h * D + (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < D / 16; kk++) qf[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(qrow + kk * 16));
  }
  floatx16 oacc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; i++) zero16(oacc[i]);
  float m = -INFINITY, l = 0.f;
  const int kend = (nb - (int)blockIdx.x) * 128;  // the longer block of the workgroup
  const int wq_last = qb * 128 + w * 32 + 31;  // last query of this wave

  Pref<D, KB, NT> pk, pv;
  pk.load(kb, ldk, 0);
  pv.load(vb, ldv, 0);
  for (int k0 = 0; k0 < kend; k0 += KB) {
    __syncthreads();
    pk.template store<true, false>(sK, nullptr);
    pv.template store<false, true>(nullptr, sVt);
    __syncthreads();
    if (k0 + KB < kend) {  // next tile in flight during this tile's MFMAs
      pk.load(kb, ldk, k0 + KB);
      pv.load(vb, ldv, k0 + KB);
    }
    if (k0 > wq_last) continue;  // whole tile masked for this wave
    floatx16 sacc[2];
    zero16(sacc[0]);
    zero16(sacc[1]);
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int kk = 0; kk < D / 16; kk++) {
        bf16x8 kf = as_bf16x8(*reinterpret_cast<const uint4*>(sK + (j * 32 + (lane & 31)) * KP + kk * 16 + (lane >> 5) * 8));
        sacc[j] = mfma16(kf, qf[kk], sacc[j]);
      }
    // raw scores: the causal mask only on tiles that reach past the wave's first query, the
    // log2 scale folded into the exponent (max(s) sl2 = max(s sl2) for sl2 > 0)
    float mx = -INFINITY;
    if (k0 + KB - 1 > wq_last - 31) {
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int key = k0 + j * 32 + acc_row(e, lane);
          if (key > qi) sacc[j][e] = -INFINITY;
          mx = fmaxf(mx, sacc[j][e]);
        }
    } else {
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) mx = fmaxf(mx, sacc[j][e]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // lazy rescaling: the reference max moves only when the running max grows by more than 8
    // (log2 units), so p <= 2^8 and the O rescale below is skipped for most key blocks; m only
    // has to be a common reference for p, l and O, and the final O / l and LSE = m + log2 l are
    // unchanged in exact arithmetic
    const float mc = fmaxf(m, mx * sl2);
    const float mnew = mc > m + 8.f ? mc : m;
    const float alpha = fexp2(m - mnew);
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        float p = fexp2(__builtin_fmaf(sacc[j][e], sl2, -mnew));
        sacc[j][e] = p;
        rs += p;
      }
    rs += __shfl_xor(rs, 32, 64);
    l = l * alpha + rs;
    m = mnew;
    // rescale only when some query's reference max moved (alpha == 1 multiplies are exact no-ops)
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int i = 0; i < D / 32; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) oacc[i][e] *= alpha;
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const bf16x8 pf = pack8(sacc[c >> 1], 8 * (c & 1));
#pragma unroll
      for (int i = 0; i < D / 32; i++) {
        const bf16x8 vf = tload<KB>(sVt, i, c * 16, lane);
        oacc[i] = mfma16(vf, pf, oacc[i]);
      }
    }
  }
  const float inv = 1.f / l;
  uint16_t* orow = o + ((int64_t)b * S + qi) * ldo + h * D;
#pragma unroll
  for (int i = 0; i < D / 32; i++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int d = i * 32 + g * 8 + (lane >> 5) * 4;
      uint2 st;
      st.x = pack_bf2(oacc[i][4 * g] * inv, oacc[i][4 * g + 1] * inv);
      st.y = pack_bf2(oacc[i][4 * g + 2] * inv, oacc[i][4 * g + 3] * inv);
      *reinterpret_cast<uint2*>(orow + d) = st;
    }
  if (lane < 32) lse[((int64_t)b * Hq + h) * S + qi] = m + log2f(l);
}

// D = 128 form of fa_fwd_kernel: key/value tiles copied global -> LDS by DMA into a double
// buffer, V^T operands read from the V row tile with ds_read_b64_tr_b16.
template <bool PAIR>
__global__ __launch_bounds__(PAIR ? 512 : 256) void fa_fwd128_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                        const uint16_t* __restrict__ v, uint16_t* __restrict__ o,
                                                        float* __restrict__ lse, int S, int Hq, int Hkv, int64_t ldq,
                                                        int64_t ldk, int64_t ldv, int64_t ldo, float sl2) {
  constexpr int D = 128, KB = 64, NT = PAIR ? 512 : 256, TB = KB * 256;
  __shared__ __attribute__((aligned(1024))) uint8_t sK[2 * TB];
  __shared__ __attribute__((aligned(1024))) uint8_t sV[2 * TB];
  const int nb = PAIR ? 2 * (int)gridDim.x : (int)gridDim.x;
  const int half = PAIR ? (int)(threadIdx.x >> 8) : 0;
  const int qb = half == 0 ? nb - 1 - (int)blockIdx.x : (int)blockIdx.x;  // longest causal rows first
  const int h = blockIdx.y, b = blockIdx.z, kvh = h / (Hq / Hkv);
  const int lane = threadIdx.x & 63, w = (threadIdx.x >> 6) & 3;
  const int qi = qb * 128 + w * 32 + (lane & 31);
  const uint16_t* kb = k + (int64_t)b * S * ldk + kvh * D;
  const uint16_t* vb = v + (int64_t)b * S * ldv + kvh * D;
  const __amdgpu_buffer_rsrc_t rk = fa_rsrc(kb, (int)((S - 1) * ldk * 2 + D * 2));
  const __amdgpu_buffer_rsrc_t rv = fa_rsrc(vb, (int)((S - 1) * ldv * 2 + D * 2));
  Dma128<NT> gk, gv;
  gk.init(ldk);
  gv.init(ldv);
  gk.fetch(rk, sK, 0);
  gv.fetch(rv, sV, 0);

  bf16x8 qf[D / 16];
  {
    const uint16_t* qrow = q + ((int64_t)b * S + qi) * ldq + h * D + (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < D / 16; kk++) qf[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(qrow + kk * 16));
  }
  floatx16 oacc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; i++) zero16(oacc[i]);
  float m = -INFINITY, l = 0.f;
  const int kend = (nb - (int)blockIdx.x) * 128;  // the longer block of the workgroup
  const int wq_last = qb * 128 + w * 32 + 31;  // last query of this wave
  int buf = 0;
  for (int k0 = 0; k0 < kend; k0 += KB, buf ^= 1) {
    fa_wait_vm();
    __syncthreads();
    if (k0 + KB < kend) {
      gk.fetch(rk, sK + (buf ^ 1) * TB, (int)((k0 + KB) * ldk * 2));
      gv.fetch(rv, sV + (buf ^ 1) * TB, (int)((k0 + KB) * ldv * 2));
    }
    if (k0 > wq_last) continue;  // whole tile masked for this wave
    const uint8_t* tK = sK + buf * TB;
    const uint8_t* tV = sV + buf * TB;
    floatx16 sacc[2];
    zero16(sacc[0]);
    zero16(sacc[1]);
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int kk = 0; kk < D / 16; kk++)
        sacc[j] = mfma16(rrow(tK, j * 32 + (lane & 31), kk * 2 + (lane >> 5)), qf[kk], sacc[j]);
    // raw scores: the causal mask only on tiles that reach past the wave's first query, the
    // log2 scale folded into the exponent (max(s) sl2 = max(s sl2) for sl2 > 0)
    float mx = -INFINITY;
    if (k0 + KB - 1 > wq_last - 31) {
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int key = k0 + j * 32 + acc_row(e, lane);
          if (key > qi) sacc[j][e] = -INFINITY;
          mx = fmaxf(mx, sacc[j][e]);
        }
    } else {
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) mx = fmaxf(mx, sacc[j][e]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // lazy rescaling: the reference max moves only when the running max grows by more than 8
    // (log2 units), so p <= 2^8 and the O rescale below is skipped for most key blocks; m only
    // has to be a common reference for p, l and O, and the final O / l and LSE = m + log2 l are
    // unchanged in exact arithmetic
    const float mc = fmaxf(m, mx * sl2);
    const float mnew = mc > m + 8.f ? mc : m;
    const float alpha = fexp2(m - mnew);
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        float p = fexp2(__builtin_fmaf(sacc[j][e], sl2, -mnew));
        sacc[j][e] = p;
        rs += p;
      }
    rs += __shfl_xor(rs, 32, 64);
    l = l * alpha + rs;
    m = mnew;
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int i = 0; i < D / 32; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) oacc[i][e] *= alpha;
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const bf16x8 pf = pack8(sacc[c >> 1], 8 * (c & 1));
#pragma unroll
      for (int i = 0; i < D / 32; i++) oacc[i] = mfma16(rtr(tV, c * 16, i, lane), pf, oacc[i]);
    }
  }
  const float inv = 1.f / l;
  uint16_t* orow = o + ((int64_t)b * S + qi) * ldo + h * D;
#pragma unroll
  for (int i = 0; i < D / 32; i++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int d = i * 32 + g * 8 + (lane >> 5) * 4;
      uint2 st;
      st.x = pack_bf2(oacc[i][4 * g] * inv, oacc[i][4 * g + 1] * inv);
      st.y = pack_bf2(oacc[i][4 * g + 2] * inv, oacc[i][4 * g + 3] * inv);
      *reinterpret_cast<uint2*>(orow + d) = st;
    }
  if (lane < 32) lse[((int64_t)b * Hq + h) * S + qi] = m + log2f(l);
}

// ============================================================================
// backward preprocessing: Di = sum_d dO*O per (b, h, q)  (the rowsum(P*dP) term)
// ============================================================================
template <int D>
__global__ __launch_bounds__(256) void fa_bwd_pre_kernel(const uint16_t* __restrict__ o, const uint16_t* __restrict__ dO,
                                                         float* __restrict__ Di, int B, int S, int Hq, int64_t ldo,
                                                         int64_t lddo) {
  const int lane = threadIdx.x & 63;
  const int64_t rows = (int64_t)B * Hq * S;
  for (int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += (int64_t)gridDim.x * 4) {
    const int qi = (int)(r % S);
    const int h = (int)((r / S) % Hq);
    const int b = (int)(r / ((int64_t)S * Hq));
    const uint16_t* orow = o + ((int64_t)b * S + qi) * ldo + h * D;
    const uint16_t* drow = dO + ((int64_t)b * S + qi) * lddo + h * D;
    float a = 0.f;
    for (int d = lane; d < D; d += 64) a += bf2f(orow[d]) * bf2f(drow[d]);
    a = wave_sum(a);
    if (lane == 0) Di[((int64_t)b * Hq + h) * S + qi] = a;
  }
}

// vectorised form: D/8 lanes per row, one 16-byte load of O and of dO per lane, the lane
// products summed in d order and then over the lane group by xor shuffles
template <int D>
__global__ __launch_bounds__(256) void fa_bwd_pre_vec_kernel(const uint16_t* __restrict__ o, const uint16_t* __restrict__ dO,
                                                             float* __restrict__ Di, int B, int S, int Hq, int64_t ldo,
                                                             int64_t lddo) {
  constexpr int L = D / 8;  // lanes per row
  const int sub = threadIdx.x % L;
  const int64_t rows = (int64_t)B * Hq * S;
  for (int64_t r = ((int64_t)blockIdx.x * 256 + threadIdx.x) / L; r - ((int)threadIdx.x % 64) / L < rows;
       r += (int64_t)gridDim.x * (256 / L)) {
    const bool live = r < rows;
    const int64_t rr = live ? r : rows - 1;
    const int qi = (int)(rr % S);
    const int h = (int)((rr / S) % Hq);
    const int b = (int)(rr / ((int64_t)S * Hq));
    const uint4 a = *reinterpret_cast<const uint4*>(o + ((int64_t)b * S + qi) * ldo + h * D + sub * 8);
    const uint4 g = *reinterpret_cast<const uint4*>(dO + ((int64_t)b * S + qi) * lddo + h * D + sub * 8);
    const uint32_t av[4] = {a.x, a.y, a.z, a.w}, gv[4] = {g.x, g.y, g.z, g.w};
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      acc += bf2f((uint16_t)(av[i] & 0xFFFFu)) * bf2f((uint16_t)(gv[i] & 0xFFFFu));
      acc += bf2f((uint16_t)(av[i] >> 16)) * bf2f((uint16_t)(gv[i] >> 16));
    }
#pragma unroll
    for (int m = 1; m < L; m <<= 1) acc += __shfl_xor(acc, m, 64);
    if (live && sub == 0) Di[((int64_t)b * Hq + h) * S + qi] = acc;
  }
}

// ============================================================================
// backward dK, dV: grid (S/128, Hq, B); 4 waves x 32 keys; query tiles of QB = 64 (two
// 32-query MFMA blocks per wave per tile).  Writes per-query-head partials dKh/dVh
// [B, S, Hq, D] fp32.
// ============================================================================
template <int D, bool PAIR, typename TG>
__global__ __launch_bounds__(PAIR ? 512 : 256) void fa_bwd_dkdv_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ Di,
    TG* __restrict__ dKh, TG* __restrict__ dVh, int S, int Hq, int Hkv, int64_t ldq, int64_t ldk,
    int64_t ldv, int64_t lddo, float sl2, float scale) {
  constexpr int QB = 64, NQ = QB / 32, RP = D + 8, TP = QB + 4, NT = PAIR ? 512 : 256;
  __shared__ __attribute__((aligned(16))) uint16_t sQ[QB * RP];
  __shared__ __attribute__((aligned(16))) uint16_t sQt[D * TP];
  __shared__ __attribute__((aligned(16))) uint16_t sdO[QB * RP];
  __shared__ __attribute__((aligned(16))) uint16_t sdOt[D * TP];
  __shared__ __attribute__((aligned(16))) float sL[QB];
  __shared__ __attribute__((aligned(16))) float sDi[QB];
  // each wave's 32 V rows: read as the B operand of dP = dO V^T from LDS rather than held in
  // registers, which keeps the wave within 256 registers (no spills in the query loop)
  __shared__ __attribute__((aligned(16))) uint16_t sV[(NT / 64) * 32 * RP];
  // key block of 128; PAIR: waves 0-3 take key block x (the most queries), waves 4-7 block nb-1-x
  const int nb = PAIR ? 2 * (int)gridDim.x : (int)gridDim.x;
  const int half = PAIR ? (int)(threadIdx.x >> 8) : 0;
  const int kbk = half == 0 ? (int)blockIdx.x : nb - 1 - (int)blockIdx.x;
  const int h = blockIdx.y, b = blockIdx.z, kvh = h / (Hq / Hkv);
  const int lane = threadIdx.x & 63, w = (threadIdx.x >> 6) & 3;
  const int kw0 = kbk * 128 + w * 32;
  const int kj = kw0 + (lane & 31);  // this lane's key (B-operand column)

  bf16x8 kf[D / 16];
  uint16_t* sVw = sV + (threadIdx.x >> 6) * 32 * RP;  // this wave's rows: key kw0 + row
  {
    const uint16_t* krow = k + ((int64_t)b * S + kj) * ldk + kvh * D + (lane >> 5) * 8;
    const uint16_t* vrow = v + ((int64_t)b * S + kj) * ldv + kvh * D + (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < D / 16; kk++) {
      kf[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(krow + kk * 16));
      *reinterpret_cast<uint4*>(sVw + (lane & 31) * RP + kk * 16 + (lane >> 5) * 8) =
          *reinterpret_cast<const uint4*>(vrow + kk * 16);
    }
  }
  floatx16 dv[D / 32], dk[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; i++) { zero16(dv[i]); zero16(dk[i]); }
  const uint16_t* qb_ = q + (int64_t)b * S * ldq + h * D;
  const uint16_t* db_ = dO + (int64_t)b * S * lddo + h * D;
  const float* lrow = lse + ((int64_t)b * Hq + h) * S;
  const float* drow = Di + ((int64_t)b * Hq + h) * S;

  Pref<D, QB, NT> pq, pd;
  float pl = 0.f, pdi = 0.f;
  const int qstart = (int)blockIdx.x * 128;  // the earlier key block of the workgroup
  pq.load(qb_, ldq, qstart);
  pd.load(db_, lddo, qstart);
  if (threadIdx.x < QB) { pl = lrow[qstart + threadIdx.x]; pdi = drow[qstart + threadIdx.x]; }
  for (int q0 = qstart; q0 < S; q0 += QB) {
    __syncthreads();
    pq.template store<true, true>(sQ, sQt);
    pd.template store<true, true>(sdO, sdOt);
    if (threadIdx.x < QB) { sL[threadIdx.x] = pl; sDi[threadIdx.x] = pdi; }
    __syncthreads();
    if (q0 + QB < S) {  // next tile in flight during this tile's MFMAs
      pq.load(qb_, ldq, q0 + QB);
      pd.load(db_, lddo, q0 + QB);
      if (threadIdx.x < QB) { pl = lrow[q0 + QB + threadIdx.x]; pdi = drow[q0 + QB + threadIdx.x]; }
    }
    if (q0 + QB - 1 < kw0) continue;  // every query precedes this wave's keys
#pragma unroll
    for (int jb = 0; jb < NQ; jb++) {
      if (q0 + jb * 32 + 31 < kw0) continue;  // this 32-query block precedes the wave's keys
      // S = Q K^T and dP = dO V^T : rows = queries, cols = keys (lane <-> key)
      floatx16 sacc, dpacc;
      zero16(sacc);
      zero16(dpacc);
#pragma unroll
      for (int kk = 0; kk < D / 16; kk++) {
        const int off = (jb * 32 + (lane & 31)) * RP + kk * 16 + (lane >> 5) * 8;
        sacc = mfma16(as_bf16x8(*reinterpret_cast<const uint4*>(sQ + off)), kf[kk], sacc);
        const bf16x8 vf = as_bf16x8(*reinterpret_cast<const uint4*>(sVw + (lane & 31) * RP + kk * 16 + (lane >> 5) * 8));
        dpacc = mfma16(as_bf16x8(*reinterpret_cast<const uint4*>(sdO + off)), vf, dpacc);
      }
      // this lane's 16 rows are 4 runs of 4 consecutive queries: row statistics as float4
      const bool diag = q0 + jb * 32 < kw0 + 31;  // some query of the block precedes some key
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++) {
        const int r0 = jb * 32 + g4 * 8 + (lane >> 5) * 4;
        const float4 L4 = *reinterpret_cast<const float4*>(sL + r0);
        const float4 D4 = *reinterpret_cast<const float4*>(sDi + r0);
        const float Lv[4] = {L4.x, L4.y, L4.z, L4.w}, Dv[4] = {D4.x, D4.y, D4.z, D4.w};
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int e = g4 * 4 + u;
          float p = fexp2(sacc[e] * sl2 - Lv[u]);
          if (diag && q0 + r0 + u < kj) p = 0.f;
          sacc[e] = p;
          dpacc[e] = p * (dpacc[e] - Dv[u]);  // dS
        }
      }
      // dV += P^T dO ; dK += dS^T Q   (A from registers: lane row = key, k-slice = its 8+8 queries)
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const bf16x8 pf = pack8(sacc, 8 * c);
        const bf16x8 sf = pack8(dpacc, 8 * c);
#pragma unroll
        for (int i = 0; i < D / 32; i++) {
          dv[i] = mfma16(pf, tload<QB>(sdOt, i, jb * 32 + c * 16, lane), dv[i]);
          dk[i] = mfma16(sf, tload<QB>(sQt, i, jb * 32 + c * 16, lane), dk[i]);
        }
        __builtin_amdgcn_sched_barrier(0);  // bounds the transposed fragments in flight
      }
    }
  }
  // outputs: rows = keys (acc_row), cols = d (lane)
#pragma unroll
  for (int i = 0; i < D / 32; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const int key = kw0 + acc_row(e, lane);
      const int64_t off = (((int64_t)b * S + key) * Hq + h) * D + i * 32 + (lane & 31);
      stg(dKh + off, dk[i][e] * scale);
      stg(dVh + off, dv[i][e]);
    }
}

// D = 128 form of fa_bwd_dkdv_kernel: the same work split, with the query tiles (Q, dO and their
// row statistics) copied global -> LDS by DMA into a double buffer (tile t+1 in flight while
// tile t is multiplied) and the transposed operands of dV += P^T dO, dK += dS^T Q read from the
// row tiles with ds_read_b64_tr_b16 (no transposed copies).
template <bool PAIR, typename TG>
__global__ __launch_bounds__(PAIR ? 512 : 256) void fa_bwd_dkdv128_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ Di,
    TG* __restrict__ dKh, TG* __restrict__ dVh, int S, int Hq, int Hkv, int64_t ldq, int64_t ldk,
    int64_t ldv, int64_t lddo, float sl2, float scale) {
  constexpr int D = 128, QB = 64, NQ = QB / 32, RP = D + 8, NT = PAIR ? 512 : 256, TB = QB * 256;
  __shared__ __attribute__((aligned(1024))) uint8_t sQ[2 * TB];
  __shared__ __attribute__((aligned(1024))) uint8_t sdO[2 * TB];
  __shared__ __attribute__((aligned(256))) float sL[2 * QB];
  __shared__ __attribute__((aligned(256))) float sDi[2 * QB];
  // each wave's 32 V rows (B operand of dP = dO V^T), padded rows: conflict-free 16-byte reads
  __shared__ __attribute__((aligned(16))) uint16_t sV[(NT / 64) * 32 * RP];
  const int nb = PAIR ? 2 * (int)gridDim.x : (int)gridDim.x;
  const int half = PAIR ? (int)(threadIdx.x >> 8) : 0;
  const int kbk = half == 0 ? (int)blockIdx.x : nb - 1 - (int)blockIdx.x;
  const int h = blockIdx.y, b = blockIdx.z, kvh = h / (Hq / Hkv);
  const int lane = threadIdx.x & 63, w = (threadIdx.x >> 6) & 3, wave = threadIdx.x >> 6;
  const int kw0 = kbk * 128 + w * 32;
  const int kj = kw0 + (lane & 31);

  const uint16_t* qb_ = q + (int64_t)b * S * ldq + h * D;
  const uint16_t* db_ = dO + (int64_t)b * S * lddo + h * D;
  const float* lrow = lse + ((int64_t)b * Hq + h) * S;
  const float* drow = Di + ((int64_t)b * Hq + h) * S;
  const __amdgpu_buffer_rsrc_t rq = fa_rsrc(qb_, (int)((S - 1) * ldq * 2 + D * 2));
  const __amdgpu_buffer_rsrc_t rd = fa_rsrc(db_, (int)((S - 1) * lddo * 2 + D * 2));
  const __amdgpu_buffer_rsrc_t rl = fa_rsrc(lrow, S * 4), rdi = fa_rsrc(drow, S * 4);
  Dma128<NT> gq, gd;
  gq.init(ldq);
  gd.init(lddo);
  const int qstart = (int)blockIdx.x * 128;  // the earlier key block of the workgroup
  auto issue = [&](int q0, int buf) {
    gq.fetch(rq, sQ + buf * TB, (int)(q0 * ldq * 2));
    gd.fetch(rd, sdO + buf * TB, (int)(q0 * lddo * 2));
    if (wave == 0) fa_dma_row64(rl, sL + buf * QB, q0 * 4);
    if (wave == 1) fa_dma_row64(rdi, sDi + buf * QB, q0 * 4);
  };
  issue(qstart, 0);

  bf16x8 kf[D / 16];
  uint16_t* sVw = sV + wave * 32 * RP;  // this wave's rows: key kw0 + row
  {
    const uint16_t* krow = k + ((int64_t)b * S + kj) * ldk + kvh * D + (lane >> 5) * 8;
    const uint16_t* vrow = v + ((int64_t)b * S + kj) * ldv + kvh * D + (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < D / 16; kk++) {
      kf[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(krow + kk * 16));
      *reinterpret_cast<uint4*>(sVw + (lane & 31) * RP + kk * 16 + (lane >> 5) * 8) =
          *reinterpret_cast<const uint4*>(vrow + kk * 16);
    }
  }
  floatx16 dv[D / 32], dk[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; i++) { zero16(dv[i]); zero16(dk[i]); }

  int buf = 0;
  for (int q0 = qstart; q0 < S; q0 += QB, buf ^= 1) {
    fa_wait_vm();     // this thread's copies of tile q0 have landed
    __syncthreads();  // ... everyone's have; and every wave is done with the other buffer
    if (q0 + QB < S) issue(q0 + QB, buf ^ 1);
    if (q0 + QB - 1 < kw0) continue;  // every query precedes this wave's keys
    const uint8_t* tQ = sQ + buf * TB;
    const uint8_t* tO = sdO + buf * TB;
    const float* tL = sL + buf * QB;
    const float* tD = sDi + buf * QB;
#pragma unroll
    for (int jb = 0; jb < NQ; jb++) {
      if (q0 + jb * 32 + 31 < kw0) continue;  // this 32-query block precedes the wave's keys
      floatx16 sacc, dpacc;
      zero16(sacc);
      zero16(dpacc);
      const int qr = jb * 32 + (lane & 31);
#pragma unroll
      for (int kk = 0; kk < D / 16; kk++) {
        const int c = kk * 2 + (lane >> 5);
        sacc = mfma16(rrow(tQ, qr, c), kf[kk], sacc);
        const bf16x8 vf = as_bf16x8(*reinterpret_cast<const uint4*>(sVw + (lane & 31) * RP + kk * 16 + (lane >> 5) * 8));
        dpacc = mfma16(rrow(tO, qr, c), vf, dpacc);
      }
      const bool diag = q0 + jb * 32 < kw0 + 31;
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++) {
        const int r0 = jb * 32 + g4 * 8 + (lane >> 5) * 4;
        const float4 L4 = *reinterpret_cast<const float4*>(tL + r0);
        const float4 D4 = *reinterpret_cast<const float4*>(tD + r0);
        const float Lv[4] = {L4.x, L4.y, L4.z, L4.w}, Dv[4] = {D4.x, D4.y, D4.z, D4.w};
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int e = g4 * 4 + u;
          float p = fexp2(sacc[e] * sl2 - Lv[u]);
          if (diag && q0 + r0 + u < kj) p = 0.f;
          sacc[e] = p;
          dpacc[e] = p * (dpacc[e] - Dv[u]);
        }
      }
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const bf16x8 pf = pack8(sacc, 8 * c);
        const bf16x8 sf = pack8(dpacc, 8 * c);
#pragma unroll
        for (int i = 0; i < D / 32; i++) {
          dv[i] = mfma16(pf, rtr(tO, jb * 32 + c * 16, i, lane), dv[i]);
          dk[i] = mfma16(sf, rtr(tQ, jb * 32 + c * 16, i, lane), dk[i]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < D / 32; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const int key = kw0 + acc_row(e, lane);
      const int64_t off = (((int64_t)b * S + key) * Hq + h) * D + i * 32 + (lane & 31);
      stg(dKh + off, dk[i][e] * scale);
      stg(dVh + off, dv[i][e]);
    }
}

// ============================================================================
// backward dQ: grid (S/128, Hq, B); 4 waves x 32 queries; key tiles of 64
// ============================================================================
template <int D, bool PAIR, typename TG>
__global__ __launch_bounds__(PAIR ? 512 : 256) void fa_bwd_dq_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ Di,
    TG* __restrict__ dq, int S, int Hq, int Hkv, int64_t ldq, int64_t ldk, int64_t ldv, int64_t lddo,
    int64_t lddq, float sl2, float scale) {
  constexpr int KB = 64, RP = D + 8, TP = KB + 4, NT = PAIR ? 512 : 256;
  __shared__ __attribute__((aligned(16))) uint16_t sK[KB * RP];
  __shared__ __attribute__((aligned(16))) uint16_t sKt[D * TP];
  __shared__ __attribute__((aligned(16))) uint16_t sV[KB * RP];
  const int nb = PAIR ? 2 * (int)gridDim.x : (int)gridDim.x;
  const int half = PAIR ? (int)(threadIdx.x >> 8) : 0;
  const int qb = half == 0 ? nb - 1 - (int)blockIdx.x : (int)blockIdx.x;
  const int h = blockIdx.y, b = blockIdx.z, kvh = h / (Hq / Hkv);
  const int lane = threadIdx.x & 63, w = (threadIdx.x >> 6) & 3;
  const int qi = qb * 128 + w * 32 + (lane & 31);
  bf16x8 qf[D / 16], of[D / 16];
  {
    const uint16_t* qrow = q + ((int64_t)b * S + qi) * ldq + h * D + (lane >> 5) * 8;
    const uint16_t* orow = dO + ((int64_t)b * S + qi) * lddo + h * D + (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < D / 16; kk++) {
      qf[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(qrow + kk * 16));
      of[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(orow + kk * 16));
    }
  }
  const float lq = lse[((int64_t)b * Hq + h) * S + qi];
  const float dq_i = Di[((int64_t)b * Hq + h) * S + qi];
  floatx16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; i++) zero16(acc[i]);
  const uint16_t* kb = k + (int64_t)b * S * ldk + kvh * D;
  const uint16_t* vb = v + (int64_t)b * S * ldv + kvh * D;
  const int kend = (nb - (int)blockIdx.x) * 128;  // the longer block of the workgroup
  const int wq_last = qb * 128 + w * 32 + 31;
  Pref<D, KB, NT> pk, pv;
  pk.load(kb, ldk, 0);
  pv.load(vb, ldv, 0);
  for (int k0 = 0; k0 < kend; k0 += KB) {
    __syncthreads();
    pk.template store<true, true>(sK, sKt);
    pv.template store<true, false>(sV, nullptr);
    __syncthreads();
    if (k0 + KB < kend) {
      pk.load(kb, ldk, k0 + KB);
      pv.load(vb, ldv, k0 + KB);
    }
    if (k0 > wq_last) continue;
    // S^T = K Q^T, dP^T = V dO^T : rows = keys, cols = queries (lane <-> query)
    floatx16 s[2], dp[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      zero16(s[j]);
      zero16(dp[j]);
#pragma unroll
      for (int kk = 0; kk < D / 16; kk++) {
        const int off = (j * 32 + (lane & 31)) * RP + kk * 16 + (lane >> 5) * 8;
        s[j] = mfma16(as_bf16x8(*reinterpret_cast<const uint4*>(sK + off)), qf[kk], s[j]);
        dp[j] = mfma16(as_bf16x8(*reinterpret_cast<const uint4*>(sV + off)), of[kk], dp[j]);
      }
    }
    const bool diag = k0 + KB - 1 > qb * 128 + w * 32;  // some key of the tile follows some query
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        float p = fexp2(s[j][e] * sl2 - lq);
        if (diag && k0 + j * 32 + acc_row(e, lane) > qi) p = 0.f;
        s[j][e] = p * (dp[j][e] - dq_i);  // dS^T
      }
    // dQ^T += K^T dS^T : A = K^T (lane row = d), B = dS^T from registers (lane col = query)
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const bf16x8 sf = pack8(s[c >> 1], 8 * (c & 1));
#pragma unroll
      for (int i = 0; i < D / 32; i++) acc[i] = mfma16(tload<KB>(sKt, i, c * 16, lane), sf, acc[i]);
    }
  }
  TG* qrow = dq + ((int64_t)b * S + qi) * lddq + h * D;
#pragma unroll
  for (int i = 0; i < D / 32; i++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int d = i * 32 + g * 8 + (lane >> 5) * 4;
      const float a0 = acc[i][4 * g] * scale, a1 = acc[i][4 * g + 1] * scale, a2 = acc[i][4 * g + 2] * scale,
                  a3 = acc[i][4 * g + 3] * scale;
      if constexpr (sizeof(TG) == 4) *reinterpret_cast<float4*>(qrow + d) = make_float4(a0, a1, a2, a3);
      else *reinterpret_cast<uint2*>(qrow + d) = make_uint2(pack_bf2(a0, a1), pack_bf2(a2, a3));
    }
}

// D = 128 form of fa_bwd_dq_kernel: key/value tiles copied global -> LDS by DMA into a double
// buffer, K^T operands read from the K row tile with ds_read_b64_tr_b16.
template <bool PAIR, typename TG>
__global__ __launch_bounds__(PAIR ? 512 : 256) void fa_bwd_dq128_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ Di,
    TG* __restrict__ dq, int S, int Hq, int Hkv, int64_t ldq, int64_t ldk, int64_t ldv, int64_t lddo,
    int64_t lddq, float sl2, float scale) {
  constexpr int D = 128, KB = 64, NT = PAIR ? 512 : 256, TB = KB * 256;
  __shared__ __attribute__((aligned(1024))) uint8_t sK[2 * TB];
  __shared__ __attribute__((aligned(1024))) uint8_t sV[2 * TB];
  const int nb = PAIR ? 2 * (int)gridDim.x : (int)gridDim.x;
  const int half = PAIR ? (int)(threadIdx.x >> 8) : 0;
  const int qb = half == 0 ? nb - 1 - (int)blockIdx.x : (int)blockIdx.x;
  const int h = blockIdx.y, b = blockIdx.z, kvh = h / (Hq / Hkv);
  const int lane = threadIdx.x & 63, w = (threadIdx.x >> 6) & 3;
  const int qi = qb * 128 + w * 32 + (lane & 31);
  const uint16_t* kb = k + (int64_t)b * S * ldk + kvh * D;
  const uint16_t* vb = v + (int64_t)b * S * ldv + kvh * D;
  const __amdgpu_buffer_rsrc_t rk = fa_rsrc(kb, (int)((S - 1) * ldk * 2 + D * 2));
  const __amdgpu_buffer_rsrc_t rv = fa_rsrc(vb, (int)((S - 1) * ldv * 2 + D * 2));
  Dma128<NT> gk, gv;
  gk.init(ldk);
  gv.init(ldv);
  gk.fetch(rk, sK, 0);
  gv.fetch(rv, sV, 0);
  bf16x8 qf[D / 16], of[D / 16];
  {
    const uint16_t* qrow = q + ((int64_t)b * S + qi) * ldq + h * D + (lane >> 5) * 8;
    const uint16_t* orow = dO + ((int64_t)b * S + qi) * lddo + h * D + (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < D / 16; kk++) {
      qf[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(qrow + kk * 16));
      of[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(orow + kk * 16));
    }
  }
  const float lq = lse[((int64_t)b * Hq + h) * S + qi];
  const float dq_i = Di[((int64_t)b * Hq + h) * S + qi];
  floatx16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; i++) zero16(acc[i]);
  const int kend = (nb - (int)blockIdx.x) * 128;  // the longer block of the workgroup
  const int wq_last = qb * 128 + w * 32 + 31;
  int buf = 0;
  for (int k0 = 0; k0 < kend; k0 += KB, buf ^= 1) {
    fa_wait_vm();
    __syncthreads();
    if (k0 + KB < kend) {
      gk.fetch(rk, sK + (buf ^ 1) * TB, (int)((k0 + KB) * ldk * 2));
      gv.fetch(rv, sV + (buf ^ 1) * TB, (int)((k0 + KB) * ldv * 2));
    }
    if (k0 > wq_last) continue;
    const uint8_t* tK = sK + buf * TB;
    const uint8_t* tV = sV + buf * TB;
    floatx16 sc[2], dp[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      zero16(sc[j]);
      zero16(dp[j]);
#pragma unroll
      for (int kk = 0; kk < D / 16; kk++) {
        const int r = j * 32 + (lane & 31), c = kk * 2 + (lane >> 5);
        sc[j] = mfma16(rrow(tK, r, c), qf[kk], sc[j]);
        dp[j] = mfma16(rrow(tV, r, c), of[kk], dp[j]);
      }
    }
    const bool diag = k0 + KB - 1 > qb * 128 + w * 32;
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        float p = fexp2(sc[j][e] * sl2 - lq);
        if (diag && k0 + j * 32 + acc_row(e, lane) > qi) p = 0.f;
        sc[j][e] = p * (dp[j][e] - dq_i);
      }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const bf16x8 sf = pack8(sc[c >> 1], 8 * (c & 1));
#pragma unroll
      for (int i = 0; i < D / 32; i++) acc[i] = mfma16(rtr(tK, c * 16, i, lane), sf, acc[i]);
    }
  }
  TG* qrow = dq + ((int64_t)b * S + qi) * lddq + h * D;
#pragma unroll
  for (int i = 0; i < D / 32; i++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int d = i * 32 + g * 8 + (lane >> 5) * 4;
      const float a0 = acc[i][4 * g] * scale, a1 = acc[i][4 * g + 1] * scale, a2 = acc[i][4 * g + 2] * scale,
                  a3 = acc[i][4 * g + 3] * scale;
      if constexpr (sizeof(TG) == 4) *reinterpret_cast<float4*>(qrow + d) = make_float4(a0, a1, a2, a3);
      else *reinterpret_cast<uint2*>(qrow + d) = make_uint2(pack_bf2(a0, a1), pack_bf2(a2, a3));
    }
}

// dK/dV [b, s, kvh, :] = sum over the group's query heads (ascending) of the per-head partials.
template <int D>
__global__ __launch_bounds__(256) void fa_group_reduce_kernel(const float* __restrict__ dKh, const float* __restrict__ dVh,
                                                              float* __restrict__ dk, float* __restrict__ dv, int B,
                                                              int S, int Hq, int Hkv, int64_t lddk, int64_t lddv) {
  const int grp = Hq / Hkv;
  const int64_t n = (int64_t)B * S * Hkv * D;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int d = (int)(i % D);
    const int kvh = (int)((i / D) % Hkv);
    const int64_t t = i / ((int64_t)D * Hkv);
    float a = 0.f, c = 0.f;
    for (int g = 0; g < grp; g++) {
      const int64_t off = (t * Hq + kvh * grp + g) * D + d;
      a += dKh[off];
      c += dVh[off];
    }
    dk[t * lddk + kvh * D + d] = a;
    dv[t * lddv + kvh * D + d] = c;
  }
}

// ---------------------------------------------------------------- launchers
int flash_forward(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, float* lse, int B,
                  int S, int Hq, int Hkv, int D, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo,
                  hipStream_t s) {
  SMHIP_REQUIRE(S % 128 == 0, "flash attention: S must be a multiple of 128");
  SMHIP_REQUIRE(Hkv > 0 && Hq % Hkv == 0, "flash attention: Hq must be a multiple of Hkv");
  const float sl2 = kLog2e / sqrtf((float)D);
  // pair the causal blocks (balanced workgroups) whenever their count is even
  const bool pair = (S / 128) % 2 == 0;
  const dim3 grid(pair ? S / 256 : S / 128, Hq, B), block(pair ? 512 : 256);
  const int ev0 = prof_mark(s);
#define FA_FWD(DD, PP) hipLaunchKernelGGL((fa_fwd_kernel<DD, PP>), grid, block, 0, s, q, k, v, o, lse, S, Hq, Hkv, ldq, ldk, ldv, ldo, sl2)
  const bool dma = D == 128 && ((uintptr_t)k | (uintptr_t)v) % 16 == 0 && (ldk | ldv) % 8 == 0 &&
                   (int64_t)S * std::max(ldk, ldv) * 2 < (int64_t)1 << 31;
  if (dma) {
    if (pair) hipLaunchKernelGGL((fa_fwd128_kernel<true>), grid, block, 0, s, q, k, v, o, lse, S, Hq, Hkv, ldq, ldk, ldv, ldo, sl2);
    else hipLaunchKernelGGL((fa_fwd128_kernel<false>), grid, block, 0, s, q, k, v, o, lse, S, Hq, Hkv, ldq, ldk, ldv, ldo, sl2);
  } else if (D == 128) { if (pair) FA_FWD(128, true); else FA_FWD(128, false); }
  else if (D == 64) { if (pair) FA_FWD(64, true); else FA_FWD(64, false); }
  else return fail(SMHIP_EUNSUPPORTED, "flash attention: head_dim must be 64 or 128");
#undef FA_FWD
  SMHIP_CHECK_LAUNCH();
  // causal: QK^T and PV over the lower triangle
  prof_add(PROF_FLASH_FWD, ev0, prof_mark(s), 2.0 * B * Hq * (double)S * S * D);
  return SMHIP_OK;
}

size_t flash_backward_workspace(int B, int S, int Hq, int D) {
  return sizeof(float) * ((size_t)B * Hq * S + 2 * (size_t)B * S * Hq * D) + 256;
}

void flash_backward_partials(void* ws, int B, int S, int Hq, int D, const void** dKh, const void** dVh) {
  const float* Di = (const float*)ws;
  const float* k = Di + (size_t)B * Hq * S;
  *dKh = k;
  *dVh = k + (size_t)B * S * Hq * D;
}

int flash_backward(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* o,
                   const uint16_t* dO, const float* lse, void* dq, float* dk, float* dv, int B, int S,
                   int Hq, int Hkv, int D, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo, int64_t lddo,
                   int64_t lddq, int64_t lddk, int64_t lddv, void* ws, hipStream_t s, int bf16_grads) {
  SMHIP_REQUIRE(S % 128 == 0, "flash attention: S must be a multiple of 128");
  SMHIP_REQUIRE(Hkv > 0 && Hq % Hkv == 0, "flash attention: Hq must be a multiple of Hkv");
  SMHIP_REQUIRE((dk == nullptr) == (dv == nullptr), "flash attention backward: dk and dv are both given or both null");
  SMHIP_REQUIRE(!bf16_grads || !dk, "flash attention backward: bf16 gradients leave dK/dV as per-head partials");
  const float scale = 1.f / sqrtf((float)D), sl2 = kLog2e * scale;
  float* Di = (float*)ws;
  float* dKh = Di + (size_t)B * Hq * S;
  float* dVh = dKh + (size_t)B * S * Hq * D;
  uint16_t* dKb = (uint16_t*)dKh;  // bf16 partials use the first half of each region
  uint16_t* dVb = (uint16_t*)dVh;
  const int64_t rows = (int64_t)B * Hq * S;
  const int gpre = (int)std::min<int64_t>((rows + 3) / 4, (int64_t)num_cus() * 8);
  const bool pre_vec = ((uintptr_t)o | (uintptr_t)dO) % 16 == 0 && ldo % 8 == 0 && lddo % 8 == 0;
  const int gpre_v = (int)std::min<int64_t>((rows * (D / 8) + 255) / 256, (int64_t)num_cus() * 8);
  const int gred = (int)std::min<int64_t>(((int64_t)B * S * Hkv * D + 255) / 256, (int64_t)num_cus() * 8);
  const bool pair = (S / 128) % 2 == 0;
  const dim3 grid(pair ? S / 256 : S / 128, Hq, B), block(pair ? 512 : 256);
  // DMA-staged D = 128 kernels: 16-byte aligned rows and one batch's rows within a 2 GiB
  // buffer resource
  const int64_t ldmax = std::max(std::max(ldq, ldk), std::max(ldv, lddo));
  const bool dma = D == 128 && ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)dO) % 16 == 0 &&
                   (ldq | ldk | ldv | lddo) % 8 == 0 && (int64_t)S * ldmax * 2 < (int64_t)1 << 31;
  const int ev0 = prof_mark(s);
#define FA_BWD(DD, PP)                                                                                          \
  if (pre_vec)                                                                                                  \
    hipLaunchKernelGGL(fa_bwd_pre_vec_kernel<DD>, dim3(gpre_v), dim3(256), 0, s, o, dO, Di, B, S, Hq, ldo, lddo); \
  else                                                                                                          \
    hipLaunchKernelGGL(fa_bwd_pre_kernel<DD>, dim3(gpre), dim3(256), 0, s, o, dO, Di, B, S, Hq, ldo, lddo);    \
  if (bf16_grads) {                                                                                             \
    if (DD == 128 && dma)                                                                                       \
      hipLaunchKernelGGL((fa_bwd_dkdv128_kernel<PP, uint16_t>), grid, block, 0, s, q, k, v, dO, lse, Di, dKb,     \
                         dVb, S, Hq, Hkv, ldq, ldk, ldv, lddo, sl2, scale);                                       \
    else                                                                                                        \
      hipLaunchKernelGGL((fa_bwd_dkdv_kernel<DD, PP, uint16_t>), grid, block, 0, s, q, k, v, dO, lse, Di, dKb,    \
                         dVb, S, Hq, Hkv, ldq, ldk, ldv, lddo, sl2, scale);                                       \
    if (DD == 128 && dma)                                                                                       \
      hipLaunchKernelGGL((fa_bwd_dq128_kernel<PP, uint16_t>), grid, block, 0, s, q, k, v, dO, lse, Di,            \
                         (uint16_t*)dq, S, Hq, Hkv, ldq, ldk, ldv, lddo, lddq, sl2, scale);                       \
    else                                                                                                        \
      hipLaunchKernelGGL((fa_bwd_dq_kernel<DD, PP, uint16_t>), grid, block, 0, s, q, k, v, dO, lse, Di,           \
                         (uint16_t*)dq, S, Hq, Hkv, ldq, ldk, ldv, lddo, lddq, sl2, scale);                       \
  } else {                                                                                                      \
    if (DD == 128 && dma)                                                                                       \
      hipLaunchKernelGGL((fa_bwd_dkdv128_kernel<PP, float>), grid, block, 0, s, q, k, v, dO, lse, Di, dKh, dVh,   \
                         S, Hq, Hkv, ldq, ldk, ldv, lddo, sl2, scale);                                            \
    else                                                                                                        \
      hipLaunchKernelGGL((fa_bwd_dkdv_kernel<DD, PP, float>), grid, block, 0, s, q, k, v, dO, lse, Di, dKh, dVh,  \
                         S, Hq, Hkv, ldq, ldk, ldv, lddo, sl2, scale);                                            \
    if (DD == 128 && dma)                                                                                       \
      hipLaunchKernelGGL((fa_bwd_dq128_kernel<PP, float>), grid, block, 0, s, q, k, v, dO, lse, Di, (float*)dq,   \
                         S, Hq, Hkv, ldq, ldk, ldv, lddo, lddq, sl2, scale);                                      \
    else                                                                                                        \
      hipLaunchKernelGGL((fa_bwd_dq_kernel<DD, PP, float>), grid, block, 0, s, q, k, v, dO, lse, Di, (float*)dq,  \
                         S, Hq, Hkv, ldq, ldk, ldv, lddo, lddq, sl2, scale);                                      \
  }                                                                                                             \
  if (dk)                                                                                                       \
    hipLaunchKernelGGL(fa_group_reduce_kernel<DD>, dim3(gred), dim3(256), 0, s, dKh, dVh, dk, dv, B, S, Hq, Hkv, \
                       lddk, lddv);
  if (D == 128) { if (pair) { FA_BWD(128, true) } else { FA_BWD(128, false) } }
  else if (D == 64) { if (pair) { FA_BWD(64, true) } else { FA_BWD(64, false) } }
  else return fail(SMHIP_EUNSUPPORTED, "flash attention: head_dim must be 64 or 128");
#undef FA_BWD
  SMHIP_CHECK_LAUNCH();
  // causal backward, algorithmic: recompute QK^T, dP = dO V^T, dV, dK, dQ (5 half-triangle products)
  prof_add(PROF_FLASH_BWD, ev0, prof_mark(s), 5.0 * B * Hq * (double)S * S * D);
  return SMHIP_OK;
}

}  // namespace smhip
