// skinny.hip — rank-sized GEMMs of the LoRA step for gfx950, streamed at HBM rate.
//
//   C[M, n] = alpha * sum_k Big(m, k) Small(r, k) + beta * C      (n = LoRA rank columns, <= 64)
//
// The four adapter products of a LoRA projection (LoRAAdapter.cs forward/backward) are all of
// this shape: one operand is a full activation or gradient (Big, T x In or T x Out, tens of
// MB) and the other has only n = r (or 2r, 3r for fused projections) rows:
//   u  = x A            Big = x  [T, In]  k-contiguous, Small = A [In, n] (n contiguous)
//   z  = dY B^T         Big = dY [T, Out] k-contiguous, Small = B [n, Out] (k contiguous)
//   dA += s x^T z       Big = x  (k = token, m contiguous), Small = z [T, n]
//   dB += s u^T dY      computed as its transpose dB^T[o, r] = sum_t dY[t, o] u[t, r]:
//                       Big = dY (k = token, m contiguous), Small = u [T, n], stored transposed
// Their cost is reading Big once, so the kernel is built for bandwidth: every workgroup
// streams a 128-row x K/S slice of Big through a 3-stage ring of direct-to-LDS buffer loads
// (buffer_load ... lds, two stages in flight, two workgroups per CU), and multiplies it
// with v_mfma_f32_16x16x32_bf16 (16-column blocks: ranks 16/32/48 waste no MFMA columns).
// Operands whose contiguous axis is m (or r) rather than k are DMA'd in their raw layout
// (k rows) and transposed by the fragment reads: Big with two ds_read_b64_tr_b16 per fragment
// (its 16-byte m-chunks XOR-swizzled by k-row so that four consecutive k-rows hit distinct
// banks), Small with eight 16-bit LDS reads; the raw Big rows are kept in 1 KiB blocks padded
// by 32 bytes.  k-contiguous tiles use the XOR-swizzled [row][64] layout of the GEMM.
// The reduction over K is split S ways (S chosen so the fp32 partials stay a small fraction
// of the bytes of Big); a second kernel sums the S partials in a fixed order, so results are
// deterministic and independent of timing.
#include <cstring>

#include "common.hpp"
#include "kernels.hpp"

namespace smhip {
namespace sk {

constexpr int MT = 128;        // Big rows per workgroup (4 waves x 32)
constexpr int BKT = 64;        // k per stage
constexpr int ST = 3;          // ring stages
constexpr int RAW_BLK = 1056;  // 1 KiB of raw Big (4 k-rows of 128 m) + 32 bytes of padding
constexpr int BIG_BYTES = 16 * RAW_BLK;  // >= 16 KiB swizzled tile
constexpr int SMALL_BYTES = 8192;        // n <= 64 rows x 64 k x 2 bytes
constexpr int STAGE = BIG_BYTES + SMALL_BYTES;
constexpr uint32_t OOB = 0x80000000u;
typedef __attribute__((address_space(3))) void lds_void;

struct Args {
  const void* big;
  int64_t ldb;      // Big row pitch (elements)
  int big_bytes;
  const void* small;
  int64_t lds;      // Small row pitch (elements)
  int small_bytes;
  int M, n, K;
  int kps;          // k tiles per split
  float* partial;   // [S][M][n] when S > 1
  SkinnyMask mask;  // block-diagonal output mask (transposed outputs of fused LoRA B gradients)
  void* C;
  int64_t ldc;
  float alpha, beta;
};

// entry (r, m) of the output is stored unless the block-diagonal mask excludes it
__device__ __forceinline__ bool mask_keep(const SkinnyMask& mk, int r, int64_t m, int M) {
  if (!mk.cols) return true;
  const int blk = r / mk.rank;
  const int lo = mk.cols[blk], hi = blk + 1 < mk.nblk ? mk.cols[blk + 1] : M;
  return m >= lo && m < hi;
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ int sw(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, uint8_t* lds, uint32_t off) {
#if defined(__HIP_DEVICE_COMPILE__)  // the LDS address-space cast exists only in the device pass
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)lds, 16, off, 0, 0, 0);
#endif
}
template <int N>
__device__ __forceinline__ void wait_vm_n() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_s4;

// Big tile loader.  BIGK: k-contiguous rows m (swizzled [128][64]); else raw k-rows.
// Each wave issues exactly 4 DMA instructions per stage.
template <bool BIGK>
struct BigLoad {
  __amdgpu_buffer_rsrc_t rs;
  uint32_t off[4];
  uint32_t kstep;  // bytes per k tile
  __device__ void init(const Args& a, int m0) {
    rs = rsrc(a.big, a.big_bytes);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int blk = j * 4 + w;
      if constexpr (BIGK) {
        const int r = blk * 8 + (l >> 3), c = (l & 7) ^ ((r >> 1) & 7);
        off[j] = m0 + r < a.M ? (uint32_t)(((int64_t)(m0 + r) * a.ldb) * 2 + c * 16) : OOB;
      } else {
        // raw k-rows, 16-byte m-chunks XOR-swizzled by 2 * (k-row % 4): the transposed fragment
        // reads of four consecutive k-rows then hit distinct banks
        const int kr = blk * 4 + (l >> 4);
        off[j] = (uint32_t)(((int64_t)kr * a.ldb + m0 + ((l & 15) ^ (2 * (l >> 4))) * 8) * 2);
      }
    }
    kstep = BIGK ? BKT * 2 : (uint32_t)(BKT * a.ldb * 2);
  }
  __device__ __forceinline__ void fetch(uint8_t* stage, int kt) {
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int blk = j * 4 + w;
      dma16(rs, stage + (BIGK ? blk * 1024 : blk * RAW_BLK), off[j] == OOB ? OOB : off[j] + kt * kstep);
    }
  }
  // A fragment of v_mfma_f32_16x16x32_bf16: row (lane & 15) of block rb, k = 8*(lane>>4) .. +8
  // of k-slice kk (0..1)
  __device__ __forceinline__ bf16x8 frag(const uint8_t* stage, int row, int kk) const {
    const int l = threadIdx.x & 63;
    if constexpr (BIGK) {
      return *reinterpret_cast<const bf16x8*>(stage + sw(row, kk * 4 + (l >> 4)));
    } else {
      // two ds_read_b64_tr_b16 over the 16 lanes of a k-group: source lane s reads 4 m of k-row
      // k0 + 4h + s/4 at m = mb + 4 (s%4); destination lane s receives m = mb + s of those rows
      const int s = l & 15, k0 = kk * 32 + 8 * (l >> 4), mb = row & ~15;
      const int slot = ((mb + 4 * (s & 3)) >> 3) ^ (2 * (s >> 2));
      const uint8_t* p = stage + (k0 >> 2) * RAW_BLK + (s >> 2) * 256 + slot * 16 + (s & 1) * 8;
      short4v lo, hi;
#if defined(__HIP_DEVICE_COMPILE__)
      lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)p);
      hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p + RAW_BLK));
#else
      lo = hi = short4v{};
#endif
      const uint2 x = __builtin_bit_cast(uint2, lo), y = __builtin_bit_cast(uint2, hi);
      return __builtin_bit_cast(bf16x8, make_uint4(x.x, x.y, y.x, y.y));
    }
  }
};

// Small tile loader (n rows, n = 16 * NB).  SMALLK: k-contiguous rows (swizzled [n][64]);
// else raw [64 k][n] (the operand's row pitch must equal n, so a tile is one contiguous
// 128*n-byte run).  NI = n / 8 DMA instructions per tile, spread over the 4 waves; waves
// beyond NI repeat an instruction (same bytes to the same place) so that every wave issues
// the same count and one vmcnt value waits for a stage.
template <bool SMALLK, int NB>
struct SmallLoad {
  static constexpr int N = 16 * NB;
  static constexpr int NI = N / 8;                   // 1 KiB instructions per tile
  static constexpr int PW = (NI + 3) / 4;            // per wave
  __amdgpu_buffer_rsrc_t rs;
  uint32_t off[PW];
  int dst[PW];
  uint32_t kstep;
  __device__ void init(const Args& a) {
    rs = rsrc(a.small, a.small_bytes);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < PW; j++) {
      const int blk = (j * 4 + w) % NI;
      dst[j] = blk * 1024;
      if constexpr (SMALLK) {
        const int r = blk * 8 + (l >> 3), c = (l & 7) ^ ((r >> 1) & 7);
        off[j] = r < a.n ? (uint32_t)(((int64_t)r * a.lds) * 2 + c * 16) : OOB;
      } else {
        off[j] = (uint32_t)(blk * 1024 + l * 16);
      }
    }
    kstep = SMALLK ? BKT * 2 : (uint32_t)(BKT * N * 2);
  }
  __device__ __forceinline__ void fetch(uint8_t* stage, int kt) {
#pragma unroll
    for (int j = 0; j < PW; j++) dma16(rs, stage + dst[j], off[j] == OOB ? OOB : off[j] + kt * kstep);
  }
  __device__ __forceinline__ bf16x8 frag(const uint8_t* stage, int col, int kk) const {
    const int l = threadIdx.x & 63;
    if constexpr (SMALLK) {
      return *reinterpret_cast<const bf16x8*>(stage + sw(col, kk * 4 + (l >> 4)));
    } else {
      const int k0 = kk * 32 + 8 * (l >> 4);
      bf16x8 v;
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = *reinterpret_cast<const __bf16*>(stage + ((k0 + j) * N + col) * 2);
      return v;
    }
  }
};

// one 128-row tile and one K split of a product (the kernels below pick which)
template <bool BIGK, bool SMALLK, int NB, bool TRANS_OUT, bool C_BF16>
__device__ __forceinline__ void skinny_tile(const Args& a, int mtile, int split, uint8_t* smem) {
  auto big_st = [&](int s) -> uint8_t* { return smem + s * STAGE; };
  auto small_st = [&](int s) -> uint8_t* { return smem + s * STAGE + BIG_BYTES; };
  const int m0 = mtile * MT;
  const int kt0 = split * a.kps;
  const int nk = max(0, min(a.K / BKT, kt0 + a.kps) - kt0);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;

  BigLoad<BIGK> lb;
  SmallLoad<SMALLK, NB> ls;
  lb.init(a, m0);
  ls.init(a);
  constexpr int PER = 4 + SmallLoad<SMALLK, NB>::PW;

  floatx4 acc[2][NB];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < NB; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int t = 0; t < ST - 1; t++)
    if (t < nk) {
      lb.fetch(big_st(t), kt0 + t);
      ls.fetch(small_st(t), kt0 + t);
    }
  for (int t = 0; t < nk; t++) {
    if (t + ST - 2 < nk) wait_vm_n<(ST - 2) * PER>();
    else wait_vm_n<0>();
    ring_barrier();  // stage t landed for every wave; stage of t-1 is free
    if (t + ST - 1 < nk) {
      const int s = (t + ST - 1) % ST;
      lb.fetch(big_st(s), kt0 + t + ST - 1);
      ls.fetch(small_st(s), kt0 + t + ST - 1);
    }
    const uint8_t* bs = big_st(t % ST);
    const uint8_t* ss = small_st(t % ST);
#pragma unroll
    for (int kk = 0; kk < BKT / 32; kk++) {
      bf16x8 fa[2], fb[NB];
#pragma unroll
      for (int i = 0; i < 2; i++) fa[i] = lb.frag(bs, wv * 32 + i * 16 + (lane & 15), kk);
#pragma unroll
      for (int j = 0; j < NB; j++) fb[j] = ls.frag(ss, j * 16 + (lane & 15), kk);
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  }

  // lane holds rows 4*(lane>>4) + e, column lane & 15 of each 16 x 16 block
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int col = j * 16 + (lane & 15);
      if (col >= a.n) continue;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int row = m0 + wv * 32 + i * 16 + 4 * (lane >> 4) + e;
        if (row >= a.M) continue;
        if (a.partial) {
          a.partial[((int64_t)split * a.M + row) * a.n + col] = acc[i][j][e];
          continue;
        }
        if (!mask_keep(a.mask, col, row, a.M)) continue;
        const int64_t ci = TRANS_OUT ? (int64_t)col * a.ldc + row : (int64_t)row * a.ldc + col;
        float o = a.alpha * acc[i][j][e];
        if constexpr (C_BF16) {
          uint16_t* c = (uint16_t*)a.C + ci;
          if (a.beta != 0.f) o += a.beta * bf2f(*c);
          *c = f2bf(o);
        } else {
          float* c = (float*)a.C + ci;
          if (a.beta != 0.f) o += a.beta * *c;
          *c = o;
        }
      }
    }
}

template <bool BIGK, bool SMALLK, int NB, bool TRANS_OUT, bool C_BF16>
__global__ __launch_bounds__(256, 2) void skinny_kernel(Args a) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[ST * STAGE];
  skinny_tile<BIGK, SMALLK, NB, TRANS_OUT, C_BF16>(a, blockIdx.x, blockIdx.y, smem);
}

// Two products of the same operand kinds and rank in one launch (a LoRA projection's dA and
// dB^T): workgroups [0, nb0) are the (tile, split) pairs of a0, the rest those of a1.
template <bool BIGK, bool SMALLK, int NB, bool T0, bool T1, bool C_BF16>
__global__ __launch_bounds__(256, 2) void skinny_pair_kernel(Args a0, Args a1, int mt0, int nb0, int mt1) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[ST * STAGE];
  const int b = blockIdx.x;
  if (b < nb0) skinny_tile<BIGK, SMALLK, NB, T0, C_BF16>(a0, b % mt0, b / mt0, smem);
  else skinny_tile<BIGK, SMALLK, NB, T1, C_BF16>(a1, (b - nb0) % mt1, (b - nb0) / mt1, smem);
}

// C (m, r) = alpha * sum_s partial[s][m][r] + beta * C, splits summed in ascending order.
// One thread per 4 consecutive r of one m (n % 16 == 0): float4 reads of the partials, which
// are contiguous for consecutive threads; the S loads of a thread are independent and issued
// together.
template <bool TRANS_OUT, bool C_BF16>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* __restrict__ partial, int S, int M, int n,
                                                            void* C, int64_t ldc, float alpha, float beta,
                                                            SkinnyMask mask) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // float4 index
  const int64_t total = (int64_t)M * n / 4;
  if (q >= total) return;
  const int n4 = n / 4;
  const int64_t m = q / n4;
  const int r = (int)(q - m * n4) * 4;
  const int64_t plane = (int64_t)M * n / 4;
  typedef float f4v __attribute__((ext_vector_type(4)));
  const f4v* p4 = reinterpret_cast<const f4v*>(partial) + q;
  f4v acc = {0.f, 0.f, 0.f, 0.f};
  int sidx = 0;
  for (; sidx + 4 <= S; sidx += 4) {
    const f4v a0 = __builtin_nontemporal_load(p4 + (sidx + 0) * plane);
    const f4v a1 = __builtin_nontemporal_load(p4 + (sidx + 1) * plane);
    const f4v a2 = __builtin_nontemporal_load(p4 + (sidx + 2) * plane);
    const f4v a3 = __builtin_nontemporal_load(p4 + (sidx + 3) * plane);
    acc += a0;
    acc += a1;
    acc += a2;
    acc += a3;
  }
  for (; sidx < S; sidx++) {
    const f4v a0 = __builtin_nontemporal_load(p4 + sidx * plane);
    acc += a0;
  }
  const float v[4] = {acc[0], acc[1], acc[2], acc[3]};
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (!mask_keep(mask, r + j, m, M)) continue;
    const int64_t ci = TRANS_OUT ? (int64_t)(r + j) * ldc + m : m * ldc + r + j;
    float o = alpha * v[j];
    if constexpr (C_BF16) {
      uint16_t* c = (uint16_t*)C + ci;
      if (beta != 0.f) o += beta * bf2f(*c);
      *c = f2bf(o);
    } else {
      float* c = (float*)C + ci;
      if (beta != 0.f) o += beta * *c;
      *c = o;
    }
  }
}

// The queued reductions of a SkinnyBatch in one launch: thread q takes float4 q of the
// concatenated outputs; the same fixed-order sum as skinny_reduce_kernel.
struct BatchArgs {
  int n;
  SkinnyJob job[SkinnyBatch::kMaxJobs];
  int64_t first4[SkinnyBatch::kMaxJobs + 1];  // prefix sums of M * n / 4
};
__global__ __launch_bounds__(256) void skinny_reduce_batch_kernel(BatchArgs b) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= b.first4[b.n]) return;
  int k = 0;
  while (g >= b.first4[k + 1]) k++;
  const SkinnyJob& j = b.job[k];
  const int64_t q = g - b.first4[k];
  const int n4 = j.n / 4;
  const int64_t m = q / n4;
  const int r = (int)(q - m * n4) * 4;
  const int64_t plane = (int64_t)j.M * j.n / 4;
  typedef float f4v __attribute__((ext_vector_type(4)));
  const f4v* p4 = reinterpret_cast<const f4v*>(j.partial) + q;
  f4v acc = {0.f, 0.f, 0.f, 0.f};
  int sidx = 0;
  for (; sidx + 4 <= j.S; sidx += 4) {  // four loads in flight, added in split order
    const f4v a0 = __builtin_nontemporal_load(p4 + (sidx + 0) * plane);
    const f4v a1 = __builtin_nontemporal_load(p4 + (sidx + 1) * plane);
    const f4v a2 = __builtin_nontemporal_load(p4 + (sidx + 2) * plane);
    const f4v a3 = __builtin_nontemporal_load(p4 + (sidx + 3) * plane);
    acc += a0;
    acc += a1;
    acc += a2;
    acc += a3;
  }
  for (; sidx < j.S; sidx++) acc += __builtin_nontemporal_load(p4 + sidx * plane);
  const float v[4] = {acc[0], acc[1], acc[2], acc[3]};
#pragma unroll
  for (int e = 0; e < 4; e++) {
    if (!mask_keep(j.mask, r + e, m, j.M)) continue;
    const int64_t ci = j.trans ? (int64_t)(r + e) * j.ldc + m : m * j.ldc + r + e;
    float o = j.alpha * v[e];
    if (j.c_bf16) {
      uint16_t* c = (uint16_t*)j.C + ci;
      if (j.beta != 0.f) o += j.beta * bf2f(*c);
      *c = f2bf(o);
    } else {
      float* c = (float*)j.C + ci;
      if (j.beta != 0.f) o += j.beta * *c;
      *c = o;
    }
  }
}

// ---------------------------------------------------------------- row-block form, no split
// For k-contiguous Big and K % 128 == 0: a workgroup owns 16 rows of C and its NW waves (8, or 4
// when K % 256 != 0) take an equal share of K each, loading v_mfma_f32_16x16x32_bf16 fragments straight from memory into
// registers (Big once from HBM, two 4-slice batches in flight per wave; Small from L2).  The
// NW 16 x n partial blocks are added in wave order through LDS and written by wave 0: one
// launch, no partial planes, a fixed summation order.  Small is read k-contiguous from memory
// (SMALLK) or, when it is [K][n] row-major, staged whole into LDS (K n 2 <= RS_SMALL bytes) and
// read with ds_read_b64_tr_b16, which hands each lane four k-rows of its column.
constexpr int RS_SMALL = 96 * 1024;

template <int NB, bool SMALLK>
__device__ __forceinline__ bf16x8 rows_small_frag(const Args& a, const uint8_t* sm, int j, int k0, int lane) {
  const int c = 16 * j + (lane & 15), g = lane >> 4;
  if constexpr (SMALLK) {
    return *reinterpret_cast<const bf16x8*>((const uint16_t*)a.small + (int64_t)c * a.lds + k0 + 8 * g);
  } else {
    // tr read over 16 lanes: source lane s reads 4 columns 16 j + 4 (s % 4) of k-row s / 4;
    // destination lane s gets column 16 j + s of the 4 rows
    const int s = lane & 15;
    const uint8_t* p = sm + ((int64_t)(k0 + 8 * g + (s >> 2)) * a.n + 16 * j + 4 * (s & 3)) * 2;
    short4v lo, hi;
#if defined(__HIP_DEVICE_COMPILE__)
    lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)p);
    hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p + 4 * a.n * 2));
#else
    lo = hi = short4v{};
#endif
    const uint2 x = __builtin_bit_cast(uint2, lo), y = __builtin_bit_cast(uint2, hi);
    return __builtin_bit_cast(bf16x8, make_uint4(x.x, x.y, y.x, y.y));
  }
}

template <int NB, bool SMALLK, bool TRANS_OUT, bool C_BF16, int NW>
__global__ __launch_bounds__(64 * NW) void skinny_rows_kernel(Args a) {
  constexpr int P = 4;  // 32-k slices per batch
  constexpr int RED = NW * NB * 64 * 16;
  __shared__ __attribute__((aligned(16))) uint8_t smem[(SMALLK ? 0 : RS_SMALL) + RED];
  uint8_t* red = smem + (SMALLK ? 0 : RS_SMALL);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int m0 = blockIdx.x * 16;
  if constexpr (!SMALLK) {  // stage Small [K][n] (contiguous, K n 2 bytes)
    const int nv = a.K * a.n / 8;
    for (int i = threadIdx.x; i < nv; i += 64 * NW)
      reinterpret_cast<uint4*>(smem)[i] = reinterpret_cast<const uint4*>(a.small)[i];
    __syncthreads();
  }
  const int row = min(m0 + (lane & 15), a.M - 1);
  const uint16_t* brow = (const uint16_t*)a.big + (int64_t)row * a.ldb + 8 * (lane >> 4);
  const int kq = a.K / NW, kb = w * kq, nsl = kq / 32;
  floatx4 acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  bf16x8 b0[P], b1[P], s0[P][SMALLK ? NB : 1], s1[P][SMALLK ? NB : 1];
  auto load = [&](bf16x8(&bb)[P], bf16x8(&ss)[P][SMALLK ? NB : 1], int sl0) {
#pragma unroll
    for (int t = 0; t < P; t++) {
      const int sl = min(sl0 + t, nsl - 1);
      bb[t] = *reinterpret_cast<const bf16x8*>(brow + kb + 32 * sl);
      if constexpr (SMALLK) {
#pragma unroll
        for (int j = 0; j < NB; j++) ss[t][j] = rows_small_frag<NB, true>(a, nullptr, j, kb + 32 * sl, lane);
      }
    }
  };
  auto compute = [&](bf16x8(&bb)[P], bf16x8(&ss)[P][SMALLK ? NB : 1], int sl0) {
#pragma unroll
    for (int t = 0; t < P; t++) {
      if (sl0 + t >= nsl) break;
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const bf16x8 f = SMALLK ? ss[t][SMALLK ? j : 0] : rows_small_frag<NB, false>(a, smem, j, kb + 32 * (sl0 + t), lane);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bb[t], f, acc[j], 0, 0, 0);
      }
    }
  };
  load(b0, s0, 0);
  for (int sl = 0; sl < nsl; sl += 2 * P) {
    if (sl + P < nsl) load(b1, s1, sl + P);
    compute(b0, s0, sl);
    if (sl + 2 * P < nsl) load(b0, s0, sl + 2 * P);
    if (sl + P < nsl) compute(b1, s1, sl + P);
  }
  // wave partials -> LDS, summed in wave order by wave 0
#pragma unroll
  for (int j = 0; j < NB; j++) *reinterpret_cast<floatx4*>(red + ((w * NB + j) * 64 + lane) * 16) = acc[j];
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int j = 0; j < NB; j++) {
    floatx4 v = *reinterpret_cast<const floatx4*>(red + (j * 64 + lane) * 16);
#pragma unroll
    for (int q = 1; q < NW; q++) v += *reinterpret_cast<const floatx4*>(red + ((q * NB + j) * 64 + lane) * 16);
    const int col = 16 * j + (lane & 15);
    if (col >= a.n) continue;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int r = m0 + 4 * (lane >> 4) + e;
      if (r >= a.M || !mask_keep(a.mask, col, r, a.M)) continue;
      const int64_t ci = TRANS_OUT ? (int64_t)col * a.ldc + r : (int64_t)r * a.ldc + col;
      float o = a.alpha * v[e];
      if constexpr (C_BF16) {
        uint16_t* c = (uint16_t*)a.C + ci;
        if (a.beta != 0.f) o += a.beta * bf2f(*c);
        *c = f2bf(o);
      } else {
        float* c = (float*)a.C + ci;
        if (a.beta != 0.f) o += a.beta * *c;
        *c = o;
      }
    }
  }
}

// RMSNorm forward fused with the LoRA down-projection of its output (the producer of x computes
// u = x A while the rows are in registers): xn = h * rinv * w (bf16 out), rinv = 1/sqrt(mean h^2 +
// eps), u[t, :] = xn[t, :] A, bf16 out, with A given transposed (At [n][D] bf16, n = 16 NB).
// Workgroup = 16 rows and 8 waves; wave w takes K columns [w D/8, (w+1) D/8) in 32-wide slices,
// each lane 8 consecutive columns of one row per slice -- the layout of the MFMA A fragment, so
// the normalised bf16 values feed v_mfma_f32_16x16x32_bf16 directly.  The B fragment of a lane
// (column 16 j + lane % 16, 8 consecutive k) is one 16-byte load of an At row, issued before the
// row statistics so it is in flight behind them; At (n D 2 bytes) stays in L2 across workgroups.
// The row's sum of squares is summed over the four lanes of a row (xor 16, 32), then over the
// waves in order.
template <int NB, int NS>  // NS = 32-wide slices per wave (D / 256)
__global__ __launch_bounds__(512) void rmsnorm_lora_u_kernel(const float* __restrict__ h, const float* __restrict__ wn,
                                                            float eps, uint16_t* __restrict__ xn, float* __restrict__ rinv,
                                                            const uint16_t* __restrict__ At, uint16_t* __restrict__ u,
                                                            int M, int D, int n) {
  constexpr int NW = 8;
  __shared__ __attribute__((aligned(16))) uint8_t red[NW * NB * 64 * 16];
  __shared__ float ssq[NW][16];
  __shared__ float sri[16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, rl = lane & 15;
  const int m0 = blockIdx.x * 16, row = min(m0 + rl, M - 1);
  const int kb = w * (D / NW);
  const float* hr = h + (int64_t)row * D + kb + 8 * g;
  float v[NS][8];
#pragma unroll
  for (int t = 0; t < NS; t++) {
    const float4 x0 = *reinterpret_cast<const float4*>(hr + 32 * t);
    const float4 x1 = *reinterpret_cast<const float4*>(hr + 32 * t + 4);
    v[t][0] = x0.x; v[t][1] = x0.y; v[t][2] = x0.z; v[t][3] = x0.w;
    v[t][4] = x1.x; v[t][5] = x1.y; v[t][6] = x1.z; v[t][7] = x1.w;
  }
  bf16x8 fb[NS][NB];
#pragma unroll
  for (int t = 0; t < NS; t++)
#pragma unroll
    for (int j = 0; j < NB; j++)
      fb[t][j] = *reinterpret_cast<const bf16x8*>(At + (int64_t)(16 * j + rl) * D + kb + 32 * t + 8 * g);
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < NS; t++)
#pragma unroll
    for (int i = 0; i < 8; i++) ss += v[t][i] * v[t][i];
  ss += __shfl_xor(ss, 16, 64);
  ss += __shfl_xor(ss, 32, 64);
  if (g == 0) ssq[w][rl] = ss;
  __syncthreads();
  if (threadIdx.x < 16) {
    float tot = 0.f;
    for (int q = 0; q < NW; q++) tot += ssq[q][threadIdx.x];
    const float ri = 1.f / sqrtf(tot / (float)D + eps);
    sri[threadIdx.x] = ri;
    if (m0 + (int)threadIdx.x < M) rinv[m0 + threadIdx.x] = ri;
  }
  __syncthreads();
  const float ri = sri[rl];
  floatx4 acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < NS; t++) {
    const int k0 = kb + 32 * t;
    const float4 w0 = *reinterpret_cast<const float4*>(wn + k0 + 8 * g);
    const float4 w1 = *reinterpret_cast<const float4*>(wn + k0 + 8 * g + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    uint32_t pk[4];
#pragma unroll
    for (int i = 0; i < 4; i++) pk[i] = pack_bf2(v[t][2 * i] * ri * wv[2 * i], v[t][2 * i + 1] * ri * wv[2 * i + 1]);
    const uint4 u4 = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    if (m0 + rl < M) *reinterpret_cast<uint4*>(xn + (int64_t)(m0 + rl) * D + k0 + 8 * g) = u4;
    const bf16x8 fa = __builtin_bit_cast(bf16x8, u4);
#pragma unroll
    for (int j = 0; j < NB; j++) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa, fb[t][j], acc[j], 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < NB; j++) *reinterpret_cast<floatx4*>(red + ((w * NB + j) * 64 + lane) * 16) = acc[j];
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int j = 0; j < NB; j++) {
    floatx4 o = *reinterpret_cast<const floatx4*>(red + (j * 64 + lane) * 16);
#pragma unroll
    for (int q = 1; q < NW; q++) o += *reinterpret_cast<const floatx4*>(red + ((q * NB + j) * 64 + lane) * 16);
    const int col = 16 * j + (lane & 15);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int r = m0 + 4 * (lane >> 4) + e;
      if (r < M) u[(int64_t)r * n + col] = f2bf(o[e]);
    }
  }
}

// SwiGLU forward fused with the LoRA down-projection of its output: act = silu(g) * u (bf16,
// the arithmetic of swiglu_fused_forward, so act is bit-identical) and uo[t, :] = act[t, :] A
// with A given transposed (At [n][F] bf16, n = 16 NB).  Same layout as rmsnorm_lora_u_kernel:
// 16 rows per workgroup, 8 waves taking equal shares of F in 32-wide slices, each lane 8
// consecutive columns of one row per slice (the MFMA A fragment), wave partials added in wave
// order through LDS.
template <int NB, int NS>  // NS = 32-wide slices per wave (F / 256), all loads issued up front
__global__ __launch_bounds__(512) void swiglu_lora_u_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ act,
                                                           const uint16_t* __restrict__ At, uint16_t* __restrict__ uo,
                                                           int M, int F, int n) {
  constexpr int NW = 8;
  __shared__ __attribute__((aligned(16))) uint8_t red[NW * NB * 64 * 16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, rl = lane & 15;
  const int m0 = blockIdx.x * 16, row = min(m0 + rl, M - 1);
  const int kb = w * (F / NW);
  const uint16_t* gr = gu + (int64_t)row * 2 * F;
  floatx4 acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  uint4 gv[NS], uv[NS];
#pragma unroll
  for (int t = 0; t < NS; t++) {
    gv[t] = *reinterpret_cast<const uint4*>(gr + kb + 32 * t + 8 * g);
    uv[t] = *reinterpret_cast<const uint4*>(gr + F + kb + 32 * t + 8 * g);
  }
#pragma unroll
  for (int t = 0; t < NS; t++) {
    const int k0 = kb + 32 * t;
    bf16x8 fb[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) fb[j] = *reinterpret_cast<const bf16x8*>(At + (int64_t)(16 * j + rl) * F + k0 + 8 * g);
    const uint32_t gw[4] = {gv[t].x, gv[t].y, gv[t].z, gv[t].w}, uw[4] = {uv[t].x, uv[t].y, uv[t].z, uv[t].w};
    uint32_t pk[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float g0 = __uint_as_float(gw[i] << 16), g1 = __uint_as_float(gw[i] & 0xFFFF0000u);
      const float u0 = __uint_as_float(uw[i] << 16), u1 = __uint_as_float(uw[i] & 0xFFFF0000u);
      pk[i] = pack_bf2((g0 / (1.f + expf(-g0))) * u0, (g1 / (1.f + expf(-g1))) * u1);
    }
    const uint4 a4 = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    if (m0 + rl < M) *reinterpret_cast<uint4*>(act + (int64_t)(m0 + rl) * F + k0 + 8 * g) = a4;
    const bf16x8 fa = __builtin_bit_cast(bf16x8, a4);
#pragma unroll
    for (int j = 0; j < NB; j++) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa, fb[j], acc[j], 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < NB; j++) *reinterpret_cast<floatx4*>(red + ((w * NB + j) * 64 + lane) * 16) = acc[j];
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int j = 0; j < NB; j++) {
    floatx4 o = *reinterpret_cast<const floatx4*>(red + (j * 64 + lane) * 16);
#pragma unroll
    for (int q = 1; q < NW; q++) o += *reinterpret_cast<const floatx4*>(red + ((q * NB + j) * 64 + lane) * 16);
    const int col = 16 * j + (lane & 15);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int r = m0 + 4 * (lane >> 4) + e;
      if (r < M) uo[(int64_t)r * n + col] = f2bf(o[e]);
    }
  }
}

template <bool SMALLK, bool TRANS_OUT, bool C_BF16, int NW>
static void launch_rows_nw(int nb, const Args& a, hipStream_t s) {
  const dim3 grid(ceil_div(a.M, 16)), block(64 * NW);
  switch (nb) {
    case 1: hipLaunchKernelGGL((skinny_rows_kernel<1, SMALLK, TRANS_OUT, C_BF16, NW>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((skinny_rows_kernel<2, SMALLK, TRANS_OUT, C_BF16, NW>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((skinny_rows_kernel<3, SMALLK, TRANS_OUT, C_BF16, NW>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((skinny_rows_kernel<4, SMALLK, TRANS_OUT, C_BF16, NW>), grid, block, 0, s, a); break;
  }
}
// eight waves (two per SIMD, twice the loads in flight) when K splits into eighths of whole
// 32-k slices, else four
template <bool SMALLK, bool TRANS_OUT, bool C_BF16>
static void launch_rows(int nb, const Args& a, hipStream_t s) {
  if (a.K % 256 == 0) launch_rows_nw<SMALLK, TRANS_OUT, C_BF16, 8>(nb, a, s);
  else launch_rows_nw<SMALLK, TRANS_OUT, C_BF16, 4>(nb, a, s);
}

template <bool BIGK, bool SMALLK, int NB>
static void launch(const Args& a, dim3 grid, bool trans, bool cbf, hipStream_t s) {
  if (trans) {
    if (cbf) hipLaunchKernelGGL((skinny_kernel<BIGK, SMALLK, NB, true, true>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((skinny_kernel<BIGK, SMALLK, NB, true, false>), grid, dim3(256), 0, s, a);
  } else {
    if (cbf) hipLaunchKernelGGL((skinny_kernel<BIGK, SMALLK, NB, false, true>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((skinny_kernel<BIGK, SMALLK, NB, false, false>), grid, dim3(256), 0, s, a);
  }
}
template <bool BIGK, bool SMALLK>
static void launch_nb(int nb, const Args& a, dim3 grid, bool trans, bool cbf, hipStream_t s) {
  switch (nb) {
    case 1: launch<BIGK, SMALLK, 1>(a, grid, trans, cbf, s); break;
    case 2: launch<BIGK, SMALLK, 2>(a, grid, trans, cbf, s); break;
    case 3: launch<BIGK, SMALLK, 3>(a, grid, trans, cbf, s); break;
    default: launch<BIGK, SMALLK, 4>(a, grid, trans, cbf, s); break;
  }
}

}  // namespace sk

// Returns 1 if the skinny path ran, 0 if the operands do not fit it (caller falls back to
// the general GEMM), < 0 on error.  big_k / small_k: operand k-contiguous.  trans_out: the
// result (m, r) is stored at C[r * ldc + m].
int skinny_flush(SkinnyBatch* b, hipStream_t s) {
  using namespace sk;
  if (!b || b->n == 0) return SMHIP_OK;
  BatchArgs a{};
  a.n = b->n;
  a.first4[0] = 0;
  for (int k = 0; k < b->n; k++) {
    a.job[k] = b->job[k];
    a.first4[k + 1] = a.first4[k] + (int64_t)b->job[k].M * b->job[k].n / 4;
  }
  b->n = 0;
  b->used = 0;
  hipLaunchKernelGGL(skinny_reduce_batch_kernel, dim3(ceil_div(a.first4[a.n], 256)), dim3(256), 0, s, a);
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

int skinny_release(SkinnyHold* h, hipStream_t s) {
  using namespace sk;
  if (!h || !h->valid) return SMHIP_OK;
  h->valid = false;
  Args a;
  memcpy(&a, h->args, sizeof(Args));
  const int ev0 = prof_mark(s);
  const dim3 grid(h->mt, h->S);
  if (h->big_k && h->small_k) launch_nb<true, true>(h->n / 16, a, grid, h->trans, h->c_bf16, s);
  else if (h->big_k) launch_nb<true, false>(h->n / 16, a, grid, h->trans, h->c_bf16, s);
  else if (h->small_k) launch_nb<false, true>(h->n / 16, a, grid, h->trans, h->c_bf16, s);
  else launch_nb<false, false>(h->n / 16, a, grid, h->trans, h->c_bf16, s);
  SMHIP_CHECK_LAUNCH();
  prof_add(PROF_GEMM, ev0, prof_mark(s), 2.0 * h->M * h->n * (double)h->K, h->M, h->n, h->K);
  return SMHIP_OK;
}

// Returns 1 when the fused kernel ran, 0 when the shapes do not fit it (the caller runs the
// RMSNorm and the rank product separately).  At is A transposed, [n][D].
int rmsnorm_lora_u(const float* h, const float* w, float eps, uint16_t* xn, float* rinv, const uint16_t* At, int n,
                   uint16_t* u, int T, int D, hipStream_t s) {
  using namespace sk;
  if (T <= 0) return 1;
  if (D % 256 || D > 1024 || n % 16 || n < 16 || n > 64) return 0;
  if (((uintptr_t)h | (uintptr_t)w | (uintptr_t)xn | (uintptr_t)At) % 16) return 0;
  const dim3 grid(ceil_div(T, 16)), block(512);
#define SMHIP_RLU(NB)                                                                                       \
  switch (D / 256) {                                                                                        \
    case 1: hipLaunchKernelGGL((rmsnorm_lora_u_kernel<NB, 1>), grid, block, 0, s, h, w, eps, xn, rinv, At, u, T, D, n); break; \
    case 2: hipLaunchKernelGGL((rmsnorm_lora_u_kernel<NB, 2>), grid, block, 0, s, h, w, eps, xn, rinv, At, u, T, D, n); break; \
    case 3: hipLaunchKernelGGL((rmsnorm_lora_u_kernel<NB, 3>), grid, block, 0, s, h, w, eps, xn, rinv, At, u, T, D, n); break; \
    default: hipLaunchKernelGGL((rmsnorm_lora_u_kernel<NB, 4>), grid, block, 0, s, h, w, eps, xn, rinv, At, u, T, D, n); break; \
  }
  switch (n / 16) {
    case 1: SMHIP_RLU(1) break;
    case 2: SMHIP_RLU(2) break;
    case 3: SMHIP_RLU(3) break;
    default: SMHIP_RLU(4) break;
  }
#undef SMHIP_RLU
  SMHIP_CHECK_LAUNCH();
  return 1;
}

// Returns 1 when the fused kernel ran, 0 when the shapes do not fit it (the caller runs the
// SwiGLU and the rank product separately).  gu [T][2F] = [gate | up] bf16, At [n][F].
int swiglu_lora_u(const uint16_t* gu, uint16_t* act, const uint16_t* At, int n, uint16_t* u, int T, int F,
                  hipStream_t s) {
  using namespace sk;
  if (T <= 0) return 1;
  if (F % 256 || n % 16 || n < 16 || n > 64) return 0;
  if (((uintptr_t)gu | (uintptr_t)act | (uintptr_t)At) % 16) return 0;
  const dim3 grid(ceil_div(T, 16)), block(512);
#define SMHIP_SLU(NB)                                                                                            \
  switch (F / 256) {                                                                                             \
    case 4: hipLaunchKernelGGL((swiglu_lora_u_kernel<NB, 4>), grid, block, 0, s, gu, act, At, u, T, F, n); break;   \
    case 8: hipLaunchKernelGGL((swiglu_lora_u_kernel<NB, 8>), grid, block, 0, s, gu, act, At, u, T, F, n); break;   \
    case 12: hipLaunchKernelGGL((swiglu_lora_u_kernel<NB, 12>), grid, block, 0, s, gu, act, At, u, T, F, n); break; \
    case 16: hipLaunchKernelGGL((swiglu_lora_u_kernel<NB, 16>), grid, block, 0, s, gu, act, At, u, T, F, n); break; \
    default: return 0;                                                                                           \
  }
  switch (n / 16) {
    case 1: SMHIP_SLU(1) break;
    case 2: SMHIP_SLU(2) break;
    case 3: SMHIP_SLU(3) break;
    default: SMHIP_SLU(4) break;
  }
#undef SMHIP_SLU
  SMHIP_CHECK_LAUNCH();
  return 1;
}

int gemm_skinny(int M, int n, int K, const void* big, int64_t ldb, bool big_k, const void* small, int64_t lds,
                bool small_k, float alpha, float beta, void* C, int64_t ldc, bool trans_out, bool c_bf16,
                SkinnyBatch* defer, hipStream_t s, SkinnyMask mask, SkinnyHold* hold) {
  using namespace sk;
  static_assert(sizeof(Args) <= sizeof(SkinnyHold::args), "SkinnyHold::args holds an sk::Args");
  if (n < 1 || n > 64 || n % 16 || M < 1 || K < BKT || K % BKT) return 0;
  if (((uintptr_t)big | (uintptr_t)small) % 16 || ldb % 8) return 0;
  if (small_k && lds % 8) return 0;
  if (!small_k && lds != n) return 0;
  // 32-bit buffer offsets
  const int64_t bb = big_k ? ((int64_t)(M - 1) * ldb + K) * 2 : ((int64_t)(K - 1) * ldb + M) * 2;
  const int64_t sb = small_k ? ((int64_t)(n - 1) * lds + K) * 2 : (int64_t)K * n * 2;
  const int64_t lim = (int64_t)1 << 31;
  if (bb + 2 * 64 * ldb * 2 >= lim || sb + 4096 >= lim) return 0;
  Args a{};
  a.big = big; a.ldb = ldb; a.big_bytes = (int)bb;
  a.small = small; a.lds = lds; a.small_bytes = (int)sb;
  a.M = M; a.n = n; a.K = K;
  a.C = C; a.ldc = ldc; a.alpha = alpha; a.beta = beta;
  a.mask = mask;
  // k-contiguous Big, K a multiple of 128 and K n <= 64Ki (Small at most 128 KiB): the row-block
  // kernel, no split and no reduction pass.  Its workgroups re-read Small once per 16 rows, which
  // for larger Small costs more than the split-K kernel's reduction pass (measured: 4096 x 48 x
  // 1024 9.7 -> 6.8 us, 4096 x 16 x 3072 8.7 -> 7.5 us, but 4096 x 48 x 4096 14.5 -> 17.7 us).
  if (big_k && K % 128 == 0 && (int64_t)K * n <= 65536 && (small_k || (int64_t)K * n * 2 <= RS_SMALL)) {
    a.partial = nullptr;
    const int ev0 = prof_mark(s);
#define SMHIP_ROWS(SK)                                                           \
  if (trans_out) { if (c_bf16) launch_rows<SK, true, true>(n / 16, a, s); else launch_rows<SK, true, false>(n / 16, a, s); } \
  else { if (c_bf16) launch_rows<SK, false, true>(n / 16, a, s); else launch_rows<SK, false, false>(n / 16, a, s); }
    if (small_k) { SMHIP_ROWS(true) } else { SMHIP_ROWS(false) }
#undef SMHIP_ROWS
    SMHIP_CHECK_LAUNCH();
    prof_add(PROF_GEMM, ev0, prof_mark(s), 2.0 * M * n * (double)K, M, n, K);
    return 1;
  }
  const int mt = ceil_div(M, MT), nk = K / BKT;
  // splits: one workgroup per CU (the engine step measured 0.3%, 0.7% and 0.9% faster than with
  // 2, 4 and 8; SMHIP_SKINNY_WPC overrides for tuning runs); fewer while the fp32 partials
  // (written and read back) exceed a quarter of the bytes of Big, as long as every CU keeps a
  // workgroup
  const int cus = num_cus();
  static const int wpc = [] { const char* v = getenv("SMHIP_SKINNY_WPC"); return v ? atoi(v) : 1; }();
  int S = std::max(1, ceil_div(wpc * cus, mt));
  S = std::min(S, std::max(1, nk / 2));
  while (S > 1 && (int64_t)S * M * n * 4 * 4 > (int64_t)M * K * 2 && mt * (S - 1) >= cus) S--;
  a.kps = ceil_div(nk, S);
  S = ceil_div(nk, a.kps);
  a.partial = nullptr;
  const size_t pbytes = (sizeof(float) * (size_t)S * M * n + 255) & ~(size_t)255;
  const bool deferred = S > 1 && defer && pbytes <= defer->cap;
  if (deferred) {
    if (defer->n == SkinnyBatch::kMaxJobs || defer->used + pbytes > defer->cap) {
      if (int rc = skinny_release(hold, s)) return rc;  // its partials are in the batch being reduced
      if (int rc = skinny_flush(defer, s)) return rc;
    }
    a.partial = (float*)((char*)defer->arena + defer->used);
    defer->job[defer->n++] = SkinnyJob{a.partial, C, ldc, S, M, n, alpha, beta, trans_out ? 1 : 0, c_bf16 ? 1 : 0, mask};
    defer->used += pbytes;
  } else if (S > 1) {
    a.partial = (float*)workspace(s, sizeof(float) * (size_t)S * M * n, 7);
    if (!a.partial) return fail(SMHIP_ENOMEM, "gemm_skinny: split workspace");
  }
  const dim3 grid(mt, S);
  // a held launch: products whose partials need no reduction launch of their own can share one
  if (hold && !(S > 1 && !deferred)) {
    if (hold->valid && hold->big_k == big_k && hold->small_k == small_k && hold->n == n &&
        hold->c_bf16 == c_bf16 && !big_k && !small_k) {
      Args a0;
      memcpy(&a0, hold->args, sizeof(Args));
      const int nb0 = hold->mt * hold->S;
      const dim3 g2(nb0 + mt * S);
      const int ev0 = prof_mark(s);
#define SMHIP_PAIR(NBV, T0, T1)                                                                                \
  if (c_bf16) hipLaunchKernelGGL((skinny_pair_kernel<false, false, NBV, T0, T1, true>), g2, dim3(256), 0, s, a0, a, hold->mt, nb0, mt); \
  else hipLaunchKernelGGL((skinny_pair_kernel<false, false, NBV, T0, T1, false>), g2, dim3(256), 0, s, a0, a, hold->mt, nb0, mt);
#define SMHIP_PAIR_T(NBV)                                                                                      \
  if (hold->trans) { if (trans_out) { SMHIP_PAIR(NBV, true, true) } else { SMHIP_PAIR(NBV, true, false) } }      \
  else { if (trans_out) { SMHIP_PAIR(NBV, false, true) } else { SMHIP_PAIR(NBV, false, false) } }
      switch (n / 16) {
        case 1: SMHIP_PAIR_T(1) break;
        case 2: SMHIP_PAIR_T(2) break;
        case 3: SMHIP_PAIR_T(3) break;
        default: SMHIP_PAIR_T(4) break;
      }
#undef SMHIP_PAIR_T
#undef SMHIP_PAIR
      SMHIP_CHECK_LAUNCH();
      prof_add(PROF_GEMM, ev0, prof_mark(s), 2.0 * ((double)hold->M * hold->n * hold->K + (double)M * n * K), M, n, K);
      hold->valid = false;
      return 1;
    }
    if (hold->valid)
      if (int rc = skinny_release(hold, s)) return rc;
    hold->valid = true;
    hold->big_k = big_k; hold->small_k = small_k; hold->trans = trans_out; hold->c_bf16 = c_bf16;
    hold->mt = mt; hold->S = S; hold->n = n; hold->M = M; hold->K = K;
    memcpy(hold->args, &a, sizeof(Args));
    return 1;
  }
  const int ev0 = prof_mark(s);
  if (big_k && small_k) launch_nb<true, true>(n / 16, a, grid, trans_out, c_bf16, s);
  else if (big_k) launch_nb<true, false>(n / 16, a, grid, trans_out, c_bf16, s);
  else if (small_k) launch_nb<false, true>(n / 16, a, grid, trans_out, c_bf16, s);
  else launch_nb<false, false>(n / 16, a, grid, trans_out, c_bf16, s);
  SMHIP_CHECK_LAUNCH();
  prof_add(PROF_GEMM, ev0, prof_mark(s), 2.0 * M * n * (double)K, M, n, K);
  if (S > 1 && !deferred) {
    const int blocks = ceil_div((int64_t)M * n / 4, 256);
    if (trans_out) {
      if (c_bf16) hipLaunchKernelGGL((skinny_reduce_kernel<true, true>), dim3(blocks), dim3(256), 0, s, a.partial, S, M, n, C, ldc, alpha, beta, mask);
      else hipLaunchKernelGGL((skinny_reduce_kernel<true, false>), dim3(blocks), dim3(256), 0, s, a.partial, S, M, n, C, ldc, alpha, beta, mask);
    } else {
      if (c_bf16) hipLaunchKernelGGL((skinny_reduce_kernel<false, true>), dim3(blocks), dim3(256), 0, s, a.partial, S, M, n, C, ldc, alpha, beta, mask);
      else hipLaunchKernelGGL((skinny_reduce_kernel<false, false>), dim3(blocks), dim3(256), 0, s, a.partial, S, M, n, C, ldc, alpha, beta, mask);
    }
    SMHIP_CHECK_LAUNCH();
  }
  return 1;
}

}  // namespace smhip
