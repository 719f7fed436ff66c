// common.hpp — shared device/host helpers for libsharpmind_hip (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>
#include <mutex>
#include <unordered_map>

#include "../../include/sharpmind_hip.h"

namespace smhip {

// ---------------------------------------------------------------- errors
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

#define SMHIP_CHECK_HIP(expr)                                                        \
  do {                                                                               \
    hipError_t _e = (expr);                                                          \
    if (_e != hipSuccess)                                                            \
      return ::smhip::fail(SMHIP_EHIP, std::string(#expr) + ": " + hipGetErrorString(_e)); \
  } while (0)

#define SMHIP_REQUIRE(cond, msg) \
  do { if (!(cond)) return ::smhip::fail(SMHIP_EINVAL, msg); } while (0)

// Launch-error check: reports the launch error (not a later fault).
#define SMHIP_CHECK_LAUNCH() SMHIP_CHECK_HIP(hipGetLastError())

// ---------------------------------------------------------------- workspace
// Per-stream growable device scratch.  Calls on one stream are ordered, so a
// buffer keyed by stream is never used by two kernels at once; calls from
// different threads must use different streams (documented in the header).
void* workspace(hipStream_t s, size_t bytes, int slot = 0);
// Frees every buffer keyed by stream s (the stream's work must be complete).
void workspace_release(hipStream_t s);

// ---------------------------------------------------------------- bf16
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// float -> bf16 bits, round to nearest even (NaN kept quiet).
// The device pass uses the hardware conversion (v_cvt_pk_bf16_f32, IEEE round to nearest
// even); the host pass rounds the same way in software.
__device__ __host__ inline uint16_t f2bf(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, (__bf16)f);
#endif
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __host__ inline float bf2f(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}
__device__ inline uint32_t pack_bf2(float lo, float hi) {
  bf16x2 v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// Bit-exact IEEE half -> float (every binary16 value is exact in binary32),
// same result as HalfToFloat_Scalar (QuantizationKernels.cs:117-146).
__device__ __host__ inline float half_bits_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      int k = 31 - __builtin_clz(m);  // msb position, 0..9
      bits = sign | ((uint32_t)(k + 103) << 23) | ((m - (1u << k)) << (23 - k));
    }
  } else if (e == 31) {
    bits = m ? 0x7FC00000u : (sign | 0x7F800000u);
  } else {
    bits = sign | ((e + 112) << 23) | (m << 13);
  }
  return __builtin_bit_cast(float, bits);
}

// ---------------------------------------------------------------- reductions (wave64)
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ inline double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }
inline int num_cus() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    hipGetDevice(&dev);
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) == hipSuccess) n = p.multiProcessorCount;
    if (n <= 0) n = 256;
  }
  return n;
}

// ---------------------------------------------------------------- GEMM operand descriptor
// Element (r, k) of an operand tile, r = row of A (m) or column of B (n).
enum SrcMode : int {
  SRC_F32_K = 0,   // float, p[r*ld + k]
  SRC_F32_R = 1,   // float, p[k*ld + r]
  SRC_BF16_K = 2,  // bf16,  p[r*ld + k]
  SRC_BF16_R = 3,  // bf16,  p[k*ld + r]
  SRC_Q8_K = 4,    // repacked Q8_0 planes, flat element e = r*ld + k
  SRC_Q8_R = 5,    // repacked Q8_0 planes, flat element e = k*ld + r
  SRC_Q4K_K = 6,   // repacked Q4_K planes, e = r*ld + k
  SRC_Q4K_R = 7,   // repacked Q4_K planes, e = k*ld + r
  // "column planes": the same quantised values stored transposed so that the k index
  // of a dX = dY W product is contiguous (bf16 GEMM only).
  SRC_Q8T = 8,     // int8 p[r*ld + k], fp32 scale s[(r/32)*ld + k]
  SRC_Q4KT = 9,    // 4-bit codes p[(r*ld + k)/2] (even k in the low nibble),
                   // (sc*d, mn*dmin) float pairs s[2*((r/32)*ld + k) + {0,1}]
  // "fragment planes" of a frozen Q8_0 base (bf16 GEMM B operand only, K = ld a multiple of 64,
  // rows a multiple of 32): int8 codes in 2048-byte blocks of 32 rows x 64 k (row-major inside),
  // block (rb, kt) at p[(rb*(ld/64) + kt)*2048], so one K tile of 32 rows is one contiguous copy;
  // fp16 block scales (the Q8_0 d, bit for bit) at half index rb*ld + k for SRC_Q8FT, whose rows
  // are the In index of W[Out][In] (dX = dY W: the block runs along the rows, one scale per
  // (k, 32 rows)), and at rb*ld + (k/64)*64 + ((k/32)%2)*32 + r%32 for SRC_Q8F (y = x W^T: the
  // block runs along k, one scale per (row, 32 k)).
  SRC_Q8F = 10,
  SRC_Q8FT = 11,
  // Q4_K fragment planes: the same 32 x 64 blocks with 4-bit codes (1024 bytes, 32 per row;
  // byte i of a row's dword j holds k = 8j + i in its low nibble and k = 8j + i + 4 in its high
  // nibble) and (sc*d, mn*dmin) fp32 pairs at pair index rb*ld + k (SRC_Q4FT, blocks along the
  // rows) or rb*ld + (k/64)*64 + ((k/32)%2)*32 + r%32 (SRC_Q4F, blocks along k).
  SRC_Q4F = 12,
  SRC_Q4FT = 13,
};

struct Operand {
  int mode;
  const void* p;       // dense data, or quant value plane (int8 for Q8, packed nibbles for Q4_K)
  const float* s;      // Q8: fp32 scale per 32-element block; Q4K: (s*d, m*dmin) float pairs per 32
  int64_t ld;          // row length in elements of the stored matrix
};

// Repacked quantized weight (device planes).  Q8_0: qs int8 [n], d f32 [n/32].
// Q4_K: qs uint8 [n/2] in Q4_K nibble order, sm float2 [n/32] = (sc*d, mn*dmin).
struct QuantPlanes {
  int kind;  // SMHIP_QTYPE_*
  int64_t n;
  void* qs;
  float* sc;
};

// GEMM: C[M,N] = alpha * op(A) op(B)^T + beta * C  (beta 0 or 1), optional second
// (rank-extension) pair A2 [M,K2] bf16/f32 and B2 so that C += alpha2 * A2 B2^T.
struct GemmArgs {
  int M, N, K;
  Operand A, B;
  int K2;              // 0 = no extension
  Operand A2, B2;
  float alpha, alpha2, beta;
  void* C;
  int64_t ldc;
  int c_bf16;          // output stored as bf16
  int precision;       // SMHIP_PREC_FP32 | SMHIP_PREC_BF16
  int split_k;         // >1: deterministic split-K through workspace
  const float* bias;   // optional per-column bias added in the epilogue
  const float* R;      // optional residual: C = alpha*AB + bias + R  (fp32 output only)
  int64_t ldr;
  int prof_cat;        // live-timing category (0: by operand kind)
  struct SkinnyBatch* defer;  // rank-sized products: queue the split reduction here (see skinny_flush)
  // block-diagonal mask of a fused LoRA B gradient, applied by the rank-sized (transposed) path;
  // *masked is set to 1 when it was applied (0: the caller masks afterwards)
  const int* mask_cols;
  int mask_rank, mask_nblk;
  int* masked;
  // rank-sized products: hold the launch so the next product with this hold shares it
  struct SkinnyHold* hold;
  // softmax row statistics of C (fp32 C, fragment-plane B, whole 128x128 tiles, at least four per
  // CU): per row and block of 64 columns the pair (max, sum_c exp(C - max)), [M][N/64][2]
  float* rowstat;
};
int gemm(const GemmArgs& g, hipStream_t s);

// ---------------------------------------------------------------- live kernel timing
// When enabled (smhip_profile_begin) the launchers bracket their main kernel with
// HIP events on the launch stream; smhip_profile_end sums the elapsed times.
// PROF_GEMM_DX: the dX products of the backward through the frozen base weights (B a
// quantised base as column planes, or tagged by the caller), counted apart from PROF_GEMM
enum ProfCat { PROF_GEMM = 0, PROF_FLASH_FWD = 1, PROF_FLASH_BWD = 2, PROF_GEMM_DX = 3, PROF_NCAT = 4 };
int prof_mark(hipStream_t s);                         // -1 when profiling is off
// two unrecorded events (indices *i0, *i1) for a launch that timestamps its own start and end
// (hipExtLaunchKernelGGL); false when profiling is off
bool prof_reserve(int* i0, int* i1, hipEvent_t* e0, hipEvent_t* e1);
bool profiling_active();
void prof_add(int cat, int i0, int i1, double flops, int M = 0, int N = 0, int K = 0);

}  // namespace smhip
