// quant.hip — Q8_0 / Q4_K handling for gfx950.
//
// Reference byte layouts (QuantizationOps.cs:37; QuantizationKernels.Q4.cs:586-624):
//   Q8_0 block  = 34 B : fp16 d @0, 32 x int8 @2; value = q * d.
//   Q4_K block  = 144 B: fp16 d @0, fp16 dmin @2, 12 B packed 6-bit scales/mins @4,
//                        128 B nibbles @16; value = (sc*v)*d - mn*dmin.
// Both formats are flat streams of blocks over the row-major [rows][K] matrix.
//
// The 34-byte Q8_0 block is not 4-byte aligned, which defeats wide loads, so
// weights that stay resident on the GPU are repacked ONCE into planes with
// exactly the same bits: an int8 (or nibble) value plane with 16-byte aligned
// rows, plus an fp32 scale plane.  fp32 scales are exact (every binary16 value
// is representable) and, for Q4_K, sc*d and mn*dmin are exact products
// (6-bit x 11-bit mantissas), so dequantising from the planes yields the same
// fp32 values bit for bit as the reference's ReadQ8_0_Scalar / ReadQ4K_Scalar.
#include "common.hpp"
#include "kernels.hpp"

namespace smhip {

__device__ inline uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

__device__ inline int k4_scale(int j, const uint8_t* s) {
  return j < 4 ? (s[j] & 0x3F) : ((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
}
__device__ inline int k4_min(int j, const uint8_t* s) {
  return j < 4 ? (s[j + 4] & 0x3F) : ((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
}

// ---------------------------------------------------------------- direct dequant (bit-exact)
__global__ void dequant_q8_0_kernel(const uint8_t* __restrict__ raw, float* __restrict__ out, int64_t n) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const uint8_t* blk = raw + (e >> 5) * 34;
    float d = half_bits_to_float(rd_u16(blk));
    out[e] = (float)(int8_t)blk[2 + (e & 31)] * d;
  }
}

__global__ void dequant_q4k_kernel(const uint8_t* __restrict__ raw, float* __restrict__ out, int64_t n) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const uint8_t* blk = raw + (e >> 8) * 144;
    const int i = (int)(e & 255);
    float dS = half_bits_to_float(rd_u16(blk)), mS = half_bits_to_float(rd_u16(blk + 2));
    float s = (float)k4_scale(i >> 5, blk + 4), m = (float)k4_min(i >> 5, blk + 4);
    int v = (blk[16 + (i >> 6) * 32 + (i & 31)] >> (((i & 63) >> 5) * 4)) & 0x0F;
    float t1 = s * (float)v;
    t1 = t1 * dS;
    out[e] = t1 - m * mS;
  }
}

int dequant_raw(int qtype, const void* raw, float* out, int64_t n, hipStream_t s) {
  if (n <= 0) return SMHIP_OK;
  int g = (int)std::min<int64_t>((n + 255) / 256, (int64_t)num_cus() * 16);
  if (qtype == SMHIP_QTYPE_Q8_0)
    hipLaunchKernelGGL(dequant_q8_0_kernel, dim3(g), dim3(256), 0, s, (const uint8_t*)raw, out, n);
  else if (qtype == SMHIP_QTYPE_Q4_K)
    hipLaunchKernelGGL(dequant_q4k_kernel, dim3(g), dim3(256), 0, s, (const uint8_t*)raw, out, n);
  else
    return fail(SMHIP_EUNSUPPORTED, "dequant: qtype must be Q8_0 (8) or Q4_K (12)");
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

// ---------------------------------------------------------------- repack to planes
// Q8_0: one thread per 32-element block; qs plane int8[n], d plane f32[n/32].
__global__ void repack_q8_0_kernel(const uint8_t* __restrict__ raw, int8_t* __restrict__ qs,
                                   float* __restrict__ d, int64_t nblocks) {
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblocks; b += (int64_t)gridDim.x * blockDim.x) {
    const uint8_t* blk = raw + b * 34;
    d[b] = half_bits_to_float(rd_u16(blk));
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; j++)
      w[j] = (uint32_t)blk[2 + 4 * j] | ((uint32_t)blk[3 + 4 * j] << 8) | ((uint32_t)blk[4 + 4 * j] << 16) |
             ((uint32_t)blk[5 + 4 * j] << 24);
    uint4* dst = reinterpret_cast<uint4*>(qs + b * 32);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
  }
}

// Q4_K: one thread per 256-element super-block; qs plane = the 128 nibble bytes,
// sm plane = 8 x (sc*d, mn*dmin) float pairs.
__global__ void repack_q4k_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ qs,
                                  float* __restrict__ sm, int64_t nblocks) {
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblocks; b += (int64_t)gridDim.x * blockDim.x) {
    const uint8_t* blk = raw + b * 144;
    float dS = half_bits_to_float(rd_u16(blk)), mS = half_bits_to_float(rd_u16(blk + 2));
#pragma unroll
    for (int j = 0; j < 8; j++) {
      sm[b * 16 + 2 * j] = (float)k4_scale(j, blk + 4) * dS;
      sm[b * 16 + 2 * j + 1] = (float)k4_min(j, blk + 4) * mS;
    }
    for (int j = 0; j < 128; j += 4) {
      uint32_t w = (uint32_t)blk[16 + j] | ((uint32_t)blk[17 + j] << 8) | ((uint32_t)blk[18 + j] << 16) |
                   ((uint32_t)blk[19 + j] << 24);
      *reinterpret_cast<uint32_t*>(qs + b * 128 + j) = w;
    }
  }
}

size_t planes_bytes(int qtype, int64_t n, size_t* qs_bytes) {
  size_t q = 0, sc = 0;
  if (qtype == SMHIP_QTYPE_Q8_0) { q = (size_t)n; sc = sizeof(float) * (size_t)(n / 32); }
  else if (qtype == SMHIP_QTYPE_Q4_K) { q = (size_t)n / 2; sc = sizeof(float) * 2 * (size_t)(n / 32); }
  q = (q + 255) & ~(size_t)255;
  if (qs_bytes) *qs_bytes = q;
  return q + sc;
}

int repack_planes(int qtype, const void* raw, int64_t n, void* dst, QuantPlanes* out, hipStream_t s) {
  size_t qb = 0;
  planes_bytes(qtype, n, &qb);
  out->kind = qtype;
  out->n = n;
  out->qs = dst;
  out->sc = (float*)((char*)dst + qb);
  if (qtype == SMHIP_QTYPE_Q8_0) {
    SMHIP_REQUIRE(n % 32 == 0, "Q8_0 repack: element count must be a multiple of 32");
    int64_t nb = n / 32;
    int g = (int)std::min<int64_t>((nb + 255) / 256, (int64_t)num_cus() * 8);
    hipLaunchKernelGGL(repack_q8_0_kernel, dim3(g), dim3(256), 0, s, (const uint8_t*)raw,
                       (int8_t*)out->qs, out->sc, nb);
  } else if (qtype == SMHIP_QTYPE_Q4_K) {
    SMHIP_REQUIRE(n % 256 == 0, "Q4_K repack: element count must be a multiple of 256");
    int64_t nb = n / 256;
    int g = (int)std::min<int64_t>((nb + 255) / 256, (int64_t)num_cus() * 8);
    hipLaunchKernelGGL(repack_q4k_kernel, dim3(g), dim3(256), 0, s, (const uint8_t*)raw,
                       (uint8_t*)out->qs, out->sc, nb);
  } else {
    return fail(SMHIP_EUNSUPPORTED, "repack: qtype must be Q8_0 (8) or Q4_K (12)");
  }
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

// ---------------------------------------------------------------- column planes
// The transposed copy of a [rows][cols] quantised matrix used by dX = dY W: element
// (o, i) of the row planes becomes element i*rows + o, with the fp32 scale (Q8_0) or the
// (sc*d, mn*dmin) pair (Q4_K) of its 32-block stored at (i/32)*rows + o, so that a run of
// consecutive o (the k index of dX) is contiguous in both planes.  Same values, same bits.
__global__ void col_planes_q8_kernel(const int8_t* __restrict__ qs, const float* __restrict__ sc, int rows, int cols,
                                     int8_t* __restrict__ qt, float* __restrict__ st) {
  const int64_t n = (int64_t)rows * cols;
  const int cb = cols / 32;
  for (int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; x < n; x += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = x / rows, o = x - i * rows;
    qt[x] = qs[o * cols + i];
    if ((i & 31) == 0) st[(i >> 5) * rows + o] = sc[o * cb + (i >> 5)];
  }
}
__device__ __forceinline__ uint32_t q4k_code(const uint8_t* qs, int64_t e) {
  const int w = (int)(e & 255);
  return (qs[(e >> 8) * 128 + (w >> 6) * 32 + (w & 31)] >> (((w & 63) >> 5) * 4)) & 0xF;
}
__global__ void col_planes_q4k_kernel(const uint8_t* __restrict__ qs, const float* __restrict__ sm, int rows, int cols,
                                      uint8_t* __restrict__ qt, float* __restrict__ st) {
  const int64_t n2 = (int64_t)rows * cols / 2;  // one output byte = codes of (o, i) and (o+1, i), o even
  const int cb = cols / 32;
  for (int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; x < n2; x += (int64_t)gridDim.x * blockDim.x) {
    const int64_t f = 2 * x, i = f / rows, o = f - i * rows;
    const uint32_t lo = q4k_code(qs, o * cols + i), hi = q4k_code(qs, (o + 1) * cols + i);
    qt[x] = (uint8_t)(lo | (hi << 4));
    if ((i & 31) == 0) {
      for (int j = 0; j < 2; j++) {
        const int64_t src = 2 * ((o + j) * cb + (i >> 5)), dst = 2 * ((i >> 5) * rows + o + j);
        st[dst] = sm[src];
        st[dst + 1] = sm[src + 1];
      }
    }
  }
}
int make_col_planes(const QuantPlanes& q, int rows, int cols, void* dst, QuantPlanes* out, hipStream_t s) {
  SMHIP_REQUIRE(q.n == (int64_t)rows * cols, "column planes: shape does not match the planes");
  SMHIP_REQUIRE(cols % 32 == 0 && rows % 2 == 0, "column planes: cols must be a multiple of 32, rows even");
  size_t qb = 0;
  planes_bytes(q.kind, q.n, &qb);
  out->kind = q.kind;
  out->n = q.n;
  out->qs = dst;
  out->sc = (float*)((char*)dst + qb);
  const int64_t n = q.kind == SMHIP_QTYPE_Q8_0 ? q.n : q.n / 2;
  const int g = (int)std::min<int64_t>((n + 255) / 256, (int64_t)num_cus() * 16);
  if (q.kind == SMHIP_QTYPE_Q8_0)
    hipLaunchKernelGGL(col_planes_q8_kernel, dim3(g), dim3(256), 0, s, (const int8_t*)q.qs, q.sc, rows, cols,
                       (int8_t*)out->qs, out->sc);
  else if (q.kind == SMHIP_QTYPE_Q4_K)
    hipLaunchKernelGGL(col_planes_q4k_kernel, dim3(g), dim3(256), 0, s, (const uint8_t*)q.qs, q.sc, rows, cols,
                       (uint8_t*)out->qs, out->sc);
  else
    return fail(SMHIP_EUNSUPPORTED, "column planes: qtype must be Q8_0 (8) or Q4_K (12)");
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

// ---------------------------------------------------------------- fragment planes (Q8_0)
// The Q8_0 base of W[rows][cols] in the order the bf16 GEMM copies it to LDS (SRC_Q8F: B = W,
// k = cols; SRC_Q8FT: B = W^T, k = rows): 2048-byte blocks of 32 B rows x 64 k, row-major, the
// K tiles of a 32-row group contiguous; scales as fp16 (each fp32 scale of the row planes is a
// binary16 value, so this is exact).
__global__ void frag_planes_q8_kernel(const int8_t* __restrict__ qs, const float* __restrict__ sc, int rows, int cols,
                                      int trans, uint8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
  const int N = trans ? cols : rows, K = trans ? rows : cols;
  const int64_t groups = (int64_t)N * K / 8, nsc = (int64_t)N * K / 32;
  const int kts = K / 64;
  for (int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; x < groups; x += (int64_t)gridDim.x * blockDim.x) {
    const int64_t blk = x >> 8;  // 256 eight-byte groups per block
    const int g8 = (int)(x & 255);
    const int64_t rb = blk / kts;
    const int kt = (int)(blk - rb * kts);
    const int64_t r = rb * 32 + (g8 >> 3);
    const int64_t k0 = (int64_t)kt * 64 + (g8 & 7) * 8;
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int64_t e = trans ? (k0 + i) * cols + r : r * cols + k0 + i;
      w[i >> 2] |= (uint32_t)(uint8_t)qs[e] << (8 * (i & 3));
    }
    *reinterpret_cast<uint2*>(codes + 8 * x) = make_uint2(w[0], w[1]);
  }
  for (int64_t y = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; y < nsc; y += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rb = y / K;
    const int rem = (int)(y - rb * K);
    float v;
    if (trans) {
      v = sc[((int64_t)rem * cols + rb * 32) / 32];
    } else {
      const int kt = rem >> 6, j = (rem >> 5) & 1, rl = rem & 31;
      v = sc[((rb * 32 + rl) * cols + kt * 64 + j * 32) / 32];
    }
    scales[y] = __builtin_bit_cast(uint16_t, (_Float16)v);
  }
}
__global__ void frag_planes_q4k_kernel(const uint8_t* __restrict__ qs, const float* __restrict__ sm, int rows,
                                       int cols, int trans, uint8_t* __restrict__ codes, float* __restrict__ pairs) {
  const int N = trans ? cols : rows, K = trans ? rows : cols;
  const int64_t words = (int64_t)N * K / 8, npair = (int64_t)N * K / 32;
  const int kts = K / 64;
  for (int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; x < words; x += (int64_t)gridDim.x * blockDim.x) {
    const int64_t blk = x >> 8;  // 256 four-byte words per 32 x 64 block
    const int g = (int)(x & 255);
    const int64_t rb = blk / kts;
    const int kt = (int)(blk - rb * kts);
    const int64_t r = rb * 32 + (g >> 3);
    const int64_t k0 = (int64_t)kt * 64 + (g & 7) * 8;
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int64_t e = trans ? (k0 + i) * cols + r : r * cols + k0 + i;
      w |= q4k_code(qs, e) << (i < 4 ? 8 * i : 8 * (i - 4) + 4);
    }
    reinterpret_cast<uint32_t*>(codes)[x] = w;
  }
  for (int64_t y = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; y < npair; y += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rb = y / K;
    const int rem = (int)(y - rb * K);
    int64_t src;
    if (trans) {
      src = ((int64_t)rem * cols + rb * 32) / 32;
    } else {
      const int kt = rem >> 6, j = (rem >> 5) & 1, rl = rem & 31;
      src = ((rb * 32 + rl) * cols + kt * 64 + j * 32) / 32;
    }
    pairs[2 * y] = sm[2 * src];
    pairs[2 * y + 1] = sm[2 * src + 1];
  }
}
size_t frag_planes_bytes(int64_t n, int qtype) {
  return qtype == SMHIP_QTYPE_Q4_K ? (size_t)n / 2 + (size_t)n / 4 : (size_t)n + (size_t)n / 16;
}
int make_frag_planes(const QuantPlanes& q, int rows, int cols, int trans, void* dst, Operand* out, hipStream_t s) {
  SMHIP_REQUIRE(q.kind == SMHIP_QTYPE_Q8_0 || q.kind == SMHIP_QTYPE_Q4_K, "fragment planes: Q8_0 or Q4_K");
  SMHIP_REQUIRE(q.n == (int64_t)rows * cols, "fragment planes: shape does not match the planes");
  const int N = trans ? cols : rows, K = trans ? rows : cols;
  SMHIP_REQUIRE(N % 32 == 0 && K % 64 == 0, "fragment planes: B rows must be a multiple of 32 and K of 64");
  SMHIP_REQUIRE(((uintptr_t)dst & 255) == 0, "fragment planes: destination must be 256-byte aligned");
  const bool q8 = q.kind == SMHIP_QTYPE_Q8_0;
  const size_t cb = q8 ? (size_t)q.n : (size_t)q.n / 2;  // code bytes
  out->mode = q8 ? (trans ? SRC_Q8FT : SRC_Q8F) : (trans ? SRC_Q4FT : SRC_Q4F);
  out->p = dst;
  out->s = (const float*)((char*)dst + cb);  // fp16 scales (Q8_0) or fp32 pairs (Q4_K), see SrcMode
  out->ld = K;
  const int64_t work = q.n / 8;
  const int g = (int)std::min<int64_t>((work + 255) / 256, (int64_t)num_cus() * 16);
  if (q8)
    hipLaunchKernelGGL(frag_planes_q8_kernel, dim3(g), dim3(256), 0, s, (const int8_t*)q.qs, q.sc, rows, cols, trans,
                       (uint8_t*)dst, (uint16_t*)((char*)dst + cb));
  else
    hipLaunchKernelGGL(frag_planes_q4k_kernel, dim3(g), dim3(256), 0, s, (const uint8_t*)q.qs, q.sc, rows, cols,
                       trans, (uint8_t*)dst, (float*)((char*)dst + cb));
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

}  // namespace smhip

namespace smhip {
// Gather + dequantise rows ids[t] of a quantised [rows][D] table (embedding lookup of a
// frozen quantised embedding, EmbeddingTable.cs:87): out[t, i] = deq(E[ids[t], i]).
__global__ void dequant_rows_kernel(QuantPlanes q, const int32_t* __restrict__ ids, float* __restrict__ out, int T,
                                    int D) {
  const int64_t n = (int64_t)T * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / D, c = i - t * D;
    const int64_t e = (int64_t)ids[t] * D + c;
    float v;
    if (q.kind == SMHIP_QTYPE_Q8_0) {
      v = (float)((const int8_t*)q.qs)[e] * q.sc[e >> 5];
    } else {
      const int w = (int)(e & 255);
      const uint8_t b = ((const uint8_t*)q.qs)[(e >> 8) * 128 + (w >> 6) * 32 + (w & 31)];
      const float sd = q.sc[2 * (e >> 5)], md = q.sc[2 * (e >> 5) + 1];
      v = sd * (float)((b >> (((w & 63) >> 5) * 4)) & 0xF) - md;
    }
    out[i] = v;
  }
}
int dequant_rows(const QuantPlanes& q, const int32_t* ids, float* out, int T, int D, hipStream_t s) {
  const int64_t n = (int64_t)T * D;
  if (!n) return SMHIP_OK;
  int g = (int)std::min<int64_t>((n + 255) / 256, (int64_t)num_cus() * 8);
  hipLaunchKernelGGL(dequant_rows_kernel, dim3(g), dim3(256), 0, s, q, ids, out, T, D);
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}
}  // namespace smhip

namespace smhip {
// ---------------------------------------------------------------- bf16 workspace of a frozen base
// Decodes a quantised [rows][cols] matrix to bf16 (the fp32 weight q*d, or sd*v - md, rounded
// once, exactly the values the fused-decode GEMM loaders stage into LDS) in the row layout
// w[o*cols + i] and/or the transposed layout wt[i*rows + o].  One workgroup per 64 x 64 tile:
// each thread decodes 16 consecutive elements of one row (one 16-byte code load, one scale),
// writes them to the row layout and to an LDS tile, from which 16 consecutive rows of one
// column are written to the transposed layout.
__device__ __forceinline__ void dequant_bf16_tile(const QuantPlanes& q, int rows, int cols, uint16_t* __restrict__ w,
                                                  uint16_t* __restrict__ wt, int bx, int by, uint16_t (*tile)[66]) {
  const int tr = threadIdx.x >> 2, tc = (threadIdx.x & 3) * 16;
  const int o = by * 64 + tr, i0 = bx * 64 + tc;
  if (o < rows && i0 < cols) {
    const int64_t e = (int64_t)o * cols + i0;
    float v[16];
    if (q.kind == SMHIP_QTYPE_Q8_0) {
      const uint4 c = *reinterpret_cast<const uint4*>((const int8_t*)q.qs + e);
      const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
      const float d = q.sc[e >> 5];
#pragma unroll
      for (int j = 0; j < 16; j++) v[j] = (float)(int8_t)(cw[j >> 2] >> ((j & 3) * 8)) * d;
    } else {
      const int wi = (int)(e & 255);
      const uint4 c = *reinterpret_cast<const uint4*>((const uint8_t*)q.qs + (e >> 8) * 128 + (wi >> 6) * 32 + (wi & 31));
      const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
      const int sh = ((wi & 63) >> 5) * 4;
      const float sd = q.sc[2 * (e >> 5)], md = q.sc[2 * (e >> 5) + 1];
#pragma unroll
      for (int j = 0; j < 16; j++) v[j] = sd * (float)((cw[j >> 2] >> ((j & 3) * 8 + sh)) & 0xF) - md;
    }
    uint32_t p[8];
#pragma unroll
    for (int j = 0; j < 8; j++) p[j] = pack_bf2(v[2 * j], v[2 * j + 1]);
    if (w) {
      uint4* dst = reinterpret_cast<uint4*>(w + e);
      dst[0] = make_uint4(p[0], p[1], p[2], p[3]);
      dst[1] = make_uint4(p[4], p[5], p[6], p[7]);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
      tile[tr][tc + 2 * j] = (uint16_t)(p[j] & 0xFFFF);
      tile[tr][tc + 2 * j + 1] = (uint16_t)(p[j] >> 16);
    }
  }
  if (!wt) return;
  __syncthreads();
  // transposed: thread -> column i = i-tile + tr, rows o0 .. o0+15
  const int i = bx * 64 + tr, o0 = by * 64 + tc;
  if (i < cols && o0 < rows) {
    uint32_t p[8];
#pragma unroll
    for (int j = 0; j < 8; j++) p[j] = (uint32_t)tile[tc + 2 * j][tr] | ((uint32_t)tile[tc + 2 * j + 1][tr] << 16);
    uint4* dst = reinterpret_cast<uint4*>(wt + (int64_t)i * rows + o0);
    dst[0] = make_uint4(p[0], p[1], p[2], p[3]);
    dst[1] = make_uint4(p[4], p[5], p[6], p[7]);
  }
}
// Many matrices in one launch: workgroup b decodes tile (b - first) of the matrix whose tile
// range [first, first + tiles) holds b (binary search over the descriptor table).
__global__ __launch_bounds__(256) void dequant_bf16_many_kernel(const DequantJob* __restrict__ jobs, int njobs) {
  __shared__ uint16_t tile[64][66];
  const int64_t b = blockIdx.x;
  int lo = 0, hi = njobs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (jobs[mid].first <= b) lo = mid; else hi = mid - 1;
  }
  const DequantJob j = jobs[lo];
  const int64_t t = b - j.first;
  const int tx = (j.cols + 63) / 64;
  dequant_bf16_tile(j.q, j.rows, j.cols, j.w, j.wt, (int)(t % tx), (int)(t / tx), tile);
}
int dequant_bf16_many(const DequantJob* jobs_dev, int njobs, int64_t total_tiles, hipStream_t s) {
  if (!njobs || !total_tiles) return SMHIP_OK;
  SMHIP_REQUIRE(total_tiles < ((int64_t)1 << 31), "dequant_bf16_many: too many tiles");
  hipLaunchKernelGGL(dequant_bf16_many_kernel, dim3((unsigned)total_tiles), dim3(256), 0, s, jobs_dev, njobs);
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}
int dequant_bf16_check(const QuantPlanes& q, int rows, int cols, const uint16_t* w, const uint16_t* wt) {
  SMHIP_REQUIRE(q.n == (int64_t)rows * cols, "dequant_bf16: shape does not match the planes");
  SMHIP_REQUIRE(rows % 16 == 0 && cols % 16 == 0, "dequant_bf16: rows and cols must be multiples of 16");
  SMHIP_REQUIRE(q.kind == SMHIP_QTYPE_Q8_0 || q.kind == SMHIP_QTYPE_Q4_K, "dequant_bf16: qtype must be Q8_0 or Q4_K");
  SMHIP_REQUIRE(((uintptr_t)w | (uintptr_t)wt) % 16 == 0, "dequant_bf16: outputs must be 16-byte aligned");
  return SMHIP_OK;
}
}  // namespace smhip
