// gemm_bf16.hip — high-throughput bf16 MFMA GEMM for gfx950 (the training step's linears).
//
//   C[M,N] = alpha * sum_k A(m,k) B(n,k) [+ alpha2 * sum_k A2(m,k) B2(n,k)] [+ bias] [+ R] [+ beta C]
//
// Block tile BM x 128 x 64 (BM = 128 or 256), 256 threads = 4 wave64s in a 2 x 2
// grid; each wave owns (BM/2) x 64 of C as 32 x 32 blocks of
// v_mfma_f32_32x32x16_bf16.  Operands are staged into LDS as bf16 [row][64]
// tiles (128-byte rows) whose 16-byte chunks are XOR-swizzled by row, so the
// MFMA fragment reads (one ds_read_b128 per lane: 8 consecutive k of one row)
// hit distinct banks.  Operand modes are template parameters:
//   *_K  k-contiguous rows: 16-byte global loads straight into LDS chunks;
//   *_R  row-contiguous (k-strided) matrices: each thread loads 4 k-rows x 8
//        columns and writes 8 LDS quads (4 consecutive k of one row, 8 bytes),
//        i.e. the transpose happens during staging;
//   Q8 / Q4_K  frozen base weights: the repacked quantisation planes are
//        decoded in registers (int8*scale, (sc*d)*v - mn*dmin; exact fp32 values
//        rounded once to bf16) and never written to HBM dequantised.
// The next K tile's global loads are issued before the current tile's MFMAs
// (register prefetch + double-buffered LDS, one barrier per K tile).
// Workgroups are numbered so that the 8 XCDs each own a contiguous band of
// output tiles (AMD dispatches consecutive workgroups round-robin over XCDs),
// keeping the operand panels a band shares in that XCD's L2.
#include "common.hpp"
#include "kernels.hpp"

namespace smhip {
namespace g2 {

constexpr int BN = 128, BK = 64, NT = 256;

struct Op {
  const void* p;
  const float* s;
  int64_t ld;
};

// swizzled byte offset of 16-byte chunk c (0..7) of row r in a [rows][64] bf16 tile
__device__ __forceinline__ int sw(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

__device__ __forceinline__ uint32_t pk(float a, float b) { return pack_bf2(a, b); }

// ---------------------------------------------------------------- decode helpers (exact fp32, then bf16)
__device__ __forceinline__ void i8x4(uint32_t w, float d, float* o) {
  o[0] = (float)(int8_t)(w & 0xFF) * d;
  o[1] = (float)(int8_t)((w >> 8) & 0xFF) * d;
  o[2] = (float)(int8_t)((w >> 16) & 0xFF) * d;
  o[3] = (float)(int8_t)(w >> 24) * d;
}
__device__ __forceinline__ void nib4(uint32_t w, int sh, float sd, float md, float* o) {
  o[0] = sd * (float)((w >> sh) & 0xF) - md;
  o[1] = sd * (float)((w >> (8 + sh)) & 0xF) - md;
  o[2] = sd * (float)((w >> (16 + sh)) & 0xF) - md;
  o[3] = sd * (float)((w >> (24 + sh)) & 0xF) - md;
}

// ---------------------------------------------------------------- K-contiguous operand (rows x 64)
// Work is split into 16-byte global "units": bf16 unit = 8 elements, Q8 unit = 16 int8
// elements; a tile row of 64 k is 8 (bf16) or 4 (Q8) units.
template <int MODE, int ROWS>
struct KLoader {
  static constexpr bool BF = MODE == SRC_BF16_K;
  static constexpr int EPU = BF ? 8 : 16;               // elements per unit
  static constexpr int UPR = BK / EPU;                  // units per row
  static constexpr int NU = ROWS * UPR / NT;            // units per thread
  uint4 raw[NU];
  float sc[NU];
  __device__ __forceinline__ void load(const Op& o, int r0, int k0, int R) {
#pragma unroll
    for (int u = 0; u < NU; u++) {
      const int id = u * NT + threadIdx.x;
      const int r = id / UPR, c = id % UPR;
      const int gr = r0 + r;
      if (gr < R) {
        const int64_t e = (int64_t)gr * o.ld + k0 + c * EPU;
        if constexpr (BF) {
          raw[u] = *reinterpret_cast<const uint4*>((const uint16_t*)o.p + e);
        } else {
          static_assert(MODE == SRC_Q8_K, "KLoader handles bf16 and Q8_0 rows");
          raw[u] = *reinterpret_cast<const uint4*>((const int8_t*)o.p + e);
          sc[u] = o.s[e >> 5];
        }
      } else {
        raw[u] = make_uint4(0, 0, 0, 0);
        sc[u] = 0.f;
      }
    }
  }
  __device__ __forceinline__ void store(uint8_t* lds) const {
#pragma unroll
    for (int u = 0; u < NU; u++) {
      const int id = u * NT + threadIdx.x;
      const int r = id / UPR, c = id % UPR;
      if constexpr (BF) {
        *reinterpret_cast<uint4*>(lds + sw(r, c)) = raw[u];
      } else {
        float v[16];
        i8x4(raw[u].x, sc[u], v); i8x4(raw[u].y, sc[u], v + 4); i8x4(raw[u].z, sc[u], v + 8); i8x4(raw[u].w, sc[u], v + 12);
        uint4 a, b;
        a.x = pk(v[0], v[1]); a.y = pk(v[2], v[3]); a.z = pk(v[4], v[5]); a.w = pk(v[6], v[7]);
        b.x = pk(v[8], v[9]); b.y = pk(v[10], v[11]); b.z = pk(v[12], v[13]); b.w = pk(v[14], v[15]);
        *reinterpret_cast<uint4*>(lds + sw(r, 2 * c)) = a;
        *reinterpret_cast<uint4*>(lds + sw(r, 2 * c + 1)) = b;
      }
    }
  }
};

// Q4_K K-contiguous needs 16 bytes of codes AND the shift: dedicated loader
template <int ROWS>
struct KLoaderQ4 {
  static constexpr int UPR = BK / 16, NU = ROWS * UPR / NT;
  uint4 raw[NU];
  float sc[NU], sm[NU];
  int sh[NU];
  __device__ __forceinline__ void load(const Op& o, int r0, int k0, int R) {
#pragma unroll
    for (int u = 0; u < NU; u++) {
      const int id = u * NT + threadIdx.x;
      const int r = id / UPR, c = id % UPR;
      const int gr = r0 + r;
      if (gr < R) {
        const int64_t e = (int64_t)gr * o.ld + k0 + c * 16;
        const int w = (int)(e & 255);
        raw[u] = *reinterpret_cast<const uint4*>((const uint8_t*)o.p + (e >> 8) * 128 + (w >> 6) * 32 + (w & 31));
        sh[u] = ((w & 63) >> 5) * 4;
        sc[u] = o.s[2 * (e >> 5)];
        sm[u] = o.s[2 * (e >> 5) + 1];
      } else {
        raw[u] = make_uint4(0, 0, 0, 0);
        sh[u] = 0; sc[u] = 0.f; sm[u] = 0.f;
      }
    }
  }
  __device__ __forceinline__ void store(uint8_t* lds) const {
#pragma unroll
    for (int u = 0; u < NU; u++) {
      const int id = u * NT + threadIdx.x;
      const int r = id / UPR, c = id % UPR;
      float v[16];
      nib4(raw[u].x, sh[u], sc[u], sm[u], v); nib4(raw[u].y, sh[u], sc[u], sm[u], v + 4);
      nib4(raw[u].z, sh[u], sc[u], sm[u], v + 8); nib4(raw[u].w, sh[u], sc[u], sm[u], v + 12);
      uint4 a, b;
      a.x = pk(v[0], v[1]); a.y = pk(v[2], v[3]); a.z = pk(v[4], v[5]); a.w = pk(v[6], v[7]);
      b.x = pk(v[8], v[9]); b.y = pk(v[10], v[11]); b.z = pk(v[12], v[13]); b.w = pk(v[14], v[15]);
      *reinterpret_cast<uint4*>(lds + sw(r, 2 * c)) = a;
      *reinterpret_cast<uint4*>(lds + sw(r, 2 * c + 1)) = b;
    }
  }
};

// ---------------------------------------------------------------- row-contiguous operand (k-strided)
// Tile element (r, k) lives at e = (k0+k)*ld + r0 + r.  Each thread owns a
// "quad": 4 consecutive k x 8 consecutive r; ROWS*64/32/256 quads per thread.
template <int MODE, int ROWS>
struct RLoader {
  static constexpr int RG = ROWS / 8;          // row groups of 8
  static constexpr int NQ = RG * (BK / 4) / NT; // quads per thread
  uint2 raw[NQ][4];                             // bf16: 4 rows of 8 bf16 = 16 B (uint4) -> use two uint2
  uint2 hi[NQ][4];
  float sc[NQ][4], sm[NQ][4];
  int sh[NQ][4];
  __device__ __forceinline__ void load(const Op& o, int r0, int k0, int R) {
#pragma unroll
    for (int q = 0; q < NQ; q++) {
      const int id = q * NT + threadIdx.x;
      const int rg = id % RG, kq = id / RG;
      const int gr = r0 + rg * 8;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int64_t e = (int64_t)(k0 + kq * 4 + j) * o.ld + gr;
        if (gr + 8 <= R) {
          if constexpr (MODE == SRC_BF16_R) {
            uint4 a = *reinterpret_cast<const uint4*>((const uint16_t*)o.p + e);
            raw[q][j] = make_uint2(a.x, a.y);
            hi[q][j] = make_uint2(a.z, a.w);
          } else if constexpr (MODE == SRC_Q8_R) {
            raw[q][j] = *reinterpret_cast<const uint2*>((const int8_t*)o.p + e);
            sc[q][j] = o.s[e >> 5];
          } else {  // Q4K_R
            const int w = (int)(e & 255);
            raw[q][j] = *reinterpret_cast<const uint2*>((const uint8_t*)o.p + (e >> 8) * 128 + (w >> 6) * 32 + (w & 31));
            sh[q][j] = ((w & 63) >> 5) * 4;
            sc[q][j] = o.s[2 * (e >> 5)];
            sm[q][j] = o.s[2 * (e >> 5) + 1];
          }
        } else {
          raw[q][j] = make_uint2(0, 0);
          hi[q][j] = make_uint2(0, 0);
          sc[q][j] = 0.f; sm[q][j] = 0.f; sh[q][j] = 0;
        }
      }
    }
  }
  // element i (0..7) of the 8 columns at k-row j, as bf16 bits
  __device__ __forceinline__ uint32_t el(int q, int j, int i) const {
    if constexpr (MODE == SRC_BF16_R) {
      const uint32_t w = i < 4 ? (i < 2 ? raw[q][j].x : raw[q][j].y) : (i < 6 ? hi[q][j].x : hi[q][j].y);
      return (i & 1) ? (w >> 16) : (w & 0xFFFF);
    } else if constexpr (MODE == SRC_Q8_R) {
      const uint32_t w = i < 4 ? raw[q][j].x : raw[q][j].y;
      return f2bf((float)(int8_t)((w >> (8 * (i & 3))) & 0xFF) * sc[q][j]);
    } else {
      const uint32_t w = i < 4 ? raw[q][j].x : raw[q][j].y;
      return f2bf(sc[q][j] * (float)((w >> (8 * (i & 3) + sh[q][j])) & 0xF) - sm[q][j]);
    }
  }
  __device__ __forceinline__ void store(uint8_t* lds) const {
#pragma unroll
    for (int q = 0; q < NQ; q++) {
      const int id = q * NT + threadIdx.x;
      const int rg = id % RG, kq = id / RG;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int r = rg * 8 + i;
        uint2 v;
        v.x = el(q, 0, i) | (el(q, 1, i) << 16);
        v.y = el(q, 2, i) | (el(q, 3, i) << 16);
        // 4 consecutive k (8 bytes) = half of chunk kq/2
        *reinterpret_cast<uint2*>(lds + sw(r, kq >> 1) + (kq & 1) * 8) = v;
      }
    }
  }
};

template <int MODE, int ROWS>
struct LoaderFor {
  using T = typename std::conditional<(MODE & 1) == 0,
                                      typename std::conditional<MODE == SRC_Q4K_K, KLoaderQ4<ROWS>, KLoader<MODE, ROWS>>::type,
                                      RLoader<MODE, ROWS>>::type;
};

// Rank-extension tile (LoRA): generic guarded element loads, any mode, K2 <= 64 per tile.
__device__ __forceinline__ float gen_elem(int mode, const Op& o, int r, int k, int R, int K) {
  if (r >= R || k >= K) return 0.f;
  switch (mode) {
    case SRC_BF16_K: return bf2f(((const uint16_t*)o.p)[(int64_t)r * o.ld + k]);
    case SRC_BF16_R: return bf2f(((const uint16_t*)o.p)[(int64_t)k * o.ld + r]);
    case SRC_F32_K: return ((const float*)o.p)[(int64_t)r * o.ld + k];
    default: return ((const float*)o.p)[(int64_t)k * o.ld + r];
  }
}
template <int ROWS>
__device__ __forceinline__ void gen_tile(int mode, const Op& o, int r0, int k0, int R, int K, float mult, uint8_t* lds) {
  // thread handles 8 consecutive k of rows (ROWS*8 chunks)
  for (int c = threadIdx.x; c < ROWS * 8; c += NT) {
    const int r = c >> 3, ch = c & 7;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = mult * gen_elem(mode, o, r0 + r, k0 + ch * 8 + i, R, K);
    uint4 a;
    a.x = pk(v[0], v[1]); a.y = pk(v[2], v[3]); a.z = pk(v[4], v[5]); a.w = pk(v[6], v[7]);
    *reinterpret_cast<uint4*>(lds + sw(r, ch)) = a;
  }
}

struct Args {
  Op A, B, A2, B2;
  int amode2, bmode2;
  int M, N, K, K2;
  float alpha, alpha2, beta;
  void* C;
  int64_t ldc;
  const float* bias;
  const float* R;
  int64_t ldr;
  int tiles_m, tiles_n;
  int kps;          // main K tiles per split (blockIdx.y = split)
  float* partial;   // non-null: write raw partial sums [split][M][N] instead of C
};

template <int BM, int AMODE, int BMODE, bool C_BF16>
__global__ __launch_bounds__(NT, BM == 128 ? 2 : 1) void gemm_bf16_kernel(Args g) {
  constexpr int WM = BM / 2;       // rows per wave
  constexpr int MB = WM / 32;      // 32-row blocks per wave
  __shared__ __attribute__((aligned(16))) uint8_t sA[2][BM * 128];
  __shared__ __attribute__((aligned(16))) uint8_t sB[2][BN * 128];

  // XCD-aware tile order: workgroup w runs on XCD w % 8; give XCD x the contiguous band
  // of tiles [x*per, (x+1)*per) (tile index = n-major within an m panel group).
  const int ntiles = g.tiles_m * g.tiles_n;
  const int wg = blockIdx.x;
  int tile = wg;
  if (ntiles % 8 == 0) tile = (wg % 8) * (ntiles / 8) + wg / 8;
  // within the band: groups of 8 m-panels swept along n (operand reuse in L2)
  constexpr int GM = 8;
  const int group = tile / (GM * g.tiles_n);
  const int first_m = group * GM;
  const int gsz = min(g.tiles_m - first_m, GM);
  const int tm = first_m + (tile % (GM * g.tiles_n)) % gsz;
  const int tn = (tile % (GM * g.tiles_n)) / gsz;
  const int m0 = tm * BM, n0 = tn * BN;

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wm = wv >> 1, wn = wv & 1;

  floatx16 acc[MB][2];
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  typename LoaderFor<AMODE, BM>::T la;
  typename LoaderFor<BMODE, BN>::T lb;
  const int nk_all = g.K / BK;
  const int split = blockIdx.y, nsplit = gridDim.y;
  const int kt0 = split * g.kps;
  const int nk1 = max(0, min(nk_all, kt0 + g.kps) - kt0);           // main K tiles of this split
  const int nk2 = split == nsplit - 1 ? (g.K2 + BK - 1) / BK : 0;   // rank extension: last split only
  const int nt = nk1 + nk2;

  auto compute = [&](int buf) {
    const uint8_t* a = sA[buf];
    const uint8_t* b = sB[buf];
#pragma unroll
    for (int kk = 0; kk < BK / 16; kk++) {
      const int ch = 2 * kk + (lane >> 5);
      bf16x8 fa[MB], fb[2];
#pragma unroll
      for (int i = 0; i < MB; i++) {
        const int r = wm * WM + i * 32 + (lane & 31);
        fa[i] = *reinterpret_cast<const bf16x8*>(a + sw(r, ch));
      }
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int r = wn * 64 + j * 32 + (lane & 31);
        fb[j] = *reinterpret_cast<const bf16x8*>(b + sw(r, ch));
      }
#pragma unroll
      for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  };

  if (nk1 > 0) {
    la.load(g.A, m0, kt0 * BK, g.M);
    lb.load(g.B, n0, kt0 * BK, g.N);
    la.store(sA[0]);
    lb.store(sB[0]);
  } else if (nk2 > 0) {
    gen_tile<BM>(g.amode2, g.A2, m0, 0, g.M, g.K2, g.alpha2, sA[0]);
    gen_tile<BN>(g.bmode2, g.B2, n0, 0, g.N, g.K2, 1.f, sB[0]);
  }
  __syncthreads();
  for (int t = 0; t < nt; t++) {
    const int buf = t & 1;
    const bool next_main = t + 1 < nk1;
    if (next_main) {
      la.load(g.A, m0, (kt0 + t + 1) * BK, g.M);
      lb.load(g.B, n0, (kt0 + t + 1) * BK, g.N);
    }
    compute(buf);
    if (next_main) {
      la.store(sA[buf ^ 1]);
      lb.store(sB[buf ^ 1]);
    } else if (t + 1 < nt) {
      const int k0 = (t + 1 - nk1) * BK;
      gen_tile<BM>(g.amode2, g.A2, m0, k0, g.M, g.K2, g.alpha2, sA[buf ^ 1]);
      gen_tile<BN>(g.bmode2, g.B2, n0, k0, g.N, g.K2, 1.f, sB[buf ^ 1]);
    }
    __syncthreads();
  }

  // epilogue: lane holds column (lane&31) and rows (e/4)*8 + (lane>>5)*4 + e%4 of each 32x32 block
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int col = n0 + wn * 64 + j * 32 + (lane & 31);
      if (col >= g.N) continue;
      const float bv = g.bias ? g.bias[col] : 0.f;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int row = m0 + wm * WM + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        if (row >= g.M) continue;
        if (g.partial) {
          g.partial[((int64_t)split * g.M + row) * g.N + col] = acc[i][j][e];
          continue;
        }
        float o = g.alpha * acc[i][j][e] + bv;
        if constexpr (C_BF16) {
          uint16_t* c = (uint16_t*)g.C + (int64_t)row * g.ldc + col;
          if (g.beta != 0.f) o = o + g.beta * bf2f(*c);
          *c = f2bf(o);
        } else {
          float* c = (float*)g.C + (int64_t)row * g.ldc + col;
          if (g.R) o = o + g.R[(int64_t)row * g.ldr + col];
          if (g.beta != 0.f) o = o + g.beta * *c;
          *c = o;
        }
      }
    }
}

template <int BM, int AM, int BMD>
static void launch_c(const Args& a, int c_bf16, int splits, hipStream_t s) {
  const dim3 grid(a.tiles_m * a.tiles_n, splits);
  if (c_bf16 && !a.partial) hipLaunchKernelGGL((gemm_bf16_kernel<BM, AM, BMD, true>), grid, dim3(NT), 0, s, a);
  else hipLaunchKernelGGL((gemm_bf16_kernel<BM, AM, BMD, false>), grid, dim3(NT), 0, s, a);
}

template <int BM>
static bool dispatch(const Args& a, int amode, int bmode, int c_bf16, int sp, hipStream_t s) {
  if (amode == SRC_BF16_K) {
    switch (bmode) {
      case SRC_BF16_K: launch_c<BM, SRC_BF16_K, SRC_BF16_K>(a, c_bf16, sp, s); return true;
      case SRC_BF16_R: launch_c<BM, SRC_BF16_K, SRC_BF16_R>(a, c_bf16, sp, s); return true;
      case SRC_Q8_K: launch_c<BM, SRC_BF16_K, SRC_Q8_K>(a, c_bf16, sp, s); return true;
      case SRC_Q8_R: launch_c<BM, SRC_BF16_K, SRC_Q8_R>(a, c_bf16, sp, s); return true;
      case SRC_Q4K_K: launch_c<BM, SRC_BF16_K, SRC_Q4K_K>(a, c_bf16, sp, s); return true;
      case SRC_Q4K_R: launch_c<BM, SRC_BF16_K, SRC_Q4K_R>(a, c_bf16, sp, s); return true;
      default: return false;
    }
  }
  if (amode == SRC_BF16_R && bmode == SRC_BF16_R && (!c_bf16 || a.partial)) {
    launch_c<BM, SRC_BF16_R, SRC_BF16_R>(a, 0, sp, s);
    return true;
  }
  return false;
}

// C = alpha * sum_s partial[s] (+ bias) (+ R) (+ beta C); splits summed in ascending order.
__global__ void splitk_epilogue_kernel(const float* __restrict__ partial, int splits, int M, int N, float alpha,
                                       float beta, void* __restrict__ Cp, int64_t ldc, int c_bf16,
                                       const float* __restrict__ bias, const float* __restrict__ R, int64_t ldr) {
  const int64_t n = (int64_t)M * N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float acc = 0.f;
    for (int k = 0; k < splits; k++) acc += partial[(int64_t)k * n + i];
    const int64_t row = i / N, col = i - row * N;
    float o = alpha * acc;
    if (bias) o = o + bias[col];
    if (c_bf16) {
      uint16_t* c = (uint16_t*)Cp + row * ldc + col;
      if (beta != 0.f) o = o + beta * bf2f(*c);
      *c = f2bf(o);
    } else {
      float* c = (float*)Cp + row * ldc + col;
      if (R) o = o + R[row * ldr + col];
      if (beta != 0.f) o = o + beta * *c;
      *c = o;
    }
  }
}

}  // namespace g2

static bool aligned_16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Returns 1 if the fast path ran, 0 if the shape/modes need the generic kernel, <0 on error.
int gemm_bf16_fast(const GemmArgs& g, hipStream_t s) {
  using namespace g2;
  if (g.precision != SMHIP_PREC_BF16) return 0;
  if (g.K % BK != 0 || g.K2 > 4 * BK) return 0;
  const int am = g.A.mode, bm = g.B.mode;
  const bool a_ok = am == SRC_BF16_K || am == SRC_BF16_R;
  const bool b_ok = bm == SRC_BF16_K || bm == SRC_BF16_R || bm == SRC_Q8_K || bm == SRC_Q8_R || bm == SRC_Q4K_K || bm == SRC_Q4K_R;
  if (!a_ok || !b_ok) return 0;
  // alignment of every vector load: rows of 16 B (bf16 K: ld%8; quant: ld%32; R-modes: 8-column groups)
  if (!aligned_16(g.A.p) || !aligned_16(g.B.p)) return 0;
  if (am == SRC_BF16_K && g.A.ld % 8) return 0;
  if (am == SRC_BF16_R && (g.A.ld % 8 || g.M % 8)) return 0;
  if ((bm == SRC_BF16_K) && g.B.ld % 8) return 0;
  if ((bm == SRC_BF16_R) && (g.B.ld % 8 || g.N % 8)) return 0;
  if (bm >= SRC_Q8_K && (g.B.ld % 32 || g.N % 8)) return 0;
  if (g.K2 > 0) {
    for (int m : {g.A2.mode, g.B2.mode})
      if (m != SRC_BF16_K && m != SRC_BF16_R && m != SRC_F32_K && m != SRC_F32_R) return 0;
  }
  Args a;
  a.A = {g.A.p, g.A.s, g.A.ld};
  a.B = {g.B.p, g.B.s, g.B.ld};
  a.A2 = {g.A2.p, g.A2.s, g.A2.ld};
  a.B2 = {g.B2.p, g.B2.s, g.B2.ld};
  a.amode2 = g.A2.mode;
  a.bmode2 = g.B2.mode;
  a.M = g.M; a.N = g.N; a.K = g.K; a.K2 = g.K2;
  a.alpha = g.alpha;
  a.alpha2 = g.alpha != 0.f ? g.alpha2 / g.alpha : 0.f;
  a.beta = g.beta;
  a.C = g.C; a.ldc = g.ldc;
  a.bias = g.bias; a.R = g.R; a.ldr = g.ldr;
  a.tiles_n = ceil_div(g.N, BN);
  // 256-row tiles when they still give >= 2 workgroups per CU worth of tiles
  const int t256 = ceil_div(g.M, 256) * a.tiles_n;
  const bool big = t256 >= 2 * num_cus();
  a.tiles_m = ceil_div(g.M, big ? 256 : 128);
  const int nk = g.K / BK;
  int sp = std::max(1, std::min(g.split_k, nk));
  a.kps = ceil_div(nk, sp);
  sp = ceil_div(nk, a.kps);
  a.partial = nullptr;
  if (sp > 1) {
    a.partial = (float*)workspace(s, sizeof(float) * (size_t)sp * g.M * g.N, 3);
    if (!a.partial) return fail(SMHIP_ENOMEM, "gemm: split-K workspace");
  }
  const int ev0 = prof_mark(s);
  const bool ok = big ? dispatch<256>(a, am, bm, g.c_bf16, sp, s) : dispatch<128>(a, am, bm, g.c_bf16, sp, s);
  if (!ok) return 0;
  SMHIP_CHECK_LAUNCH();
  prof_add(PROF_GEMM, ev0, prof_mark(s), 2.0 * g.M * g.N * ((double)g.K + g.K2), g.M, g.N, g.K + g.K2);
  if (sp > 1) {
    const int blocks = (int)std::min<int64_t>(((int64_t)g.M * g.N + 255) / 256, (int64_t)num_cus() * 8);
    hipLaunchKernelGGL(splitk_epilogue_kernel, dim3(blocks), dim3(256), 0, s, a.partial, sp, g.M, g.N, g.alpha,
                       g.beta, g.C, g.ldc, g.c_bf16, g.bias, g.R, g.ldr);
    SMHIP_CHECK_LAUNCH();
  }
  return 1;
}

}  // namespace smhip
