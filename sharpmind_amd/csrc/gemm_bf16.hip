// gemm_bf16.hip — bf16 MFMA GEMM for gfx950: split-K epilogues, tile / split choice and the
// operand checks of the fast path (the kernel template is in gemm_bf16.hpp, instantiated per
// B-operand mode by gemm_bf16_m*.hip).
#include "gemm_bf16.hpp"

namespace smhip {
namespace g3 {

thread_local hipEvent_t tl_ev0 = nullptr, tl_ev1 = nullptr;

// float4 form (N % 4 == 0, ldc / ldr % 4 == 0): 4 consecutive columns per thread, the
// partial loads of 8 splits in flight at once; sums still in ascending split order.
__device__ __forceinline__ void add4(float4& a, const float4& b) { a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w; }
__global__ void splitk_epilogue4_kernel(const float* __restrict__ partial, int splits, int M, int N, float alpha,
                                        float beta, void* __restrict__ Cp, int64_t ldc, int c_bf16,
                                        const float* __restrict__ bias, const float* __restrict__ R, int64_t ldr) {
  const int64_t n = (int64_t)M * N, n4 = n / 4;
  for (int64_t i4 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i4 < n4; i4 += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = 4 * i4;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k0 = 0; k0 < splits; k0 += 8) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (k0 + u < splits) v[u] = *reinterpret_cast<const float4*>(partial + (int64_t)(k0 + u) * n + i);
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (k0 + u < splits) add4(acc, v[u]);
    }
    const int64_t row = i / N, col = i - row * N;
    float o[4] = {alpha * acc.x, alpha * acc.y, alpha * acc.z, alpha * acc.w};
    if (bias) {
#pragma unroll
      for (int u = 0; u < 4; u++) o[u] = o[u] + bias[col + u];
    }
    if (c_bf16) {
      uint16_t* c = (uint16_t*)Cp + row * ldc + col;
      if (beta != 0.f) {
        const uint2 w = *reinterpret_cast<const uint2*>(c);
        o[0] = o[0] + beta * bf2f((uint16_t)(w.x & 0xFFFFu));
        o[1] = o[1] + beta * bf2f((uint16_t)(w.x >> 16));
        o[2] = o[2] + beta * bf2f((uint16_t)(w.y & 0xFFFFu));
        o[3] = o[3] + beta * bf2f((uint16_t)(w.y >> 16));
      }
      *reinterpret_cast<uint2*>(c) = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
    } else {
      float* c = (float*)Cp + row * ldc + col;
      if (R) {
        const float4 r = *reinterpret_cast<const float4*>(R + row * ldr + col);
        o[0] = o[0] + r.x; o[1] = o[1] + r.y; o[2] = o[2] + r.z; o[3] = o[3] + r.w;
      }
      if (beta != 0.f) {
        const float4 cv = *reinterpret_cast<const float4*>(c);
        o[0] = o[0] + beta * cv.x; o[1] = o[1] + beta * cv.y; o[2] = o[2] + beta * cv.z; o[3] = o[3] + beta * cv.w;
      }
      *reinterpret_cast<float4*>(c) = make_float4(o[0], o[1], o[2], o[3]);
    }
  }
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

// ---------------------------------------------------------------- host dispatch
// 256x256 runs 8 waves (2 x 4, each 128 x 64), 256x192 8 waves (4 x 2, each 64 x 96, for
// N = 3072: one tile per CU at M = 4096), 128x128W8 8 waves; the others 4.  64x128 and 128x64 are
// for skinny products (LoRA rank on one side), which are bandwidth-bound: many small
// workgroups plus split-K keep every CU streaming.
static bool dispatch(int tile, const Args& a, int amode, int bmode, int c_bf16, int sp, bool dx, hipStream_t s) {
  if (amode == SRC_BF16_K) {
    if (bmode == SRC_BF16_K) return dispatch_bf16k(tile, a, bmode, c_bf16, sp, dx, s);
    if (bmode == SRC_BF16_R) return dispatch_bf16r(tile, a, amode, bmode, c_bf16, sp, s);
    if (bmode == SRC_Q8_K || bmode == SRC_Q8T) return dispatch_q8(tile, a, bmode, c_bf16, sp, s);
    if (bmode == SRC_Q4K_K || bmode == SRC_Q4KT) return dispatch_q4k(tile, a, bmode, c_bf16, sp, s);
    if (bmode == SRC_Q8F || bmode == SRC_Q8FT || bmode == SRC_Q4F || bmode == SRC_Q4FT)
      return dispatch_q8f(tile, a, bmode, c_bf16, sp, dx, s);
    return false;
  }
  if (amode == SRC_BF16_R && bmode == SRC_BF16_R && (!c_bf16 || a.partial))
    return dispatch_bf16r(tile, a, amode, bmode, 0, sp, s);
  return false;
}

static bool skinny(int M, int N) { return M <= 64 || N <= 64; }
static int pick_tile(int M, int N, int splits, int bmode) {
  static const int forced = [] {  // SMHIP_GEMM_TILE=0..5 pins the tile shape (tuning runs)
    const char* v = getenv("SMHIP_GEMM_TILE");
    return v ? atoi(v) : -1;
  }();
  if (forced >= 0 && forced < NTILE && !(forced == T256x64 && N > 64)) return forced;
  if (M <= 64) return T64x128;
  if (N <= 64) return T128x64;
  const int cus = num_cus();
  int best = T128x128;
  double best_t = 1e300;
  for (int t : {T256x256, T256x128, T128x128, T256x64, T256x192}) {
    const TileInfo& ti = kTiles[t];
    if (t == T256x64 && N > 64) continue;
    const int64_t tiles = (int64_t)ceil_div(M, ti.bm) * ceil_div(N, ti.bn) * splits;
    const int64_t slots = (int64_t)cus * ti.occ;
    const double rounds = (double)((tiles + slots - 1) / slots);
    const double est = rounds * ti.occ * (double)ti.bm * ti.bn / ti.eff;
    if (est < best_t * 0.999) { best_t = est; best = t; }
  }
  return best;
}

}  // namespace g3

static bool aligned_16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// bytes spanned by an operand with rows x K elements (element width by mode)
static int64_t op_bytes(const Operand& o, int rows, int K, int64_t* sbytes) {
  *sbytes = 0;
  switch (o.mode) {
    case SRC_BF16_K: return ((int64_t)(rows - 1) * o.ld + K) * 2;
    case SRC_BF16_R: return ((int64_t)(K - 1) * o.ld + rows) * 2;
    case SRC_Q8_K: *sbytes = ((int64_t)(rows - 1) * o.ld + K) / 32 * 4; return (int64_t)(rows - 1) * o.ld + K;
    case SRC_Q8T: *sbytes = ((int64_t)((rows - 1) / 32) * o.ld + K) * 4; return (int64_t)(rows - 1) * o.ld + K;
    case SRC_Q4K_K: *sbytes = ((int64_t)(rows - 1) * o.ld + K) / 32 * 8; return ((int64_t)(rows - 1) * o.ld + K) / 2;
    case SRC_Q4KT: *sbytes = ((int64_t)((rows - 1) / 32) * o.ld + K) * 8; return ((int64_t)(rows - 1) * o.ld + K) / 2;
    case SRC_Q8F:
    case SRC_Q8FT: *sbytes = (int64_t)rows * o.ld / 16; return (int64_t)rows * o.ld;
    case SRC_Q4F:
    case SRC_Q4FT: *sbytes = (int64_t)rows * o.ld / 4; return (int64_t)rows * o.ld / 2;
    default: return -1;
  }
}

// Returns 1 if the fast path ran, 0 if the shape/modes need the generic kernel, <0 on error.
int gemm_bf16_fast(const GemmArgs& g, hipStream_t s) {
  using namespace g3;
  if (g.precision != SMHIP_PREC_BF16) return 0;
  if (g.K % BK != 0 || g.K2 > 4 * BK) return 0;
  const int am = g.A.mode, bm = g.B.mode;
  const bool a_ok = am == SRC_BF16_K || am == SRC_BF16_R;
  const bool frag = bm == SRC_Q8F || bm == SRC_Q8FT || bm == SRC_Q4F || bm == SRC_Q4FT;
  const bool b_ok = bm == SRC_BF16_K || bm == SRC_BF16_R || bm == SRC_Q8_K || bm == SRC_Q8T || bm == SRC_Q4K_K ||
                    bm == SRC_Q4KT || frag;
  if (!a_ok || !b_ok) return 0;
  // a side of at most 64 (the LoRA rank products): the bandwidth-bound skinny kernel
  if (g.K2 == 0 && !g.bias && !g.R && (g.N <= 64 || g.M <= 64) && (bm == SRC_BF16_K || bm == SRC_BF16_R)) {
    const int r = g.N <= 64
        ? gemm_skinny(g.M, g.N, g.K, g.A.p, g.A.ld, am == SRC_BF16_K, g.B.p, g.B.ld, bm == SRC_BF16_K, g.alpha,
                      g.beta, g.C, g.ldc, false, g.c_bf16 != 0, g.defer, s, SkinnyMask{}, g.hold)
        : gemm_skinny(g.N, g.M, g.K, g.B.p, g.B.ld, bm == SRC_BF16_K, g.A.p, g.A.ld, am == SRC_BF16_K, g.alpha,
                      g.beta, g.C, g.ldc, true, g.c_bf16 != 0, g.defer, s,
                      SkinnyMask{g.mask_cols, g.mask_rank, g.mask_nblk}, g.hold);
    if (r > 0 && g.M <= 64 && g.N > 64 && g.mask_cols && g.masked) *g.masked = 1;
    if (r != 0) return r;
  }
  if (am == SRC_BF16_R && bm != SRC_BF16_R) return 0;
  if (!aligned_16(g.A.p) || !aligned_16(g.B.p)) return 0;
  if (am == SRC_BF16_K && g.A.ld % 8) return 0;
  if (am == SRC_BF16_R && (g.A.ld % 8 || (uintptr_t)g.A.p % 16)) return 0;
  if (bm == SRC_BF16_K && g.B.ld % 8) return 0;
  if (bm == SRC_BF16_R && g.B.ld % 8) return 0;
  if ((bm == SRC_Q8_K || bm == SRC_Q8T || bm == SRC_Q4KT) && g.B.ld % 32) return 0;
  if (bm == SRC_Q4K_K && g.B.ld % 256) return 0;
  if ((bm == SRC_Q8T || bm == SRC_Q4KT) && !aligned_16(g.B.s)) return 0;
  // fragment planes: whole 32-row groups, the plane's K is the product's, A k-contiguous bf16
  if (frag && (g.B.ld != g.K || g.N % 32 || !aligned_16(g.B.s) || am != SRC_BF16_K)) return 0;
  if (g.K2 > 0) {
    for (int m : {g.A2.mode, g.B2.mode})
      if (m != SRC_BF16_K && m != SRC_BF16_R && m != SRC_F32_K && m != SRC_F32_R) return 0;
  }
  int64_t asb = 0, bsb = 0;
  const int64_t ab = op_bytes(g.A, g.M, g.K, &asb), bb = op_bytes(g.B, g.N, g.K, &bsb);
  // 32-bit buffer offsets: every operand (and any row beyond it) below 2 GiB
  const int64_t lim = (int64_t)1 << 31;
  if (ab < 0 || bb < 0 || ab + 256 * 4 * g.A.ld >= lim || bb + 256 * 4 * g.B.ld >= lim || bsb >= lim) return 0;

  Args a;
  a.A = {g.A.p, g.A.s, g.A.ld, (int)ab, 0};
  a.B = {g.B.p, g.B.s, g.B.ld, (int)bb, (int)bsb};
  a.A2 = {g.A2.p, g.A2.s, g.A2.ld, 0, 0};
  a.B2 = {g.B2.p, g.B2.s, g.B2.ld, 0, 0};
  a.amode2 = g.A2.mode;
  a.bmode2 = g.B2.mode;
  a.ext_vec = 0;
  if (g.K2 > 0 && g.K2 % 8 == 0) {
    bool ok = true;
    for (const Operand* o : {&g.A2, &g.B2})
      ok = ok && (o->mode == SRC_BF16_K || o->mode == SRC_BF16_R) && o->ld % 8 == 0 && aligned_16(o->p);
    // row-contiguous chunks are 8 rows wide: the row count must not end inside one
    if (g.A2.mode == SRC_BF16_R && g.M % 8) ok = false;
    if (g.B2.mode == SRC_BF16_R && g.N % 8) ok = false;
    a.ext_vec = ok ? 1 : 0;
  }
  a.M = g.M; a.N = g.N; a.K = g.K; a.K2 = g.K2;
  a.alpha = g.alpha;
  a.alpha2 = g.alpha != 0.f ? g.alpha2 / g.alpha : 0.f;
  a.beta = g.beta;
  a.C = g.C; a.ldc = g.ldc;
  a.bias = g.bias; a.R = g.R; a.ldr = g.ldr;
  const int nk = g.K / BK;
  int sp = std::max(1, std::min(g.split_k, nk));
  int tile;
  if (frag) {
    // fragment-plane B: 128x128 tiles (4 MFMA waves, 4 decoder waves, 2 loader waves); split-K
    // only to fill the machine
    tile = T128x128;
    const int64_t tiles = (int64_t)ceil_div(g.M, kTiles[tile].bm) * ceil_div(g.N, kTiles[tile].bn);
    sp = 1;
    if (g.split_k > 0) sp = std::max(1, std::min(g.split_k, nk));
    else if (tiles < num_cus()) sp = (int)std::max<int64_t>(1, std::min<int64_t>((num_cus() + tiles - 1) / tiles, nk / 8));
    while (sp > 1 && (int64_t)sp * g.M * g.N * 4 > ((int64_t)64 << 20)) sp--;
    a.kps = ceil_div(nk, sp);
    sp = ceil_div(nk, a.kps);
  } else if (g.split_k <= 0) {
    // automatic split-K: fill the machine (2 workgroups per CU slot for skinny, bandwidth-bound
    // products), keep >= 8 (skinny: 2) K tiles per split and the partials under 64 MiB
    tile = pick_tile(g.M, g.N, 1, bm);
    const bool sk = skinny(g.M, g.N);
    // at most one 128x128 tile per CU and a moderate K: the 8-wave tile (two waves per SIMD
    // hide LDS and barrier latency) with a ring, whole K per workgroup, beats split-K
    // (k-contiguous operands only: with a row-contiguous operand split-K measured faster)
    const bool w8 = tile == T128x128 && am == SRC_BF16_K && bm == SRC_BF16_K && !sk &&
                    (int64_t)ceil_div(g.M, 128) * ceil_div(g.N, 128) <= num_cus() && nk < 96;
    if (w8) tile = T128x128W8;
    const int64_t tiles = (int64_t)ceil_div(g.M, kTiles[tile].bm) * ceil_div(g.N, kTiles[tile].bn);
    const int64_t target = (int64_t)num_cus() * kTiles[tile].occ * (sk ? 2 : 1);
    sp = 1;
    if (tiles < target && !w8) {
      sp = (int)std::min<int64_t>((target + tiles - 1) / tiles, nk / (sk ? 2 : 8));
      sp = std::max(1, std::min(sp, 64));
      if (!sk) {
        // fewest rounds of resident workgroups per unit of K work; ties go to fewer splits (less
        // partial traffic).  E.g. 192 tiles: 2 splits fill 384 of 512 slots in one round, 3 need
        // two rounds (measured 46 against 53 us for the down-projection weight gradient)
        int best = 1;
        double best_c = 1e300;
        for (int c = 1; c <= sp; c++) {
          const double cost = (double)((tiles * c + target - 1) / target) / c;
          if (cost < best_c * 0.999) { best_c = cost; best = c; }
        }
        sp = best;
      }
      while (sp > 1 && (int64_t)sp * g.M * g.N * 4 > ((int64_t)64 << 20)) sp--;
    }
    a.kps = ceil_div(nk, sp);
    sp = ceil_div(nk, a.kps);
  } else {
    a.kps = ceil_div(nk, sp);
    sp = ceil_div(nk, a.kps);
    tile = pick_tile(g.M, g.N, sp, bm);
  }
  a.tiles_m = ceil_div(g.M, kTiles[tile].bm);
  a.tiles_n = ceil_div(g.N, kTiles[tile].bn);
  a.partial = nullptr;
  a.rowstat = g.rowstat;
  if (g.rowstat) {
    SMHIP_REQUIRE(frag && sp == 1 && g.K2 == 0 && !g.c_bf16 && !g.bias && !g.R && g.beta == 0.f && g.M % 128 == 0 &&
                      g.N % 128 == 0 && (int64_t)a.tiles_m * a.tiles_n >= 4 * num_cus(),
                  "gemm: softmax row statistics need the persistent fragment-plane form (fp32 C, whole tiles, "
                  "at least four per CU, no extension)");
  }
  if (sp > 1) {
    a.partial = (float*)workspace(s, sizeof(float) * (size_t)sp * g.M * g.N, 3);
    if (!a.partial) return fail(SMHIP_ENOMEM, "gemm: split-K workspace");
  }
  int ev0 = -1, ev1 = -1;
  if (!prof_reserve(&ev0, &ev1, &tl_ev0, &tl_ev1)) tl_ev0 = tl_ev1 = nullptr;
  const bool ok = dispatch(tile, a, am, bm, g.c_bf16, sp, g.prof_cat == PROF_GEMM_DX || bm == SRC_Q8FT || bm == SRC_Q4FT, s);
  tl_ev0 = tl_ev1 = nullptr;
  if (!ok) return 0;
  SMHIP_CHECK_LAUNCH();
  prof_add(g.prof_cat ? g.prof_cat : (bm == SRC_Q8T || bm == SRC_Q4KT || bm == SRC_Q8FT || bm == SRC_Q4FT ? PROF_GEMM_DX : PROF_GEMM), ev0, ev1,
           2.0 * g.M * g.N * ((double)g.K + g.K2), g.M, g.N, g.K + g.K2);
  if (sp > 1) {
    const bool v4 = g.N % 4 == 0 && g.ldc % 4 == 0 && (!g.R || g.ldr % 4 == 0) && aligned_16(g.C) &&
                    (!g.R || aligned_16(g.R));
    const int64_t work = v4 ? (int64_t)g.M * g.N / 4 : (int64_t)g.M * g.N;
    const int blocks = (int)std::min<int64_t>((work + 255) / 256, (int64_t)num_cus() * 8);
    if (v4)
      hipLaunchKernelGGL(splitk_epilogue4_kernel, dim3(blocks), dim3(256), 0, s, a.partial, sp, g.M, g.N, g.alpha,
                         g.beta, g.C, g.ldc, g.c_bf16, g.bias, g.R, g.ldr);
    else
      hipLaunchKernelGGL(splitk_epilogue_kernel, dim3(blocks), dim3(256), 0, s, a.partial, sp, g.M, g.N, g.alpha,
                         g.beta, g.C, g.ldc, g.c_bf16, g.bias, g.R, g.ldr);
    SMHIP_CHECK_LAUNCH();
  }
  return 1;
}

}  // namespace smhip
