// gemm_bf16_mq8f.hip — bf16 MFMA GEMM whose B operand is a frozen Q8_0 base held as fragment
// planes (SRC_Q8F: B = W for y = x W^T; SRC_Q8FT: B = W^T for dX = dY W).  The base is never
// expanded in HBM: its int8 codes (1 byte per weight) and fp16 block scales are copied straight
// into LDS (buffer_load ... lds, no registers), and each K tile is decoded once per workgroup,
// to the exact fp32 weight q*d rounded once to bf16 (the value the dense path would hold), into
// a bf16 tile of the layout the MFMA fragment reads expect.
//
// Warp-specialised workgroup: NWM MFMA waves own the output tile (as in the dense 8-wave 128x128
// kernel) and never touch global memory in the main loop; NWP producer waves issue every LDS copy
// (A tile, codes, scales) and decode.  With one producer wave per SIMD, the decode's VALU work
// runs beside the MFMA waves' matrix instructions instead of between them.  Per K tile t (one
// barrier each): MFMA waves multiply A(t) by decoded B(t); producers start the copies of tile
// t+ST-1, decode B(t+1) into the other bf16 buffer and wait for tile t+2 to land.  A decode unit
// is 8 consecutive k of one B row: one ds_read_b64 of codes, one shared read of the scales,
// v_cvt_f32_i32 with a sign-extending byte select, v_fma_mix_f32 with the fp16 scale operand
// (exact product), v_cvt_pk_bf16_f32, one 16-byte store at the row's swizzled slot; a wave's
// reads and stores each cover whole 128-byte LDS rows (no bank conflicts).
#include "gemm_bf16.hpp"

namespace smhip {
namespace g3 {

// exact q * s for an fp16 scale in the low / high half of s (the product fits in fp32)
__device__ __forceinline__ float mix_lo(float q, uint32_t s) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(q), "v"(s));
  return r;
}
__device__ __forceinline__ float mix_hi(float q, uint32_t s) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(q), "v"(s));
  return r;
}
// signed byte B of w as float: one v_cvt_f32_i32 with a sign-extending byte select (written out:
// left to itself the compiler hoists shifts and bit-field extracts into the loop)
template <int B>
__device__ __forceinline__ float i8f(uint32_t w) {
  float r;
  if constexpr (B == 0) asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
  else if constexpr (B == 1) asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
  else if constexpr (B == 2) asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
  else asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
  return r;
}
__device__ __forceinline__ void wait_lgkm() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Loader-side copies.  p = loader thread index (0 .. 64*NWP-1).
// A: bf16 k-contiguous rows, 1 KiB direct copies (8 rows x 128 bytes), each lane fetching the
// global chunk that belongs at its swizzled slot (as DmaLoad).
template <int ROWS, int NWP>
struct ProdA {
  static constexpr int NI = ROWS / 8 / NWP;
  static_assert((ROWS / 8) % NWP == 0, "A copies must split evenly over the producer waves");
  uint32_t off[NI];
  __amdgpu_buffer_rsrc_t rs;
  __device__ __forceinline__ void init(const Op& o, int r0, int R, int p) {
    rs = rsrc(o.p, o.bytes);
    const int w = p >> 6, l = p & 63;
#pragma unroll
    for (int j = 0; j < NI; j++) {
      const int r = (j * NWP + w) * 8 + (l >> 3);
      const int c = (l & 7) ^ ((r >> 1) & 7);
      off[j] = (r0 + r < R) ? (uint32_t)(((int64_t)(r0 + r) * o.ld) * 2 + c * 16) : OOB;
    }
  }
  __device__ __forceinline__ void fetch(uint8_t* tile, int k0, int p) {
#if defined(__HIP_DEVICE_COMPILE__)
    const int w = p >> 6;
#pragma unroll
    for (int j = 0; j < NI; j++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(tile + (j * NWP + w) * 1024), 16, off[j] + k0 * 2, 0, 0, 0);
#endif
  }
};

// B tile loader (NWL waves) and decoder (NWD waves) of the fragment planes.  Raw stage: BN*64
// code bytes in plane order, then one 256-byte scale slice per loader wave (BN*4 bytes used:
// 128 bytes per 32 B rows).
template <int BN, int NWL, int NWD, bool TRANS>
struct FragQ8 {
  static constexpr int NW = NWL;
  static constexpr int NC = BN / 16;  // 1 KiB code copies per tile
  static_assert(NC % NW == 0, "code copies must split evenly over the waves");
  static constexpr int NI = NC / NW;
  static constexpr int CODE = BN * 64;
  static constexpr int SCB = NW * 256;
  static_assert(BN * 4 <= SCB, "scale slice too small");
  static constexpr int STAGE = CODE + SCB;
  static constexpr int PER = NI + 1;               // LDS copies per loader wave per tile
  static constexpr int UPT = BN * 8 / (64 * NWD);  // decode units (8 weights) per decoder thread per tile
  static_assert(UPT >= 1 && UPT <= 8, "decode units per thread");
  uint32_t coff[NI], soff;
  __amdgpu_buffer_rsrc_t rc, rs;
  struct Raw {
    u32x2 c;
    u32x4 s;
  };

  __device__ __forceinline__ void init(const Op& o, int n0, int N, int p) {
    rc = rsrc(o.p, o.bytes);
    rs = rsrc(o.s, o.sbytes);
    const int w = p >> 6, l = p & 63;
    const int K = (int)o.ld;
#pragma unroll
    for (int j = 0; j < NI; j++) {
      const int jj = j * NW + w, nb = n0 / 32 + jj / 2;
      coff[j] = nb < N / 32 ? (uint32_t)((int64_t)nb * (K / 16) * 512 + (jj & 1) * 1024 + l * 16) : OOB;
    }
    const int b = w * 256 + l * 4, nbl = b >> 7, nb = n0 / 32 + nbl;
    soff = (nbl < BN / 32 && nb < N / 32) ? (uint32_t)((int64_t)nb * K * 2 + (b & 127)) : OOB;
  }
  __device__ __forceinline__ void fetch(uint8_t* st, int k0, int p) {
#if defined(__HIP_DEVICE_COMPILE__)
    const int w = p >> 6;
#pragma unroll
    for (int j = 0; j < NI; j++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (lds_void*)(st + (j * NW + w) * 1024), 16, coff[j] + k0 * 32, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(st + CODE + w * 256), 4, soff + k0 * 2, 0, 0, 0);
#endif
  }
  // unit j of decoder thread p: 8 consecutive k (chunk l%8) of B row 8*(j*NWD + w) + l/8; a wave's
  // 64 lanes read 512 contiguous code bytes and store two whole 128-byte LDS rows per 16 lanes
  // (conflict-free both ways)
  __device__ __forceinline__ Raw read(const uint8_t* st, int j, int p) const {
    const int w = p >> 6, l = p & 63;
    const int g = j * NWD + w, nbl = g >> 2, ch = l & 7;
    Raw r;
    r.c = *reinterpret_cast<const u32x2*>(st + g * 512 + l * 8);
    if constexpr (TRANS) {
      r.s = *reinterpret_cast<const u32x4*>(st + CODE + nbl * 128 + ch * 16);
    } else {
      r.s[0] = *reinterpret_cast<const uint16_t*>(st + CODE + nbl * 128 + ((ch >> 2) * 32 + (g & 3) * 8 + (l >> 3)) * 2);
    }
    return r;
  }
  __device__ __forceinline__ void write(const Raw& r, uint8_t* bf, int j, int p) const {
    const int w = p >> 6, l = p & 63;
    const int g = j * NWD + w;
    const float q[8] = {i8f<0>(r.c[0]), i8f<1>(r.c[0]), i8f<2>(r.c[0]), i8f<3>(r.c[0]),
                        i8f<0>(r.c[1]), i8f<1>(r.c[1]), i8f<2>(r.c[1]), i8f<3>(r.c[1])};
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      if constexpr (TRANS) f[i] = (i & 1) ? mix_hi(q[i], r.s[i >> 1]) : mix_lo(q[i], r.s[i >> 1]);
      else f[i] = mix_lo(q[i], r.s[0]);
    }
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = pk(f[2 * i], f[2 * i + 1]);
    *reinterpret_cast<u32x4*>(bf + sw(g * 8 + (l >> 3), l & 7)) = o;
  }
  __device__ __forceinline__ void decode(const uint8_t* st, uint8_t* bf, int p) const {
    Raw r[UPT];
#pragma unroll
    for (int j = 0; j < UPT; j++) r[j] = read(st, j, p);
#pragma unroll
    for (int j = 0; j < UPT; j++) write(r[j], bf, j, p);
  }
};

// rank-extension staging: the vectorised forms, or (GEN instantiations, operands the engine never
// passes) the element-wise general form, whose register demand would otherwise shape the kernel's
template <int ROWS, int NT, bool GEN>
__device__ __forceinline__ void ext_stage(int mode, const Op& o, int r0, int k0, int R, int K, float mult, uint8_t* lds) {
  if constexpr (GEN) gen_tile<ROWS, NT>(mode, o, r0, k0, R, K, mult, lds);
  else if (mode == SRC_BF16_K) ext_tile_k<ROWS, NT>(o, r0, k0, R, K, mult, lds, threadIdx.x);
  else ext_tile_r<ROWS, NT>(o, r0, k0, R, K, mult, lds, threadIdx.x);
}

// Q4_K fragment planes: raw stage = BN*32 code bytes (32 per row of a 32 x 64 block) and BN*16
// bytes of (sc*d, mn*dmin) fp32 pairs (512 bytes per 32 B rows).  A decode unit is one code
// dword (8 consecutive k of a row: low nibbles k..k+3, high nibbles k+4..k+7); the weight is
// fma(sc*d, v, -mn*dmin), one rounding of the exact (sc*d)*v - mn*dmin, which is the value the
// reference forms.
template <int BN, int NWL, int NWD, bool TRANS>
struct FragQ4 {
  static constexpr int NW = NWL;
  static constexpr int NC = BN / 32;  // 1 KiB code copies per tile (one per 32 B rows)
  static_assert(NC % NW == 0, "code copies must split evenly over the waves");
  static constexpr int NI = NC / NW;
  static constexpr int CODE = BN * 32;
  static constexpr int NS = BN / 64;  // 1 KiB pair copies per tile
  static_assert(NS % NW == 0, "pair copies must split evenly over the waves");
  static constexpr int NIS = NS / NW;
  static constexpr int STAGE = CODE + BN * 16;
  static constexpr int PER = NI + NIS;
  static constexpr int UPT = BN * 8 / (64 * NWD);
  static_assert(UPT >= 1 && UPT <= 8, "decode units per thread");
  uint32_t coff[NI], soff[NIS];
  __amdgpu_buffer_rsrc_t rc, rs;
  struct Raw {
    uint32_t c;
    u32x4 s[4];  // TRANS: 8 (s, m) pairs; otherwise one pair in s[0].xy
  };
  __device__ __forceinline__ void init(const Op& o, int n0, int N, int p) {
    rc = rsrc(o.p, o.bytes);
    rs = rsrc(o.s, o.sbytes);
    const int w = p >> 6, l = p & 63;
    const int K = (int)o.ld;
#pragma unroll
    for (int j = 0; j < NI; j++) {
      const int nb = n0 / 32 + j * NW + w;
      coff[j] = nb < N / 32 ? (uint32_t)((int64_t)nb * (K / 64) * 1024 + l * 16) : OOB;
    }
#pragma unroll
    for (int j = 0; j < NIS; j++) {
      const int b = (j * NW + w) * 1024 + l * 16, nb = n0 / 32 + b / 512;
      soff[j] = nb < N / 32 ? (uint32_t)((int64_t)nb * K * 8 + (b & 511)) : OOB;
    }
  }
  __device__ __forceinline__ void fetch(uint8_t* st, int k0, int p) {
#if defined(__HIP_DEVICE_COMPILE__)
    const int w = p >> 6;
#pragma unroll
    for (int j = 0; j < NI; j++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (lds_void*)(st + (j * NW + w) * 1024), 16, coff[j] + k0 * 16, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < NIS; j++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(st + CODE + (j * NW + w) * 1024), 16, soff[j] + k0 * 8, 0, 0, 0);
#endif
  }
  __device__ __forceinline__ Raw read(const uint8_t* st, int j, int p) const {
    const int w = p >> 6, l = p & 63;
    const int g = j * NWD + w, nbl = g >> 2, ch = l & 7;
    Raw r;
    r.c = *reinterpret_cast<const uint32_t*>(st + g * 256 + l * 4);
    if constexpr (TRANS) {
#pragma unroll
      for (int i = 0; i < 4; i++) r.s[i] = *reinterpret_cast<const u32x4*>(st + CODE + nbl * 512 + ch * 64 + i * 16);
    } else {
      const u32x2 pr = *reinterpret_cast<const u32x2*>(st + CODE + nbl * 512 + ((ch >> 2) * 32 + (g & 3) * 8 + (l >> 3)) * 8);
      r.s[0][0] = pr[0];
      r.s[0][1] = pr[1];
    }
    return r;
  }
  __device__ __forceinline__ void write(const Raw& r, uint8_t* bf, int j, int p) const {
    const int w = p >> 6, l = p & 63;
    const int g = j * NWD + w;
    const uint32_t lo = r.c & 0x0F0F0F0Fu, hi = (r.c >> 4) & 0x0F0F0F0Fu;
    const float v[8] = {(float)(lo & 0xFFu), (float)((lo >> 8) & 0xFFu), (float)((lo >> 16) & 0xFFu), (float)(lo >> 24),
                        (float)(hi & 0xFFu), (float)((hi >> 8) & 0xFFu), (float)((hi >> 16) & 0xFFu), (float)(hi >> 24)};
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      float sc, mn;
      if constexpr (TRANS) {
        sc = as_f(r.s[i >> 1][(i & 1) * 2]);
        mn = as_f(r.s[i >> 1][(i & 1) * 2 + 1]);
      } else {
        sc = as_f(r.s[0][0]);
        mn = as_f(r.s[0][1]);
      }
      f[i] = __builtin_fmaf(sc, v[i], -mn);
    }
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = pk(f[2 * i], f[2 * i + 1]);
    *reinterpret_cast<u32x4*>(bf + sw(g * 8 + (l >> 3), l & 7)) = o;
  }
  __device__ __forceinline__ void decode(const uint8_t* st, uint8_t* bf, int p) const {
    Raw r[UPT];
#pragma unroll
    for (int j = 0; j < UPT; j++) r[j] = read(st, j, p);
#pragma unroll
    for (int j = 0; j < UPT; j++) write(r[j], bf, j, p);
  }
};

// Epilogue of a transposed accumulator tile (STAT): block acc[i][j] holds rows wm*WM + i*32 +
// lane%32 of C and its columns wn*WN + j*32 + acc_row(e).  C = alpha * acc is stored 16 bytes at a
// time, and each (row, 64 columns of the wave) gets its softmax statistics: the lane's 32 values
// and those of lane ^ 32 (the other half of the columns) give (max, sum exp(c - max)) with the
// hardware exponential.
template <class S>
__device__ __forceinline__ void stat_epilogue(const Args& g, floatx16 (&acc)[S::MB][S::NB], int m0, int n0) {
  static_assert(S::WN == 64, "one statistics pair per wave and row");
  constexpr int MB = S::MB, NB = S::NB;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wm = wv / S::WGN, wn = wv % S::WGN;
  const int nst = g.N / 64;
#pragma unroll
  for (int i = 0; i < MB; i++) {
    const int64_t row = m0 + wm * S::WM + i * 32 + (lane & 31);
    float* crow = (float*)g.C + row * g.ldc + n0 + wn * S::WN + (lane >> 5) * 4;
    float mx = -INFINITY;
    if (g.alpha != 1.f) {
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[i][j][e] *= g.alpha;
    }
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) mx = fmaxf(mx, acc[i][j][e]);
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int q = 0; q < 4; q++)
        *reinterpret_cast<float4*>(crow + j * 32 + q * 8) =
            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float sm = 0.f;
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) sm += __expf(acc[i][j][e] - mx);
    sm += __shfl_xor(sm, 32, 64);
    if (lane < 32) *reinterpret_cast<float2*>(g.rowstat + (row * nst + n0 / 64 + wn) * 2) = make_float2(mx, sm);
  }
}

template <int BM, int BN, int WGM, int NWM, int NWD, int NWL, bool TRANS, bool C_BF16, int ST, int TAG, bool FULL, bool GEN,
          bool Q4, bool PERS = false, bool STAT = false>
__global__ __launch_bounds__(64 * (NWM + NWD + NWL), 1) void gemm_q8f_kernel(Args g) {
  using S = Shape<BM, BN, WGM, NWM>;  // the MFMA waves' layout (epilogue included)
  constexpr int MB = S::MB, NB = S::NB, NT = 64 * (NWM + NWD + NWL);
  constexpr int LW = NWL ? NWL : NWM;  // NWL = 0: the MFMA waves issue the copies
  using LA = ProdA<BM, LW>;
  using LB = typename std::conditional<Q4, FragQ4<BN, LW, NWD, TRANS>, FragQ8<BN, LW, NWD, TRANS>>::type;
  static_assert(ST >= 3, "the loaders run two tiles ahead of the MFMA waves");
  constexpr int RAW = BM * 128 + LB::STAGE;
  constexpr int LDS = ST * RAW + 2 * BN * 128;
  static_assert(LDS <= 160 * 1024, "LDS budget");
  constexpr int PER = LA::NI + LB::PER;  // copies per loader wave per tile
  __shared__ __attribute__((aligned(1024))) uint8_t smem[LDS];
  auto sA = [&](int st) -> uint8_t* { return smem + st * RAW; };
  auto sQ = [&](int st) -> uint8_t* { return smem + st * RAW + BM * 128; };
  auto sB = [&](int b) -> uint8_t* { return smem + ST * RAW + b * (BN * 128); };

  const int ntiles = g.tiles_m * g.tiles_n;
  const int wg = blockIdx.x;
  // linear index -> tile origin: launch order i goes to XCD i % 8, each XCD owning a contiguous
  // band of tiles, swept GM m-panels at a time
  auto tile_origin = [&](int lin, int& om0, int& on0) {
    int tile = lin;
    if (ntiles % 8 == 0) tile = (lin % 8) * (ntiles / 8) + lin / 8;
    constexpr int GM = 8;
    const int group = tile / (GM * g.tiles_n);
    const int first_m = group * GM;
    const int gsz = min(g.tiles_m - first_m, GM);
    om0 = (first_m + (tile % (GM * g.tiles_n)) % gsz) * BM;
    on0 = ((tile % (GM * g.tiles_n)) / gsz) * BN;
  };
  int m0, n0;
  tile_origin(wg, m0, n0);

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  // wave-uniform roles: MFMA waves [0, NWM), decoders [NWM, NWM+NWD) (one per SIMD), loaders after
  const int role = wv < NWM ? 0 : (wv < NWM + NWD ? 1 : 2);
  const int pd = threadIdx.x - 64 * NWM, pl = NWL ? threadIdx.x - 64 * (NWM + NWD) : threadIdx.x;
  const int wm = wv / S::WGN, wn = wv % S::WGN;

  const int nk_all = g.K / BK;
  const int split = blockIdx.y, nsplit = gridDim.y;
  const int kt0 = split * g.kps;
  const int nk1 = max(0, min(nk_all, kt0 + g.kps) - kt0);
  const int nk2 = split == nsplit - 1 ? (g.K2 + BK - 1) / BK : 0;

  floatx16 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  // MFMA waves: the fragments of k slice kk+1 are read while the MFMAs of slice kk run
  auto compute = [&](const uint8_t* a, const uint8_t* b) {
    bf16x8 fa[2][MB], fb[2][NB];
    auto rd = [&](int kk, int q) {
      const int ch = 2 * kk + (lane >> 5);
#pragma unroll
      for (int i = 0; i < MB; i++) fa[q][i] = *reinterpret_cast<const bf16x8*>(a + sw(wm * S::WM + i * 32 + (lane & 31), ch));
#pragma unroll
      for (int j = 0; j < NB; j++) fb[q][j] = *reinterpret_cast<const bf16x8*>(b + sw(wn * S::WN + j * 32 + (lane & 31), ch));
    };
    rd(0, 0);
#pragma unroll
    for (int kk = 0; kk < BK / 16; kk++) {
      if (kk + 1 < BK / 16) rd(kk + 1, (kk + 1) & 1);
      __builtin_amdgcn_sched_barrier(0);
      const int q = kk & 1;
#pragma unroll
      for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) {
          // STAT: the transposed block (lane = one row of C, its 16 values along N), so a row's
          // softmax statistics are lane-local
          if constexpr (STAT) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[q][j], fa[q][i], acc[i][j], 0, 0, 0);
          else acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[q][i], fb[q][j], acc[i][j], 0, 0, 0);
        }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Three loops with the same barrier sequence: two before the first tile (raw tiles 0 and 1
  // landed; tile 0 decoded), one after each tile.  The loaders are the only waves with copies in
  // flight: an LDS copy also counts against the issuing wave's LDS counter, so a wave that waited
  // for its own LDS reads would drain the ring.
  if constexpr (PERS) {
    // Persistent form (no split; at most one rank-extension K tile, element-wise staging not
    // used): workgroup wg takes output tiles wg, wg + G, ... and runs their K tiles as one
    // sequence u = 0 .. ntl*sp-1 (sp = main K tiles + the extension tile, last), so the copies
    // and the decode of the next output tile are in flight while the MFMA waves store the
    // previous one.  The extension tile has no copies: the decoder waves stage its two operands
    // into the ring stage and the decoded buffer it would have used.  Every role passes the same
    // 2 + ntl*sp barriers.
    static_assert(NWL > 0 && ST == 4 && !GEN, "persistent form: loader waves, a 4-stage ring");
    const int G = gridDim.x;
    const int ntl = (ntiles - wg + G - 1) / G;
    const int nk = nk1, sp = nk1 + nk2, total = ntl * sp;
    auto is_ext = [&](int u) { return u % sp >= nk; };
    if (total > 0 && role == 2) {
      LA la;
      LB lb;
      auto fetch = [&](int u) {
        const int kt = u % sp;
        if (kt >= nk) return;
        if (kt == 0) {
          int fm0, fn0;
          tile_origin(wg + (u / sp) * G, fm0, fn0);
          la.init(g.A, fm0, g.M, pl);
          lb.init(g.B, fn0, g.N, pl);
        }
        la.fetch(sA(u % ST), kt * BK, pl);
        lb.fetch(sQ(u % ST), kt * BK, pl);
      };
      // steps up to v issued: step v - 1 (and older) landed; v itself may be in flight when it
      // has copies (loads complete in order)
      auto wait_upto = [&](int v) {
        if (v < total && !is_ext(v)) wait_vm_n<PER>();
        else wait_vm();
      };
#pragma unroll
      for (int u = 0; u < ST - 1; u++)
        if (u < total) fetch(u);
      wait_upto(ST - 2);
      ring_barrier();
      ring_barrier();
      for (int u = 0; u < total; u++) {
        if (u + ST - 1 < total) fetch(u + ST - 1);
        wait_upto(u + ST - 1);
        ring_barrier();
      }
    } else if (total > 0 && role == 1) {
      LB lb;
      auto prep = [&](int u) {  // step u's B tile (and, for the extension, its A tile)
        if (is_ext(u)) {
          int em0, en0;
          tile_origin(wg + (u / sp) * G, em0, en0);
          const int tid = pd, k0 = (u % sp - nk) * BK;
          if (g.amode2 == SRC_BF16_K) ext_tile_k<BM, 64 * NWD>(g.A2, em0, k0, g.M, g.K2, g.alpha2, sA(u % ST), tid);
          else ext_tile_r<BM, 64 * NWD>(g.A2, em0, k0, g.M, g.K2, g.alpha2, sA(u % ST), tid);
          if (g.bmode2 == SRC_BF16_K) ext_tile_k<BN, 64 * NWD>(g.B2, en0, k0, g.N, g.K2, 1.f, sB(u & 1), tid);
          else ext_tile_r<BN, 64 * NWD>(g.B2, en0, k0, g.N, g.K2, 1.f, sB(u & 1), tid);
        } else {
          lb.decode(sQ(u % ST), sB(u & 1), pd);
        }
        wait_lgkm();
      };
      ring_barrier();
      prep(0);
      ring_barrier();
      for (int u = 0; u < total; u++) {
        if (u + 1 < total) prep(u + 1);
        ring_barrier();
      }
    } else if (total > 0) {
      ring_barrier();
      ring_barrier();
      for (int u = 0; u < total; u++) {
        compute(sA(u % ST), sB(u & 1));
        if (u % sp == sp - 1) {
          int em0, en0;
          tile_origin(wg + (u / sp) * G, em0, en0);
          if constexpr (STAT) stat_epilogue<S>(g, acc, em0, en0);
          else gemm_epilogue<S, C_BF16, FULL>(g, acc, em0, en0, 0);
#pragma unroll
          for (int i = 0; i < MB; i++)
#pragma unroll
            for (int j = 0; j < NB; j++)
#pragma unroll
              for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;
        }
        ring_barrier();
      }
    }
    return;
  }
  // rank extension (LoRA) first, from stage 0 and decoded buffer 0: every thread stages, the MFMA
  // waves multiply.  The accumulators are live through the role loops that follow, which the
  // 168-register budget of a 10-wave workgroup holds without spilling.
  for (int t = 0; t < nk2; t++) {
    ext_stage<BM, NT, GEN>(g.amode2, g.A2, m0, t * BK, g.M, g.K2, g.alpha2, sA(0));
    ext_stage<BN, NT, GEN>(g.bmode2, g.B2, n0, t * BK, g.N, g.K2, 1.f, sB(0));
    __syncthreads();
    if (role == 0) compute(sA(0), sB(0));
    __syncthreads();
  }
  // copies of tiles 0 .. ST-2, then per tile t the copies of tile t+ST-1 and a wait for tile t+2
  // (decoded next, multiplied next-but-one)
  auto load_prologue = [&](LA& la, LB& lb) {
    la.init(g.A, m0, g.M, pl);
    lb.init(g.B, n0, g.N, pl);
#pragma unroll
    for (int t = 0; t < ST - 1; t++)
      if (t < nk1) {
        la.fetch(sA(t), (kt0 + t) * BK, pl);
        lb.fetch(sQ(t), (kt0 + t) * BK, pl);
      }
    if (nk1 >= ST - 1) wait_vm_n<(ST - 3) * PER>();  // tiles 0 and 1
    else wait_vm();
  };
  auto load_issue = [&](LA& la, LB& lb, int t) {
    if (t + ST - 1 < nk1) {
      const int st = (t + ST - 1) % ST;
      la.fetch(sA(st), (kt0 + t + ST - 1) * BK, pl);
      lb.fetch(sQ(st), (kt0 + t + ST - 1) * BK, pl);
    }
  };
  auto load_wait = [&](int t) {
    if (t + ST - 1 < nk1) wait_vm_n<(ST - 3) * PER>();
    else wait_vm();
  };
  if (nk1 > 0 && role == 2) {
    LA la;
    LB lb;
    load_prologue(la, lb);
    ring_barrier();
    ring_barrier();
    for (int t = 0; t < nk1; t++) {
      load_issue(la, lb, t);
      load_wait(t);
      ring_barrier();
    }
  } else if (nk1 > 0 && role == 1) {
    LB lb;
    ring_barrier();
    lb.decode(sQ(0), sB(0), pd);
    wait_lgkm();
    ring_barrier();
    for (int t = 0; t < nk1; t++) {
      if (t + 1 < nk1) {
        lb.decode(sQ((t + 1) % ST), sB((t + 1) & 1), pd);
        wait_lgkm();
      }
      ring_barrier();
    }
  } else if (nk1 > 0 && NWL == 0) {
    LA la;
    LB lb;
    load_prologue(la, lb);
    ring_barrier();
    ring_barrier();
    for (int t = 0; t < nk1; t++) {
      load_issue(la, lb, t);
      compute(sA(t % ST), sB(t & 1));
      load_wait(t);
      ring_barrier();
    }
  } else if (nk1 > 0) {
    ring_barrier();
    ring_barrier();
    for (int t = 0; t < nk1; t++) {
      compute(sA(t % ST), sB(t & 1));
      ring_barrier();
    }
  }
  // fp32 C with a residual (y = x W^T + R): every wave copies a share of the tile's R rows to
  // the now idle LDS ring with buffer_load ... lds before the epilogue, so the MFMA waves add R
  // from LDS (one coalesced burst per workgroup instead of a memory round trip per few
  // elements between the C stores)
  const float* rl = nullptr;
  if constexpr (!C_BF16) {
    if (g.R && g.beta == 0.f && !g.partial && m0 + BM <= g.M && n0 + BN <= g.N) {
      static_assert(BM * BN * 4 <= LDS, "residual tile fits the LDS ring");
      ring_barrier();  // every role is done with the ring
#if defined(__HIP_DEVICE_COMPILE__)
      const __amdgpu_buffer_rsrc_t rr =
          rsrc(g.R + (int64_t)m0 * g.ldr + n0, (int)(((int64_t)(BM - 1) * g.ldr + BN) * 4));
      constexpr int RPI = 1024 / (BN * 4);  // tile rows per 1 KiB copy
      constexpr int NI = BM / RPI;
      for (int i = wv; i < NI; i += NT / 64) {
        const int row = i * RPI + lane / (BN / 4), c4 = lane % (BN / 4);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void*)(smem + i * 1024), 16,
                                                 (uint32_t)((row * g.ldr + 4 * c4) * 4), 0, 0, 0);
      }
#endif
      wait_vm();
      ring_barrier();
      rl = reinterpret_cast<const float*>(smem);
    }
  }
  if (role == 0) gemm_epilogue<S, C_BF16, FULL>(g, acc, m0, n0, split, rl);
}

template <int BM, int BN, int WGM, int NWM, int NWD, int NWL, bool TRANS, int ST, int TAG, bool Q4>
static void launch_q8f_t(const Args& a, int c_bf16, int splits, hipStream_t s) {
  const dim3 grid(a.tiles_m * a.tiles_n, splits), block(64 * (NWM + NWD + NWL));
  const bool full = a.M % BM == 0 && a.N % BN == 0;
  const bool cb = c_bf16 && !a.partial;
  if (a.K2 > 0 && !a.ext_vec) {  // element-wise extension staging, general epilogue
    if (cb) launch_main(gemm_q8f_kernel<BM, BN, WGM, NWM, NWD, NWL, TRANS, true, ST, TAG, false, true, Q4>, grid, block, s, a);
    else launch_main(gemm_q8f_kernel<BM, BN, WGM, NWM, NWD, NWL, TRANS, false, ST, TAG, false, true, Q4>, grid, block, s, a);
  } else if (a.rowstat) {  // the caller checked the conditions of the persistent form, fp32 C
    const dim3 pgrid(num_cus() / 8 * 8);
    launch_main(gemm_q8f_kernel<BM, BN, WGM, NWM, NWD, NWL, TRANS, false, ST, TAG, true, false, Q4, true, true>, pgrid, block, s, a);
  } else if (full && a.K2 <= BK && splits == 1 && !a.partial && a.tiles_m * a.tiles_n >= 4 * num_cus()) {
    // many tiles per CU: the persistent form, one workgroup per CU
    const dim3 pgrid(num_cus() / 8 * 8);
    if (cb) launch_main(gemm_q8f_kernel<BM, BN, WGM, NWM, NWD, NWL, TRANS, true, ST, TAG, true, false, Q4, true>, pgrid, block, s, a);
    else launch_main(gemm_q8f_kernel<BM, BN, WGM, NWM, NWD, NWL, TRANS, false, ST, TAG, true, false, Q4, true>, pgrid, block, s, a);
  } else if (full) {
    if (cb) launch_main(gemm_q8f_kernel<BM, BN, WGM, NWM, NWD, NWL, TRANS, true, ST, TAG, true, false, Q4>, grid, block, s, a);
    else launch_main(gemm_q8f_kernel<BM, BN, WGM, NWM, NWD, NWL, TRANS, false, ST, TAG, true, false, Q4>, grid, block, s, a);
  } else {
    if (cb) launch_main(gemm_q8f_kernel<BM, BN, WGM, NWM, NWD, NWL, TRANS, true, ST, TAG, false, false, Q4>, grid, block, s, a);
    else launch_main(gemm_q8f_kernel<BM, BN, WGM, NWM, NWD, NWL, TRANS, false, ST, TAG, false, false, Q4>, grid, block, s, a);
  }
}
template <int BM, int BN, int WGM, int NWM, int NWD, int NWL, bool TRANS, int ST, bool Q4>
static void launch_q8f(const Args& a, int c_bf16, int splits, bool dx, hipStream_t s) {
  if (dx) launch_q8f_t<BM, BN, WGM, NWM, NWD, NWL, TRANS, ST, 1, Q4>(a, c_bf16, splits, s);
  else launch_q8f_t<BM, BN, WGM, NWM, NWD, NWL, TRANS, ST, 0, Q4>(a, c_bf16, splits, s);
}

// One shape: 128x128 output tiles, 4 MFMA waves of 64x64 (2x2), 4 decoder waves (one per SIMD),
// 2 loader waves; a 4-stage ring of raw tiles and two decoded tiles (132 KiB of LDS).  Larger
// tiles would halve the decode work per MFMA but need more than the 168 registers per lane that
// a workgroup of 10 waves leaves (measured: the 8-MFMA-wave 256x128 form spills).
bool dispatch_q8f(int tile, const Args& a, int bmode, int c_bf16, int sp, bool dx, hipStream_t s) {
  if (tile != T128x128) return false;
  switch (bmode) {
    case SRC_Q8FT: launch_q8f<128, 128, 2, 4, 4, 2, true, 4, false>(a, c_bf16, sp, dx, s); return true;
    case SRC_Q8F: launch_q8f<128, 128, 2, 4, 4, 2, false, 4, false>(a, c_bf16, sp, dx, s); return true;
    case SRC_Q4FT: launch_q8f<128, 128, 2, 4, 4, 2, true, 4, true>(a, c_bf16, sp, dx, s); return true;
    case SRC_Q4F: launch_q8f<128, 128, 2, 4, 4, 2, false, 4, true>(a, c_bf16, sp, dx, s); return true;
    default: return false;
  }
}

}  // namespace g3
}  // namespace smhip
