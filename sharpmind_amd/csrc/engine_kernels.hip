// engine_kernels.hip — fused elementwise kernels used by the training engine.
//
//  * qk_norm + RoPE forward / backward on the fused q|k|v projection output
//    (per-head RMSNorm as in AttentionLayer.cs:284, then RoPE.cs:168-259; the
//    backward is RoPE.cs:300-347 followed by the RMSNorm-slot formula
//    GradientKernels.cs:303-337 applied per head row);
//  * SwiGLU forward/backward on the fused [gate | up] row layout
//    (BackpropEngine.cs:409-431 forward, :623-657 backward);
//  * LoRA block-diagonal gradient masking, global-norm clipping
//    (Gradients.cs:92-116), bf16 shadow casts;
//  * synthetic initialisation: a counter-based normal generator and the
//    Q8_0 / Q4_K encoders of TensorQuantizer (TensorQuantizer.cs:80-144,
//    TensorQuantizer.KQuant.cs:173-225,451-459) so quantised bases are built
//    on the device with the reference's exact bytes.
#include "common.hpp"
#include "kernels.hpp"

namespace smhip {

template <typename T> __device__ inline void st(T* p, float v);
template <> __device__ inline void st<float>(float* p, float v) { *p = v; }
template <> __device__ inline void st<uint16_t>(uint16_t* p, float v) { *p = f2bf(v); }
template <typename T> __device__ inline float ldv(const T* p);
template <> __device__ inline float ldv<float>(const float* p) { return *p; }
template <> __device__ inline float ldv<uint16_t>(const uint16_t* p) { return bf2f(*p); }

static int gridn(int64_t n, int per = 256, int cap = 8) {
  int64_t g = (n + per - 1) / per;
  int64_t c = (int64_t)num_cus() * cap;
  return (int)std::max<int64_t>(1, std::min(g, c));
}

// ============================================================================
// q/k/v split + optional per-head RMSNorm + RoPE.  One wave per (token, head) row;
// rows 0..Hq-1 are query heads, Hq..Hq+Hkv-1 key heads, then Hkv value heads.
// ============================================================================
template <typename TA>
__global__ __launch_bounds__(256) void qkv_prep_fwd_kernel(
    const float* __restrict__ qkv, TA* __restrict__ qo, TA* __restrict__ ko, TA* __restrict__ vo,
    float* __restrict__ rinv, const float* __restrict__ wq, const float* __restrict__ wk,
    const float* __restrict__ cosT, const float* __restrict__ sinT, int T, int S, int Hq, int Hkv,
    int D, int qk_norm, int neox, float eps) {
  const int lane = threadIdx.x & 63;
  const int H = Hq + 2 * Hkv, nqkv = H * D;
  const int64_t rows = (int64_t)T * H;
  const int pairs = D / 2;
  for (int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += (int64_t)gridDim.x * 4) {
    const int t = (int)(r / H), hh = (int)(r % H);
    const float* x = qkv + (int64_t)t * nqkv + hh * D;
    if (hh >= Hq + Hkv) {  // value head: copy
      TA* dst = vo + (int64_t)t * Hkv * D + (hh - Hq - Hkv) * D;
      for (int d = lane; d < D; d += 64) st(dst + d, x[d]);
      continue;
    }
    const bool isq = hh < Hq;
    const float* w = isq ? wq : wk;
    TA* dst = isq ? qo + (int64_t)t * Hq * D + hh * D : ko + (int64_t)t * Hkv * D + (hh - Hq) * D;
    float ri = 1.f;
    if (qk_norm) {
      float ss = 0.f;
      for (int d = lane; d < D; d += 64) ss += x[d] * x[d];
      ss = wave_sum(ss);
      ri = 1.f / sqrtf(ss / (float)D + eps);
      if (lane == 0) rinv[(int64_t)t * (Hq + Hkv) + hh] = ri;
    }
    const int pos = t % S;
    for (int p = lane; p < pairs; p += 64) {
      const int i0 = neox ? p : 2 * p, i1 = neox ? p + pairs : 2 * p + 1;
      float a = x[i0], b = x[i1];
      if (qk_norm) {
        a = a * ri * w[i0];
        b = b * ri * w[i1];
      }
      const float c = cosT[(int64_t)pos * pairs + p], sn = sinT[(int64_t)pos * pairs + p];
      st(dst + i0, a * c - b * sn);
      st(dst + i1, b * c + a * sn);
    }
  }
}

// Backward: dq/dk/dv (fp32, attention outputs) -> dqkv (TA) fused [T, nqkv];
// dwq/dwk partials per block (deterministic, reduced afterwards).
template <typename TA>
__global__ __launch_bounds__(256) void qkv_prep_bwd_kernel(
    const float* __restrict__ dq, const float* __restrict__ dk, const float* __restrict__ dv,
    const float* __restrict__ qkv, const float* __restrict__ rinv, const float* __restrict__ wq,
    const float* __restrict__ wk, const float* __restrict__ cosT, const float* __restrict__ sinT,
    TA* __restrict__ dqkv, float* __restrict__ part, int T, int S, int Hq, int Hkv, int D, int qk_norm,
    int neox) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int H = Hq + 2 * Hkv, nqkv = H * D;
  const int64_t rows = (int64_t)T * H;
  const int pairs = D / 2;
  // per-lane dw accumulators for columns lane, lane+64 (D <= 128) of q and k weights
  float aq0 = 0.f, aq1 = 0.f, ak0 = 0.f, ak1 = 0.f;
  for (int64_t r = (int64_t)blockIdx.x * 4 + wv; r < rows; r += (int64_t)gridDim.x * 4) {
    const int t = (int)(r / H), hh = (int)(r % H);
    TA* dst = dqkv + (int64_t)t * nqkv + hh * D;
    if (hh >= Hq + Hkv) {
      const float* g = dv + (int64_t)t * Hkv * D + (hh - Hq - Hkv) * D;
      for (int d = lane; d < D; d += 64) st(dst + d, g[d]);
      continue;
    }
    const bool isq = hh < Hq;
    const float* g = isq ? dq + (int64_t)t * Hq * D + hh * D : dk + (int64_t)t * Hkv * D + (hh - Hq) * D;
    const int pos = t % S;
    // inverse rotation into registers: element d = lane + 64*j
    float gr[2] = {0.f, 0.f};
    for (int j = 0; j < 2; j++) {
      const int d = lane + 64 * j;
      if (d >= D) break;
      int p, first;
      if (neox) { p = d < pairs ? d : d - pairs; first = d < pairs; }
      else { p = d >> 1; first = (d & 1) == 0; }
      const int i0 = neox ? p : 2 * p, i1 = neox ? p + pairs : 2 * p + 1;
      const float c = cosT[(int64_t)pos * pairs + p], sn = sinT[(int64_t)pos * pairs + p];
      const float g0 = g[i0], g1 = g[i1];
      gr[j] = first ? c * g0 + sn * g1 : -sn * g0 + c * g1;
    }
    if (!qk_norm) {
      for (int j = 0; j < 2; j++) if (lane + 64 * j < D) st(dst + lane + 64 * j, gr[j]);
      continue;
    }
    const float* x = qkv + (int64_t)t * nqkv + hh * D;
    const float* w = isq ? wq : wk;
    const float ri = rinv[(int64_t)t * (Hq + Hkv) + hh];
    float xn[2] = {0.f, 0.f}, dot = 0.f;
    for (int j = 0; j < 2; j++) {
      const int d = lane + 64 * j;
      if (d >= D) break;
      xn[j] = x[d] * ri;
      dot += gr[j] * w[d] * xn[j];
      if (isq) { if (j == 0) aq0 += gr[j] * xn[j]; else aq1 += gr[j] * xn[j]; }
      else { if (j == 0) ak0 += gr[j] * xn[j]; else ak1 += gr[j] * xn[j]; }
    }
    dot = wave_sum(dot) / (float)D;
    for (int j = 0; j < 2; j++) {
      const int d = lane + 64 * j;
      if (d >= D) break;
      st(dst + d, ri * (gr[j] * w[d] - xn[j] * dot));
    }
  }
  if (part) {
    __shared__ float sh[4][4][64];
    sh[wv][0][lane] = aq0; sh[wv][1][lane] = aq1; sh[wv][2][lane] = ak0; sh[wv][3][lane] = ak1;
    __syncthreads();
    if (threadIdx.x < 4 * 64) {
      const int which = threadIdx.x >> 6, l = threadIdx.x & 63;
      float s = sh[0][which][l] + sh[1][which][l] + sh[2][which][l] + sh[3][which][l];
      const int col = (which & 1) * 64 + l;  // column within head
      if (col < D) part[(int64_t)blockIdx.x * 2 * D + (which >> 1) * D + col] = s;
    }
  }
}

// dq[c] += sum_g part[g][c] (c < D), dk[c - D] += ... (c >= D): 64 columns per workgroup,
// 16 row groups of 64 lanes each sum a strided share of the G partial rows (coalesced 256-byte
// rows), then the 16 group sums combine in a fixed order (deterministic)
__global__ __launch_bounds__(1024) void colsum_add2_kernel(const float* __restrict__ part, float* __restrict__ dq,
                                                           float* __restrict__ dk, int G, int D) {
  __shared__ float sh[16][64];
  const int l = threadIdx.x & 63, rg = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + l;
  float s0 = 0.f, s1 = 0.f;
  if (c < 2 * D) {
    int g = rg;
    for (; g + 16 < G; g += 32) {
      s0 += part[(int64_t)g * 2 * D + c];
      s1 += part[(int64_t)(g + 16) * 2 * D + c];
    }
    if (g < G) s0 += part[(int64_t)g * 2 * D + c];
  }
  sh[rg][l] = s0 + s1;
  __syncthreads();
  if (rg == 0 && c < 2 * D) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 16; q++) s += sh[q][l];
    float* dst = c < D ? dq + c : dk + (c - D);
    *dst += s;
  }
}

// ---------------------------------------------------------------- vectorised form, D = 64 / 128
// Half a wave (32 lanes) per (token, head) row, E = D/32 consecutive elements per lane, two
// rows per wave.  Lane l holds elements (l % 2) D/2 + E (l / 2) ..: NeoX rotation partners
// (d, d + D/2) sit in lanes l and l ^ 1 (one DPP move, no LDS round trip); adjacent pairs
// (2p, 2p+1) sit in one lane.  Same arithmetic per element as the generic kernels above; the
// sum of squares / dot products reduce in a different order.
template <int E> struct VecF;
template <> struct VecF<2> { typedef float2 T; };
template <> struct VecF<4> { typedef float4 T; };
template <int E> __device__ __forceinline__ void ldE(const float* p, float* v) {
  if constexpr (E == 8) {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    return;
  } else {
    const typename VecF<E>::T t = *reinterpret_cast<const typename VecF<E>::T*>(p);
    const float* f = reinterpret_cast<const float*>(&t);
#pragma unroll
    for (int i = 0; i < E; i++) v[i] = f[i];
  }
}
// E bf16 values (4 or 8 bytes) widened to fp32
template <int E> __device__ __forceinline__ void ldE(const uint16_t* p, float* v) {
  uint32_t w[E / 2];
  if constexpr (E == 8) {
    const uint4 t = *reinterpret_cast<const uint4*>(p);
    w[0] = t.x; w[1] = t.y; w[2] = t.z; w[3] = t.w;
  } else if constexpr (E == 4) {
    const uint2 t = *reinterpret_cast<const uint2*>(p);
    w[0] = t.x;
    w[1] = t.y;
  } else {
    w[0] = *reinterpret_cast<const uint32_t*>(p);
  }
#pragma unroll
  for (int i = 0; i < E / 2; i++) {
    v[2 * i] = __builtin_bit_cast(float, w[i] << 16);
    v[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xFFFF0000u);
  }
}
template <int E, typename TA> __device__ __forceinline__ void stE(TA* p, const float* v) {
  if constexpr (sizeof(TA) == 4 && E == 8) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else if constexpr (sizeof(TA) == 4) {
    typename VecF<E>::T t;
    float* f = reinterpret_cast<float*>(&t);
#pragma unroll
    for (int i = 0; i < E; i++) f[i] = v[i];
    *reinterpret_cast<typename VecF<E>::T*>(p) = t;
  } else {
    uint32_t w[E / 2];
#pragma unroll
    for (int i = 0; i < E / 2; i++) w[i] = pack_bf2(v[2 * i], v[2 * i + 1]);
    if constexpr (E == 8) *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    else if constexpr (E == 4) *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint32_t*>(p) = w[0];
  }
}
// lane l ^ 1's value (DPP quad permute, no LDS round trip)
__device__ __forceinline__ float dpp_xor1(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
}
// sum over the 32 lanes of a half wave: quad permutes (xor 1, xor 2), the 8- and 16-lane mirrors
// by DPP, one cross-row shuffle; every lane ends with the same bits
// sum over the 16 lanes of a row group (the DPP steps of half_sum without the xor-16 shuffle)
__device__ __forceinline__ float quarter_sum(float v) {
  v += dpp_xor1(v);
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
  return v;
}
template <int L> __device__ __forceinline__ float group_sum(float v);
__device__ __forceinline__ float half_sum(float v) {
  v += dpp_xor1(v);
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
  v += __shfl_xor(v, 16, 64);
  return v;
}
template <> __device__ __forceinline__ float group_sum<32>(float v) { return half_sum(v); }
template <> __device__ __forceinline__ float group_sum<16>(float v) { return quarter_sum(v); }

// L = lanes per head row (32, or 16 for 16-byte bf16 accesses at D = 128)
template <int D, typename TA, typename TQ, int L = 32>
__global__ __launch_bounds__(256) void qkv_prep_fwd_vec_kernel(
    const TQ* __restrict__ qkv, TA* __restrict__ qo, TA* __restrict__ ko, TA* __restrict__ vo,
    float* __restrict__ rinv, const float* __restrict__ wq, const float* __restrict__ wk,
    const float* __restrict__ cosT, const float* __restrict__ sinT, int T, int S, int Hq, int Hkv,
    int qk_norm, int neox, float eps) {
  constexpr int E = D / L, P = D / 2, NG = 256 / L;
  constexpr int R = L == 32 ? 4 : 2;  // rows in flight per row group
  const int l = threadIdx.x & (L - 1), hw = threadIdx.x / L;
  // lane l holds elements eo .. eo + E - 1 of a head row, the halves interleaved so that NeoX
  // partners (i, i + D/2) sit in lanes l and l ^ 1
  const int eo = (l & 1) * P + E * (l >> 1);
  const int H = Hq + 2 * Hkv, nqkv = H * D;
  // vo null: V is read where the projection wrote it (no copy), only q and k rows are processed
  const int Hl = vo ? H : Hq + Hkv;
  // workgroup per token: the half-waves take heads hw, hw + 8, ...; the lane's RoPE factors
  // depend only on the lane and the position, so they are loaded once per token
  for (int t = blockIdx.x; t < T; t += gridDim.x) {
    const int pos = t % S;
    float cs[E], sn[E];
    if (neox) {
      ldE<E>(cosT + (int64_t)pos * P + eo % P, cs);
      ldE<E>(sinT + (int64_t)pos * P + eo % P, sn);
    } else {
#pragma unroll
      for (int i = 0; i < E; i += 2) {
        const int p = (eo + i) / 2;
        cs[i] = cs[i + 1] = cosT[(int64_t)pos * P + p];
        sn[i] = sn[i + 1] = sinT[(int64_t)pos * P + p];
      }
    }
    const TQ* xt = qkv + (int64_t)t * nqkv;
    for (int h0 = hw; h0 < Hl; h0 += NG * R) {
      float v[R][E];
#pragma unroll
      for (int r = 0; r < R; r++)
        if (h0 + NG * r < Hl) ldE<E>(xt + (h0 + NG * r) * D + eo, v[r]);
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int hh = h0 + NG * r;
        if (hh >= Hl) break;
        if (hh >= Hq + Hkv) {
          stE<E>(vo + (int64_t)t * Hkv * D + (hh - Hq - Hkv) * D + eo, v[r]);
          continue;
        }
        const bool isq = hh < Hq;
        const float* w = (isq ? wq : wk) + eo;
        if (qk_norm) {
          float ss = 0.f;
#pragma unroll
          for (int i = 0; i < E; i++) ss += v[r][i] * v[r][i];
          ss = group_sum<L>(ss);
          const float ri = 1.f / sqrtf(ss / (float)D + eps);
          if (l == 0) rinv[(int64_t)t * (Hq + Hkv) + hh] = ri;
#pragma unroll
          for (int i = 0; i < E; i++) v[r][i] = v[r][i] * ri * w[i];
        }
        float o[E];
        if (neox) {
          const bool lo = eo < P;
#pragma unroll
          for (int i = 0; i < E; i++) {
            const float partner = dpp_xor1(v[r][i]);
            o[i] = lo ? v[r][i] * cs[i] - partner * sn[i] : v[r][i] * cs[i] + partner * sn[i];
          }
        } else {
#pragma unroll
          for (int i = 0; i < E; i += 2) {
            o[i] = v[r][i] * cs[i] - v[r][i + 1] * sn[i];
            o[i + 1] = v[r][i + 1] * cs[i] + v[r][i] * sn[i];
          }
        }
        stE<E>((isq ? qo + (int64_t)t * Hq * D + hh * D : ko + (int64_t)t * Hkv * D + (hh - Hq) * D) + eo, o);
      }
    }
  }
}

// L = lanes per head row: 32 (E = D/32 elements per lane) or 16 (E = D/16: 16-byte bf16 accesses
// at D = 128, 16 row groups per workgroup)
template <int D, typename TA, typename TQ, typename TG, int L = 32>
__global__ __launch_bounds__(256) void qkv_prep_bwd_vec_kernel(
    const TG* __restrict__ dq, const TG* __restrict__ dk, const TG* __restrict__ dv,
    const TQ* __restrict__ qkv, const float* __restrict__ rinv, const float* __restrict__ wq,
    const float* __restrict__ wk, const float* __restrict__ cosT, const float* __restrict__ sinT,
    TA* __restrict__ dqkv, float* __restrict__ part, int T, int S, int Hq, int Hkv, int qk_norm, int neox,
    int kv_grp) {
  constexpr int E = D / L, P = D / 2, NG = 256 / L;
  const int l = threadIdx.x & (L - 1), hw = threadIdx.x / L;  // row group 0 .. NG-1
  const int eo = (l & 1) * P + E * (l >> 1);  // as in the forward: NeoX partners in lanes l, l ^ 1
  // kv_grp > 0: dk / dv are the attention backward's per-query-head partials [T, Hq, D]; a KV
  // head's gradient is the sum of its kv_grp query heads, added in ascending head order
  auto ld_kv = [&](const TG* base, int t, int kvh, float* g) {
    if (kv_grp == 0) {
      ldE<E>(base + (int64_t)t * Hkv * D + kvh * D + eo, g);
      return;
    }
    const TG* p0 = base + ((int64_t)t * Hq + (int64_t)kvh * kv_grp) * D + eo;
    float h[E];
#pragma unroll
    for (int i = 0; i < E; i++) g[i] = 0.f;
    if (kv_grp == 2) {  // both loads in flight before the (ordered) adds
      float h1[E];
      ldE<E>(p0, h);
      ldE<E>(p0 + D, h1);
#pragma unroll
      for (int i = 0; i < E; i++) g[i] = (g[i] + h[i]) + h1[i];
      return;
    }
    for (int j = 0; j < kv_grp; j++) {
      ldE<E>(p0 + (int64_t)j * D, h);
#pragma unroll
      for (int i = 0; i < E; i++) g[i] += h[i];
    }
  };
  const int H = Hq + 2 * Hkv, nqkv = H * D;
  constexpr int R = 2;  // rows in flight per half-wave (4 costs occupancy: 135 registers)
  float aq[E], ak[E];
#pragma unroll
  for (int i = 0; i < E; i++) { aq[i] = 0.f; ak[i] = 0.f; }
  // workgroup per token: the half-waves take heads hw, hw + 8, ...; RoPE factors once per token
  for (int t = blockIdx.x; t < T; t += gridDim.x) {
    const int pos = t % S;
    float cs[E], sn[E];
    if (neox) {
      ldE<E>(cosT + (int64_t)pos * P + eo % P, cs);
      ldE<E>(sinT + (int64_t)pos * P + eo % P, sn);
    } else {
#pragma unroll
      for (int i = 0; i < E; i += 2) {
        const int p = (eo + i) / 2;
        cs[i] = cs[i + 1] = cosT[(int64_t)pos * P + p];
        sn[i] = sn[i + 1] = sinT[(int64_t)pos * P + p];
      }
    }
    for (int h0 = hw; h0 < H; h0 += NG * R) {
      float g[R][E], x[R][E], ri[R];
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int hh = h0 + NG * r;
        if (hh >= H) break;
        if (hh >= Hq + Hkv) {
          ld_kv(dv, t, hh - Hq - Hkv, g[r]);
          continue;
        }
        if (hh < Hq) ldE<E>(dq + (int64_t)t * Hq * D + hh * D + eo, g[r]);
        else ld_kv(dk, t, hh - Hq, g[r]);
        if (qk_norm) {
          ldE<E>(qkv + (int64_t)t * nqkv + hh * D + eo, x[r]);
          ri[r] = rinv[(int64_t)t * (Hq + Hkv) + hh];
        }
      }
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int hh = h0 + NG * r;
        if (hh >= H) break;
        TA* dst = dqkv + (int64_t)t * nqkv + hh * D + eo;
        if (hh >= Hq + Hkv) {
          stE<E>(dst, g[r]);
          continue;
        }
        const bool isq = hh < Hq;
        float gr[E];
        if (neox) {
          const bool lo = eo < P;
#pragma unroll
          for (int i = 0; i < E; i++) {
            const float partner = dpp_xor1(g[r][i]);
            gr[i] = lo ? cs[i] * g[r][i] + sn[i] * partner : -sn[i] * partner + cs[i] * g[r][i];
          }
        } else {
#pragma unroll
          for (int i = 0; i < E; i += 2) {
            gr[i] = cs[i] * g[r][i] + sn[i] * g[r][i + 1];
            gr[i + 1] = -sn[i] * g[r][i] + cs[i] * g[r][i + 1];
          }
        }
        if (!qk_norm) {
          stE<E>(dst, gr);
          continue;
        }
        const float* w = (isq ? wq : wk) + eo;
        float dot = 0.f, xn[E];
#pragma unroll
        for (int i = 0; i < E; i++) {
          xn[i] = x[r][i] * ri[r];
          dot += gr[i] * w[i] * xn[i];
          if (isq) aq[i] += gr[i] * xn[i];
          else ak[i] += gr[i] * xn[i];
        }
        dot = group_sum<L>(dot) / (float)D;
        float o[E];
#pragma unroll
        for (int i = 0; i < E; i++) o[i] = ri[r] * (gr[i] * w[i] - xn[i] * dot);
        stE<E>(dst, o);
      }
    }
  }
  if (part) {  // block partial of dw: sum the NG row groups in a fixed order
    __shared__ float sh[NG][2][D];
#pragma unroll
    for (int i = 0; i < E; i++) {
      sh[hw][0][eo + i] = aq[i];
      sh[hw][1][eo + i] = ak[i];
    }
    __syncthreads();
    for (int c = threadIdx.x; c < 2 * D; c += 256) {
      float acc = 0.f;
      for (int h = 0; h < NG; h++) acc += sh[h][c / D][c % D];
      part[(int64_t)blockIdx.x * 2 * D + c] = acc;
    }
  }
}

int qkv_prep_forward(const void* qkv, int qkv_bf16, void* q, void* k, void* v, float* rinv, const float* wq,
                     const float* wk, const float* cosT, const float* sinT, int T, int S, int Hq, int Hkv,
                     int D, int qk_norm, int neox, float eps, int bf16, hipStream_t s) {
  SMHIP_REQUIRE(D <= 128 && D % 2 == 0, "qkv prep: head_dim must be even and <= 128");
  const int64_t rows = (int64_t)T * (Hq + 2 * Hkv);
  SMHIP_REQUIRE(v || (D == 128 || D == 64), "qkv prep: v may be omitted only for head_dim 64 or 128");
  if (D == 128 || D == 64) {
    const int gv = (int)std::min<int64_t>(T, (int64_t)num_cus() * 8);  // workgroup per token
#define SMHIP_QKV_FWD(DD, TT, TQ) \
  hipLaunchKernelGGL((qkv_prep_fwd_vec_kernel<DD, TT, TQ>), dim3(gv), dim3(256), 0, s, (const TQ*)qkv, (TT*)q, (TT*)k, (TT*)v, rinv, wq, wk, cosT, sinT, T, S, Hq, Hkv, qk_norm, neox, eps)
    if (qkv_bf16) {
      SMHIP_REQUIRE(bf16, "qkv prep: bf16 projections need bf16 outputs");
      if (D == 128)  // 16 lanes per row: 16-byte accesses
        hipLaunchKernelGGL((qkv_prep_fwd_vec_kernel<128, uint16_t, uint16_t, 16>), dim3(gv), dim3(256), 0, s,
                           (const uint16_t*)qkv, (uint16_t*)q, (uint16_t*)k, (uint16_t*)v, rinv, wq, wk, cosT, sinT, T,
                           S, Hq, Hkv, qk_norm, neox, eps);
      else SMHIP_QKV_FWD(64, uint16_t, uint16_t);
    } else if (D == 128) { if (bf16) SMHIP_QKV_FWD(128, uint16_t, float); else SMHIP_QKV_FWD(128, float, float); }
    else { if (bf16) SMHIP_QKV_FWD(64, uint16_t, float); else SMHIP_QKV_FWD(64, float, float); }
#undef SMHIP_QKV_FWD
    SMHIP_CHECK_LAUNCH();
    return SMHIP_OK;
  }
  SMHIP_REQUIRE(!qkv_bf16, "qkv prep: bf16 projections need head_dim 64 or 128");
  const int g = gridn(rows, 4);
  if (bf16)
    hipLaunchKernelGGL(qkv_prep_fwd_kernel<uint16_t>, dim3(g), dim3(256), 0, s, (const float*)qkv, (uint16_t*)q, (uint16_t*)k, (uint16_t*)v, rinv, wq, wk, cosT, sinT, T, S, Hq, Hkv, D, qk_norm, neox, eps);
  else
    hipLaunchKernelGGL(qkv_prep_fwd_kernel<float>, dim3(g), dim3(256), 0, s, (const float*)qkv, (float*)q, (float*)k, (float*)v, rinv, wq, wk, cosT, sinT, T, S, Hq, Hkv, D, qk_norm, neox, eps);
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

int qkv_prep_backward(const void* dq_, const void* dk_, const void* dv_, int grads_bf16, const void* qkv, int qkv_bf16,
                      const float* rinv,
                      const float* wq, const float* wk, float* dwq, float* dwk, const float* cosT,
                      const float* sinT, void* dqkv, int T, int S, int Hq, int Hkv, int D, int qk_norm,
                      int neox, int bf16, int kv_grp, hipStream_t s) {
  SMHIP_REQUIRE(D <= 128 && D % 2 == 0, "qkv prep: head_dim must be even and <= 128");
  SMHIP_REQUIRE(!grads_bf16 || D == 128 || D == 64, "qkv prep: bf16 attention gradients need head_dim 64 or 128");
  const float *dq = (const float*)dq_, *dk = (const float*)dk_, *dv = (const float*)dv_;
  SMHIP_REQUIRE(kv_grp == 0 || ((D == 128 || D == 64) && kv_grp * Hkv == Hq),
                "qkv prep: per-query-head K/V partials need head_dim 64 or 128 and kv_grp = Hq / Hkv");
  const int64_t rows = (int64_t)T * (Hq + 2 * Hkv);
  const bool want_dw = qk_norm && (dwq || dwk);
  const bool vec = D == 128 || D == 64;
  // dw partials: one row of 2*D per block, so fewer (larger) blocks when they are needed; the
  // vectorised kernel runs a workgroup per token
  const int g = vec ? (int)std::min<int64_t>(T, (int64_t)num_cus() * (want_dw ? 4 : 8)) : gridn(rows, 4, 2);
  float* part = nullptr;
  if (want_dw) {
    part = (float*)workspace(s, sizeof(float) * (size_t)g * 2 * D, 7);
    if (!part) return fail(SMHIP_ENOMEM, "qkv prep backward: workspace");
  }
  SMHIP_REQUIRE(vec || !qkv_bf16, "qkv prep: bf16 projections need head_dim 64 or 128");
  SMHIP_REQUIRE(bf16 || !qkv_bf16, "qkv prep: bf16 projections need bf16 outputs");
  if (vec) {
#define SMHIP_QKV_BWD(DD, TT, TQ)                                                                                  \
  if (grads_bf16)                                                                                                  \
    hipLaunchKernelGGL((qkv_prep_bwd_vec_kernel<DD, TT, TQ, uint16_t>), dim3(g), dim3(256), 0, s,                  \
                       (const uint16_t*)dq_, (const uint16_t*)dk_, (const uint16_t*)dv_, (const TQ*)qkv, rinv, wq, \
                       wk, cosT, sinT, (TT*)dqkv, part, T, S, Hq, Hkv, qk_norm, neox, kv_grp);                     \
  else                                                                                                             \
    hipLaunchKernelGGL((qkv_prep_bwd_vec_kernel<DD, TT, TQ, float>), dim3(g), dim3(256), 0, s, dq, dk, dv,         \
                       (const TQ*)qkv, rinv, wq, wk, cosT, sinT, (TT*)dqkv, part, T, S, Hq, Hkv, qk_norm, neox, kv_grp)
    if (qkv_bf16 && grads_bf16 && D == 128)  // 16 lanes per row: 16-byte accesses
      hipLaunchKernelGGL((qkv_prep_bwd_vec_kernel<128, uint16_t, uint16_t, uint16_t, 16>), dim3(g), dim3(256), 0, s,
                         (const uint16_t*)dq_, (const uint16_t*)dk_, (const uint16_t*)dv_, (const uint16_t*)qkv, rinv,
                         wq, wk, cosT, sinT, (uint16_t*)dqkv, part, T, S, Hq, Hkv, qk_norm, neox, kv_grp);
    else if (qkv_bf16) { if (D == 128) SMHIP_QKV_BWD(128, uint16_t, uint16_t); else SMHIP_QKV_BWD(64, uint16_t, uint16_t); }
    else if (D == 128) { if (bf16) SMHIP_QKV_BWD(128, uint16_t, float); else SMHIP_QKV_BWD(128, float, float); }
    else { if (bf16) SMHIP_QKV_BWD(64, uint16_t, float); else SMHIP_QKV_BWD(64, float, float); }
#undef SMHIP_QKV_BWD
  } else if (bf16)
    hipLaunchKernelGGL(qkv_prep_bwd_kernel<uint16_t>, dim3(g), dim3(256), 0, s, dq, dk, dv, (const float*)qkv, rinv, wq, wk, cosT, sinT, (uint16_t*)dqkv, part, T, S, Hq, Hkv, D, qk_norm, neox);
  else
    hipLaunchKernelGGL(qkv_prep_bwd_kernel<float>, dim3(g), dim3(256), 0, s, dq, dk, dv, (const float*)qkv, rinv, wq, wk, cosT, sinT, (float*)dqkv, part, T, S, Hq, Hkv, D, qk_norm, neox);
  SMHIP_CHECK_LAUNCH();
  if (part) {
    hipLaunchKernelGGL(colsum_add2_kernel, dim3(ceil_div(2 * D, 64)), dim3(1024), 0, s, part, dwq, dwk, g, D);
    SMHIP_CHECK_LAUNCH();
  }
  return SMHIP_OK;
}

// ============================================================================
// SwiGLU on the fused [gate | up] layout
// ============================================================================
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void swiglu_fused_fwd_kernel(const TI* __restrict__ gu, TO* __restrict__ act, int T, int F) {
  const int64_t n = (int64_t)T * F;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t t = i / F, d = i - t * F;
    const float g = ldv(gu + t * 2 * F + d), u = ldv(gu + t * 2 * F + F + d);
    st(act + i, (g / (1.f + expf(-g))) * u);
  }
}
template <typename TD, typename TI, typename TO>
__global__ __launch_bounds__(256) void swiglu_fused_bwd_kernel(const TD* __restrict__ dA, const TI* __restrict__ gu,
                                                               TO* __restrict__ dgu, int T, int F) {
  const int64_t n = (int64_t)T * F;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t t = i / F, d = i - t * F;
    const float g = ldv(gu + t * 2 * F + d), u = ldv(gu + t * 2 * F + F + d), da = ldv(dA + i);
    const float sig = 1.f / (1.f + expf(-g));
    st(dgu + t * 2 * F + F + d, da * (g * sig));
    st(dgu + t * 2 * F + d, da * (sig * (1.f + g * (1.f - sig))) * u);
  }
}

// 8 consecutive elements per thread (F % 8 == 0, 16-byte aligned rows): 16-byte loads and
// stores for bf16, two float4 for fp32; the same per-element arithmetic as the scalar kernels
__device__ inline void ld8(const uint16_t* p, float* f) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    f[2 * i] = bf2f((uint16_t)(w[i] & 0xFFFFu));
    f[2 * i + 1] = bf2f((uint16_t)(w[i] >> 16));
  }
}
__device__ inline void ld8(const float* p, float* f) {
  const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
__device__ inline void st8(uint16_t* p, const float* f) {
  *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf2(f[0], f[1]), pack_bf2(f[2], f[3]), pack_bf2(f[4], f[5]), pack_bf2(f[6], f[7]));
}
__device__ inline void st8(float* p, const float* f) {
  *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(f[4], f[5], f[6], f[7]);
}
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void swiglu_fused_fwd_vec_kernel(const TI* __restrict__ gu, TO* __restrict__ act, int T, int F) {
  const int64_t n8 = (int64_t)T * F / 8;
  for (int64_t i8 = (int64_t)blockIdx.x * 256 + threadIdx.x; i8 < n8; i8 += (int64_t)gridDim.x * 256) {
    const int64_t i = i8 * 8, t = i / F, d = i - t * F;
    float g[8], u[8], o[8];
    ld8(gu + t * 2 * F + d, g);
    ld8(gu + t * 2 * F + F + d, u);
#pragma unroll
    for (int k = 0; k < 8; k++) o[k] = (g[k] / (1.f + expf(-g[k]))) * u[k];
    st8(act + i, o);
  }
}
template <typename TD, typename TI, typename TO>
__global__ __launch_bounds__(256) void swiglu_fused_bwd_vec_kernel(const TD* __restrict__ dA, const TI* __restrict__ gu,
                                                                   TO* __restrict__ dgu, int T, int F) {
  const int64_t n8 = (int64_t)T * F / 8;
  for (int64_t i8 = (int64_t)blockIdx.x * 256 + threadIdx.x; i8 < n8; i8 += (int64_t)gridDim.x * 256) {
    const int64_t i = i8 * 8, t = i / F, d = i - t * F;
    float g[8], u[8], da[8], og[8], ou[8];
    ld8(gu + t * 2 * F + d, g);
    ld8(gu + t * 2 * F + F + d, u);
    ld8(dA + i, da);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const float sig = 1.f / (1.f + expf(-g[k]));
      ou[k] = da[k] * (g[k] * sig);
      og[k] = da[k] * (sig * (1.f + g[k] * (1.f - sig))) * u[k];
    }
    st8(dgu + t * 2 * F + F + d, ou);
    st8(dgu + t * 2 * F + d, og);
  }
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int swiglu_fused_forward(const void* gu, void* act, int T, int F, int bf16, hipStream_t s) {
  const bool vec = F % 8 == 0 && al16(gu) && al16(act);
  const int g = gridn((int64_t)T * F / (vec ? 8 : 1));
  if (vec) {
    if (bf16) hipLaunchKernelGGL((swiglu_fused_fwd_vec_kernel<uint16_t, uint16_t>), dim3(g), dim3(256), 0, s, (const uint16_t*)gu, (uint16_t*)act, T, F);
    else hipLaunchKernelGGL((swiglu_fused_fwd_vec_kernel<float, float>), dim3(g), dim3(256), 0, s, (const float*)gu, (float*)act, T, F);
  } else if (bf16) {
    hipLaunchKernelGGL((swiglu_fused_fwd_kernel<uint16_t, uint16_t>), dim3(g), dim3(256), 0, s, (const uint16_t*)gu, (uint16_t*)act, T, F);
  } else {
    hipLaunchKernelGGL((swiglu_fused_fwd_kernel<float, float>), dim3(g), dim3(256), 0, s, (const float*)gu, (float*)act, T, F);
  }
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}
int swiglu_fused_backward(const void* dA, const void* gu, void* dgu, int T, int F, int bf16, hipStream_t s) {
  const bool vec = F % 8 == 0 && al16(dA) && al16(gu) && al16(dgu);
  const int g = gridn((int64_t)T * F / (vec ? 8 : 1));
  if (vec) {
    if (bf16) hipLaunchKernelGGL((swiglu_fused_bwd_vec_kernel<uint16_t, uint16_t, uint16_t>), dim3(g), dim3(256), 0, s, (const uint16_t*)dA, (const uint16_t*)gu, (uint16_t*)dgu, T, F);
    else hipLaunchKernelGGL((swiglu_fused_bwd_vec_kernel<float, float, float>), dim3(g), dim3(256), 0, s, (const float*)dA, (const float*)gu, (float*)dgu, T, F);
  } else if (bf16) {
    hipLaunchKernelGGL((swiglu_fused_bwd_kernel<uint16_t, uint16_t, uint16_t>), dim3(g), dim3(256), 0, s, (const uint16_t*)dA, (const uint16_t*)gu, (uint16_t*)dgu, T, F);
  } else {
    hipLaunchKernelGGL((swiglu_fused_bwd_kernel<float, float, float>), dim3(g), dim3(256), 0, s, (const float*)dA, (const float*)gu, (float*)dgu, T, F);
  }
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

// ============================================================================
// LoRA block-diagonal mask: zero dB[j, n] unless row block (j / r) == column block
// ============================================================================
__global__ void lora_mask_kernel(float* __restrict__ dB, int nr, int r, int Out, const int* __restrict__ col_starts,
                                 int nblocks) {
  const int64_t n = (int64_t)nr * Out;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int j = (int)(i / Out), c = (int)(i % Out);
    const int blk = j / r;
    const int lo = col_starts[blk], hi = blk + 1 < nblocks ? col_starts[blk + 1] : Out;
    if (c < lo || c >= hi) dB[i] = 0.f;
  }
}
int lora_mask(float* dB, int nr, int r, int Out, const int* col_starts_dev, int nblocks, hipStream_t s) {
  hipLaunchKernelGGL(lora_mask_kernel, dim3(gridn((int64_t)nr * Out)), dim3(256), 0, s, dB, nr, r, Out, col_starts_dev, nblocks);
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

__global__ void cast_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) y[i] = f2bf(x[i]);
}
int cast_bf16(const float* x, uint16_t* y, int64_t n, hipStream_t s) {
  if (n <= 0) return SMHIP_OK;
  hipLaunchKernelGGL(cast_bf16_kernel, dim3(gridn(n)), dim3(256), 0, s, x, y, n);
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

// ============================================================================
// synthetic data: counter-based normal generator (splitmix64 hash of (seed, index),
// Box-Muller in double) and uniform integers for token ids
// ============================================================================
__device__ inline uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__global__ void fill_normal_kernel(float* __restrict__ x, int64_t n, uint64_t seed, float mean, float std) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    uint64_t a = mix64(seed * 0x100000001B3ull + 2 * (uint64_t)i), b = mix64(seed * 0x100000001B3ull + 2 * (uint64_t)i + 1);
    double u1 = ((a >> 11) + 1) * (1.0 / 9007199254740993.0);
    double u2 = (b >> 11) * (1.0 / 9007199254740992.0);
    x[i] = mean + std * (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
  }
}
__global__ void fill_uniform_kernel(float* __restrict__ x, int64_t n, uint64_t seed, float lo, float hi) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    double u = (mix64(seed * 0x100000001B3ull + (uint64_t)i) >> 11) * (1.0 / 9007199254740992.0);
    x[i] = lo + (hi - lo) * (float)u;
  }
}
__global__ void fill_ids_kernel(int32_t* __restrict__ x, int64_t n, uint64_t seed, int V) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    x[i] = (int32_t)(mix64(seed * 0x100000001B3ull + (uint64_t)i) % (uint64_t)V);
}
int fill_normal(float* x, int64_t n, uint64_t seed, float mean, float std, hipStream_t s) {
  hipLaunchKernelGGL(fill_normal_kernel, dim3(gridn(n)), dim3(256), 0, s, x, n, seed, mean, std);
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}
int fill_uniform(float* x, int64_t n, uint64_t seed, float lo, float hi, hipStream_t s) {
  hipLaunchKernelGGL(fill_uniform_kernel, dim3(gridn(n)), dim3(256), 0, s, x, n, seed, lo, hi);
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}
int fill_ids(int32_t* x, int64_t n, uint64_t seed, int V, hipStream_t s) {
  hipLaunchKernelGGL(fill_ids_kernel, dim3(gridn(n)), dim3(256), 0, s, x, n, seed, V);
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

// ============================================================================
// encoders (bit-identical to the reference byte layout)
// ============================================================================
// float -> IEEE binary16 bits, round to nearest even ((Half)f, QuantizationKernels.cs:149)
__device__ inline uint16_t f2h_rne(float f) {
  uint32_t x = __builtin_bit_cast(uint32_t, f);
  uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax == 0x7F800000u ? 0x7C00u : (0x7E00u | ((ax >> 13) & 0x3FFu))));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
  if (ax >= 0x38800000u) {
    uint32_t mant = ax & 0x7FFFFFu, h = (((ax >> 23) - 112) << 10) | (mant >> 13), rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  if (ax < 0x33000000u) return (uint16_t)sign;
  uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
  int shift = 126 - (int)(ax >> 23);
  uint32_t h = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}
__device__ inline int round_away(float x) { return (int)roundf(x); }
__device__ inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

__global__ void encode_q8_0_kernel(const float* __restrict__ x, uint8_t* __restrict__ out, int64_t nb) {
  for (int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x; b < nb; b += (int64_t)gridDim.x * 256) {
    const float* v = x + b * 32;
    uint8_t* o = out + b * 34;
    float amax = 0.f;
    for (int j = 0; j < 32; j++) { float a = fabsf(v[j]); if (a > amax) amax = a; }
    if (amax == 0.f) {
      for (int j = 0; j < 34; j++) o[j] = 0;
      continue;
    }
    const float d = amax / 127.f;
    const uint16_t h = f2h_rne(d);
    o[0] = (uint8_t)h;
    o[1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t)(int8_t)clampi(round_away(v[j] / d), -128, 127);
  }
}

__global__ void encode_q4k_kernel(const float* __restrict__ x, uint8_t* __restrict__ out, int64_t nb) {
  for (int64_t b = (int64_t)blockIdx.x * 64 + threadIdx.x; b < nb; b += (int64_t)gridDim.x * 64) {
    const float* v = x + b * 256;
    uint8_t* o = out + b * 144;
    for (int j = 0; j < 144; j++) o[j] = 0;
    float amax = 0.f;
    for (int j = 0; j < 256; j++) { float a = fabsf(v[j]); if (a > amax) amax = a; }
    if (amax == 0.f) continue;
    const float step = amax / 63.f;
    const uint16_t h = f2h_rne(step);
    o[0] = o[2] = (uint8_t)h;
    o[1] = o[3] = (uint8_t)(h >> 8);
    int sc[8], mn[8];
    for (int sub = 0; sub < 8; sub++) {
      const float* g = v + sub * 32;
      float gmn = 3.40282347e+38f, gmx = -3.40282347e+38f;
      for (int j = 0; j < 32; j++) { if (g[j] < gmn) gmn = g[j]; if (g[j] > gmx) gmx = g[j]; }
      const float range = gmx - gmn;
      mn[sub] = clampi(round_away(-gmn / step), 0, 63);
      if (range <= 0.f) { sc[sub] = 0; continue; }
      sc[sub] = clampi(round_away(range / (15.f * step)), 1, 63);
      const float scF = (float)sc[sub] * step;
      for (int j = 0; j < 32; j++) {
        const int code = clampi(round_away((g[j] + (float)mn[sub] * step) / scF), 0, 15);
        const int i = sub * 32 + j;
        o[16 + (i / 64) * 32 + (i % 32)] |= (uint8_t)(code << (((i % 64) / 32) * 4));
      }
    }
    for (int j = 0; j < 4; j++) {
      o[4 + j] = (uint8_t)((sc[j] & 0x3F) | ((sc[4 + j] >> 4) << 6));
      o[8 + j] = (uint8_t)((mn[j] & 0x3F) | ((mn[4 + j] >> 4) << 6));
      o[12 + j] = (uint8_t)((sc[4 + j] & 0x0F) | ((mn[4 + j] & 0x0F) << 4));
    }
  }
}

int encode_quant(int qtype, const float* x, int64_t n, void* out, hipStream_t s) {
  if (qtype == SMHIP_QTYPE_Q8_0) {
    SMHIP_REQUIRE(n % 32 == 0, "Q8_0 encode: length must be a multiple of 32");
    hipLaunchKernelGGL(encode_q8_0_kernel, dim3(gridn(n / 32)), dim3(256), 0, s, x, (uint8_t*)out, n / 32);
  } else if (qtype == SMHIP_QTYPE_Q4_K) {
    SMHIP_REQUIRE(n % 256 == 0, "Q4_K encode: length must be a multiple of 256");
    hipLaunchKernelGGL(encode_q4k_kernel, dim3(gridn(n / 256, 64)), dim3(64), 0, s, x, (uint8_t*)out, n / 256);
  } else {
    return fail(SMHIP_EUNSUPPORTED, "encode: qtype must be Q8_0 (8) or Q4_K (12)");
  }
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

}  // namespace smhip

namespace smhip {
__global__ void zero_kernel(uint32_t* __restrict__ x, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) x[i] = 0u;
}
// Graph-capture-safe clear (a kernel, not a memset node).  bytes must be a multiple of 4.
int zero_bytes(void* p, size_t bytes, hipStream_t s) {
  if (!bytes) return SMHIP_OK;
  const int64_t n = (int64_t)(bytes / 4);
  hipLaunchKernelGGL(zero_kernel, dim3(gridn(n)), dim3(256), 0, s, (uint32_t*)p, n);
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}
// ---------------------------------------------------------------- batched bf16 transposes
// grid (element blocks, jobs): destination-ordered (coalesced stores), the small source rows
// gathered
__global__ __launch_bounds__(256) void transpose_bf16_jobs_kernel(const BfTJob* __restrict__ jobs) {
  const BfTJob j = jobs[blockIdx.y];
  const int64_t n = (int64_t)j.rows * j.cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t c = i / j.rows, r = i - c * j.rows;
    j.dst[i] = j.src[r * j.cols + c];
  }
}

int transpose_bf16_jobs(const BfTJob* jobs_dev, int njobs, int64_t max_elems, hipStream_t s) {
  if (njobs <= 0) return SMHIP_OK;
  const int gx = (int)std::min<int64_t>((max_elems + 255) / 256, 64);
  hipLaunchKernelGGL(transpose_bf16_jobs_kernel, dim3(gx, njobs), dim3(256), 0, s, jobs_dev);
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

}  // namespace smhip
