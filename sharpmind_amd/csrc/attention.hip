// attention.hip — attention forward/backward for gfx950.
//
// Slot form (GradientMapping.Attention, GradientKernels.cs:408-481): one head
// with materialised probabilities P [S,S].  The four S x S x D products run on
// the fp32 MFMA GEMM (transposed operands are read in place, no copies) and the
// softmax-Jacobian row step dS = P*(dP - rowsum(P*dP)) is one wave per row.
#include "common.hpp"
#include "kernels.hpp"

namespace smhip {

__global__ __launch_bounds__(256) void softmax_jacobian_rows(const float* __restrict__ P,
                                                             float* __restrict__ dP, int S) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int i = blockIdx.x * 4 + wv; i < S; i += gridDim.x * 4) {
    const float* p = P + (int64_t)i * S;
    float* d = dP + (int64_t)i * S;
    float dot = 0.f;
    for (int j = lane; j < S; j += 64) dot += p[j] * d[j];
    dot = wave_sum(dot);
    for (int j = lane; j < S; j += 64) d[j] = p[j] * (d[j] - dot);
  }
}

int attention_slot_backward(const float* dO, const float* q, const float* k, const float* v,
                            const float* P, float* dQ, float* dK, float* dV, int S, int D,
                            float scale, hipStream_t s) {
  if (S <= 0 || D <= 0) return SMHIP_OK;
  float* dP = (float*)workspace(s, sizeof(float) * (size_t)S * S, 4);
  if (!dP) return fail(SMHIP_ENOMEM, "attention backward: workspace");
  GemmArgs g{};
  g.precision = SMHIP_PREC_FP32;
  g.alpha = 1.f;
  g.beta = 0.f;
  g.split_k = 1;
  // dV[j,d] = sum_i P[i,j] dO[i,d]
  g.M = S; g.N = D; g.K = S;
  g.A = {SRC_F32_R, P, nullptr, S};
  g.B = {SRC_F32_R, dO, nullptr, D};
  g.C = dV; g.ldc = D;
  int rc = gemm(g, s);
  if (rc) return rc;
  // dP[i,j] = sum_d dO[i,d] V[j,d]
  g.M = S; g.N = S; g.K = D;
  g.A = {SRC_F32_K, dO, nullptr, D};
  g.B = {SRC_F32_K, v, nullptr, D};
  g.C = dP; g.ldc = S;
  if ((rc = gemm(g, s))) return rc;
  hipLaunchKernelGGL(softmax_jacobian_rows, dim3(std::min(ceil_div(S, 4), num_cus() * 4)), dim3(256), 0, s, P, dP, S);
  SMHIP_CHECK_LAUNCH();
  // dQ = scale * dS K
  g.M = S; g.N = D; g.K = S;
  g.alpha = scale;
  g.A = {SRC_F32_K, dP, nullptr, S};
  g.B = {SRC_F32_R, k, nullptr, D};
  g.C = dQ; g.ldc = D;
  if ((rc = gemm(g, s))) return rc;
  // dK = scale * dS^T Q
  g.A = {SRC_F32_R, dP, nullptr, S};
  g.B = {SRC_F32_R, q, nullptr, D};
  g.C = dK; g.ldc = D;
  return gemm(g, s);
}

// ---------------------------------------------------------------------------
// Causal forward with materialised probs (BackpropEngine.cs:237-388, exact-exp
// branch): one block per (b, h, i) row group; used for the exactness config
// whose recorded probabilities feed the slot backward.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void attention_fwd_probs_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ probs, float* __restrict__ out, int B, int S, int Hq, int Hkv, int D) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int group = Hq / Hkv;
  const float scale = 1.f / sqrtf((float)D);
  const int64_t rows = (int64_t)B * Hq * S;
  for (int64_t row = (int64_t)blockIdx.x * 4 + wv; row < rows; row += (int64_t)gridDim.x * 4) {
    const int i = (int)(row % S);
    const int h = (int)((row / S) % Hq);
    const int b = (int)(row / ((int64_t)S * Hq));
    const int kvh = h / group;
    float* p = probs + ((int64_t)(b * Hq + h) * S + i) * S;
    const float* qi = q + (((int64_t)b * S + i) * Hq + h) * D;
    float mx = -INFINITY;
    for (int j = lane; j <= i; j += 64) {
      const float* kj = k + (((int64_t)b * S + j) * Hkv + kvh) * D;
      float sc = 0.f;
      for (int d = 0; d < D; d++) sc += qi[d] * kj[d];
      sc *= scale;
      p[j] = sc;
      mx = fmaxf(mx, sc);
    }
    for (int j = i + 1 + lane; j < S; j += 64) p[j] = 0.f;
    mx = wave_max(mx);
    float sum = 0.f;
    for (int j = lane; j <= i; j += 64) {
      float e = expf(p[j] - mx);
      p[j] = e;
      sum += e;
    }
    sum = wave_sum(sum);
    const float inv = 1.f / sum;
    for (int j = lane; j <= i; j += 64) p[j] *= inv;
    __threadfence_block();  // this wave's probability stores are read back by all its lanes
    float* o = out + ((int64_t)b * S + i) * (Hq * D) + h * D;
    for (int d = lane; d < D; d += 64) {
      float acc = 0.f;
      for (int j = 0; j <= i; j++) acc += p[j] * v[(((int64_t)b * S + j) * Hkv + kvh) * D + d];
      o[d] = acc;
    }
  }
}

int attention_forward_probs(const float* q, const float* k, const float* v, float* probs, float* out,
                            int B, int S, int Hq, int Hkv, int D, hipStream_t s) {
  SMHIP_REQUIRE(Hkv > 0 && Hq % Hkv == 0, "attention forward: Hq must be a multiple of Hkv");
  int64_t rows = (int64_t)B * Hq * S;
  if (!rows) return SMHIP_OK;
  int g = (int)std::min<int64_t>((rows + 3) / 4, (int64_t)num_cus() * 8);
  hipLaunchKernelGGL(attention_fwd_probs_kernel, dim3(g), dim3(256), 0, s, q, k, v, probs, out, B, S, Hq, Hkv, D);
  SMHIP_CHECK_LAUNCH();
  return SMHIP_OK;
}

}  // namespace smhip

namespace smhip {

// Head-strided form of the slot backward for the exactness engine: q/dq [B*S, Hq*D],
// k/v/dk/dv [B*S, Hkv*D], probs [B, Hq, S, S].  dK/dV of query heads sharing a kv
// head are summed in head order (BackpropEngine.cs:563-582 AddHead order).
int attention_probs_backward(const float* dO, const float* q, const float* k, const float* v,
                             const float* probs, float* dq, float* dk, float* dv, int B, int S, int Hq,
                             int Hkv, int D, hipStream_t s) {
  const int grp = Hq / Hkv;
  const int64_t qd = (int64_t)Hq * D, kvd = (int64_t)Hkv * D;
  float* dP = (float*)workspace(s, sizeof(float) * (size_t)S * S, 4);
  if (!dP) return fail(SMHIP_ENOMEM, "attention backward: workspace");
  int rz = zero_bytes(dk, sizeof(float) * (size_t)B * S * kvd, s);
  if (!rz) rz = zero_bytes(dv, sizeof(float) * (size_t)B * S * kvd, s);
  if (rz) return rz;
  const float scale = 1.f / sqrtf((float)D);
  for (int b = 0; b < B; b++)
    for (int h = 0; h < Hq; h++) {
      const int kvh = h / grp;
      const float* P = probs + ((int64_t)b * Hq + h) * S * S;
      const float* dOh = dO + (int64_t)b * S * qd + h * D;
      const float* qh = q + (int64_t)b * S * qd + h * D;
      const float* kh = k + (int64_t)b * S * kvd + kvh * D;
      const float* vh = v + (int64_t)b * S * kvd + kvh * D;
      GemmArgs g{};
      g.precision = SMHIP_PREC_FP32;
      g.split_k = 1;
      g.alpha = 1.f;
      // dV += P^T dO
      g.M = S; g.N = D; g.K = S; g.beta = 1.f;
      g.A = {SRC_F32_R, P, nullptr, S};
      g.B = {SRC_F32_R, dOh, nullptr, qd};
      g.C = dv + (int64_t)b * S * kvd + kvh * D; g.ldc = kvd;
      int rc = gemm(g, s);
      if (rc) return rc;
      // dP = dO V^T
      g.M = S; g.N = S; g.K = D; g.beta = 0.f;
      g.A = {SRC_F32_K, dOh, nullptr, qd};
      g.B = {SRC_F32_K, vh, nullptr, kvd};
      g.C = dP; g.ldc = S;
      if ((rc = gemm(g, s))) return rc;
      hipLaunchKernelGGL(softmax_jacobian_rows, dim3(std::min(ceil_div(S, 4), num_cus() * 4)), dim3(256), 0, s, P, dP, S);
      SMHIP_CHECK_LAUNCH();
      // dQ = scale dS K
      g.M = S; g.N = D; g.K = S; g.alpha = scale; g.beta = 0.f;
      g.A = {SRC_F32_K, dP, nullptr, S};
      g.B = {SRC_F32_R, kh, nullptr, kvd};
      g.C = dq + (int64_t)b * S * qd + h * D; g.ldc = qd;
      if ((rc = gemm(g, s))) return rc;
      // dK += scale dS^T Q
      g.beta = 1.f;
      g.A = {SRC_F32_R, dP, nullptr, S};
      g.B = {SRC_F32_R, qh, nullptr, qd};
      g.C = dk + (int64_t)b * S * kvd + kvh * D; g.ldc = kvd;
      if ((rc = gemm(g, s))) return rc;
    }
  return SMHIP_OK;
}

}  // namespace smhip
