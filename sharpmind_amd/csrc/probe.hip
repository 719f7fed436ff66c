// probe.hip — the sustained bf16 MFMA rate of the device (a measurement for the roofline).
//
// Eight independent 32x32x16 bf16 accumulators per wave, operands in registers, no memory
// traffic in the loop, 8 waves per workgroup, one workgroup per CU: the rate the matrix
// cores sustain under this load (clocks included), against which the GEMM kernels' fraction
// of the published dense peak can be read.
#include "common.hpp"
#include "kernels.hpp"

namespace smhip {

__global__ __launch_bounds__(512) void mfma_rate_kernel(int iters, float* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    a[j] = (__bf16)(float)((lane + j) & 7);
    b[j] = (__bf16)(float)((lane * 3 + j) & 7);
  }
  floatx16 acc[8];
#pragma unroll
  for (int j = 0; j < 8; j++)
#pragma unroll
    for (int e = 0; e < 16; e++) acc[j][e] = 0.f;
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; j++) s += acc[j][lane & 15];
  if (s == -1.f) sink[threadIdx.x] = s;  // never true: keeps the loop
}

int probe_mfma_bf16(double* tflops) {
  float* sink = (float*)workspace(nullptr, 4096, 6);
  SMHIP_REQUIRE(sink, "probe: workspace");
  hipEvent_t a, b;
  SMHIP_CHECK_HIP(hipEventCreate(&a));
  SMHIP_CHECK_HIP(hipEventCreate(&b));
  const int iters = 20000, wgs = num_cus();
  hipLaunchKernelGGL(mfma_rate_kernel, dim3(wgs), dim3(512), 0, nullptr, 2000, sink);  // clocks up
  hipEventRecord(a, nullptr);
  hipLaunchKernelGGL(mfma_rate_kernel, dim3(wgs), dim3(512), 0, nullptr, iters, sink);
  hipEventRecord(b, nullptr);
  SMHIP_CHECK_HIP(hipEventSynchronize(b));
  float ms = 0.f;
  hipEventElapsedTime(&ms, a, b);
  hipEventDestroy(a);
  hipEventDestroy(b);
  const double flops = 2.0 * 32 * 32 * 16 * 8 * (double)iters * 8 * wgs;  // per wave: 8 MFMAs x iters
  *tflops = flops / (ms * 1e-3) / 1e12;
  return SMHIP_OK;
}

}  // namespace smhip

extern "C" int smhip_probe_mfma_bf16(double* tflops) {
  SMHIP_REQUIRE(tflops, "probe_mfma_bf16: null output");
  return smhip::probe_mfma_bf16(tflops);
}
