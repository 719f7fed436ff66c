// gemm_bf16_mbk.hip — GEMM instantiations with a bf16 k-contiguous B operand (TAG 1: the
// backward dX products through the frozen base, named apart for profilers).
#include "gemm_bf16.hpp"

namespace smhip {
namespace g3 {
bool dispatch_bf16k(int tile, const Args& a, int bmode, int c_bf16, int sp, bool dx, hipStream_t s) {
  if (bmode != SRC_BF16_K) return false;
  if (dx) launch_tile<SRC_BF16_K, SRC_BF16_K, 1>(tile, a, c_bf16, sp, s);
  else launch_tile<SRC_BF16_K, SRC_BF16_K>(tile, a, c_bf16, sp, s);
  return true;
}
}  // namespace g3
}  // namespace smhip
