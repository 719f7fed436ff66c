// gemm_bf16_mbr.hip — GEMM instantiations with a bf16 row-contiguous B operand (and the
// row-contiguous A of the weight-gradient products).
#include "gemm_bf16.hpp"

namespace smhip {
namespace g3 {
bool dispatch_bf16r(int tile, const Args& a, int amode, int bmode, int c_bf16, int sp, hipStream_t s) {
  if (bmode != SRC_BF16_R) return false;
  if (amode == SRC_BF16_K) launch_tile<SRC_BF16_K, SRC_BF16_R>(tile, a, c_bf16, sp, s);
  else launch_tile<SRC_BF16_R, SRC_BF16_R>(tile, a, 0, sp, s);
  return true;
}
}  // namespace g3
}  // namespace smhip
