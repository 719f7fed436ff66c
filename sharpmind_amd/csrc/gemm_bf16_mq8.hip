// gemm_bf16_mq8.hip — GEMM instantiations with a frozen Q8_0 B operand decoded in the loader.
#include "gemm_bf16.hpp"

namespace smhip {
namespace g3 {
bool dispatch_q8(int tile, const Args& a, int bmode, int c_bf16, int sp, hipStream_t s) {
  if (bmode == SRC_Q8_K) launch_tile<SRC_BF16_K, SRC_Q8_K>(tile, a, c_bf16, sp, s);
  else if (bmode == SRC_Q8T) launch_tile<SRC_BF16_K, SRC_Q8T>(tile, a, c_bf16, sp, s);
  else return false;
  return true;
}
}  // namespace g3
}  // namespace smhip
