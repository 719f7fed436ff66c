// gemm_bf16_mq4k.hip — GEMM instantiations with a frozen Q4_K B operand decoded in the loader.
#include "gemm_bf16.hpp"

namespace smhip {
namespace g3 {
bool dispatch_q4k(int tile, const Args& a, int bmode, int c_bf16, int sp, hipStream_t s) {
  if (bmode == SRC_Q4K_K) launch_tile<SRC_BF16_K, SRC_Q4K_K>(tile, a, c_bf16, sp, s);
  else if (bmode == SRC_Q4KT) launch_tile<SRC_BF16_K, SRC_Q4KT>(tile, a, c_bf16, sp, s);
  else return false;
  return true;
}
}  // namespace g3
}  // namespace smhip
