// Verify-attention kernels for bf16 and head dim 256 (one translation unit per pair, so the
// build compiles them in parallel).
#include "dspark_attn.h"

namespace dspark {
namespace attn {
DSPARK_ATTN_LAUNCH(BF16, 256) {
  return launch_impl<BF16, 256>(a, p, B, tree, qbits, s);
}
}  // namespace attn
}  // namespace dspark
