// Verify-attention kernels for f16 and head dim 64 (one translation unit per pair, so the
// build compiles them in parallel).
#include "dspark_attn.h"

namespace dspark {
namespace attn {
DSPARK_ATTN_LAUNCH(F16, 64) {
  return launch_impl<F16, 64>(a, p, B, tree, qbits, s);
}
}  // namespace attn
}  // namespace dspark
