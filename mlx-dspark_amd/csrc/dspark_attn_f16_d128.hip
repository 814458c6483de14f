// Verify-attention kernels for f16 and head dim 128 (one translation unit per pair, so the
// build compiles them in parallel).
#include "dspark_attn.h"

namespace dspark {
namespace attn {
DSPARK_ATTN_LAUNCH(F16, 128) {
  return launch_impl<F16, 128>(a, p, B, tree, qbits, s);
}
}  // namespace attn
}  // namespace dspark
