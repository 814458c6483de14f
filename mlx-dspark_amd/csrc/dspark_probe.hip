// Streaming-read bandwidth probe: the measured denominator of the roofline fractions bench.py
// reports (the reference measures its own with an fp16 matvec, calibrate.py:871-894).
//
// Grid-stride 16-byte non-temporal loads, eight in flight per thread, folded with XOR; the sink
// is written only if the fold equals a sentinel, so the loads cannot be removed and the store
// almost never happens.
#include <algorithm>

#include "dspark_common.h"

namespace dspark {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;
constexpr u32 kProbeSentinel = 0x9E3779B9u;

__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const u32x4_t* __restrict__ p, long n16,
                                                                   u32* __restrict__ sink) {
  u32x4_t acc = {0u, 0u, 0u, 0u};
  const long stride = (long)gridDim.x * kProbeThreads * kProbeUnroll;
  for (long base = (long)blockIdx.x * kProbeThreads * kProbeUnroll + threadIdx.x; base < n16; base += stride) {
    u32x4_t v[kProbeUnroll];
#pragma unroll
    for (int j = 0; j < kProbeUnroll; ++j) {
      const long i = base + (long)j * kProbeThreads;
      v[j] = i < n16 ? ldg128_nt(p + i) : acc;
    }
#pragma unroll
    for (int j = 0; j < kProbeUnroll; ++j) acc ^= v[j];
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == kProbeSentinel) sink[0] = 1u;
}

}  // namespace
}  // namespace dspark

using namespace dspark;

extern "C" int dspark_stream_read(const void* p, size_t bytes, uint32_t* sink, dspark_stream stream) {
  if (!p || !sink) return fail(DSPARK_ERR_ARG, "stream_read: null pointer");
  if (!aligned(p, 16) || bytes % 16 || bytes == 0)
    return fail(DSPARK_ERR_ALIGN, "stream_read: 16-byte aligned pointer and a positive multiple of 16 bytes");
  const long n16 = (long)(bytes / 16);
  const long per_block = (long)kProbeThreads * kProbeUnroll;
  const unsigned blocks = (unsigned)std::min<long>((n16 + per_block - 1) / per_block, 4096L);
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(kProbeThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4_t*>(p), n16, sink);
  return check_launch("dspark_stream_read");
}
