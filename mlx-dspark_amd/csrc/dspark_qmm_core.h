// Dequantization pieces of the small-M affine qmm shared by the dense split-K kernel
// (dspark_qmm_splitk.h) and the expert kernels (dspark_moe.hip, dspark_moe_sk.h): packed
// fields -> exact bf16 MFMA operands, and the matching order of the x fragments.
#pragma once

#include "dspark_common.h"

namespace dspark {

// bf16 pair (128 + nibble t, 128 + nibble t+4) of a packed 4-bit word, for t = 0..3.
__device__ __forceinline__ u32x4_t unpack_u4(u32 w) {
  const u32 m = opaque_sgpr(0x000F000Fu), c = opaque_vgpr(0x43004300u);
  return u32x4_t{and_or(w, m, c), and_or(w >> 4, m, c), and_or(w >> 8, m, c), and_or(w >> 12, m, c)};
}

// Reorders 8 consecutive bf16 x-values [x0..x7] into [x0,x4,x1,x5,x2,x6,x3,x7], the field
// order unpack_u4 produces.
__device__ __forceinline__ u32x4_t perm_x_u4(u32x4_t u) {
  return u32x4_t{__builtin_amdgcn_perm(u.z, u.x, 0x05040100u), __builtin_amdgcn_perm(u.z, u.x, 0x07060302u),
                 __builtin_amdgcn_perm(u.w, u.y, 0x05040100u), __builtin_amdgcn_perm(u.w, u.y, 0x07060302u)};
}

__device__ __forceinline__ u32 cvt_u8_pair(u32 w, int byte) {
  const float f0 = (float)((w >> (8 * byte)) & 0xFFu);
  const float f1 = (float)((w >> (8 * byte + 8)) & 0xFFu);
  return pack_bf16x2(f0, f1);
}

// Two words of 8-bit fields -> 8 bf16 in natural order (exact: integers 0..255).
__device__ __forceinline__ u32x4_t unpack_u8(u32 lo, u32 hi) {
  return u32x4_t{cvt_u8_pair(lo, 0), cvt_u8_pair(lo, 2), cvt_u8_pair(hi, 0), cvt_u8_pair(hi, 2)};
}

template <int BITS>
struct WFrag;
template <>
struct WFrag<4> {
  u32x2_t v;
};
template <>
struct WFrag<8> {
  u32x4_t v;
};

// Lane pointers for weight row n (clamped by the caller) and quarter q.
template <int BITS>
__device__ __forceinline__ const u32* wrow_ptr(const u32* w, long n, int K, int q) {
  constexpr int WPR_SHIFT = (BITS == 4) ? 3 : 2;  // words per row = K >> WPR_SHIFT
  return w + n * (K >> WPR_SHIFT) + (BITS == 4 ? 2 * q : 4 * q);
}

}  // namespace dspark
