// Inner loop of the small-M affine qmm shared by the dense kernel (dspark_qmm.hip) and the
// grouped expert kernels (dspark_moe.hip).
//
// One wave accumulates, for NT tiles of 16 output features and one 16-row tile of x, the
// partial sums over quantization groups [g0, g1):
//     acc[j][r] (lane l) = y[row 4*(l>>4) + r][feature 16*j + (l & 15)]  (partial over groups)
// Per group (64 k): the x fragment (A operand, 2 x 16 bytes per lane) is loaded once and
// reused for the NT weight fragments; sum_k x (or -128 * sum_k x for 4-bit, see below) is one
// MFMA pair against a constant operand and reused too.
#pragma once

#include "dspark_common.h"

namespace dspark {

// bf16 pair (128 + nibble t, 128 + nibble t+4) of a packed 4-bit word, for t = 0..3.
__device__ __forceinline__ u32x4_t unpack_u4(u32 w) {
  const u32 m = 0x000F000Fu, c = 0x43004300u;
  return u32x4_t{(w & m) | c, ((w >> 4) & m) | c, ((w >> 8) & m) | c, ((w >> 12) & m) | c};
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

// Pointers one lane reads, already offset to its own row and quarter:
//   xr    = x row (clamped to a valid row) + 16*q     (bf16)
//   wr[j] = packed row n_j + (BITS == 4 ? 2*q : 4*q)  (words)
//   sr[j], br[j] = scales / biases row n_j            (bf16)
template <int BITS, int NT, int CH>
__device__ __forceinline__ void qmm_wave_partial(const u16* __restrict__ xr, const u32* const (&wr)[NT],
                                                 const u16* const (&sr)[NT], const u16* const (&br)[NT], int g0,
                                                 int g1, f32x4_t (&acc)[NT]) {
  // constant B operand that turns an MFMA into a row sum: -128 (4-bit offset) or 1.0
  constexpr u32 kconst = (BITS == 4) ? 0xC300C300u : 0x3F803F80u;
  const u32x4_t kb = {kconst, kconst, kconst, kconst};
  constexpr float bias_mul = (BITS == 4) ? (-1.0f / 128.0f) : 1.0f;
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};

  for (int gc = g0; gc < g1; gc += CH) {
    u32x4_t xa[CH][2];
    WFrag<BITS> wf[CH][NT];
    u32 sv[CH][NT], bv[CH][NT];
    // loads: unconditional (clamped group index) so the wait counts stay static
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int g = min(gc + i, g1 - 1);
      xa[i][0] = ldg128(xr + 64 * g);
      xa[i][1] = ldg128(xr + 64 * g + 8);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if constexpr (BITS == 4)
          wf[i][j].v = ldg64(wr[j] + 8 * g);
        else
          wf[i][j].v = ldg128(wr[j] + 16 * g);
        sv[i][j] = sr[j][g];
        bv[i][j] = br[j][g];
      }
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      if (gc + i < g1) {
        u32x4_t a0 = xa[i][0], a1 = xa[i][1];
        if constexpr (BITS == 4) {
          a0 = perm_x_u4(a0);
          a1 = perm_x_u4(a1);
        }
        // 4-bit: c = -128 * sum x seeds the product MFMA, cancelling the +128 field offset;
        // 8-bit: c = sum x.  Either way the bias term is (bias * bias_mul) * c.
        f32x4_t c = mfma16x16x32(a0, kb, zero);
        c = mfma16x16x32(a1, kb, c);
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          f32x4_t p;
          if constexpr (BITS == 4) {
            p = mfma16x16x32(a0, unpack_u4(wf[i][j].v.x), c);
            p = mfma16x16x32(a1, unpack_u4(wf[i][j].v.y), p);
          } else {
            p = mfma16x16x32(a0, unpack_u8(wf[i][j].v.x, wf[i][j].v.y), zero);
            p = mfma16x16x32(a1, unpack_u8(wf[i][j].v.z, wf[i][j].v.w), p);
          }
          const float s = bf2f(sv[i][j]);
          const float b = bf2f(bv[i][j]) * bias_mul;
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[j][r] = __builtin_fmaf(b, c[r], __builtin_fmaf(s, p[r], acc[j][r]));
        }
      }
    }
  }
}

// Lane pointers for weight row n (clamped by the caller) and quarter q.
template <int BITS>
__device__ __forceinline__ const u32* wrow_ptr(const u32* w, long n, int K, int q) {
  constexpr int WPR_SHIFT = (BITS == 4) ? 3 : 2;  // words per row = K >> WPR_SHIFT
  return w + n * (K >> WPR_SHIFT) + (BITS == 4 ? 2 * q : 4 * q);
}

}  // namespace dspark
