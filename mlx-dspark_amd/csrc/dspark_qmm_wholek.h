// Dense small-M affine qmm without split-K (gfx950): one workgroup per 16-row output tile over
// all of K, for the launches where one such workgroup per CU beats the split-K kernel (a
// [4096, 4096] 8-bit matrix: 256 tiles, one per CU, 64 KB of weights each). Its NW waves split
// K into contiguous octet ranges (8 groups = 512 k each), multiply their ranges, and the NW
// partial tiles are summed in LDS in wave order. Nothing leaves the workgroup but the bf16 tile:
// no fp32 partials, no arrival counters, no workspace.
//
// Per lane (row c16 of the tile, quarter q) and group g: the x fragments (rows of x in the MFMA's
// A operand) are read straight from global memory (x is small and stays in L2), the weight
// fragment from the row (or the packed tile stream), and the bias term's per-row sum of x comes
// from the same MFMA against an all-ones B operand, in the output layout. Same per-group
// arithmetic as qmm_sk_kernel (acc = fma(b, sum x, fma(s, P, acc)) with P exact in fp32). With
// one octet per wave (NW = G / 8) the octet partials and their wave-order sum are the split-K
// plan's 8-group slices summed in slice order, so the two kernels agree bit for bit wherever the
// per-group sums of x (here an MFMA against ones, there lane sums) are exact in fp32, as they are
// for bf16 x of ordinary range. Row-major and packed weights give the same bits, at every M.
#pragma once

#include "dspark_qmm_splitk.h"

namespace dspark {

// One octet (8 groups) of a lane's operands.
template <int BITS>
struct WkOctet {
  u32x4_t x[16];                         // a0, a1 of each group
  u32x4_t w[BITS == 8 ? 8 : 4];          // 8-bit: one 16-byte fragment per group; 4-bit: per pair
  u32x4_t s, b;                          // scales / biases of the lane's row, 8 groups
};

// SBVEC: the row-major scales and biases are 16-byte aligned (one 16-byte load per octet),
// else they are read as 8 bf16 each.
template <int BITS, int NW, bool PACKED, bool SBVEC>
__global__ __launch_bounds__(64 * NW) void qmm_wk_kernel(const QmmSkArgs args) {
  const int bx = blockIdx.x;
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kQmmMaxProblems; ++i)
    if (i < args.count && bx >= args.p[i].strip0) pi = i;
  const QmmSkProb& P = args.p[pi];
  const int N = P.N, K = P.K, G = K >> 6;
  const int tile = bx - P.strip0;
  const int mt = blockIdx.y;
  const int m_base = mt * 16;
  const int m_rows = min(16, args.M - m_base);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = uniform(tid >> 6);
  const int c16 = lane & 15, q = lane >> 4;
  const int n = min(tile * 16 + c16, N - 1);
  const int U = G >> 3;  // octets
  const int o0 = (wave * U) / NW, o1 = ((wave + 1) * U) / NW;

  const u16* xrow = P.x + (long)(m_base + min(c16, m_rows - 1)) * P.ldx + k_quarter<BITS>(q);
  const u32x4_t ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0 pairs

  auto load = [&](WkOctet<BITS>& r, int o) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const u16* xp = xrow + 64 * (8 * o + j);
      r.x[2 * j] = ldg128(xp);
      r.x[2 * j + 1] = ldg128(xp + 8);
    }
    if constexpr (PACKED) {
      const long t16 = n >> 4;
      const u16* blk = P.s + ((t16 * U + o) * 2) * 128 + 8 * c16;
      r.s = ldg128_nt(blk);
      r.b = ldg128_nt(blk + 128);
      constexpr int NL = BITS == 4 ? 4 : 8;
      const int per_tile = BITS == 4 ? (G >> 1) : G;
      const char* tb = reinterpret_cast<const char*>(P.w) + ((t16 * per_tile + NL * o) * 64 + lane) * 16;
#pragma unroll
      for (int j = 0; j < NL; ++j) r.w[j] = ldg128_nt(tb + j * 1024);
    } else {
      if constexpr (SBVEC) {
        r.s = ldg128(P.s + (long)n * G + 8 * o);
        r.b = ldg128(P.b + (long)n * G + 8 * o);
      } else {
        const u16* sp = P.s + (long)n * G + 8 * o;
        const u16* bp = P.b + (long)n * G + 8 * o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          r.s[i] = (u32)sp[2 * i] | ((u32)sp[2 * i + 1] << 16);
          r.b[i] = (u32)bp[2 * i] | ((u32)bp[2 * i + 1] << 16);
        }
      }
      const u32* wrow = P.w + (long)n * (K * BITS / 32);
      if constexpr (BITS == 8) {
#pragma unroll
        for (int j = 0; j < 8; ++j) r.w[j] = ldg128_nt(wrow + 16 * (8 * o + j) + 4 * q);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) r.w[j] = ldg128_nt(wrow + 8 * (8 * o + 2 * j) + 4 * q);
      }
    }
  };

  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const WkOctet<BITS>& r) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      u32x4_t a0 = r.x[2 * j], a1 = r.x[2 * j + 1];
      if constexpr (BITS == 4) {
        a0 = perm_x_u4(a0);
        a1 = perm_x_u4(a1);
      }
      const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
      f32x4_t c = mfma16x16x32(a1, ones, mfma16x16x32(a0, ones, zero));  // sum x of rows 4q + r
      u32x2_t w4 = {0u, 0u};
      if constexpr (BITS == 4) {
        if constexpr (PACKED) {
          w4 = (j & 1) ? u32x2_t{r.w[j >> 1].z, r.w[j >> 1].w} : u32x2_t{r.w[j >> 1].x, r.w[j >> 1].y};
        } else {
          u32x2_t f0, f1;
          frag_u4(r.w[j >> 1], f0, f1);
          w4 = (j & 1) ? f1 : f0;
        }
        c *= -128.0f;
      }
      const u32 sbits = (r.s[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
      const u32 bbits = (r.b[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
      group_fma<BITS>(a0, a1, c, r.w[BITS == 8 ? j : 0], w4, bf2f(sbits), bf2f(bbits), acc);
    }
  };

  WkOctet<BITS> ra;
  for (int o = o0; o < o1; ++o) {
    load(ra, o);
    // every load of the octet is issued before any is consumed
    __builtin_amdgcn_sched_barrier(0);
    compute(ra);
  }

  __shared__ f32x4_t red[NW][64];
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  f32x4_t v = red[0][lane];
#pragma unroll
  for (int w = 1; w < NW; ++w) v += red[w][lane];
  const int ncol = tile * 16 + c16;
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const int m = 4 * q + rr;
    if (m < m_rows && ncol < N) P.y[(long)(m_base + m) * P.ldy + ncol] = f2bf(v[rr]);
  }
}

}  // namespace dspark
