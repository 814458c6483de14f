// Grouped expert qmm for small buckets (gfx950): the fused MoE block's projections when each
// expert sees a few rows (the verify regime: M <= 16 tokens, top-k of many experts, so a
// bucket holds ~M*k/E rows).
//
// Workgroup = 4 waves = one expert x one strip of output columns x the whole K, so no
// partial sums leave the workgroup. Wave w takes column tile w % NT and K part w / NT (KW
// parts, NT = 4 / KW tiles); the KW partial tiles are summed in LDS in part order. SwiGLU mode:
// even tiles read gate rows, odd tiles the up rows of the same 16 columns, and the strip's
// reduced tiles become h = swiglu(gate, up).
// The bucket's rows go through the MFMA in passes of RC = 4: x rows are gathered into LDS
// (4 rows x K, with their per-group sums; rows past the bucket are not read and staged as
// zeros) and MFMA A rows 4..15 repeat row 3; their outputs are dropped. One pass covers buckets
// of up to 4 rows; larger tiles loop, reusing the weights held in registers.
// Issue order of a workgroup: bucket bounds -> x row indices (pass 0) -> every weight load
// -> the tiles' scale and bias rows (contiguous 16-byte chunks, one or two per thread, kept in
// LDS) -> x loads (waiting only for the row indices, which were issued first)
// -> LDS staging -> MFMA -> LDS reduction -> output.
#pragma once

#include "dspark_qmm_splitk.h"

namespace dspark {

struct MoeRcArgs {
  const u16* x;          // [rows, K] activations
  const int* row_index;  // nullable: x row of bucket position p is row_index[p] / row_div
  const int* offsets;    // [E + 1] bucket starts (sorted pair positions)
  const u32* w0;         // [E, N, K*bits/32] plain / gate
  const u16* s0;
  const u16* b0;
  const u32* w1;         // up (SwiGLU)
  const u16* s1;
  const u16* b1;
  u16* y;                // [P, N] bf16
  long ldx, ldy;
  int K, N, row_div, P_max, mtiles;
};

// Requires K % 128 == 0, K <= KW * KSMAX * 64, N * K / 64 % 8 == 0 and 16-byte aligned scales
// and biases. KSMAX (even) is the largest K part in groups.
// PW: the weights are dspark_moe_pack's form (each expert's 16-row tiles in the MFMA lane order,
// one contiguous 1 KB wave read per group, or group pair at 4 bits), the same bytes per expert as
// the row-major layout; scales and biases keep their layout. Same products, bit for bit.
template <int BITS, int KSMAX, int KW, bool SWIGLU, bool PW = false>
__global__ __launch_bounds__(256, (KSMAX >= 24 || BITS == 8) ? 2 : 3) void moe_rc_kernel(const MoeRcArgs a) {
  constexpr int NT = 4 / KW;  // 16-column tiles per workgroup
  static_assert(KW == 1 || KW == 2 || KW == 4, "K parts");
  static_assert(!SWIGLU || NT % 2 == 0, "SwiGLU pairs gate and up tiles");
  static_assert(KSMAX % 2 == 0, "groups come in pairs");
  constexpr int RC = 4;                              // bucket rows per pass
  constexpr int KMAX = KW * KSMAX * 64;              // x elements per row
  constexpr int XP = KMAX + 8;                       // LDS row pitch (elements): rows 16 bytes apart in banks
  constexpr int XCH = (RC * KMAX / 8 + 255) / 256;   // 16-byte x chunks per thread per pass
  constexpr int GMAX = KW * KSMAX;
  __shared__ __attribute__((aligned(16))) u16 xs[RC * XP];
  __shared__ __attribute__((aligned(16))) float xsum[GMAX][RC];  // 4-bit: -128 * sum x
  __shared__ float red[4][RC * 16];
  // scales (array 0) and biases (array 1) of each tile's 16 rows, all groups, as stored:
  // row r of tile t at [t][r * G + g]
  __shared__ __attribute__((aligned(16))) u16 sbl[2][NT][16 * GMAX];

  const int strip = blockIdx.x;
  const int e = blockIdx.y / a.mtiles, mt = blockIdx.y - e * a.mtiles;
  const int p0 = a.offsets[e] + 16 * mt;
  const int p1 = min(a.offsets[e + 1], a.P_max);
  if (p0 >= p1) return;
  const int m_rows = min(16, p1 - p0);
  const int K = a.K, N = a.N, G = K >> 6;
  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
  const int c16 = lane & 15, q = lane >> 4;
  const int tile = wave % NT, kp = wave / NT;
  // K parts start on even groups (G is even): weights of 4-bit rows and the scale/bias
  // pairs are read two groups at a time
  int gs, ge;
  slice_groups(kp, KW, G, 2, gs, ge);
  const int gcount = ge - gs;  // even, >= 2
  const bool up = SWIGLU && (tile & 1);
  const int ncol = SWIGLU ? strip * (8 * NT) + 16 * (tile >> 1) + c16 : strip * (16 * NT) + 16 * tile + c16;
  const int n = min(ncol, N - 1);
  const long wstride = (long)N * (K * BITS / 32), sstride = (long)N * G;
  const u32* wmat = (up ? a.w1 : a.w0) + e * wstride;

  // x chunk i of this thread: row r (of the pass), column chunk col (8 elements)
  const int cpr = K >> 3;
  const int xtotal = RC * cpr;
  int xrow[XCH], xcol[XCH];
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    const int c = min(tid + 256 * i, xtotal - 1);
    xrow[i] = c / cpr;
    xcol[i] = c - xrow[i] * cpr;
  }
  auto src_row = [&](int r0, int r) {
    const int pr = p0 + min(r0 + r, m_rows - 1);
    return (a.row_index ? a.row_index[pr] : pr) / a.row_div;
  };
  // ---- 1. x row indices of pass 0
  int src[XCH];
#pragma unroll
  for (int i = 0; i < XCH; ++i) src[i] = src_row(0, xrow[i]);
  // ---- 2. weights of this wave's rows and K part
  WSlice<BITS, KSMAX> wsl;
  if constexpr (PW) {
    constexpr int NL = BITS == 4 ? KSMAX / 2 : KSMAX;
    const int per_tile = BITS == 4 ? (G >> 1) : G, first = BITS == 4 ? (gs >> 1) : gs;
    const int nl = BITS == 4 ? (gcount >> 1) : gcount;
    const char* tb = reinterpret_cast<const char*>(wmat) + (((long)(n >> 4) * per_tile + first) * 64 + lane) * 16;
#pragma unroll
    for (int j = 0; j < NL; ++j) wsl.v[j] = ldg128_nt(tb + (long)min(j, nl - 1) * 1024);
  } else {
    wsl.load(wmat + (long)n * (K * BITS / 32), q, gs, gcount, G);
  }
  // ---- 3. scale / bias blocks of the workgroup's tiles: 16 rows x G contiguous bf16 per
  // (array, tile), read in 16-byte chunks (2G per block; the last strip's block stops at the
  // matrix end)
  constexpr int SBCH = (4 * NT * GMAX + 255) / 256;
  const int nblk = 2 * G;
  u32x4_t sbv[SBCH];
#pragma unroll
  for (int j = 0; j < SBCH; ++j) {
    const int ci = min(tid + 256 * j, 2 * NT * nblk - 1);
    const int arr = ci / (NT * nblk), t = (ci / nblk) % NT, cc = ci % nblk;
    const bool tup = SWIGLU && (t & 1);
    const int n0 = SWIGLU ? strip * (8 * NT) + 16 * (t >> 1) : strip * (16 * NT) + 16 * t;
    const u16* base = arr == 0 ? (tup ? a.s1 : a.s0) : (tup ? a.b1 : a.b0);
    const long off = min((long)n0 * G + 8 * cc, (long)N * G - 8);  // in bounds of expert e's block
    sbv[j] = ldg128(base + e * sstride + off);
  }
  // ---- 4. x rows of pass 0 (waits only for the row indices, issued first). Only the bucket's
  // rows are read: rows past it are staged as zeros (their MFMA rows are dropped)
  u32x4_t xv[XCH];
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    xv[i] = u32x4_t{0u, 0u, 0u, 0u};
    if (xrow[i] < m_rows) xv[i] = ldg128(a.x + (long)src[i] * a.ldx + 8 * xcol[i]);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (BITS == 4 && !PW) swap_pairs(wsl);  // the packed form is stored swapped

  const u16* xl = &xs[min(c16, RC - 1) * XP + k_quarter<BITS>(q)];
  const int nrow = max(n - (ncol - c16), 0);  // this lane's row in its tile block (0 past N)
  const u32* sp = reinterpret_cast<const u32*>(&sbl[0][tile][nrow * G + gs]);
  const u32* bp = reinterpret_cast<const u32*>(&sbl[1][tile][nrow * G + gs]);
  for (int r0 = 0; r0 < m_rows; r0 += RC) {
    const int rows = min(RC, m_rows - r0);
    if (r0 > 0) {
#pragma unroll
      for (int i = 0; i < XCH; ++i) src[i] = src_row(r0, xrow[i]);
#pragma unroll
      for (int i = 0; i < XCH; ++i) {
        xv[i] = u32x4_t{0u, 0u, 0u, 0u};
        if (r0 + xrow[i] < m_rows) xv[i] = ldg128(a.x + (long)src[i] * a.ldx + 8 * xcol[i]);
      }
      __syncthreads();  // the previous pass has finished with xs, xsum and red
    }
    // ---- 5. x rows -> LDS with their per-group sums (8 lanes per (row, group))
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const bool valid = tid + 256 * i < xtotal;
      u32x4_t v = xv[i];
      float s8 = sum8_lanes(sum_bf16x8(v));
      if (BITS == 4) {
        v = perm_x_u4(v);
        s8 *= -128.0f;
      }
      if (valid) {
        *reinterpret_cast<u32x4_t*>(&xs[xrow[i] * XP + 8 * xcol[i]]) = v;
        if ((xcol[i] & 7) == 0) xsum[xcol[i] >> 3][xrow[i]] = s8;
      }
    }
    if (r0 == 0) {
#pragma unroll
      for (int j = 0; j < SBCH; ++j) {
        const int ci = tid + 256 * j;
        if (ci < 2 * NT * nblk) {
          const int arr = ci / (NT * nblk), t = (ci / nblk) % NT, cc = ci % nblk;
          *reinterpret_cast<u32x4_t*>(&sbl[arr][t][8 * cc]) = sbv[j];
        }
      }
    }
    __syncthreads();
    // ---- 6. MFMA over the wave's groups, two at a time (the part's group count is even and
    // wave-uniform). A rows >= RC repeat row RC-1. The empty asm makes the weight registers
    // opaque per pass, so the compiler cannot hoist every group's dequantized fragments out of
    // the pass loop.
#pragma unroll
    for (int j = 0; j < (BITS == 4 ? KSMAX / 2 : KSMAX); ++j) asm volatile("" : "+v"(wsl.v[j]));
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int gl = 0; gl < KSMAX; gl += 2) {
      if (gl >= gcount) break;  // wave-uniform
      const int gp = gl;
      const u32 s2 = sp[gp >> 1], b2 = bp[gp >> 1];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int g = gs + gp + h;
        const u32x4_t a0 = lds128(xl + 64 * g), a1 = lds128(xl + 64 * g + 8);
        const f32x4_t c = *reinterpret_cast<const f32x4_t*>(&xsum[g][0]);
        u32x2_t w4 = {};
        u32x4_t w8 = {};
        if constexpr (BITS == 4) {
          const u32x4_t& v = wsl.v[gl >> 1];
          w4 = h ? u32x2_t{v.z, v.w} : u32x2_t{v.x, v.y};
        } else {
          w8 = wsl.v[gl + h];
        }
        const u32 sb = h ? (s2 >> 16) : (s2 & 0xFFFFu);
        const u32 bb = h ? (b2 >> 16) : (b2 & 0xFFFFu);
        group_fma<BITS>(a0, a1, c, w8, w4, bf2f(sb), bf2f(bb), acc);
      }
    }
    // ---- 7. partial tiles (rows 0..RC-1 live in lanes q == 0) -> LDS, summed in part order
    if (q == 0) {
#pragma unroll
      for (int r = 0; r < RC; ++r) red[wave][r * 16 + c16] = acc[r];
    }
    __syncthreads();
    constexpr int OUT_TILES = SWIGLU ? NT / 2 : NT;
    if (tid < OUT_TILES * RC * 16) {
      const int ot = tid / (RC * 16), el = tid - ot * (RC * 16);
      const int r = el >> 4, cc = el & 15;
      float v0 = 0.f, v1 = 0.f;
#pragma unroll
      for (int k2 = 0; k2 < KW; ++k2) {
        if constexpr (SWIGLU) {
          v0 += red[k2 * NT + 2 * ot][el];
          v1 += red[k2 * NT + 2 * ot + 1][el];
        } else {
          v0 += red[k2 * NT + ot][el];
        }
      }
      const int col = strip * (16 * OUT_TILES) + 16 * ot + cc;
      if (r < rows && col < N) {
        float out = v0;
        if constexpr (SWIGLU) {
          // h = silu(gate) * up with the bf16 rounding of each elementwise op
          const float g = bf2f(f2bf(v0)), u = bf2f(f2bf(v1));
          const float sg = bf2f(f2bf(1.0f / (1.0f + expf(-g))));
          out = bf2f(f2bf(g * sg)) * u;
        }
        a.y[(long)(p0 + r0 + r) * a.ldy + col] = f2bf(out);
      }
    }
  }
}

}  // namespace dspark
