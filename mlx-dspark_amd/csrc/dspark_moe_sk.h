// Grouped expert qmm for the fused MoE block (gfx950): the dense split-K qmm's structure
// (dspark_qmm_splitk.h) applied per expert over its bucket of (token, slot) rows.
//
// Workgroup = 4 waves = one 64-row strip of ONE expert's weights x one K slice x one 16-row
// tile of that expert's bucket. Plain mode: the strip is 64 consecutive output rows. SwiGLU
// mode: waves 0/1 take gate rows [32s, 32s+32), waves 2/3 the up rows of the same 32 columns,
// and the strip's reduced tile is turned into h = swiglu(gate, up) for those 32 columns.
// The bucket's x rows (gathered through the sorted pair list) are staged in LDS with their
// per-group sums, every x load issued before the weight stream, exactly as in the dense kernel.
// Slices of a strip are combined by the last workgroup to arrive (device-scope counter per
// (expert, strip, row tile)), in slice order, so results are deterministic. Workgroups of an
// expert with no rows in their tile exit at once.
#pragma once

#include "dspark_qmm_splitk.h"

namespace dspark {

struct MoeSkArgs {
  const u16* x;          // [rows, K] activations
  const int* row_index;  // nullable: x row of bucket position p is row_index[p] / row_div
  const int* offsets;    // [E + 1] bucket starts (sorted pair positions)
  const u32* w0;         // [E, N0, K*bits/32] plain / gate
  const u16* s0;
  const u16* b0;
  const u32* w1;         // up (SwiGLU)
  const u16* s1;
  const u16* b1;
  u16* y;                // [P, ncols] bf16
  float* part;           // [E][strips][mtiles][S][16][64]
  int* ctr;              // [E][strips][mtiles]
  long ldx, ldy;
  int K, N, row_div, P_max, strips, mtiles, S;
};

template <int BITS, int KSMAX, bool SBVEC, bool SWIGLU>
__global__ __launch_bounds__(256) void moe_sk_kernel(const MoeSkArgs a) {
  constexpr int NS = 4;
  constexpr int XP = KSMAX * 64 + 8;
  __shared__ __attribute__((aligned(16))) u16 xs[16 * XP];
  __shared__ __attribute__((aligned(16))) float xsum[KSMAX * 16];
  __shared__ float tile_out[SWIGLU ? 16 * 64 : 1];
  __shared__ int last_flag;

  const int strip = blockIdx.x, sl = blockIdx.y;
  const int e = blockIdx.z / a.mtiles, mt = blockIdx.z - e * a.mtiles;
  const int p0 = a.offsets[e] + 16 * mt;
  const int p1 = min(a.offsets[e + 1], a.P_max);
  if (p0 >= p1) return;
  const int m_rows = min(16, p1 - p0);
  const int S = a.S, K = a.K, N = a.N;
  const int G = K >> 6;
  int gs, ge;
  slice_groups(sl, S, G, slice_unit(G, BITS), gs, ge);
  const int gcount = ge - gs;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, q = lane >> 4;
  // output column this lane's tile row maps to, and which matrix it reads
  const bool up = SWIGLU && (wave >= 2);
  const int ncol = SWIGLU ? strip * 32 + 16 * (wave & 1) + c16 : strip * 64 + 16 * wave + c16;
  const int n = min(ncol, N - 1);
  const long wstride = (long)N * (K * BITS / 32), sstride = (long)N * G;
  const u32* wmat = (up ? a.w1 : a.w0) + e * wstride;
  const u16* smat = (up ? a.s1 : a.s0) + e * sstride;
  const u16* bmat = (up ? a.b1 : a.b0) + e * sstride;

  // ---- 1. x slice of the bucket tile, every load first
  constexpr int XCH = (2 * KSMAX) / NS;
  const int cpr = gcount * 8;
  const int xtotal = 16 * cpr;
  u32x4_t xv[XCH];
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    const int c = min(tid + i * 64 * NS, xtotal - 1);
    const int row = c / cpr, col = c - row * cpr;
    const int pr = p0 + min(row, m_rows - 1);
    const int src = (a.row_index ? a.row_index[pr] : pr) / a.row_div;
    xv[i] = ldg128(a.x + (long)src * a.ldx + (long)gs * 64 + 8 * col);
  }
  // ---- 2. weights of this lane's row in the slice
  WSlice<BITS, KSMAX> wsl;
  wsl.load(wmat + (long)n * (K * BITS / 32), q, gs, gcount, G);
  // ---- 3. scales / biases
  constexpr int SBV = (KSMAX + 7) / 8;
  u32x4_t svv[SBV], bvv[SBV];
  u32 svs[SBVEC ? 1 : KSMAX], bvs[SBVEC ? 1 : KSMAX];
  const u16* srow = smat + (long)n * G + gs;
  const u16* brow = bmat + (long)n * G + gs;
  if constexpr (SBVEC) {
#pragma unroll
    for (int j = 0; j < SBV; ++j) {
      const int jj = min(j, (gcount >> 3) - 1);
      svv[j] = ldg128(srow + 8 * jj);
      bvv[j] = ldg128(brow + 8 * jj);
    }
  } else {
#pragma unroll
    for (int gl = 0; gl < KSMAX; ++gl) {
      const int g = min(gl, gcount - 1);
      svs[gl] = srow[g];
      bvs[gl] = brow[g];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // ---- 4. x -> LDS with the group sums (branch-free; a chunk past the slice goes to the pad)
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    const int c0 = tid + i * 64 * NS;
    const bool valid = c0 < xtotal;
    const int c = min(c0, xtotal - 1);
    const int row = c / cpr, col = c - row * cpr;
    u32x4_t v = xv[i];
    float s8 = sum_bf16x8(v);
    s8 += shfl_xor(s8, 1);
    s8 += shfl_xor(s8, 2);
    s8 += shfl_xor(s8, 4);
    if (BITS == 4) {
      v = perm_x_u4(v);
      s8 *= -128.0f;
    }
    *reinterpret_cast<u32x4_t*>(&xs[row * XP + (valid ? 8 * col : KSMAX * 64)]) = v;
    if (valid && (c & 7) == 0) xsum[(col >> 3) * 16 + row] = s8;
  }
  __syncthreads();
  // ---- 5. MFMA over the slice
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  const u16* xl = &xs[c16 * XP + k_quarter<BITS>(q)];
  u32x2_t w4[2] = {};
#pragma unroll
  for (int gl = 0; gl < KSMAX; ++gl) {
    if (gl < gcount) {
      if (BITS == 4 && (gl & 1) == 0) frag_u4(wsl.v[gl >> 1], w4[0], w4[1]);
      const u32x4_t a0 = lds128(xl + 64 * gl), a1 = lds128(xl + 64 * gl + 8);
      const f32x4_t c = *reinterpret_cast<const f32x4_t*>(&xsum[gl * 16 + 4 * q]);
      u32 sbits, bbits;
      if constexpr (SBVEC) {
        sbits = bf_field(svv[gl >> 3], gl & 7);
        bbits = bf_field(bvv[gl >> 3], gl & 7);
      } else {
        sbits = svs[gl];
        bbits = bvs[gl];
      }
      group_fma<BITS>(a0, a1, c, wsl.v[BITS == 4 ? 0 : gl], w4[gl & 1], bf2f(sbits), bf2f(bbits), acc);
    }
  }
  // ---- 6. epilogue. tile column t (0..63) of this workgroup = wave * 16 + c16
  const int tcol = 16 * wave + c16;
  float v[4];
  if (S == 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = acc[r];
  } else {
    const long tix = ((long)e * a.strips + strip) * a.mtiles + mt;
    float* part = a.part + tix * S * (16 * 64);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      __hip_atomic_store(&part[(long)sl * 1024 + (4 * q + r) * 64 + tcol], acc[r], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
      last_flag = (__hip_atomic_fetch_add(&a.ctr[tix], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1);
    __syncthreads();
    if (!last_flag) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = 0.f;
    for (int s0 = 0; s0 < S; s0 += kSliceChunk) {  // slice order, kSliceChunk requests at a time
      float pv[4][kSliceChunk];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int s2 = 0; s2 < kSliceChunk; ++s2)
          pv[r][s2] = __hip_atomic_load(&part[(long)min(s0 + s2, S - 1) * 1024 + (4 * q + r) * 64 + tcol],
                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int s2 = 0; s2 < kSliceChunk; ++s2)
          if (s0 + s2 < S) v[r] += pv[r][s2];
    }
    if (tid == 0) __hip_atomic_store(&a.ctr[tix], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if constexpr (!SWIGLU) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * q + r;
      if (m < m_rows && ncol < N) a.y[(long)(p0 + m) * a.ldy + ncol] = f2bf(v[r]);
    }
  } else {
    // gate tile columns 0..31 (waves 0, 1), up tile columns 32..63 (waves 2, 3)
#pragma unroll
    for (int r = 0; r < 4; ++r) tile_out[(4 * q + r) * 64 + tcol] = v[r];
    __syncthreads();
    for (int t = tid; t < 16 * 32; t += 256) {
      const int m = t >> 5, cc = t & 31;
      const int col = strip * 32 + cc;
      if (m < m_rows && col < N) {
        const float g = bf2f(f2bf(tile_out[m * 64 + cc])), u = bf2f(f2bf(tile_out[m * 64 + 32 + cc]));
        const float sg = bf2f(f2bf(1.0f / (1.0f + expf(-g))));
        a.y[(long)(p0 + m) * a.ldy + col] = f2bf(bf2f(f2bf(g * sg)) * u);
      }
    }
  }
}

}  // namespace dspark
