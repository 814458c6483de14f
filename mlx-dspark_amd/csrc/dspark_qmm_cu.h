// Dense small-M affine qmm, one workgroup per CU over all of K (gfx950), for packed weights
// with K = 4096 and one to six 16-row tiles per CU (the 8B-class MLP's gate+up pair: 1536
// tiles, six per CU; a [4096, 4096] matrix: one per CU); or over one of KP parts of a larger K,
// the KP workgroups of a tile group meeting through the split-K workspace (the [4096, 12288]
// down projection: 4 tiles per CU, K in 4 parts of 3072).
//
// A workgroup of TPW * KH waves owns TPW consecutive 16-row tiles; wave w works tile w % TPW
// over K part w / TPW (64 / KH groups). The 16 rows of x (128 KB) and the tiles' scale/bias
// blocks go straight into LDS (global_load_lds_dwordx4, no registers) first, so the CU's
// in-order request stream carries x once, ahead of the weights. Each wave then keeps 8 groups
// of weights in flight: it requests its first 8 groups, and one more group each time it
// multiplies one, so no wave stalls issuing far ahead of its work, the waves of a SIMD multiply
// side by side as their groups land, and there is no split-K exchange at all. (Requesting a
// wave's whole part at once stalled the issue behind the CU's full request queue and left each
// SIMD multiplying one wave after another: slower than split-K.)
//
// Bitwise the split-K kernel's results (dspark_qmm_splitk.h) for the same slice count S: the
// per-group arithmetic is the same (acc = fma(b, sum x, fma(s, P, acc)), P from the same two
// MFMAs), each wave keeps one accumulator per split-K slice of its part (acc from zero at the
// slice's first group), the group sums of x are formed in the staging kernel's order (8-value
// chunk sums, then the 8 chunks pairwise), and the slice accumulators are summed in slice order
// from zero before the bf16 rounding, as the split-K last arriver does.
#pragma once

#include "dspark_qmm_splitk.h"

namespace dspark {

constexpr int kCuK = 4096;  // K a workgroup covers at most (16 x rows fit LDS)
// LDS row pitch of x (elements): 32 bytes of padding per row
constexpr int cu_xpitch(int kc) { return kc + 16; }
// LDS bytes of a workgroup of `tpw` tiles over `kc` columns of K: x, the tiles' scale/bias
// blocks, the group sums
constexpr size_t cu_lds_bytes(int tpw, int kc = kCuK) {
  return (size_t)16 * cu_xpitch(kc) * 2 + (size_t)tpw * (kc / 512) * 512 + (size_t)(kc / 64) * 16 * 4;
}

// GSL: groups per split-K slice (8, 16 or 32). Tiles are numbered across the problems
// (args.p[i].strip0 = first tile of problem i); every problem reads the same x.
// KC: the columns of K a workgroup covers; a K of KP x KC runs KP workgroups per tile group
// (blockIdx.z = K part), which leave their slices' partials in the split-K workspace
// (args.p[0].part, [M tile][tile][slice][64 lanes] x 16 bytes) and count themselves on the tile
// group's counter (args.p[0].ctr); the last to arrive sums every slice in order, as the
// split-K kernel's last arriver does.
template <int BITS, int TPW, int KH, int GSL, int KC = kCuK, int KP = 1>
__global__ __launch_bounds__(64 * TPW * KH) void qmm_cu_kernel(const QmmSkArgs args, int tiles) {
  constexpr int kparts = KP;
  constexpr int NW = KH * TPW;
  constexpr int G = KC / 64;             // groups of this workgroup's K part
  constexpr int GPW = G / KH;            // groups per wave (its part of K)
  constexpr int SPW = GPW / GSL;         // split-K slices per wave
  constexpr int S = G / GSL;             // slices of this workgroup's K part
  constexpr int XP = cu_xpitch(KC);
  constexpr int OCT = G / 8;             // scale/bias octets per tile and K part
  static_assert(KC % 512 == 0 && OCT % 2 == 0 && GPW % GSL == 0, "whole 1 KB chunks and slices");
  static_assert(GPW % GSL == 0 && GSL % 2 == 0, "slices within a K part");
  extern __shared__ __attribute__((aligned(16))) char lds[];
  u16* const xs = reinterpret_cast<u16*>(lds);                          // [16][XP]
  char* const sbl = lds + 16 * XP * 2;                                  // [TPW][OCT][512 B]
  float* const xsum = reinterpret_cast<float*>(sbl + TPW * OCT * 512);  // [G][16]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = uniform(tid >> 6);
  const int c16 = lane & 15, q = lane >> 4;
  const int tl = wave % TPW, kp = wave / TPW;
  const int mt = blockIdx.y;
  const int kpw = blockIdx.z;  // this workgroup's K part
  const int m_base = mt * 16;
  const int m_rows = min(16, args.M - m_base);
  // the tile of this wave and its problem; a tile past the last one re-reads the last
  const int t = min((int)blockIdx.x * TPW + tl, tiles - 1);
  auto prob_of = [&](int tt) {
    int pi = 0;
#pragma unroll
    for (int i = 1; i < kQmmMaxProblems; ++i)
      if (i < args.count && tt >= args.p[i].strip0) pi = i;
    return pi;
  };
  const QmmSkProb& P = args.p[prob_of(t)];
  const long t16 = t - P.strip0;  // tile within its problem

  // ---- 1. x (16 rows, clamped to the last real row) and the tiles' scale/bias blocks -> LDS.
  // One wave instruction moves 1 KB: 64 lanes x 16 bytes to consecutive LDS addresses.
  {
    constexpr int CPRW = KC / 512;             // 1 KB chunks per row
    constexpr int XCH = 16 * CPRW;
    constexpr int XPER = (XCH + NW - 1) / NW;
    const u16* x = args.p[0].x + (long)kpw * KC;
    const long ldx = args.p[0].ldx;
#pragma unroll
    for (int i = 0; i < XPER; ++i) {
      const int c = min(wave + NW * i, XCH - 1);
      const int row = c / CPRW, part = c - row * CPRW;
      const u16* src = x + (long)(m_base + min(row, m_rows - 1)) * ldx + 512 * part + 8 * lane;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(xs + row * XP + 512 * part), 16, 0, 0);
    }
    constexpr int SCH = TPW * OCT / 2;  // 1 KB chunks: two octets of one tile
    constexpr int SPER = (SCH + NW - 1) / NW;
#pragma unroll
    for (int i = 0; i < SPER; ++i) {
      const int c = min(wave + NW * i, SCH - 1);
      const int ct = c / (OCT / 2), co = 2 * (c % (OCT / 2));
      const int tt = min((int)blockIdx.x * TPW + ct, tiles - 1);
      const QmmSkProb& Q = args.p[prob_of(tt)];
      const u16* src = Q.s + (((long)(tt - Q.strip0) * kparts + kpw) * OCT + co) * 256 + 8 * lane;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(sbl + (ct * OCT + co) * 512), 16, 0,
                                       0);
    }
  }
  // ---- 2. the first PF weight fragments of this wave's part of its tile; the rest are requested one
  // per group as the multiply consumes them, so a wave never stalls issuing far ahead of its
  // work and the copies into LDS land before most weight requests are queued
  __builtin_amdgcn_sched_barrier(0);
  constexpr int NL = BITS == 4 ? GPW / 2 : GPW;
  constexpr int PF = BITS == 4 ? 4 : 8;  // 8 groups in flight per wave
  u32x4_t wv[NL];
  const int per_part = BITS == 4 ? (G >> 1) : G;  // loads per tile and K part
  const char* tb =
      reinterpret_cast<const char*>(P.w) + (((t16 * kparts + kpw) * per_part + kp * NL) * 64 + lane) * 16;
#pragma unroll
  for (int j = 0; j < PF; ++j) {
    wv[j] = ldg128_nt(tb + (long)j * 1024);
    __builtin_amdgcn_sched_barrier(0);
  }
  static_assert(PF < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(PF | (7 << 4) | (15 << 8));
  __builtin_amdgcn_s_barrier();

  // ---- 3. group sums of x, in the split-K staging's order: each 8-value chunk summed in order,
  // the 8 chunks of a group then pairwise (c0+c1)+(c2+c3), + ((c4+c5)+(c6+c7)); 4-bit: times
  // -128, and every chunk rewritten in place in the (t, t+4) order unpack_u4 produces (as the
  // split-K staging stores it)
  for (int i = tid; i < 16 * G; i += 64 * NW) {
    const int row = i & 15, g = i >> 4;
    u16* src = xs + row * XP + 64 * g;
    float cs[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const u32x4_t v = lds128(src + 8 * c);
      cs[c] = sum_bf16x8(v);
      if (BITS == 4) *reinterpret_cast<u32x4_t*>(src + 8 * c) = perm_x_u4(v);
    }
    float s = ((cs[0] + cs[1]) + (cs[2] + cs[3])) + ((cs[4] + cs[5]) + (cs[6] + cs[7]));
    if (BITS == 4) s *= -128.0f;
    xsum[g * 16 + row] = s;
  }
  // the sums' LDS writes done (lgkmcnt(0), vmcnt not waited on), then every wave's are visible
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();

  // ---- 4. the multiply: groups kp*GPW .. +GPW-1, one accumulator per split-K slice; load j + PF
  // is requested just before load j's groups are multiplied
  f32x4_t accs[SPW];
  const u16* xl = xs + c16 * XP + k_quarter<BITS>(q);
  const char* sb_t = sbl + tl * OCT * 512 + 16 * c16;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    if (j + PF < NL) {
      wv[j + PF] = ldg128_nt(tb + (long)(j + PF) * 1024);
      __builtin_amdgcn_sched_barrier(0);
    }
    constexpr int GPL = BITS == 4 ? 2 : 1;  // groups per load
#pragma unroll
    for (int h = 0; h < GPL; ++h) {
      const int gw = GPL * j + h;  // group within the wave's K part
      const int g = kp * GPW + gw;
      if (gw % GSL == 0) acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const char* sbo = sb_t + (g >> 3) * 512 + 2 * (g & 7);
      const u32 sbits = *reinterpret_cast<const u16*>(sbo);
      const u32 bbits = *reinterpret_cast<const u16*>(sbo + 256);
      u32x2_t w4 = {0u, 0u};
      if constexpr (BITS == 4) w4 = h ? u32x2_t{wv[j].z, wv[j].w} : u32x2_t{wv[j].x, wv[j].y};
      const u32x4_t a0 = lds128(xl + 64 * g), a1 = lds128(xl + 64 * g + 8);
      const f32x4_t c = *reinterpret_cast<const f32x4_t*>(&xsum[g * 16 + 4 * q]);
      group_fma<BITS>(a0, a1, c, wv[j], w4, bf2f(sbits), bf2f(bbits), acc);
      if (gw % GSL == GSL - 1) accs[gw / GSL] = acc;
    }
  }

  if constexpr (KP > 1) {
    // ---- 5'. the slices' partials leave the workgroup: device-coherent stores, this thread's
    // complete before the workgroup counts itself; the last of the kparts workgroups of the
    // tile group reads every slice (coherent loads) and sums them in order from zero
    __shared__ int last_flag;
    const int S_all = S * kparts;
    const bool real = (int)blockIdx.x * TPW + tl < tiles;
    const long tile_all = (long)mt * tiles + t;
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        args.p[0].part, 0, (int)min((long)gridDim.y * tiles * S_all * 1024, 0x7FFFFFF0L), kBufferRsrcWord3);
    if (real) {
#pragma unroll
      for (int s = 0; s < SPW; ++s)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, accs[s]), prs,
                                               (int)(((tile_all * S_all + kpw * S + kp * SPW + s) * 64 + lane) * 16), 0,
                                               kCoherentSc1);
    }
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0): this thread's partial stores are complete
    __syncthreads();
    int* const ctr = args.p[0].ctr + (long)mt * gridDim.x + blockIdx.x;
    if (tid == 0) last_flag = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kparts - 1;
    __syncthreads();
    if (!last_flag) return;
    if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // zero for the next call
    if (kp != 0 || !real) return;
    f32x4_t v = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < S_all; s0 += kSliceChunk) {
      u32x4_t pv[kSliceChunk];
#pragma unroll
      for (int s2 = 0; s2 < kSliceChunk; ++s2)
        if (s0 + s2 < S_all)  // wave-uniform
          pv[s2] = __builtin_amdgcn_raw_buffer_load_b128(prs, (int)(((tile_all * S_all + s0 + s2) * 64 + lane) * 16), 0,
                                                         kCoherentSc1);
#pragma unroll
      for (int s2 = 0; s2 < kSliceChunk; ++s2)
        if (s0 + s2 < S_all) v += __builtin_bit_cast(f32x4_t, pv[s2]);
    }
    const int ncol = (int)t16 * 16 + c16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * q + r;
      if (m < m_rows && ncol < P.N) P.y[(long)(m_base + m) * P.ldy + ncol] = f2bf(v[r]);
    }
    return;
  }

  // ---- 5. the slice accumulators of the tile's K parts meet in LDS (x's area, free once
  // every wave is done multiplying); the wave of the first part sums them in slice order
  __syncthreads();
  f32x4_t* red = reinterpret_cast<f32x4_t*>(lds);  // [TPW][S][64 lanes]
#pragma unroll
  for (int s = 0; s < SPW; ++s) red[(tl * S + kp * SPW + s) * 64 + lane] = accs[s];
  __syncthreads();
  if (kp != 0 || (int)blockIdx.x * TPW + tl >= tiles) return;
  f32x4_t v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < S; ++s) v += red[(tl * S + s) * 64 + lane];
  const int ncol = (int)t16 * 16 + c16;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * q + r;
    if (m < m_rows && ncol < P.N) P.y[(long)(m_base + m) * P.ldy + ncol] = f2bf(v[r]);
  }
}

}  // namespace dspark
