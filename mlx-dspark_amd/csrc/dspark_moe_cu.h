// The fused MoE block's gate/up projection (SwiGLU) in the verify regime (M <= 16 tokens), one
// workgroup per CU (gfx950), for dspark_moe_pack weights.
//
// Unit = one live expert x one 16-column strip of h: the gate tile and the up tile of those 16
// columns over the whole K, SwiGLU applied in place. Units are numbered over the experts some
// token selected (the bucket bounds say which), expert by expert, and every CU takes a
// contiguous range of them, so each CU streams the same number of weight bytes whatever the
// routing. Each of the NW waves of a CU works every NW-th unit of the range on its own, with no
// barrier after the set-up: it keeps PF loads of 1 KB in flight (the unit's four scale/bias
// blocks, then its gate and up weight loads interleaved in group order), requesting one more each
// time it has used one, across unit boundaries. The M token rows of x go into LDS once per CU
// (with their per-group sums); a unit's bucket row p reads token sorted[p] / k.
//
// One workgroup per (expert, strip) (dspark_moe_rc.h) stages its own x rows and requests its
// few weights at once; this kernel carries x once per CU and keeps the CU's request stream
// busy between units. The block's time is mostly the 4-bit unpack and the per-group FMAs, not
// the stream: the same loop with its arithmetic removed takes under half the time.
//
// Bitwise the small-bucket kernel's results: bucket row r goes through MFMA row r (a single pass
// covers a bucket of up to 16 rows), every group's arithmetic is group_fma's, each K part
// (slice_groups(kp, KW, G, 2)) accumulates from zero in group order, the parts are summed in
// order from zero, and SwiGLU rounds each elementwise op to bf16 as that kernel does.
#pragma once

#include "dspark_moe_rc.h"

namespace dspark {

constexpr int kMoeCuMaxE = 256;                 // experts the unit numbering covers (4 ballots)
constexpr int kMoeCuMaxPairs = 512;             // M * k
constexpr int kMoeCuOffsInts = kMoeCuMaxE + 4;  // bucket starts in LDS (E + 1, 16-byte multiple)
constexpr int kMoeCuRows = 16;                  // token rows of x staged (M <= 16)

struct MoeCuArgs {
  const u16* x;          // [M, K] token rows
  const int* sorted;     // pair id of bucket position p (token = sorted[p] / k)
  const int* offsets;    // [E + 1] bucket starts
  const char* wg;        // packed gate tiles of expert e at wg + e * wstride
  const u16* sg;         // [E, N, G]
  const u16* bg;
  const char* wu;        // up
  const u16* su;
  const u16* bu;
  u16* h;                // [P, N] bf16
  long ldx, ldh, wstride;
  int M, E, N, k, strips;
};

// LDS row pitch of x (elements), the bytes of one wave's scale/bias slot (four [16][G] blocks)
// and the workgroup's total (with each wave's [G][16] table of its unit's MFMA seeds, 64 G bytes)
template <int G>
constexpr int moe_cu_xpitch() { return 64 * G + 8; }
template <int G>
constexpr int moe_cu_slot() { return 4 * 32 * G; }
template <int G, int NW>
constexpr size_t moe_cu_lds_bytes() {
  return (size_t)kMoeCuRows * moe_cu_xpitch<G>() * 2 + (size_t)kMoeCuRows * G * 4 + 4 * kMoeCuOffsInts +
         4 * kMoeCuMaxPairs + (size_t)NW * (moe_cu_slot<G>() + 64 * G);
}
// loads per unit (four scale/bias blocks, then the two weight tiles) and the fewest units
// (<= 8) whose loads fill whole windows of PF, or 0
template <int BITS, int G>
constexpr int moe_cu_loads() { return 4 + 2 * (BITS == 4 ? G / 2 : G); }
constexpr int moe_cu_trip_units(int L, int PF) {
  for (int r = 1; r <= 8; ++r)
    if ((r * L) % PF == 0) return r;
  return 0;
}
// first group of K part kp of KW (the small-bucket kernel's slice_groups with unit 2)
template <int G, int KW>
constexpr int moe_cu_part_start(int kp) { return 2 * ((kp * (G / 2)) / KW); }

// One unit's wave-uniform description: bucket rows and the byte offsets of its weight tiles (the
// same in wg and wu) and scale/bias blocks (the same in sg, bg, su, bu). A unit past the wave's
// last has offsets past every buffer: its loads return zeros without reading memory.
constexpr u32 kMoeCuNoUnit = 0x80000000u;
struct MoeCuUnit {
  int valid, strip, p0, rows;
  u32 wo, so;
};

// PF: loads in flight per wave. NW: waves of the workgroup (one workgroup per CU).
template <int BITS, int G, int KW, int PF, int NW>
__global__ __launch_bounds__(64 * NW) void moe_cu_kernel(const MoeCuArgs a) {
  constexpr int PT = BITS == 4 ? G / 2 : G;       // 1 KB loads per tile
  constexpr int SBB = moe_cu_slot<G>();           // scale/bias bytes per unit
  constexpr int NSB = 4;                          // their loads: one per [16 rows][G] block
  static_assert(32 * G <= 1024, "a scale/bias block in one wave load");
  constexpr int L = NSB + 2 * PT;                 // loads per unit
  static_assert(L == moe_cu_loads<BITS, G>(), "load count");
  constexpr int D = (L - 1 + PF) / L;             // units ahead the window reaches
  constexpr int R = moe_cu_trip_units(L, PF);     // units per loop trip
  static_assert(R > 0, "PF must divide R * L for some R <= 8");
  constexpr int XP = moe_cu_xpitch<G>();
  constexpr int K = 64 * G;
  constexpr int CPR = K / 8;                      // 16-byte x chunks per row
  constexpr int XCH = (kMoeCuRows * CPR + 64 * NW - 1) / (64 * NW);
  constexpr int NC = kMoeCuMaxE / 64;
  constexpr int GPL = BITS == 4 ? 2 : 1;          // groups per load
  static_assert(G % 2 == 0 && (KW == 1 || KW == 2), "K parts of whole group pairs");
  extern __shared__ __attribute__((aligned(16))) char lds[];
  u16* const xs = reinterpret_cast<u16*>(lds);                             // [16][XP]
  float* const xsum = reinterpret_cast<float*>(lds + kMoeCuRows * XP * 2);  // [16][G]
  int* const offs = reinterpret_cast<int*>(xsum + kMoeCuRows * G);         // [E + 1] bucket starts
  int* const tok = offs + kMoeCuOffsInts;                                  // token of bucket position
  char* const slots = reinterpret_cast<char*>(tok + kMoeCuMaxPairs);        // [NW][SBB]
  float* const seeds = reinterpret_cast<float*>(slots + NW * SBB);          // [NW][G][16 rows]

  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
  const int c16 = lane & 15, q = lane >> 4;

  // ---- 1. bucket bounds -> LDS; the token rows of x and the bucket order, which do not depend
  // on the routing's counts, requested at once (every 16-byte chunk of the M rows)
  const int off_t = tid <= a.E ? a.offsets[tid] : 0;
  u32x4_t xv[XCH];
  int xr[XCH], xc[XCH];
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    const int c = min(tid + 64 * NW * i, kMoeCuRows * CPR - 1);
    xr[i] = c / CPR;
    xc[i] = c - xr[i] * CPR;
    xv[i] = u32x4_t{0u, 0u, 0u, 0u};
    if (xr[i] < a.M) xv[i] = ldg128(a.x + (long)xr[i] * a.ldx + 8 * xc[i]);
  }
  const int tk = tid < a.M * a.k ? a.sorted[tid] / a.k : 0;
  __builtin_amdgcn_sched_barrier(0);
  if (tid <= a.E) offs[tid] = off_t;
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the LDS writes done, the x loads in flight
  __builtin_amdgcn_s_barrier();

  // live experts (4 ballots over E <= 256) -> this CU's contiguous range of units
  uint64_t live[NC];
  int nlive = 0;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int e = 64 * c + lane;
    live[c] = __ballot(e < a.E && offs[e + 1] > offs[e]);
    nlive += __builtin_popcountll(live[c]);
  }
  const int U = nlive * a.strips;
  const int ub = (int)((long)U * blockIdx.x / gridDim.x), ue = (int)((long)U * (blockIdx.x + 1) / gridDim.x);
  if (ub >= ue) return;  // the whole workgroup: no unit here

  // unit u: the (u / strips)-th live expert, strip u % strips
  auto unit = [&](int u) {
    MoeCuUnit d{0, 0, 0, 0, kMoeCuNoUnit, kMoeCuNoUnit};
    if (u >= ue) return d;
    int li = u / a.strips;
    d.strip = u - li * a.strips;
    int e = 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int cnt = __builtin_popcountll(live[c]);
      if (li >= 0 && li < cnt) {
        // the li-th set bit: the set bit with li set bits below it
        const uint64_t m = live[c];
        const int below = __builtin_amdgcn_mbcnt_hi((u32)(m >> 32), __builtin_amdgcn_mbcnt_lo((u32)m, 0));
        e = 64 * c + __builtin_ctzll(__ballot(((m >> lane) & 1) && below == li));
      }
      li -= cnt;
    }
    e = uniform(e);
    d.valid = 1;
    d.p0 = uniform(offs[e]);
    d.rows = uniform(offs[e + 1]) - d.p0;
    d.strip = uniform(d.strip);
    d.wo = (u32)((long)e * a.wstride + (long)d.strip * PT * 1024);
    d.so = (u32)(((long)e * a.N + 16L * d.strip) * G * 2);
    return d;
  };

  // ---- 2. this wave's first PF loads: load j (0..L-1) of a unit, 16 bytes per lane, through
  // buffer resources (byte offsets below 2^31, checked by the launcher). Scale/bias block j is
  // 32G bytes: lanes past it re-read its last 16 bytes.
  char* const slot = slots + wave * SBB;
  MoeCuUnit cur = unit(ub + wave);
  MoeCuUnit nxt[D];
#pragma unroll
  for (int d = 0; d < D; ++d) nxt[d] = unit(ub + wave + NW * (d + 1));

  auto rsrc = [](const void* p, long bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
  };
  const long wbytes = (long)a.E * a.wstride, sbytes = (long)a.E * a.N * G * 2;
  const __amdgpu_buffer_rsrc_t rw[2] = {rsrc(a.wg, wbytes), rsrc(a.wu, wbytes)};
  const __amdgpu_buffer_rsrc_t rsb[4] = {rsrc(a.sg, sbytes), rsrc(a.bg, sbytes), rsrc(a.su, sbytes),
                                         rsrc(a.bu, sbytes)};
  const u32 w_off = 16 * lane, sb_off = 16 * min(lane, 2 * G - 1);
  auto issue = [&](const MoeCuUnit& u, int j) -> u32x4_t {
    if (j < NSB) return __builtin_amdgcn_raw_buffer_load_b128(rsb[j], u.so + sb_off, 0, 0);
    const int t = (j - NSB) / 2, m = (j - NSB) % 2;
    return __builtin_amdgcn_raw_buffer_load_b128(rw[m], u.wo + w_off, t * 1024, 2);  // streamed: nt
  };
  u32x4_t buf[PF];
#pragma unroll
  for (int n = 0; n < PF; ++n) {
    const int d = n / L, j = n % L;
    buf[n] = issue(d == 0 ? cur : nxt[d - 1], j);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- 3. stage x (its loads were requested before the weights'): the 4-bit chunks permuted
  // to the order unpack_u4 produces, the per-(row, group) sums over 8 lanes (-128x at 4 bits),
  // as the small-bucket kernel stages them
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    u32x4_t v = xv[i];
    float s8 = sum8_lanes(sum_bf16x8(v));
    if (BITS == 4) {
      v = perm_x_u4(v);
      s8 *= -128.0f;
    }
    if (tid + 64 * NW * i < kMoeCuRows * CPR && xr[i] < a.M) {
      *reinterpret_cast<u32x4_t*>(&xs[xr[i] * XP + 8 * xc[i]]) = v;
      if ((xc[i] & 7) == 0) xsum[xr[i] * G + (xc[i] >> 3)] = s8;
    }
  }
  if (tid < a.M * a.k) tok[tid] = tk;
  // the LDS writes done (lgkmcnt(0); the weight loads stay in flight), then every wave's seen
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();

  // ---- 4. the units of this wave, R per loop trip so that the window's slots line up again
  // at the trip's end (R * L a multiple of PF): moving registers whose loads are still in
  // flight from slot to slot would wait for those loads
  for (int u0 = ub + wave; u0 < ue; u0 += NW * R) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int ui = u0 + NW * r;  // a unit past the range (cur.valid == 0) computes on zeros, stores nothing
      // LDS row (token) of bucket row rr (rows past the bucket repeat its last row; their
      // outputs are dropped)
      auto xrow = [&](int rr) { return tok[min(cur.p0 + max(min(rr, cur.rows - 1), 0), kMoeCuMaxPairs - 1)]; };
      const u16* xl = xs + xrow(c16) * XP + k_quarter<BITS>(q);
      // the unit's MFMA seeds (the group sums of its bucket rows) gathered once into this wave's
      // table [G][16 rows], so each group reads its lane's 4 rows with one 16-byte read
      float* const seed = seeds + wave * (G * 16);
      {
        constexpr int GL = G / 4;  // groups per lane: lane (row l % 16, groups (l / 16) * GL ..)
        const float* src = xsum + xrow(c16) * G + q * GL;
#pragma unroll
        for (int i = 0; i < GL; ++i) seed[(q * GL + i) * 16 + c16] = src[i];
        asm volatile("" ::: "memory");
      }

      f32x4_t acc[2], part[2][KW];
      u32x4_t a0[GPL], a1[GPL];  // x fragments and sums of the load's groups, read once for
      f32x4_t cs[GPL];           // both matrices
      // once load j is used, request load j + PF of the stream (this unit's or one ahead) into
      // its registers (reusing them keeps every slot in the same registers from trip to trip)
      auto refill = [&](int j) {
        const int n = j + PF, d = n / L, jj = n % L;
        __builtin_amdgcn_sched_barrier(0);
        buf[(r * L + j) % PF] = issue(d == 0 ? cur : nxt[d - 1], jj);
        __builtin_amdgcn_sched_barrier(0);
      };
      // scale/bias blocks -> this wave's slot: [sg | bg | su | bu], each [16 rows][G]
#pragma unroll
      for (int j = 0; j < NSB; ++j) {
        const u32x4_t v = buf[(r * L + j) % PF];
        if (lane < 2 * G) *reinterpret_cast<u32x4_t*>(slot + 32 * G * j + 16 * lane) = v;
        refill(j);
      }
      // weight loads: group order, the gate and up loads of a group (pair) one after the other
#pragma unroll
      for (int j = NSB; j < L; ++j) {
        const u32x4_t v = buf[(r * L + j) % PF];
        const int t = (j - NSB) / 2, m = (j - NSB) % 2;
#pragma unroll
        for (int h = 0; h < GPL; ++h) {
          const int g = GPL * t + h;
          if (m == 0) {
            a0[h] = lds128(xl + 64 * g);
            a1[h] = lds128(xl + 64 * g + 8);
            cs[h] = *reinterpret_cast<const f32x4_t*>(&seed[g * 16 + 4 * q]);
          }
          const char* sbo = slot + 2 * m * 32 * G + c16 * 2 * G + 2 * (g & ~1);
          const u32 s2 = *reinterpret_cast<const u32*>(sbo);
          const u32 b2 = *reinterpret_cast<const u32*>(sbo + 32 * G);
          const u32 sbits = (g & 1) ? (s2 >> 16) : (s2 & 0xFFFFu);
          const u32 bbits = (g & 1) ? (b2 >> 16) : (b2 & 0xFFFFu);
          u32x2_t w4 = {0u, 0u};
          if constexpr (BITS == 4) w4 = h ? u32x2_t{v.z, v.w} : u32x2_t{v.x, v.y};
#pragma unroll
          for (int kp = 0; kp < KW; ++kp)
            if (g == moe_cu_part_start<G, KW>(kp)) acc[m] = f32x4_t{0.f, 0.f, 0.f, 0.f};
          group_fma<BITS>(a0[h], a1[h], cs[h], v, w4, bf2f(sbits), bf2f(bbits), acc[m]);
#pragma unroll
          for (int kp = 0; kp < KW; ++kp)
            if (g == moe_cu_part_start<G, KW>(kp + 1) - 1) part[m][kp] = acc[m];
        }
        refill(j);
      }
      // parts summed in order from zero; SwiGLU with each elementwise op rounded to bf16
      f32x4_t vs[2];
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        vs[m] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kp = 0; kp < KW; ++kp) vs[m] += part[m][kp];
      }
      const int col = cur.strip * 16 + c16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = 4 * q + i;
        if (rr < cur.rows) {
          const float g = bf2f(f2bf(vs[0][i])), u = bf2f(f2bf(vs[1][i]));
          const float sg = bf2f(f2bf(1.0f / (1.0f + expf(-g))));
          a.h[(long)(cur.p0 + rr) * a.ldh + col] = f2bf(bf2f(f2bf(g * sg)) * u);
        }
      }
      // next unit: the look-ahead units shift by one
      cur = nxt[0];
#pragma unroll
      for (int d = 0; d + 1 < D; ++d) nxt[d] = nxt[d + 1];
      nxt[D - 1] = unit(ui + NW * (D + 1));
    }
  }
}

// ---- host side (dspark_moe_cu.hip)
// Whether the packed block's gate/up projection at these shapes runs moe_cu_kernel
bool moe_cu_gate_up(long M, long H, long I, long E, long k, int bits);
// The gate/up projection (K = H) on stream s
int launch_moe_cu(const MoeCuArgs& a, long K, int bits, hipStream_t s);

}  // namespace dspark
