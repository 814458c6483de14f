// Dense small-M affine qmm, split-K across workgroups (gfx950).
//
// Workgroup = NS waves = NS tiles of 16 output features ("strip" of 16*NS rows) x one slice of
// K (blockIdx.y). The slice of x (16 rows x slice) is staged once in LDS and shared by the NS
// waves, together with its per-group row sums (the bias term's sum_j x[m, j], reduced across
// 8 lanes during staging). Load order is what keeps this a single memory round trip: every
// x-slice load of the thread is issued first, then the strip's scales and biases, then every
// weight load of its 16 rows x slice (16-byte loads straight from the packed rows).
// Vector-memory completion is counted in issue order, so staging x, scales and biases in LDS
// does not wait for the weight stream; the MFMA loop then consumes weights as they land.
// Slices of one strip are combined by the last workgroup to finish (a device-scope arrival
// counter per strip), always in slice order 0..S-1, so the result is deterministic and
// independent of M and of arrival order.
#pragma once

#include "dspark_qmm_core.h"

namespace dspark {

constexpr int kQmmMaxProblems = DSPARK_QMM_MAX_PROBLEMS;
constexpr int kQmmMaxSlices = 32;
constexpr int kSliceChunk = 16;  // partials the last arriver requests at a time
// buffer resource word 3 for gfx9-family raw buffers, and the sc1 (device-coherent) cache
// policy of buffer loads and stores
constexpr int kBufferRsrcWord3 = 0x00020000;
constexpr int kCoherentSc1 = 16;

struct QmmSkProb {
  const u16* x;
  const u32* w;
  const u16* s;
  const u16* b;
  u16* y;
  float* part;  // [mtiles][strips][S][16*NS columns][16 rows] fp32 partials (S > 1)
  int* ctr;     // [mtiles][strips] arrival counters (zero between calls)
  long ldx;
  long ldy;
  int N;
  int K;
  int strip0;  // first blockIdx.x of this problem
  int strips;
  int hN;      // SWIGLU: width of y (= h), the unpadded gate / up rows
};

struct QmmSkArgs {
  QmmSkProb p[kQmmMaxProblems];
  int count;
  int M;
  int S;  // K slices (<= kQmmMaxSlices)
};

__device__ __forceinline__ u32x4_t lds128(const void* p) { return *reinterpret_cast<const u32x4_t*>(p); }

// bf16 field `i` (0..7) of a 16-byte vector of 8 bf16
__device__ __forceinline__ u32 bf_field(u32x4_t v, int i) {
  const u32 wd = v[i >> 1];
  return (i & 1) ? (wd >> 16) : (wd & 0xFFFFu);
}

__device__ __forceinline__ float sum_bf16x8(u32x4_t v) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) s += bf2f(v[i] & 0xFFFFu) + bf2f(v[i] >> 16);
  return s;
}

// K slices are cut on multiples of `unit` groups: 8 when G is a multiple of 8 (every slice's
// scale/bias run is then whole 16-byte chunks), else 2 for 4-bit rows (their weights are read
// two groups per load, see WSlice), else 1.
__host__ __device__ inline int slice_unit(int G, int bits) { return G % 8 == 0 ? 8 : bits == 4 ? 2 : 1; }

// Groups [gs, ge) of K slice sl of S (S <= ceil(G / unit), so no slice is empty).
__host__ __device__ inline void slice_groups(int sl, int S, int G, int unit, int& gs, int& ge) {
  const int units = (G + unit - 1) / unit;
  gs = unit * ((sl * units) / S);
  ge = min(unit * (((sl + 1) * units) / S), G);
}

// Most slices G groups can be cut into with none of them empty.
inline long max_slices(long G, int bits) {
  const long unit = slice_unit((int)G, bits);
  return (G + unit - 1) / unit;
}

// Kernel instantiation (8 or 16 groups) that holds the largest of S slices of G groups, or 0
// when a slice would exceed 16 groups (K > 32768 at 32 slices) or S would leave a slice empty
// (the kernels read group gs - 1 of an empty slice).
inline int slice_capacity(long G, long S, int bits) {
  const long unit = slice_unit((int)G, bits), units = (G + unit - 1) / unit;
  if (S < 1 || S > units) return 0;
  const long per = unit * ((units + S - 1) / S);
  return per <= 8 ? 8 : per <= 16 ? 16 : 0;
}

// The weight fragments of one row over a K slice, loaded with 16-byte loads.
//  8-bit: load gl = group gs+gl; lane quarter q holds bytes [16q, 16q+16), k [16q, 16q+16).
//  4-bit: load j covers groups gs+2j and gs+2j+1 (64 bytes of the row): quarters 0,1 read
//    bytes [16q, 16q+16) of the first group, quarters 2,3 bytes [16(q-2), ...) of the second,
//    so one wave instruction reads 64 contiguous bytes of each of its 16 rows. frag_u4()
//    swaps the halves between lanes l and l+32 (v_permlane32_swap), after which every lane
//    holds 8 bytes of each group: bytes [8qs, 8qs+8), k [16qs, 16qs+16), qs = 2(q&1) + (q>>1).
//  Loads past the slice repeat its last group (pair); their fragments are never used.
template <int BITS, int KSMAX>
struct WSlice {
  static_assert(BITS == 8 || KSMAX % 2 == 0, "4-bit slices hold whole pairs");
  u32x4_t v[BITS == 4 ? KSMAX / 2 : KSMAX];

  // wrow: packed row (words); G: groups per row
  __device__ __forceinline__ void load(const u32* wrow, int q, int gs, int gcount, int G) {
    if constexpr (BITS == 4) {
      const int pairs = (gcount + 1) >> 1;
#pragma unroll
      for (int j = 0; j < KSMAX / 2; ++j) {
        const int g = gs + 2 * min(j, pairs - 1);
        const int qq = (g + 1 < G) ? q : (q & 1);  // no second group at the row end: re-read the first
        v[j] = ldg128_nt(wrow + 8 * g + 4 * qq);
      }
    } else {
#pragma unroll
      for (int gl = 0; gl < KSMAX; ++gl) v[gl] = ldg128_nt(wrow + 16 * (gs + min(gl, gcount - 1)) + 4 * q);
    }
  }
};

// In place: every 4-bit load j becomes {group 2j lo, hi, group 2j+1 lo, hi} of this lane
// (the exchange frag_u4 performs).
template <int KSMAX>
__device__ __forceinline__ void swap_pairs(WSlice<4, KSMAX>& w) {
#pragma unroll
  for (int j = 0; j < KSMAX / 2; ++j) {
    const auto r0 = __builtin_amdgcn_permlane32_swap(w.v[j].x, w.v[j].z, false, false);
    const auto r1 = __builtin_amdgcn_permlane32_swap(w.v[j].y, w.v[j].w, false, false);
    w.v[j] = u32x4_t{r0[0], r1[0], r0[1], r1[1]};
  }
}

// (words of group 2j, words of group 2j+1) of 4-bit load j, each {k 16qs..+7, k 16qs+8..+15}
__device__ __forceinline__ void frag_u4(u32x4_t v, u32x2_t& f0, u32x2_t& f1) {
  const auto r0 = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
  const auto r1 = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
  f0 = u32x2_t{r0[0], r1[0]};
  f1 = u32x2_t{r0[1], r1[1]};
}

// lane quarter q's k offset inside a group: 16q (8-bit), 16qs (4-bit, after frag_u4)
template <int BITS>
__device__ __forceinline__ int k_quarter(int q) {
  return BITS == 4 ? 16 * (2 * (q & 1) + (q >> 1)) : 16 * q;
}

// One group's contribution to a lane's 4 outputs: acc += s * (x . q) + b * sum x, with the
// x fragments a0/a1 (from LDS) and c = the row sums (4-bit: -128 * sum x, the MFMA seed).
template <int BITS>
__device__ __forceinline__ void group_fma(u32x4_t a0, u32x4_t a1, f32x4_t c, u32x4_t w8, u32x2_t w4, float sf,
                                          float bfv, f32x4_t& acc) {
  f32x4_t p;
  if constexpr (BITS == 4) {
    p = mfma16x16x32(a0, unpack_u4(w4.x), c);
    p = mfma16x16x32(a1, unpack_u4(w4.y), p);
  } else {
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    p = mfma16x16x32(a0, unpack_u8(w8.x, w8.y), zero);
    p = mfma16x16x32(a1, unpack_u8(w8.z, w8.w), p);
  }
  constexpr float bias_mul = (BITS == 4) ? (-1.0f / 128.0f) : 1.0f;
  const float bm = bfv * bias_mul;
#pragma unroll
  for (int r = 0; r < 4; ++r) acc[r] = __builtin_fmaf(bm, c[r], __builtin_fmaf(sf, p[r], acc[r]));
}

// PACKED: the weights and scales/biases come in the tiled form dspark_qmm_pack writes (see
// pack_* below): P.w is the tile stream, P.s the scale/bias tiles (P.b unused); requires
// SBVEC (G % 8 == 0). Same products, bit for bit, as the reference layout.
// SWIGLU (packed only): the tiles alternate gate tile t, up tile t (dspark_qmm_pack_swiglu),
// so a strip holds 2 gate and 2 up tiles and its finished sums become
// h = bf16(swiglu(bf16(gate), bf16(up))) for 32 columns of h, the same values an unfused
// gate / up launch and the SwiGLU kernel produce.
template <int BITS, int NS, int KSMAX, bool SBVEC, bool PACKED = false, bool SWIGLU = false>
__global__ __launch_bounds__(64 * NS) void qmm_sk_kernel(const QmmSkArgs args) {
  static_assert(!PACKED || SBVEC, "the packed form needs 8-group slices");
  static_assert(!SWIGLU || PACKED, "the fused SwiGLU reads the interleaved packed form");
  constexpr int XP = KSMAX * 64 + 8;  // LDS row pitch of the staged x slice (elements)
  __shared__ __attribute__((aligned(16))) u16 xs[16 * XP];
  // per group: 16 row sums (8-bit: sum x; 4-bit: -128 * sum x, the MFMA seed)
  __shared__ __attribute__((aligned(16))) float xsum[KSMAX * 16];
  __shared__ int last_flag;
  // SWIGLU: the strip's finished sums, [16*NS columns][16 rows] (pitch 17)
  __shared__ float hsum[SWIGLU ? 16 * NS * 17 : 1];
  // SBVEC: scales (0) and biases (1) of the strip's 16*NS rows over the slice, row pitch
  // SBP (16-byte rows; 4-byte reads of 16 consecutive rows fall in distinct banks)
  constexpr int SBP = KSMAX + 8;
  constexpr bool SBLDS = SBVEC && !PACKED;
  __shared__ __attribute__((aligned(16))) u16 sbl[SBLDS ? 2 : 1][SBLDS ? 16 * NS : 1][SBLDS ? SBP : 1];

  const int bx = blockIdx.x;
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kQmmMaxProblems; ++i)
    if (i < args.count && bx >= args.p[i].strip0) pi = i;
  const QmmSkProb& P = args.p[pi];
  const int N = P.N, K = P.K;
  const int strip = bx - P.strip0;
  const int S = args.S;
  const int sl = blockIdx.y;
  const int mt = blockIdx.z;
  const int G = K >> 6;
  int gs, ge;
  slice_groups(sl, S, G, slice_unit(G, BITS), gs, ge);
  const int gcount = ge - gs;
  const int m_base = mt * 16;
  const int m_rows = min(16, args.M - m_base);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = uniform(tid >> 6);
  const int c16 = lane & 15, q = lane >> 4;
  const int ncol = strip * 16 * NS + 16 * wave + c16;
  const int n = min(ncol, N - 1);

  // ---- 1. the x slice (16 rows; rows >= M are clamped duplicates): issue every load now.
  // 16-byte chunk c covers row c / (8*gcount), group (c / 8) % gcount, eighth c % 8; the 8
  // chunks of one (row, group) sit in 8 consecutive lanes. The chunk count 128*gcount is a
  // multiple of 64, so each wave either handles a whole iteration or skips it.
  constexpr int XCH = (2 * KSMAX) / NS;  // max chunks per thread (128 * KSMAX / (64 * NS))
  static_assert(XCH >= 1 && (2 * KSMAX) % NS == 0, "x staging shape");
  const int cpr = gcount * 8;  // chunks per row
  const int xtotal = 16 * cpr;
  u32x4_t xv[XCH];
  {
    const u16* xb = P.x + (long)gs * 64;
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int c = min(tid + i * 64 * NS, xtotal - 1);
      const int row = c / cpr, col = c - row * cpr;
      const int src = m_base + min(row, m_rows - 1);
      xv[i] = ldg128(xb + (long)src * P.ldx + 8 * col);
    }
  }
  // ---- 2. scales / biases of the strip's rows over the slice. SBVEC (G a multiple of 8, so
  // slices are too; 16-byte aligned arrays): the workgroup reads them as 16-byte chunks,
  // one (array, row, 8 groups) each, into LDS. Otherwise every lane reads its own row's.
  constexpr int SBCH = SBLDS ? (2 * 16 * NS * (KSMAX / 8) + 64 * NS - 1) / (64 * NS) : 1;
  u32x4_t sbv[SBCH];
  u32 svs[SBVEC ? 1 : KSMAX], bvs[SBVEC ? 1 : KSMAX];
  u32x4_t tsv[PACKED ? KSMAX / 8 : 1], tbv[PACKED ? KSMAX / 8 : 1];  // packed: 8 groups per load
  const int cpa = 16 * NS * (gcount >> 3);  // chunks per array
  const long tile16 = n >> 4;                 // packed: this wave's 16-row tile
  if constexpr (PACKED) {
    // tile (t, octet j): 256 B of scales then 256 B of biases, row r at 16 r
#pragma unroll
    for (int j = 0; j < KSMAX / 8; ++j) {
      const int jj = min(j, (gcount >> 3) - 1);
      const u16* blk = P.s + ((tile16 * (G >> 3) + (gs >> 3) + jj) * 2) * 128 + 8 * c16;
      tsv[j] = ldg128_nt(blk);
      tbv[j] = ldg128_nt(blk + 128);
    }
  } else if constexpr (SBVEC) {
#pragma unroll
    for (int j = 0; j < SBCH; ++j) {
      const int ci = min(tid + 64 * NS * j, 2 * cpa - 1);
      const int arr = ci / cpa, r = (ci % cpa) / (gcount >> 3), jj = ci % (gcount >> 3);
      const int nr = min(strip * 16 * NS + r, N - 1);
      sbv[j] = ldg128((arr ? P.b : P.s) + (long)nr * G + gs + 8 * jj);
    }
  } else {
    const u16* srow = P.s + (long)n * G + gs;
    const u16* brow = P.b + (long)n * G + gs;
#pragma unroll
    for (int gl = 0; gl < KSMAX; ++gl) {
      const int g = min(gl, gcount - 1);
      svs[gl] = srow[g];
      bvs[gl] = brow[g];
    }
  }
  // ---- 3. every weight load of this lane's row in the slice (clamped, unconditional)
  WSlice<BITS, KSMAX> wsl;
  if constexpr (PACKED) {
    // tile stream: 1 KB per (16-row tile, group) for 8-bit, per (tile, group pair) for 4-bit,
    // lane l's 16 bytes at 16 l, already in the order the MFMA B operand takes
    constexpr int NL = BITS == 4 ? KSMAX / 2 : KSMAX;
    const int per_tile = BITS == 4 ? (G >> 1) : G, first = BITS == 4 ? (gs >> 1) : gs;
    const int nl = BITS == 4 ? (gcount >> 1) : gcount;
    const char* tb = reinterpret_cast<const char*>(P.w) + ((tile16 * per_tile + first) * 64 + lane) * 16;
#pragma unroll
    for (int j = 0; j < NL; ++j) wsl.v[j] = ldg128_nt(tb + (long)min(j, nl - 1) * 1024);
  } else {
    wsl.load(P.w + (long)n * (K * BITS / 32), q, gs, gcount, G);
  }
  // every load above is issued before anything consumes one (keeps the scheduler from
  // interleaving the x processing, and its waits, into the load sequence)
  __builtin_amdgcn_sched_barrier(0);
  // ---- 4. x slice -> LDS with the group sums (8-lane butterfly reduction). Branch-free, so
  // the compiler cannot sink a load into a conditional block behind the weight stream: a chunk
  // past the slice (whole waves only) lands in the row's unused 16-byte pad.
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    const int c0 = tid + i * 64 * NS;
    const bool valid = c0 < xtotal;
    const int c = min(c0, xtotal - 1);
    const int row = c / cpr, col = c - row * cpr;
    u32x4_t v = xv[i];
    float s8 = sum8_lanes(sum_bf16x8(v));
    if (BITS == 4) {
      // store the 8 values in the (t, t+4) order unpack_u4 produces
      v = perm_x_u4(v);
      s8 *= -128.0f;
    }
    *reinterpret_cast<u32x4_t*>(&xs[row * XP + (valid ? 8 * col : KSMAX * 64)]) = v;
    if (valid && (c & 7) == 0) xsum[(col >> 3) * 16 + row] = s8;
  }
  if constexpr (SBLDS) {
#pragma unroll
    for (int j = 0; j < SBCH; ++j) {
      const int ci = tid + 64 * NS * j;
      if (ci < 2 * cpa) {
        const int arr = ci / cpa, r = (ci % cpa) / (gcount >> 3), jj = ci % (gcount >> 3);
        *reinterpret_cast<u32x4_t*>(&sbl[arr][r][8 * jj]) = sbv[j];
      }
    }
  }
  __syncthreads();

  // ---- 5. MFMA loop over the slice, a pair of groups per step (gcount is wave-uniform)
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  const u16* xl = &xs[c16 * XP + k_quarter<BITS>(q)];
  const int srow_l = SBVEC ? 16 * wave + c16 : 0;
#pragma unroll
  for (int gl = 0; gl < KSMAX; gl += 2) {
    if (gl >= gcount) break;
    u32x2_t w4[2] = {};
    if constexpr (BITS == 4) {
      if constexpr (PACKED) {
        w4[0] = u32x2_t{wsl.v[gl >> 1].x, wsl.v[gl >> 1].y};
        w4[1] = u32x2_t{wsl.v[gl >> 1].z, wsl.v[gl >> 1].w};
      } else {
        frag_u4(wsl.v[gl >> 1], w4[0], w4[1]);
      }
    }
    u32 s2 = 0, b2 = 0;
    if constexpr (PACKED) {
      s2 = tsv[gl >> 3][(gl & 7) >> 1];
      b2 = tbv[gl >> 3][(gl & 7) >> 1];
    } else if constexpr (SBVEC) {
      s2 = *reinterpret_cast<const u32*>(&sbl[0][srow_l][gl]);
      b2 = *reinterpret_cast<const u32*>(&sbl[1][srow_l][gl]);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h == 1 && gl + 1 >= gcount) break;
      const int g = gl + h;
      const u32x4_t a0 = lds128(xl + 64 * g), a1 = lds128(xl + 64 * g + 8);
      // rows 4q..4q+3. (Read as a float vector: bit-casting ext-vector elements one by one
      // miscompiles to a single-dword read.)
      const f32x4_t c = *reinterpret_cast<const f32x4_t*>(&xsum[g * 16 + 4 * q]);
      u32 sbits, bbits;
      if constexpr (SBVEC) {
        sbits = h ? (s2 >> 16) : (s2 & 0xFFFFu);
        bbits = h ? (b2 >> 16) : (b2 & 0xFFFFu);
      } else {
        sbits = svs[g];
        bbits = bvs[g];
      }
      group_fma<BITS>(a0, a1, c, wsl.v[BITS == 4 ? 0 : g], w4[h], bf2f(sbits), bf2f(bbits), acc);
    }
  }

  // ---- 6. epilogue: lane holds y[m_base + 4q + r][ncol]
  constexpr int TW = 16 * NS;  // strip width
  // SWIGLU: thread -> h columns 32 * strip + (tid >> 3) of rows 2 (tid & 7), +1; gate tile 2s + j
  // of the strip is its columns 32 j .. 32 j + 15, the matching up tile the next 16
  auto swiglu_out = [&]() {
    const int hc = tid >> 3, r0 = 2 * (tid & 7);
    const int gc = 32 * (hc >> 4) + (hc & 15);
    const int col = strip * (TW / 2) + hc;
#pragma unroll
    for (int r = r0; r < r0 + 2; ++r) {
      const float g = bf2f(f2bf(hsum[gc * 17 + r])), u = bf2f(f2bf(hsum[(gc + 16) * 17 + r]));
      if (r < m_rows && col < P.hN) P.y[(long)(m_base + r) * P.ldy + col] = f2bf(swiglu_bf16(g, u));
    }
  };
  static_assert(!SWIGLU || TW * 8 == 2 * 64 * NS, "two SwiGLU outputs per thread");
  if (S == 1) {
    if constexpr (SWIGLU) {
#pragma unroll
      for (int r = 0; r < 4; ++r) hsum[(16 * wave + c16) * 17 + 4 * q + r] = acc[r];
      __syncthreads();
      swiglu_out();
      return;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * q + r;
      if (m < m_rows && ncol < N) P.y[(long)(m_base + m) * P.ldy + ncol] = f2bf(acc[r]);
    }
    return;
  }
  // Partials travel through device-coherent (sc1) stores and loads, so no L2 write-back or
  // invalidate is needed: each thread waits for its stores to complete before the workgroup
  // arrives on the strip's counter (device-scope atomic), and the last arriver reads the other
  // slices with coherent loads, summing in slice order. A strip's partials are
  // [S][TW columns][16 rows] fp32: a lane's 4 rows of one column are one 16-byte chunk, so each
  // wave stores 1 KB contiguous and the last arriver reads one chunk per slice per thread.
  const long tile = (long)mt * P.strips + strip;
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc(P.part + (tile * S) * (16 * TW), 0, S * 16 * TW * 4, kBufferRsrcWord3);
  const f32x4_t accv = acc;
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, accv), prs,
                                         ((sl * TW + 16 * wave + c16) * 16 + 4 * q) * 4, 0, kCoherentSc1);
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0): this thread's partial stores are complete
  __syncthreads();
  if (tid == 0)
    last_flag = (__hip_atomic_fetch_add(&P.ctr[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1);
  __syncthreads();
  if (!last_flag) return;
  // thread -> (column tid / 4, rows 4 (tid % 4) .. + 3): one chunk per slice, summed in slice
  // order; kSliceChunk slices are requested at a time
  static_assert(TW * 4 == 64 * NS, "one 4-row chunk per thread");
  const int col = tid >> 2, rq = tid & 3;
  f32x4_t v = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < S; s0 += kSliceChunk) {
    u32x4_t pv[kSliceChunk];
#pragma unroll
    for (int s2 = 0; s2 < kSliceChunk; ++s2)
      if (s0 + s2 < S)  // wave-uniform: no request past the last slice
        pv[s2] = __builtin_amdgcn_raw_buffer_load_b128(prs, (((s0 + s2) * TW + col) * 16 + 4 * rq) * 4, 0,
                                                       kCoherentSc1);
#pragma unroll
    for (int s2 = 0; s2 < kSliceChunk; ++s2)
      if (s0 + s2 < S) v += __builtin_bit_cast(f32x4_t, pv[s2]);
  }
  if constexpr (SWIGLU) {
#pragma unroll
    for (int r = 0; r < 4; ++r) hsum[col * 17 + 4 * rq + r] = v[r];
    __syncthreads();
    swiglu_out();
  } else {
    const int nc = strip * TW + col;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * rq + r;
      if (m < m_rows && nc < N) P.y[(long)(m_base + m) * P.ldy + nc] = f2bf(v[r]);
    }
  }
  if (tid == 0) __hip_atomic_store(&P.ctr[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace dspark
