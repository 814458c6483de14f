// MoE top-k routing, expert bucketing and grouped expert qmm for gfx950 (MI355X).
//
// The reference routes A3B targets through mlx-lm's SparseMoeBlock + SwitchGLU (third-party,
// not vendored; call stack in the reference's load.py:111-123 routing and roofline.py:190-245
// accounting):
//     gates  = softmax(router(x), precise=True)            (fp32 math, bf16 result)
//     inds   = argpartition(-gates, k-1)[..., :k]          (unordered top-k)
//     scores = take_along_axis(gates, inds); scores /= scores.sum(-1)
//     y      = SwitchGLU(x, inds)   # pairs sorted by expert when inds.size >= 64, gather_qmm
//     out    = (y * scores[..., None]).sum(-2)
// Tie rule used here (argpartition leaves it unspecified): experts are ranked by router logit
// (descending), then expert id (ascending). Softmax is monotone, so this is one of the orders
// argpartition may return on the bf16 gates, and it is bit-reproducible.
//
// MI355X mapping: one tiny workgroup routes all M tokens and builds the expert buckets
// (counting sort, stable in pair id). The grouped qmm launches one workgroup per
// (expert, 16-feature tile); workgroups of unselected experts exit at once, every selected
// expert's weight tile is streamed once for all of its tokens (<= 16 at verify widths).
#include <initializer_list>

#include "dspark_moe_cu.h"
#include "dspark_moe_rc.h"
#include "dspark_moe_sk.h"

namespace dspark {
namespace {

constexpr int kRouteThreads = 1024;  // one wave per token, 16 tokens at a time

struct RouteArgs {
  const u16* logits;
  int* inds;
  u16* scores;
  int* offsets;
  int* sorted;
  int* pos;
  int* ctr;   // nullable: arrival counters of the grouped qmm, cleared here
  int nctr;
  int M, E, k, renorm;
};

__device__ __forceinline__ float bf16r(float f) { return bf2f(f2bf(f)); }

// Routing key of expert e with bf16 logit bits b: orders by logit (NaN as -inf, -0 as +0),
// then by smaller expert id, as one unsigned 32-bit value (larger = chosen first).
__device__ __forceinline__ u32 route_key(u32 b, int e) {
  if ((b & 0x7F80u) == 0x7F80u && (b & 0x7Fu)) b = 0xFF80u;
  if (b == 0x8000u) b = 0u;
  const u32 ord = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
  return (ord << 16) | (0xFFFFu - (u32)e);
}
// logit (as float) of a routing key
__device__ __forceinline__ float route_key_logit(u32 key) {
  const u32 ord = key >> 16;
  return bf2f((ord & 0x8000u) ? (ord & 0x7FFFu) : (~ord & 0xFFFFu));
}

// Maximum of v over the wave: DPP within each row of 16 lanes, then the four row results.
__device__ __forceinline__ u32 wave_max_u32(u32 v) {
  v = max(v, (u32)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  v = max(v, (u32)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  v = max(v, (u32)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  v = max(v, (u32)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xF, 0xF, false));  // row_mirror
  const u32 r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const u32 r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return max(max(r0, r1), max(r2, r3));
}

// One 1024-thread workgroup routes all M tokens (a wave per token, 16 at a time) and buckets
// the (token, slot) pairs by expert. NPL = experts per lane (E <= 64 * NPL).
// Top-k: k rounds of a wave-wide maximum over the routing keys; slot j holds the j-th largest
// (ties to the smaller id), the order of the reference's descending sort.
template <int NPL>
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(const RouteArgs a) {
  extern __shared__ int lds[];
  int* pair_e = lds;                                                 // [M*k]
  int* counts = lds + a.M * a.k;                                     // [kRouteThreads]
  u32* tmask = reinterpret_cast<u32*>(counts + kRouteThreads);       // [2][kRouteThreads] bits of 64 tokens
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int P = a.M * a.k;

  counts[threadIdx.x] = 0;

  for (int t = wave; t < a.M; t += kRouteThreads / 64) {
    float xv[NPL];
    u32 key[NPL];
    u32 kmax = 0;
    u16 lg[NPL];  // every lane's logits requested together (clamped index, no branch)
#pragma unroll
    for (int i = 0; i < NPL; ++i) lg[i] = a.logits[(long)t * a.E + min(lane + 64 * i, a.E - 1)];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int e = lane + 64 * i;
      const u32 b = (e < a.E) ? (u32)lg[i] : 0xFF80u;
      key[i] = (e < a.E) ? route_key(b, e) : 0u;  // every real key is > 0
      xv[i] = route_key_logit(key[i]);
      kmax = max(kmax, key[i]);
    }
    u32 m = wave_max_u32(kmax);
    const float mx = route_key_logit(m);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NPL; ++i)
      if (lane + 64 * i < a.E) sum += expf(xv[i] - mx);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum += shfl_xor(sum, o);
    u32 mine = 0;  // lane j < k keeps the key of slot j
    for (int j = 0; j < a.k; ++j) {
      if (j > 0) {
        kmax = 0;
#pragma unroll
        for (int i = 0; i < NPL; ++i) kmax = max(kmax, key[i]);
        m = wave_max_u32(kmax);
      }
      const int e = 0xFFFF - (int)(m & 0xFFFFu);
#pragma unroll
      for (int i = 0; i < NPL; ++i)
        if (lane + 64 * i == e) key[i] = 0u;
      if (lane == j) mine = m;
    }
    // lanes 0..k-1 finish their slots together: expert, gate value, and the renormalised
    // score over the slot-order fp32 sum of the k gate values
    const int e_mine = 0xFFFF - (int)(mine & 0xFFFFu);
    const float g_mine = bf16r(expf(route_key_logit(mine) - mx) / sum);
    float gsum = 0.f;
    for (int j = 0; j < a.k; ++j) gsum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, g_mine), j));
    const float denom = bf16r(gsum);
    if (lane < a.k) {
      a.inds[t * a.k + lane] = e_mine;
      pair_e[t * a.k + lane] = e_mine;
      a.scores[t * a.k + lane] = f2bf(a.renorm ? bf16r(g_mine / denom) : g_mine);
    }
    __builtin_amdgcn_wave_barrier();
  }
  // the grouped qmm's arrival counters (after the logits loads, which would otherwise wait
  // behind these stores)
  for (int i = threadIdx.x; i < a.nctr; i += kRouteThreads) a.ctr[i] = 0;
  if (!a.offsets) return;
  // ---- bucket the (token, slot) pairs by expert, stable in pair id. A token selects an
  // expert at most once, so a pair's place in its bucket is the number of earlier tokens that
  // selected the same expert. Bucket sizes first (order-free), then an exclusive scan, then
  // the tokens in chunks of 64: one bit per (expert, token of the chunk) gives each pair its
  // rank among the chunk's earlier tokens, and a running per-expert total carries the
  // earlier chunks. Cost: M/64 chunks of four barriers, whatever M is.
  __syncthreads();
  for (int p = threadIdx.x; p < P; p += kRouteThreads) atomicAdd(&counts[pair_e[p]], 1);
  __syncthreads();
  // exclusive scan of the bucket sizes by wave 0, 64 experts at a time; counts[e] becomes the
  // bucket start
  if (wave == 0) {
    int carry = 0;
    for (int c0 = 0; c0 < a.E; c0 += 64) {
      const int e = c0 + lane;
      const int cnt = (e < a.E) ? counts[e] : 0;
      int incl = cnt;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d);
        if (lane >= d) incl += o;
      }
      if (e < a.E) {
        a.offsets[e] = carry + incl - cnt;
        counts[e] = carry + incl - cnt;
      }
      carry += __shfl(incl, 63);
    }
    if (lane == 0) a.offsets[a.E] = carry;
  }
  for (int t0 = 0; t0 < a.M; t0 += 64) {
    tmask[threadIdx.x] = 0;
    tmask[kRouteThreads + threadIdx.x] = 0;
    __syncthreads();  // also orders the scan's counts before the first chunk's reads
    const int q0 = t0 * a.k, q1 = min(t0 + 64, a.M) * a.k;
    for (int p = q0 + threadIdx.x; p < q1; p += kRouteThreads) {
      const int tl = p / a.k - t0;
      atomicOr(&tmask[(tl >> 5) * kRouteThreads + pair_e[p]], 1u << (tl & 31));
    }
    __syncthreads();
    for (int p = q0 + threadIdx.x; p < q1; p += kRouteThreads) {
      const int pe = pair_e[p], tl = p / a.k - t0;
      const u32 lo = tmask[pe], hi = tmask[kRouteThreads + pe];
      const int before = (tl < 32) ? __builtin_popcount(lo & ((1u << tl) - 1u))
                                   : __builtin_popcount(lo) + __builtin_popcount(hi & ((1u << (tl - 32)) - 1u));
      const int slot = counts[pe] + before;  // bucket start + earlier chunks + earlier tokens here
      if (a.sorted) a.sorted[slot] = p;
      if (a.pos) a.pos[p] = slot;
    }
    __syncthreads();
    counts[threadIdx.x] += __builtin_popcount(tmask[threadIdx.x]) + __builtin_popcount(tmask[kRouteThreads + threadIdx.x]);
  }
}

// ---------------------------------------------------------------- grouped expert qmm

enum GatherMode { kPlain = 0, kSwiGLU = 1 };

struct GatherArgs {
  const u16* x;
  const int* row_index;  // nullable: x row of sorted position p (else p)
  const int* offsets;    // [E + 1]
  const u32* w0;         // [E, N, K*bits/32] (gate for SwiGLU)
  const u16* s0;
  const u16* b0;
  const u32* w1;         // up (SwiGLU only)
  const u16* s1;
  const u16* b1;
  u16* y;                // [P, N]
  long ldx, ldy;
  int K, N, row_div, P_max;
};

// One workgroup = one expert x CT tiles of 16 output features (SwiGLU: one tile, for gate and
// for up), K split over the W waves. Each wave walks its K slice in chunks of KSW groups,
// issuing the chunk's weight / scale-bias / x loads before its MFMAs; the W partial tiles are
// summed in LDS in wave order. Workgroups of experts no token selected exit at once. Rows
// are the expert's bucket, 16 at a time.
template <int BITS, int MODE, int CT, int KSW, int W>
__global__ __launch_bounds__(64 * W) void gather_qmm_kernel(const GatherArgs a) {
  constexpr int NTW = (MODE == kSwiGLU) ? 2 * CT : CT;  // weight tiles per wave
  const int e = blockIdx.x;
  const int p0 = a.offsets[e], p1 = min(a.offsets[e + 1], a.P_max);
  if (p0 >= p1) return;
  const int n_base = blockIdx.y * 16 * CT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c16 = lane & 15, q = lane >> 4;
  const int G = a.K >> 6;
  const int g0 = (wave * G) / W, g1 = ((wave + 1) * G) / W;
  const long wstride = (long)a.N * (a.K * BITS / 32);
  const long sstride = (long)a.N * G;

  const u32* wr[NTW];
  const u16* sr[NTW];
  const u16* br[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    const int ct = (MODE == kSwiGLU) ? (j >> 1) : j;
    const bool up = (MODE == kSwiGLU) && (j & 1);
    const int n = min(n_base + 16 * ct + c16, a.N - 1);
    wr[j] = wrow_ptr<BITS>((up ? a.w1 : a.w0) + e * wstride, n, a.K, q);
    sr[j] = (up ? a.s1 : a.s0) + e * sstride + (long)n * G;
    br[j] = (up ? a.b1 : a.b0) + e * sstride + (long)n * G;
  }
  constexpr u32 kconst = (BITS == 4) ? 0xC300C300u : 0x3F803F80u;
  const u32x4_t kb = {kconst, kconst, kconst, kconst};
  constexpr float bias_mul = (BITS == 4) ? (-1.0f / 128.0f) : 1.0f;
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  __shared__ float red[W][NTW][256];
  for (int mb = p0; mb < p1; mb += 16) {
    const int pr = min(mb + c16, p1 - 1);
    const int src = (a.row_index ? a.row_index[pr] : pr) / a.row_div;
    const u16* xr = a.x + (long)src * a.ldx + 16 * q;
    f32x4_t acc[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[j] = zero;
    for (int gc = g0; gc < g1; gc += KSW) {
      const int cnt = min(KSW, g1 - gc);
      WFrag<BITS> wf[KSW][NTW];
      u32 sb[KSW][NTW];  // scale (low half) and bias (high half) bf16 bits
      u32x4_t xa[KSW][2];
#pragma unroll
      for (int i = 0; i < KSW; ++i) {
        const int g = gc + min(i, cnt - 1);
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          if constexpr (BITS == 4)
            wf[i][j].v = ldg64(wr[j] + 8 * g);
          else
            wf[i][j].v = ldg128(wr[j] + 16 * g);
        }
      }
#pragma unroll
      for (int i = 0; i < KSW; ++i) {
        const int g = gc + min(i, cnt - 1);
        xa[i][0] = ldg128(xr + 64 * g);
        xa[i][1] = ldg128(xr + 64 * g + 8);
#pragma unroll
        for (int j = 0; j < NTW; ++j) sb[i][j] = (u32)sr[j][g] | ((u32)br[j][g] << 16);
      }
#pragma unroll
      for (int i = 0; i < KSW; ++i) {
        if (i < cnt) {
          u32x4_t a0 = xa[i][0], a1 = xa[i][1];
          if constexpr (BITS == 4) {
            a0 = perm_x_u4(a0);
            a1 = perm_x_u4(a1);
          }
          f32x4_t c = mfma16x16x32(a0, kb, zero);
          c = mfma16x16x32(a1, kb, c);
#pragma unroll
          for (int j = 0; j < NTW; ++j) {
            f32x4_t p;
            if constexpr (BITS == 4) {
              p = mfma16x16x32(a0, unpack_u4(wf[i][j].v.x), c);
              p = mfma16x16x32(a1, unpack_u4(wf[i][j].v.y), p);
            } else {
              p = mfma16x16x32(a0, unpack_u8(wf[i][j].v.x, wf[i][j].v.y), zero);
              p = mfma16x16x32(a1, unpack_u8(wf[i][j].v.z, wf[i][j].v.w), p);
            }
            const float sf = bf2f(sb[i][j] & 0xFFFFu), bf = bf2f(sb[i][j] >> 16) * bias_mul;
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[j][r] = __builtin_fmaf(bf, c[r], __builtin_fmaf(sf, p[r], acc[j][r]));
          }
        }
      }
    }
    __syncthreads();  // the previous row tile's reduction has read red
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][j][(4 * q + r) * 16 + c16] = acc[j][r];
    __syncthreads();
    for (int t = threadIdx.x; t < 256 * CT; t += 64 * W) {
      const int ct = t >> 8, el = t & 255;
      const int m = el >> 4, nn = el & 15;
      float v0 = 0.f, v1 = 0.f;
#pragma unroll
      for (int ww = 0; ww < W; ++ww) {
        if constexpr (MODE == kSwiGLU) {
          v0 += red[ww][2 * ct][el];
          v1 += red[ww][2 * ct + 1][el];
        } else {
          v0 += red[ww][ct][el];
        }
      }
      const int pp = mb + m, nf = n_base + 16 * ct + nn;
      if (pp < p1 && nf < a.N) {
        float out = v0;
        if constexpr (MODE == kSwiGLU) {
          // h = silu(gate) * up with the bf16 rounding of each elementwise op
          const float g = bf16r(v0), u = bf16r(v1);
          const float sg = bf16r(1.0f / (1.0f + expf(-g)));
          out = bf16r(g * sg) * u;
        }
        a.y[(long)pp * a.ldy + nf] = f2bf(out);
      }
    }
  }
}

// out[t, n] = sum_j bf16(scores[t, j] * y[pos[t*k + j], n])   (fp32 sum in slot order)
__global__ __launch_bounds__(256) void moe_combine_kernel(const u16* __restrict__ y, const int* __restrict__ pos,
                                                          const u16* __restrict__ scores, u16* __restrict__ out,
                                                          int H, int k) {
  const int t = blockIdx.x;
  const int n = blockIdx.y * 256 + threadIdx.x;
  if (n >= H) return;
  float acc = 0.f;
  for (int j = 0; j < k; ++j) {
    const int p = pos[t * k + j];
    acc += bf16r(bf2f(scores[t * k + j]) * bf2f(y[(long)p * H + n]));
  }
  out[(long)t * H + n] = f2bf(acc);
}

int check_route(long M, long E, long k) {
  if (M < 1 || E < 1 || k < 1) return fail(DSPARK_ERR_SHAPE, "moe_route: M=%ld E=%ld k=%ld", M, E, k);
  if (k > 32 || k > E || E > 1024) return fail(DSPARK_ERR_SHAPE, "moe_route: need 1 <= k <= 32, k <= E <= 1024 (E=%ld k=%ld)", E, k);
  if (M * k > 8192) return fail(DSPARK_ERR_SHAPE, "moe_route: M*k=%ld > 8192", M * k);
  return DSPARK_OK;
}

int launch_route(const RouteArgs& a, hipStream_t s) {
  const size_t lds = sizeof(int) * ((size_t)a.M * a.k + 3 * kRouteThreads);
  const dim3 g(1), b(kRouteThreads);
  if (a.E <= 64) hipLaunchKernelGGL(moe_route_kernel<1>, g, b, lds, s, a);
  else if (a.E <= 128) hipLaunchKernelGGL(moe_route_kernel<2>, g, b, lds, s, a);
  else if (a.E <= 256) hipLaunchKernelGGL(moe_route_kernel<4>, g, b, lds, s, a);
  else if (a.E <= 512) hipLaunchKernelGGL(moe_route_kernel<8>, g, b, lds, s, a);
  else hipLaunchKernelGGL(moe_route_kernel<16>, g, b, lds, s, a);
  return check_launch("moe_route_topk");
}

template <int MODE, int W>
int launch_gather_k(const GatherArgs& a, int E, int bits, hipStream_t s) {
  constexpr int CT = (MODE == kSwiGLU) ? 1 : 2;  // 16 (gate + up) or 32 output features
  constexpr int KSW = 4;                         // groups per load chunk
  const dim3 grid((unsigned)E, (unsigned)((a.N + 16 * CT - 1) / (16 * CT)));
  if (bits == 4) hipLaunchKernelGGL((gather_qmm_kernel<4, MODE, CT, KSW, W>), grid, dim3(64 * W), 0, s, a);
  else hipLaunchKernelGGL((gather_qmm_kernel<8, MODE, CT, KSW, W>), grid, dim3(64 * W), 0, s, a);
  return check_launch(MODE == kSwiGLU ? "moe gate/up" : "gather_qmm");
}

// K split over W in {4, 8, 16} waves: each wave's slice is about one 4-group load chunk.
template <int MODE>
int launch_gather(const GatherArgs& a, int E, int bits, hipStream_t s) {
  const int G = a.K / 64;
  if (G <= 16) return launch_gather_k<MODE, 4>(a, E, bits, s);
  if (G <= 32) return launch_gather_k<MODE, 8>(a, E, bits, s);
  return launch_gather_k<MODE, 16>(a, E, bits, s);
}

int check_qmm_format(long K, long N, int bits, int group_size) {
  if (bits != 4 && bits != 8) return fail(DSPARK_ERR_UNSUPPORTED, "gather_qmm: bits=%d", bits);
  if (group_size != 64) return fail(DSPARK_ERR_UNSUPPORTED, "gather_qmm: group_size=%d", group_size);
  if (K < 64 || K % 64 || N < 1) return fail(DSPARK_ERR_SHAPE, "gather_qmm: K=%ld N=%ld", K, N);
  return DSPARK_OK;
}

inline size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

// Launch plan of the grouped split-K qmm (moe_sk_kernel) for one projection of every expert.
struct MoePlan {
  int S, ksmax, strips, mtiles;
  bool sbvec;
  size_t ctrs, part_floats;
};

MoePlan moe_plan(long K, long N, long E, long M, bool swiglu, int bits) {
  MoePlan p{};
  const long G = K / 64;
  p.strips = (int)(swiglu ? (N + 31) / 32 : (N + 63) / 64);
  p.mtiles = (int)((M + 15) / 16);  // a token selects an expert at most once: <= M rows per bucket
  long s = (G + 15) / 16;
  if (E * p.strips * p.mtiles * s < 512) s = (G + 7) / 8;
  if (s > kQmmMaxSlices) s = kQmmMaxSlices;
  if (s > max_slices(G, bits)) s = max_slices(G, bits);
  if (s < 1) s = 1;
  p.S = (int)s;
  p.ksmax = slice_capacity(G, s, bits);
  p.sbvec = G % 8 == 0;
  p.ctrs = (size_t)E * p.strips * p.mtiles;
  p.part_floats = p.S > 1 ? p.ctrs * p.S * 1024 : 0;
  return p;
}

struct MoeWorkspace {
  size_t offsets, sorted, pos, inds, scores, h, y, ctr, part, total;
  MoePlan gu, dn;
};

// (bits only picks the kernel instantiation; the sizes do not depend on it)
MoeWorkspace moe_layout(long M, long H, long I, long E, long k, int bits) {
  MoeWorkspace w{};
  w.gu = moe_plan(H, I, E, M, true, bits);
  w.dn = moe_plan(I, H, E, M, false, bits);
  const size_t P = (size_t)M * k;
  size_t o = 0;
  w.offsets = o; o += align256(sizeof(int) * (E + 1));
  w.sorted = o;  o += align256(sizeof(int) * P);
  w.pos = o;     o += align256(sizeof(int) * P);
  w.inds = o;    o += align256(sizeof(int) * P);
  w.scores = o;  o += align256(sizeof(u16) * P);
  w.h = o;       o += align256(sizeof(u16) * P * I);
  w.y = o;       o += align256(sizeof(u16) * P * H);
  w.ctr = o;     o += align256(sizeof(int) * (w.gu.ctrs > w.dn.ctrs ? w.gu.ctrs : w.dn.ctrs));
  w.part = o;    o += align256(sizeof(float) * (w.gu.part_floats > w.dn.part_floats ? w.gu.part_floats : w.dn.part_floats));
  w.total = o;
  return w;
}

// The plan with 16-byte scale/bias loads only if every scale/bias array is 16-byte aligned.
MoePlan sb_checked(MoePlan p, std::initializer_list<const void*> arrays) {
  for (const void* a : arrays) p.sbvec = p.sbvec && aligned(a, 16);
  return p;
}

MoeRcArgs rc_args(const MoeSkArgs& a) {
  MoeRcArgs r{};
  r.x = a.x;
  r.row_index = a.row_index;
  r.offsets = a.offsets;
  r.w0 = a.w0;
  r.s0 = a.s0;
  r.b0 = a.b0;
  r.w1 = a.w1;
  r.s1 = a.s1;
  r.b1 = a.b1;
  r.y = a.y;
  r.ldx = a.ldx;
  r.ldy = a.ldy;
  r.K = a.K;
  r.N = a.N;
  r.row_div = a.row_div;
  r.P_max = a.P_max;
  r.mtiles = a.mtiles;
  return r;
}

// Small-bucket plan (moe_rc_kernel): K parts per workgroup and groups per part, or kw = 0
// when the whole-K workgroup does not apply (the split-K kernel then runs).
struct RcPlan {
  int kw, ksmax, strips;
};

RcPlan rc_plan(long K, long N, bool swiglu, const void* s, const void* b) {
  RcPlan p{};
  const long G = K / 64;
  if (K % 128 || (N * G) % 8 || !aligned(s, 16) || !aligned(b, 16)) return p;
  // fewest K parts whose largest part has <= 16 groups, else <= 32; the kernel instance is
  // the smallest of 8, 12, 16, 24, 32 groups that holds the part
  const int kws[3] = {1, 2, 4};
  for (int cap : {16, 32}) {
    for (int kw : kws) {
      if (swiglu && kw == 4) break;
      const long per = 2 * ((G / 2 + kw - 1) / kw);
      if (per <= cap) {
        p.kw = kw;
        p.ksmax = per <= 8 ? 8 : per <= 12 ? 12 : per <= 16 ? 16 : per <= 24 ? 24 : 32;
        const long cols = swiglu ? 8 * (4 / kw) : 16 * (4 / kw);  // output columns per workgroup
        p.strips = (int)((N + cols - 1) / cols);
        return p;
      }
    }
  }
  return p;
}

template <bool SWIGLU, bool PW = false>
int launch_moe_rc(const MoeRcArgs& a, const RcPlan& p, int E, int bits, hipStream_t s) {
  const dim3 grid((unsigned)p.strips, (unsigned)(E * a.mtiles));
#define MOE_RC(B, KS, KW) hipLaunchKernelGGL((moe_rc_kernel<B, KS, KW, SWIGLU, PW>), grid, dim3(256), 0, s, a)
#define MOE_RC_KW(B, KS)                                     \
  if (p.kw == 1) MOE_RC(B, KS, 1);                           \
  else if (SWIGLU || p.kw == 2) MOE_RC(B, KS, 2);            \
  else MOE_RC(B, KS, (SWIGLU ? 2 : 4));
#define MOE_RC_BITS(B)                   \
  if (p.ksmax == 8) { MOE_RC_KW(B, 8) }          \
  else if (p.ksmax == 12) { MOE_RC_KW(B, 12) }   \
  else if (p.ksmax == 16) { MOE_RC_KW(B, 16) }   \
  else if (p.ksmax == 24) { MOE_RC_KW(B, 24) }   \
  else { MOE_RC_KW(B, 32) }
  if (bits == 4) { MOE_RC_BITS(4) } else { MOE_RC_BITS(8) }
#undef MOE_RC_BITS
#undef MOE_RC_KW
#undef MOE_RC
  return check_launch(SWIGLU ? "moe gate/up" : "moe down");
}

template <bool SWIGLU>
int launch_moe_sk(const MoeSkArgs& a, const MoePlan& p, int E, int bits, hipStream_t s) {
  const dim3 grid((unsigned)p.strips, (unsigned)p.S, (unsigned)(E * p.mtiles));
#define MOE_SK(B, KS, SB) hipLaunchKernelGGL((moe_sk_kernel<B, KS, SB, SWIGLU>), grid, dim3(256), 0, s, a)
#define MOE_SK_BITS(B)                                                   \
  if (p.ksmax == 8) { if (p.sbvec) MOE_SK(B, 8, true); else MOE_SK(B, 8, false); }     \
  else { if (p.sbvec) MOE_SK(B, 16, true); else MOE_SK(B, 16, false); }
  if (bits == 4) { MOE_SK_BITS(4) } else { MOE_SK_BITS(8) }
#undef MOE_SK_BITS
#undef MOE_SK
  return check_launch(SWIGLU ? "moe gate/up" : "moe down");
}

// The per-CU gate/up kernel's arguments (the small-bucket kernel's, plus the routing's pair order
// and the expert stride of the packed weights)
MoeCuArgs cu_args(const MoeSkArgs& g, const int* sorted, long M, long E, long k, int bits) {
  MoeCuArgs a{};
  a.x = g.x;
  a.sorted = sorted;
  a.offsets = g.offsets;
  a.wg = reinterpret_cast<const char*>(g.w0);
  a.sg = g.s0;
  a.bg = g.b0;
  a.wu = reinterpret_cast<const char*>(g.w1);
  a.su = g.s1;
  a.bu = g.b1;
  a.h = g.y;
  a.ldx = g.ldx;
  a.ldh = g.ldy;
  a.wstride = (long)g.N * g.K * bits / 8;
  a.M = (int)M;
  a.E = (int)E;
  a.N = g.N;
  a.k = (int)k;
  a.strips = g.N / 16;
  return a;
}

}  // namespace
}  // namespace dspark

using namespace dspark;

extern "C" int dspark_moe_route_topk(const void* logits, int64_t M, int64_t E, int64_t k, int renorm, int32_t* inds,
                                     void* scores, int32_t* expert_offsets, int32_t* sorted_pairs, int32_t* pair_pos,
                                     dspark_stream stream) {
  if (!logits || !inds || !scores) return fail(DSPARK_ERR_ARG, "moe_route: null pointer");
  int st = check_route(M, E, k);
  if (st) return st;
  if ((sorted_pairs || pair_pos) && !expert_offsets)
    return fail(DSPARK_ERR_ARG, "moe_route: sorted_pairs/pair_pos need expert_offsets");
  RouteArgs a{};
  a.logits = static_cast<const u16*>(logits);
  a.inds = inds;
  a.scores = static_cast<u16*>(scores);
  a.offsets = expert_offsets;
  a.sorted = sorted_pairs;
  a.pos = pair_pos;
  a.M = (int)M;
  a.E = (int)E;
  a.k = (int)k;
  a.renorm = renorm ? 1 : 0;
  return launch_route(a, static_cast<hipStream_t>(stream));
}

extern "C" int dspark_gather_qmm(const void* x, int64_t ldx, int64_t K, const int32_t* row_index,
                                 const int32_t* expert_offsets, int64_t E, int64_t P_max, const uint32_t* w,
                                 const void* scales, const void* biases, int64_t N, int bits, int group_size, void* y,
                                 int64_t ldy, dspark_stream stream) {
  if (!x || !expert_offsets || !w || !scales || !biases || !y) return fail(DSPARK_ERR_ARG, "gather_qmm: null pointer");
  int st = check_qmm_format(K, N, bits, group_size);
  if (st) return st;
  if (E < 1 || P_max < 1) return fail(DSPARK_ERR_SHAPE, "gather_qmm: E=%lld P_max=%lld", (long long)E, (long long)P_max);
  if (!aligned(x, 16) || ldx % 8 || ldx < K || !aligned(w, 16) || ldy < N)
    return fail(DSPARK_ERR_ALIGN, "gather_qmm: x/w must be 16-byte aligned, ldx %% 8 == 0, ldx >= K, ldy >= N");
  GatherArgs a{};
  a.x = static_cast<const u16*>(x);
  a.row_index = row_index;
  a.offsets = expert_offsets;
  a.w0 = w;
  a.s0 = static_cast<const u16*>(scales);
  a.b0 = static_cast<const u16*>(biases);
  a.y = static_cast<u16*>(y);
  a.ldx = ldx;
  a.ldy = ldy;
  a.K = (int)K;
  a.N = (int)N;
  a.row_div = 1;
  a.P_max = (int)P_max;
  return launch_gather<kPlain>(a, (int)E, bits, static_cast<hipStream_t>(stream));
}

extern "C" size_t dspark_moe_workspace(int64_t M, int64_t H, int64_t I, int64_t E, int64_t k) {
  if (check_route(M, E, k)) return 0;
  return moe_layout(M, H, I, E, k, 4).total;
}

namespace dspark {
namespace {
// The fused MoE block over row-major (packed = false) or dspark_moe_pack weights.
int switch_glu_impl(const void* x, const void* logits, int64_t M, int64_t H, int64_t I, int64_t E, int64_t k,
                    int renorm, const uint32_t* w_gate, const void* s_gate, const void* b_gate, const uint32_t* w_up,
                    const void* s_up, const void* b_up, const uint32_t* w_down, const void* s_down,
                    const void* b_down, int bits, int group_size, void* out, int32_t* inds, void* scores,
                    void* workspace, size_t workspace_bytes, dspark_stream stream, bool packed) {
  if (!x || !logits || !w_gate || !s_gate || !b_gate || !w_up || !s_up || !b_up || !w_down || !s_down || !b_down || !out)
    return fail(DSPARK_ERR_ARG, "moe_switch_glu: null pointer");
  int st = check_route(M, E, k);
  if (st) return st;
  if ((st = check_qmm_format(H, I, bits, group_size))) return st;
  if ((st = check_qmm_format(I, H, bits, group_size))) return st;
  if (H > 32 * 16 * 64 || I > 32 * 16 * 64)
    return fail(DSPARK_ERR_SHAPE, "moe_switch_glu: H=%lld I=%lld (each <= 32768)", (long long)H, (long long)I);
  if (E * ((I + 31) / 32) * ((M + 15) / 16) > 65535L * 64 || (M + 15) / 16 * E > 65535)
    return fail(DSPARK_ERR_SHAPE, "moe_switch_glu: too many experts x tiles");
  if (!aligned(x, 16) || !aligned(w_gate, 16) || !aligned(w_up, 16) || !aligned(w_down, 16) || !aligned(out, 2))
    return fail(DSPARK_ERR_ALIGN, "moe_switch_glu: x and packed weights must be 16-byte aligned");
  const MoeWorkspace L = moe_layout(M, H, I, E, k, bits);
  if (!workspace || workspace_bytes < L.total)
    return fail(DSPARK_ERR_WORKSPACE, "moe_switch_glu: workspace %zu < %zu bytes", workspace_bytes, L.total);
  if (!aligned(workspace, 256)) return fail(DSPARK_ERR_ALIGN, "moe_switch_glu: workspace must be 256-byte aligned");
  char* ws = static_cast<char*>(workspace);
  int* offsets = reinterpret_cast<int*>(ws + L.offsets);
  int* sorted = reinterpret_cast<int*>(ws + L.sorted);
  int* pos = reinterpret_cast<int*>(ws + L.pos);
  int* inds_ws = inds ? inds : reinterpret_cast<int*>(ws + L.inds);
  u16* scores_ws = scores ? static_cast<u16*>(scores) : reinterpret_cast<u16*>(ws + L.scores);
  u16* h = reinterpret_cast<u16*>(ws + L.h);
  u16* ypair = reinterpret_cast<u16*>(ws + L.y);
  hipStream_t s = static_cast<hipStream_t>(stream);

  RouteArgs r{};
  r.logits = static_cast<const u16*>(logits);
  r.inds = inds_ws;
  r.scores = scores_ws;
  r.offsets = offsets;
  r.sorted = sorted;
  r.pos = pos;
  r.M = (int)M;
  r.E = (int)E;
  r.k = (int)k;
  r.renorm = renorm ? 1 : 0;
  int* ctr = reinterpret_cast<int*>(ws + L.ctr);
  r.ctr = ctr;  // the grouped qmm's arrival counters start every block at zero
  r.nctr = (int)(L.gu.ctrs > L.dn.ctrs ? L.gu.ctrs : L.dn.ctrs);
  if ((st = launch_route(r, s))) return st;

  const int P = (int)(M * k);
  float* part = reinterpret_cast<float*>(ws + L.part);
  MoeSkArgs g{};
  g.x = static_cast<const u16*>(x);
  g.row_index = sorted;
  g.offsets = offsets;
  g.w0 = w_gate;
  g.s0 = static_cast<const u16*>(s_gate);
  g.b0 = static_cast<const u16*>(b_gate);
  g.w1 = w_up;
  g.s1 = static_cast<const u16*>(s_up);
  g.b1 = static_cast<const u16*>(b_up);
  g.y = h;
  g.part = part;
  g.ctr = ctr;
  g.ldx = H;
  g.ldy = I;
  g.K = (int)H;
  g.N = (int)I;
  g.row_div = (int)k;
  g.P_max = P;
  g.strips = L.gu.strips;
  g.mtiles = L.gu.mtiles;
  g.S = L.gu.S;
  const RcPlan rgu = rc_plan(H, I, true, s_gate, b_gate), rgu2 = rc_plan(H, I, true, s_up, b_up);
  const RcPlan rdn = rc_plan(I, H, false, s_down, b_down);
  if (packed && (!rgu.kw || !rgu2.kw || !rdn.kw))
    return fail(DSPARK_ERR_UNSUPPORTED,
                "moe_switch_glu_packed: H=%lld I=%lld need K %% 128 == 0 and 16-byte aligned scales and biases",
                (long long)H, (long long)I);
  if (packed && moe_cu_gate_up(M, H, I, E, k, bits)) {
    if ((st = launch_moe_cu(cu_args(g, sorted, M, E, k, bits), H, bits, s))) return st;
  } else if (packed) {
    if ((st = launch_moe_rc<true, true>(rc_args(g), rgu, (int)E, bits, s))) return st;
  } else if (rgu.kw && rgu2.kw) {
    if ((st = launch_moe_rc<true>(rc_args(g), rgu, (int)E, bits, s))) return st;
  } else if ((st = launch_moe_sk<true>(g, sb_checked(L.gu, {s_gate, b_gate, s_up, b_up}), (int)E, bits, s))) {
    return st;
  }

  MoeSkArgs d{};
  d.x = h;
  d.row_index = nullptr;
  d.offsets = offsets;
  d.w0 = w_down;
  d.s0 = static_cast<const u16*>(s_down);
  d.b0 = static_cast<const u16*>(b_down);
  d.y = ypair;
  d.part = part;
  d.ctr = ctr;
  d.ldx = I;
  d.ldy = H;
  d.K = (int)I;
  d.N = (int)H;
  d.row_div = 1;
  d.P_max = P;
  d.strips = L.dn.strips;
  d.mtiles = L.dn.mtiles;
  d.S = L.dn.S;
  if (packed) {
    if ((st = launch_moe_rc<false, true>(rc_args(d), rdn, (int)E, bits, s))) return st;
  } else if (rdn.kw) {
    if ((st = launch_moe_rc<false>(rc_args(d), rdn, (int)E, bits, s))) return st;
  } else if ((st = launch_moe_sk<false>(d, sb_checked(L.dn, {s_down, b_down}), (int)E, bits, s))) {
    return st;
  }

  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)M, (unsigned)((H + 255) / 256)), dim3(256), 0, s, ypair, pos,
                     scores_ws, static_cast<u16*>(out), (int)H, (int)k);
  return check_launch("moe combine");
}
}  // namespace
}  // namespace dspark

extern "C" int dspark_moe_switch_glu(const void* x, const void* logits, int64_t M, int64_t H, int64_t I, int64_t E,
                                     int64_t k, int renorm, const uint32_t* w_gate, const void* s_gate,
                                     const void* b_gate, const uint32_t* w_up, const void* s_up, const void* b_up,
                                     const uint32_t* w_down, const void* s_down, const void* b_down, int bits,
                                     int group_size, void* out, int32_t* inds, void* scores, void* workspace,
                                     size_t workspace_bytes, dspark_stream stream) {
  return switch_glu_impl(x, logits, M, H, I, E, k, renorm, w_gate, s_gate, b_gate, w_up, s_up, b_up, w_down, s_down,
                         b_down, bits, group_size, out, inds, scores, workspace, workspace_bytes, stream, false);
}

extern "C" int dspark_moe_switch_glu_packed(const void* x, const void* logits, int64_t M, int64_t H, int64_t I,
                                            int64_t E, int64_t k, int renorm, const void* w_gate,
                                            const void* s_gate, const void* b_gate, const void* w_up,
                                            const void* s_up, const void* b_up, const void* w_down,
                                            const void* s_down, const void* b_down, int bits, int group_size,
                                            void* out, int32_t* inds, void* scores, void* workspace,
                                            size_t workspace_bytes, dspark_stream stream) {
  if (H % 16 || I % 16)
    return fail(DSPARK_ERR_SHAPE, "moe_switch_glu_packed: H=%lld and I=%lld must be multiples of 16", (long long)H,
                (long long)I);
  return switch_glu_impl(x, logits, M, H, I, E, k, renorm, static_cast<const uint32_t*>(w_gate), s_gate, b_gate,
                         static_cast<const uint32_t*>(w_up), s_up, b_up, static_cast<const uint32_t*>(w_down), s_down,
                         b_down, bits, group_size, out, inds, scores, workspace, workspace_bytes, stream, true);
}
