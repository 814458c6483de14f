// Small-M affine-quantized matmul for gfx950 (MI355X).
//
//   y[m, n] = sum_g ( s[n,g] * sum_{j in g} q[n,j] x[m,j]  +  b[n,g] * sum_{j in g} x[m,j] )
//
// Same factored form as the reference's skinny kernel (skinny_qmm.py:138-145): the per-group
// product P = sum q*x is formed from exact bf16 x exact-integer products in fp32, then
// acc = fma(b, sum x, fma(s, P, acc)). Format (skinny_qmm.py:95-119): element j of weight row
// n is field j % (32/bits) of uint32 word j / (32/bits), low bits first; groups of 64 along K.
//
// MI355X mapping (independent of the Metal kernel's 8x8 simdgroup layout):
//   * one v_mfma_f32_16x16x32_bf16 consumes 16 weight rows x 32 k. The A operand is x
//     (16 verify rows; rows >= M are clamped duplicates whose outputs are dropped), the B
//     operand is the dequantized weight fragment. Lane (c16 = l & 15, q = l >> 4) owns weight
//     row n0 + c16 and the 16 (8-bit) / 16 (4-bit) k-values of quarter q inside a group, read
//     as one 16-byte (8-bit) or 8-byte (4-bit) load straight from the packed row.
//   * integer fields become bf16 without int->float converts where possible:
//       4-bit: (w >> 4t) & 0x000F000F | 0x43004300 is the bf16 pair (128 + q_t, 128 + q_{t+4});
//              the +128 offset is removed exactly by seeding the MFMA accumulator with
//              -128 * sum x (itself an MFMA of x against a constant -128 operand), and the
//              x fragment is permuted once to match the (t, t+4) field order.
//       8-bit: v_cvt_f32_ubyte{0..3} + v_cvt_pk_bf16_f32 (exact for 0..255).
//     Integers 0..255 are exact in bf16, so every product is exact in fp32, as in the
//     reference's pre-scaled masked-field trick.
//   * sum_{j in g} x[m, j] (the bias term) comes out of the same MFMA in the output layout.
//   * a workgroup = 4 waves = a 64-row strip x one slice of K; the x slice and its group sums
//     are staged once in LDS and shared by the 4 waves (dspark_qmm_splitk.h). Slices of a
//     strip are summed by the last workgroup to arrive, in slice order: deterministic and
//     independent of M. The slice count depends only on the strips and K.
#include <algorithm>
#include <mutex>

#include "dspark_qmm_cu.h"
#include "dspark_qmm_splitk.h"
#include "dspark_qmm_wholek.h"

namespace dspark {
namespace {

constexpr int kNS = 4;             // waves (16-row output tiles) per workgroup: 64-row strips
constexpr int kStripRows = 16 * kNS;
constexpr long kCUs = 256;         // MI355X
// Split-K arrival counters live in a fixed region at the start of the workspace, the same bytes
// for every shape, so partials of one shape never land on another shape's counters (each
// launch leaves its counters at zero).
constexpr size_t kCtrRegionBytes = 256 * 1024;
constexpr size_t kMaxCounters = kCtrRegionBytes / sizeof(int);

// Launch plan shared by the workspace query and the launch: S depends only on the strips and
// K, never on M, so a row's result does not depend on how many rows ride with it.
struct Plan {
  bool wholek;  // 16-row whole-K workgroups (qmm_wk_kernel), no split-K and no workspace
  int tiles;    // wholek: 16-row output tiles over all problems
  int S;       // K slices
  int ksmax;   // groups per slice the kernel is instantiated for (8, 16 or 32)
  int strips;  // 64-row strips over all problems
  int mtiles;
  size_t ctr_bytes;
  size_t part_bytes;
};

// wholek_ok: the launch may take the whole-K kernel (the plain qmm entry points, not the fused
// SwiGLU pair, whose epilogue only the split-K kernel has).
Plan make_plan(const long* Ns, int count, long K, long M, int bits, bool wholek_ok = false) {
  Plan p{};
  const long G = K / 64;
  long strips = 0;
  for (int i = 0; i < count; ++i) strips += (Ns[i] + kStripRows - 1) / kStripRows;
  p.strips = (int)strips;
  p.mtiles = (int)((M + 15) / 16);
  // One 16-row whole-K workgroup per CU where it was measured faster than split-K: 8- or 4-bit
  // rows, K = 4096, 240..256 tiles (a [4096, 4096] matrix, or problems adding up to it; 4-bit
  // 8.6 -> 8.4 us at M = 16, its packed o projection in the 4-bit layer set too). The choice
  // depends on the shape only, never on M, so a row's bits do not depend on its company.
  if (wholek_ok && (bits == 8 || bits == 4) && K == 4096) {
    long tiles = 0;
    for (int i = 0; i < count; ++i) tiles += (Ns[i] + 15) / 16;
    if (tiles >= 240 && tiles <= kCUs) {
      p.wholek = true;
      p.tiles = (int)tiles;
      p.S = 1;
      p.ksmax = (int)G;
      return p;
    }
  }
  // 16 groups (1024 k) per slice, unless those workgroups fill their last resident round
  // (one or two rounds) poorly and 8-group slices, whose kernels keep more workgroups per CU,
  // fill theirs better. Resident workgroups per CU of the instantiations (VGPR-limited, as
  // compiled): 16-group 3 (8-bit) / 4 (4-bit), 8-group 5.
  long s = (G + 15) / 16;
  {
    auto fill = [&](long w, long slots) { return (double)w / (double)(((w + slots - 1) / slots) * slots); };
    const long slots16 = kCUs * (bits == 8 ? 3 : 4), slots8 = kCUs * 5;
    const long w16 = strips * s, s8 = (G + 7) / 8;
    if (w16 <= 2 * slots16 && fill(w16, slots16) < 0.9 && fill(strips * s8, slots8) > fill(w16, slots16)) s = s8;
  }
  if (s > kQmmMaxSlices) s = kQmmMaxSlices;
  if (s > max_slices(G, bits)) s = max_slices(G, bits);
  if (s < 1) s = 1;
  p.S = (int)s;
  p.ksmax = slice_capacity(G, s, bits);
  if (!p.ksmax) {
    p.S = 0;  // refused: K too large for 32 slices of 16 groups
    return p;
  }
  if (p.S > 1) {
    const size_t ctrs = (size_t)strips * p.mtiles;
    if (ctrs > kMaxCounters) {
      p.S = 0;  // refused: more output tiles than counters
      return p;
    }
    p.ctr_bytes = kCtrRegionBytes;
    p.part_bytes = ctrs * p.S * 16 * kStripRows * sizeof(float);
  }
  return p;
}

template <int BITS, int KSMAX, bool SBVEC, bool PACKED = false, bool SWIGLU = false>
int launch(const QmmSkArgs& a, const Plan& p, hipStream_t st) {
  hipLaunchKernelGGL((qmm_sk_kernel<BITS, kNS, KSMAX, SBVEC, PACKED, SWIGLU>), dim3(p.strips, p.S, p.mtiles),
                     dim3(64 * kNS), 0, st, a);
  return check_launch(SWIGLU ? "dspark_qmm_swiglu_packed" : PACKED ? "dspark_qmm_packed" : "dspark_qmm_affine");
}

template <int BITS>
int launch_bits(const QmmSkArgs& a, const Plan& p, bool sbvec, hipStream_t st) {
  if (p.ksmax == 8) return sbvec ? launch<BITS, 8, true>(a, p, st) : launch<BITS, 8, false>(a, p, st);
  return sbvec ? launch<BITS, 16, true>(a, p, st) : launch<BITS, 16, false>(a, p, st);
}

constexpr int kWkWaves = 8;  // whole-K: one K octet per wave at K = 4096

template <bool PACKED, bool SBVEC>
int launch_wk(const QmmSkArgs& a, const Plan& p, int bits, hipStream_t st) {
  if (bits == 4)
    hipLaunchKernelGGL((qmm_wk_kernel<4, kWkWaves, PACKED, SBVEC>), dim3(p.tiles, p.mtiles), dim3(64 * kWkWaves), 0,
                       st, a);
  else
    hipLaunchKernelGGL((qmm_wk_kernel<8, kWkWaves, PACKED, SBVEC>), dim3(p.tiles, p.mtiles), dim3(64 * kWkWaves), 0,
                       st, a);
  return check_launch(PACKED ? "dspark_qmm_packed" : "dspark_qmm_affine");
}

// One workgroup per CU (dspark_qmm_cu.h): packed weights, one x for every problem, TPW row
// tiles per workgroup split over KH K parts, on at least 180 CUs; the slices of the split-K plan
// fix the association, so the bits are that plan's.
//   K = 4096: TPW = ceil(tiles / 256) (2 tiles x 4 parts, or 3..6 tiles x 2 parts: 8 or 12
//   waves) over all of K. Where measured faster than the other kernels: 3..6 tiles (the gate+up
//   pair 2 x [12288, 4096] at M = 16: 25.5 -> 21.3 us, 4-bit 17.9 -> 16.3), and 2 tiles at 8
//   bits (q+k+v, [6144, 4096]: 9.7 -> 9.2 us; at 4
//   bits 8.3 -> 8.7, not taken). One tile per CU (x 8 K parts) measured slower than the whole-K
//   tile kernel (7.9 -> 8.2 us) and is not taken.
//   K = 12288 with 16-group slices, up to 256 tiles (the [4096, 12288] down
//   projection): four workgroups per tile group,
//   each over 3072 columns of K (three slices), 4 tiles x 3 waves, their partials summed by the
//   last to arrive. (Three parts of 4096 at 3 tiles per workgroup would need 258 workgroups.)
// Returns the shape, or tpw = 0 when the launch keeps the split-K or whole-K tile kernel.
struct CuShape {
  int tpw, kh, kparts, kc;
};
CuShape cu_shape(const dspark_qmm_problem* problems, int count, const long* Ns, long K, int bits, const Plan& p) {
  if (p.wholek) return {0, 0, 0, 0};
  const long G = K / 64;
  const long gsl = p.S >= 2 && G % p.S == 0 ? G / p.S : 0;
  if (gsl != 8 && gsl != 16) return {0, 0, 0, 0};
  long tiles = 0;
  for (int i = 0; i < count; ++i) {
    if (problems[i].x != problems[0].x || problems[i].ldx != problems[0].ldx) return {0, 0, 0, 0};
    tiles += (Ns[i] + 15) / 16;
  }
  if (K == 12288 && gsl == 16 && tiles <= kCUs && (tiles + 3) / 4 * 4 >= 180) return {4, 3, 4, 3072};
  if (K != kCuK) return {0, 0, 0, 0};
  const long tpw = (tiles + kCUs - 1) / kCUs;
  if (tpw < 2 || tpw > 6 || (tpw == 2 && bits != 8) || (tiles + tpw - 1) / tpw < 180) return {0, 0, 0, 0};
  const int kh = tpw == 2 ? 4 : 2;
  if ((G / kh) % gsl) return {0, 0, 0, 0};
  return {(int)tpw, kh, 1, (int)kCuK};
}

template <int BITS, int TPW, int KH, int GSL, int KC = kCuK, int KP = 1>
int launch_cu_t(const QmmSkArgs& a, const Plan& p, int tiles, hipStream_t st) {
  constexpr size_t lds = cu_lds_bytes(TPW, KC);
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&qmm_cu_kernel<BITS, TPW, KH, GSL, KC, KP>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  });
  if (attr != hipSuccess) return fail(DSPARK_ERR_LAUNCH, "dspark_qmm_packed: LDS attribute: %s", hipGetErrorString(attr));
  hipLaunchKernelGGL((qmm_cu_kernel<BITS, TPW, KH, GSL, KC, KP>),
                     dim3((unsigned)((tiles + TPW - 1) / TPW), p.mtiles, (unsigned)KP), dim3(64 * TPW * KH), lds, st, a,
                     tiles);
  return check_launch("dspark_qmm_packed");
}

template <int BITS, int GSL>
int launch_cu_g(const QmmSkArgs& a, const Plan& p, CuShape c, int tiles, hipStream_t st) {
  if (c.kc == 3072) {
    if constexpr (GSL == 16) return launch_cu_t<BITS, 4, 3, 16, 3072, 4>(a, p, tiles, st);
    return fail(DSPARK_ERR_SHAPE, "dspark_qmm_packed: no per-CU instance for 3072-column parts of %d groups", GSL);
  }
  switch (c.tpw) {
    case 2: return launch_cu_t<BITS, 2, 4, GSL>(a, p, tiles, st);
    case 3: return launch_cu_t<BITS, 3, 2, GSL>(a, p, tiles, st);
    case 4: return launch_cu_t<BITS, 4, 2, GSL>(a, p, tiles, st);
    case 5: return launch_cu_t<BITS, 5, 2, GSL>(a, p, tiles, st);
    case 6: return launch_cu_t<BITS, 6, 2, GSL>(a, p, tiles, st);
    default: break;
  }
  return fail(DSPARK_ERR_SHAPE, "dspark_qmm_packed: no per-CU instance for %d tiles per workgroup", c.tpw);
}

int launch_cu(const QmmSkArgs& a, const Plan& p, int bits, CuShape c, int tiles, hipStream_t st) {
  const bool g16 = (a.p[0].K / 64) / p.S == 16;
  if (bits == 8) return g16 ? launch_cu_g<8, 16>(a, p, c, tiles, st) : launch_cu_g<8, 8>(a, p, c, tiles, st);
  return g16 ? launch_cu_g<4, 16>(a, p, c, tiles, st) : launch_cu_g<4, 8>(a, p, c, tiles, st);
}

template <int BITS, bool SWIGLU = false>
int launch_packed(const QmmSkArgs& a, const Plan& p, hipStream_t st) {
  if (p.ksmax == 8) return launch<BITS, 8, true, true, SWIGLU>(a, p, st);
  return launch<BITS, 16, true, true, SWIGLU>(a, p, st);
}

// ---- the packed form (dspark_qmm_pack). Per matrix, T = ceil(N/16) row tiles, G = K/64:
//   tile stream  T x (8-bit: G groups | 4-bit: G/2 group pairs) x 64 lanes x 16 B: lane l of
//                tile t holds row 16t + (l & 15), quarter q = l >> 4:
//                  8-bit: bytes [16q, 16q+16) of the group;
//                  4-bit: bytes [8qs, 8qs+8) of group 2j then of group 2j+1, qs = 2(q&1) + (q>>1)
//                  (the lane order the MFMA loop uses; see WSlice);
//   scale/bias   T x G/8 octets x {scales, biases} x 16 rows x 8 bf16.
// Rows >= N are zero. The SwiGLU pair form (dspark_qmm_pack_swiglu) is this layout for 2T tiles,
// tile 2t = gate tile t, tile 2t + 1 = up tile t.
struct PackedLayout {
  long tiles, wchunks, schunks;
  size_t bytes() const { return (size_t)(wchunks + schunks) * 16; }
};
PackedLayout packed_layout(long N, long K, int bits) {
  PackedLayout L{};
  const long G = K / 64;
  L.tiles = (N + 15) / 16;
  L.wchunks = L.tiles * (bits == 4 ? G / 2 : G) * 64;
  L.schunks = L.tiles * (G / 8) * 32;
  return L;
}

// pair (w2 != null): destination tile t takes tile t / 2 of the first matrix (t even) or of
// the second (t odd)
__global__ __launch_bounds__(256) void pack_kernel(const unsigned char* __restrict__ w1, const u16* __restrict__ s1,
                                                   const u16* __restrict__ b1, const unsigned char* __restrict__ w2,
                                                   const u16* __restrict__ s2, const u16* __restrict__ b2, long N,
                                                   int K, int bits, long wchunks, long schunks,
                                                   unsigned char* __restrict__ out) {
  const long c = (long)blockIdx.x * 256 + threadIdx.x;
  const int G = K >> 6;
  const bool pair = w2 != nullptr;
  u32x4_t v = {0u, 0u, 0u, 0u};
  if (c < wchunks) {
    const int per_tile = bits == 4 ? (G >> 1) : G;
    const long tt = c / (per_tile * 64);
    const int rem = (int)(c - tt * per_tile * 64), j = rem >> 6, l = rem & 63;
    const long t = pair ? tt >> 1 : tt;
    const unsigned char* w = (pair && (tt & 1)) ? w2 : w1;
    const long r = 16 * t + (l & 15);
    const int q = l >> 4;
    if (r < N) {
      if (bits == 8) {
        v = ldg128(w + r * K + j * 64 + 16 * q);
      } else {
        const int qs = 2 * (q & 1) + (q >> 1);
        const unsigned char* row = w + r * (K / 2);
        const u32x2_t lo = ldg64(row + (2 * j) * 32 + 8 * qs), hi = ldg64(row + (2 * j + 1) * 32 + 8 * qs);
        v = u32x4_t{lo.x, lo.y, hi.x, hi.y};
      }
    }
  } else if (c < wchunks + schunks) {
    const long c2 = c - wchunks;
    const long blk = c2 >> 5;
    const int rem = (int)(c2 & 31), arr = rem >> 4, r16 = rem & 15;
    const long tt = blk / (G >> 3);
    const int o = (int)(blk - tt * (G >> 3));
    const long t = pair ? tt >> 1 : tt;
    const bool second = pair && (tt & 1);
    const long r = 16 * t + r16;
    if (r < N) v = ldg128((arr ? (second ? b2 : b1) : (second ? s2 : s1)) + r * G + 8 * o);
  } else {
    return;
  }
  *reinterpret_cast<u32x4_t*>(out + c * 16) = v;
}

int check_common(int64_t M, int64_t K, int64_t N, int bits, int group_size) {
  if (bits != 4 && bits != 8) return fail(DSPARK_ERR_UNSUPPORTED, "qmm: bits=%d (4 or 8 supported)", bits);
  if (group_size != 64) return fail(DSPARK_ERR_UNSUPPORTED, "qmm: group_size=%d (64 supported)", group_size);
  if (M < 1 || N < 1 || K < 64) return fail(DSPARK_ERR_SHAPE, "qmm: M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  if (K % 64) return fail(DSPARK_ERR_SHAPE, "qmm: K=%lld is not a multiple of 64", (long long)K);
  if (K > 32 * 16 * 64) return fail(DSPARK_ERR_SHAPE, "qmm: K=%lld > 32768", (long long)K);
  if (M > 65535L * 16 || N > (1L << 30) / 16)  // 16-row tiles index grid.z
    return fail(DSPARK_ERR_SHAPE, "qmm: shape too large (M=%lld N=%lld)", (long long)M, (long long)N);
  return DSPARK_OK;
}

int check_problem(const dspark_qmm_problem& p) {
  if (!p.x || !p.w || !p.scales || !p.biases || !p.y) return fail(DSPARK_ERR_ARG, "qmm: null pointer");
  if (!aligned(p.x, 16) || (p.ldx % 8) != 0)
    return fail(DSPARK_ERR_ALIGN, "qmm: x must be 16-byte aligned with ldx %% 8 == 0 (ldx=%lld)", (long long)p.ldx);
  if (!aligned(p.w, 16)) return fail(DSPARK_ERR_ALIGN, "qmm: packed weights must be 16-byte aligned");
  if (!aligned(p.scales, 2) || !aligned(p.biases, 2) || !aligned(p.y, 2))
    return fail(DSPARK_ERR_ALIGN, "qmm: bf16 buffers must be 2-byte aligned");
  if (p.ldx < p.K || p.ldy < p.N)
    return fail(DSPARK_ERR_SHAPE, "qmm: ldx=%lld < K=%lld or ldy=%lld < N=%lld", (long long)p.ldx, (long long)p.K,
                (long long)p.ldy, (long long)p.N);
  return DSPARK_OK;
}

int validate(const dspark_qmm_problem* problems, int count, int64_t M, int bits, int group_size, long* Ns,
             bool packed = false) {
  if (!problems || count < 1 || count > kQmmMaxProblems)
    return fail(DSPARK_ERR_ARG, "qmm: problem count %d (1..%d)", count, kQmmMaxProblems);
  for (int i = 0; i < count; ++i) {
    int st = check_common(M, problems[i].K, problems[i].N, bits, group_size);
    if (st) return st;
    if (packed && problems[i].K % 512)
      return fail(DSPARK_ERR_SHAPE, "qmm_packed: K=%lld is not a multiple of 512", (long long)problems[i].K);
    if ((st = check_problem(problems[i]))) return st;
    if (problems[i].K != problems[0].K) return fail(DSPARK_ERR_SHAPE, "qmm: all problems of one launch must share K");
    Ns[i] = problems[i].N;
  }
  return DSPARK_OK;
}

}  // namespace
}  // namespace dspark

using namespace dspark;

extern "C" int dspark_qmm_affine_supported(int64_t M, int64_t K, int64_t N, int bits, int group_size) {
  const int st = check_common(M, K, N, bits, group_size);
  if (st) return st;
  long Ns[1] = {(long)N};
  if (make_plan(Ns, 1, K, M, bits, true).S == 0)
    return fail(DSPARK_ERR_SHAPE, "qmm: M=%lld x N=%lld x K=%lld needs more than %zu split-K counters or 32 slices",
                (long long)M, (long long)N, (long long)K, kMaxCounters);
  return DSPARK_OK;
}

extern "C" int dspark_qmm_affine_plan(int64_t M, int64_t K, int64_t N, int bits, int group_size, int32_t* out) {
  if (!out) return fail(DSPARK_ERR_ARG, "qmm_plan: null output");
  const int st = dspark_qmm_affine_supported(M, K, N, bits, group_size);
  if (st) return st;
  long Ns[1] = {(long)N};
  const Plan p = make_plan(Ns, 1, K, M, bits, true);
  out[0] = p.S;
  out[1] = p.ksmax;
  out[2] = p.strips;
  out[3] = p.wholek ? p.tiles * p.mtiles : p.S * p.strips * p.mtiles;
  return DSPARK_OK;
}

extern "C" size_t dspark_qmm_affine_multi_workspace(const dspark_qmm_problem* problems, int count, int64_t M,
                                                    int bits, int group_size) {
  long Ns[kQmmMaxProblems];
  if (validate(problems, count, M, bits, group_size, Ns)) return 0;
  const Plan p = make_plan(Ns, count, problems[0].K, M, bits, true);
  return p.ctr_bytes + p.part_bytes;
}

extern "C" size_t dspark_qmm_affine_workspace(int64_t M, int64_t K, int64_t N, int bits, int group_size) {
  if (check_common(M, K, N, bits, group_size)) return 0;
  long Ns[1] = {(long)N};
  const Plan p = make_plan(Ns, 1, K, M, bits, true);
  return p.ctr_bytes + p.part_bytes;
}

namespace dspark {
namespace {
// One launch over `count` problems; problems[i].w / .scales / .biases are the reference layout,
// or (packed) the tile stream / the scale-bias tiles / unused.
int multi_impl(const dspark_qmm_problem* problems, int count, int64_t M, int bits, int group_size, bool packed,
               void* workspace, size_t workspace_bytes, hipStream_t s) {
  long Ns[kQmmMaxProblems];
  int st = validate(problems, count, M, bits, group_size, Ns, packed);
  if (st) return st;
  const long K = problems[0].K;
  const Plan p = make_plan(Ns, count, K, M, bits, true);
  if (p.S == 0)
    return fail(DSPARK_ERR_SHAPE, "qmm: M=%lld K=%lld needs more than %zu split-K counters or 32 slices", (long long)M,
                (long long)K, kMaxCounters);
  const size_t need = p.ctr_bytes + p.part_bytes;
  if (need && (!workspace || workspace_bytes < need))
    return fail(DSPARK_ERR_WORKSPACE, "qmm: workspace %zu < %zu bytes", workspace_bytes, need);
  if (need && !aligned(workspace, 256)) return fail(DSPARK_ERR_ALIGN, "qmm: workspace must be 256-byte aligned");
  const long G = K / 64;
  bool sbvec = G % 8 == 0;
  QmmSkArgs a{};
  a.count = count;
  a.M = (int)M;
  a.S = p.S;
  int strip0 = 0;
  int* ctr = static_cast<int*>(workspace);
  float* part = need ? reinterpret_cast<float*>(static_cast<char*>(workspace) + p.ctr_bytes) : nullptr;
  for (int i = 0; i < count; ++i) {
    const dspark_qmm_problem& q = problems[i];
    QmmSkProb& d = a.p[i];
    d.x = static_cast<const u16*>(q.x);
    d.w = q.w;
    d.s = static_cast<const u16*>(q.scales);
    d.b = static_cast<const u16*>(q.biases);
    d.y = static_cast<u16*>(q.y);
    d.ldx = q.ldx;
    d.ldy = q.ldy;
    d.N = (int)q.N;
    d.K = (int)K;
    d.strips = (int)((q.N + kStripRows - 1) / kStripRows);
    d.strip0 = strip0;
    if (need) {
      d.ctr = ctr;
      d.part = part;
      ctr += (size_t)d.strips * p.mtiles;
      part += (size_t)d.strips * p.mtiles * p.S * 16 * kStripRows;
    }
    strip0 += d.strips;
    if (!packed) sbvec = sbvec && aligned(q.scales, 16) && aligned(q.biases, 16);
  }
  for (int i = count; i < kQmmMaxProblems; ++i) {
    a.p[i] = a.p[0];
    a.p[i].strip0 = 1 << 30;
  }
  if (packed) {
    if (const CuShape c = cu_shape(problems, count, Ns, K, bits, p); c.tpw) {  // blockIdx.x counts TPW-tile groups
      int t0 = 0;
      for (int i = 0; i < count; ++i) {
        a.p[i].strip0 = t0;
        t0 += (int)((problems[i].N + 15) / 16);
      }
      return launch_cu(a, p, bits, c, t0, s);
    }
  }
  if (p.wholek) {  // blockIdx.x counts 16-row tiles
    int t0 = 0;
    for (int i = 0; i < count; ++i) {
      a.p[i].strip0 = t0;
      t0 += (int)((problems[i].N + 15) / 16);
    }
    if (packed) return launch_wk<true, true>(a, p, bits, s);
    return sbvec ? launch_wk<false, true>(a, p, bits, s) : launch_wk<false, false>(a, p, bits, s);
  }
  if (packed) return bits == 4 ? launch_packed<4>(a, p, s) : launch_packed<8>(a, p, s);
  return bits == 4 ? launch_bits<4>(a, p, sbvec, s) : launch_bits<8>(a, p, sbvec, s);
}

int to_views(const dspark_qmm_packed_problem* pp, int count, dspark_qmm_problem* out) {
  if (!pp || count < 1 || count > kQmmMaxProblems)
    return fail(DSPARK_ERR_ARG, "qmm_packed: problem count %d (1..%d)", count, kQmmMaxProblems);
  for (int i = 0; i < count; ++i) {
    out[i].x = pp[i].x;
    out[i].ldx = pp[i].ldx;
    out[i].w = static_cast<const uint32_t*>(pp[i].packed);
    out[i].scales = nullptr;  // set once bits are known
    out[i].biases = nullptr;
    out[i].y = pp[i].y;
    out[i].ldy = pp[i].ldy;
    out[i].N = pp[i].N;
    out[i].K = pp[i].K;
  }
  return DSPARK_OK;
}

int packed_views(const dspark_qmm_packed_problem* pp, int count, int bits, dspark_qmm_problem* out) {
  int st = to_views(pp, count, out);
  if (st) return st;
  for (int i = 0; i < count; ++i) {
    if (!pp[i].packed) return fail(DSPARK_ERR_ARG, "qmm_packed: null packed pointer");
    if (!aligned(pp[i].packed, 16)) return fail(DSPARK_ERR_ALIGN, "qmm_packed: packed buffer must be 16-byte aligned");
    const PackedLayout L = packed_layout(pp[i].N, pp[i].K, bits);
    out[i].scales = static_cast<const char*>(pp[i].packed) + (size_t)L.wchunks * 16;
    out[i].biases = out[i].scales;
  }
  return DSPARK_OK;
}
}  // namespace
}  // namespace dspark

extern "C" int dspark_qmm_affine_multi(const dspark_qmm_problem* problems, int count, int64_t M, int bits,
                                       int group_size, void* workspace, size_t workspace_bytes,
                                       dspark_stream stream) {
  return multi_impl(problems, count, M, bits, group_size, false, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

extern "C" size_t dspark_qmm_packed_bytes(int64_t N, int64_t K, int bits, int group_size) {
  if (check_common(1, K, N, bits, group_size) || K % 512) return 0;
  return packed_layout(N, K, bits).bytes();
}

extern "C" int dspark_qmm_pack(const uint32_t* w, const void* scales, const void* biases, int64_t N, int64_t K,
                               int bits, int group_size, void* packed, size_t packed_bytes, dspark_stream stream) {
  int st = check_common(1, K, N, bits, group_size);
  if (st) return st;
  if (K % 512) return fail(DSPARK_ERR_SHAPE, "qmm_pack: K=%lld is not a multiple of 512", (long long)K);
  if (!w || !scales || !biases || !packed) return fail(DSPARK_ERR_ARG, "qmm_pack: null pointer");
  if (!aligned(w, 16) || !aligned(scales, 16) || !aligned(biases, 16) || !aligned(packed, 16))
    return fail(DSPARK_ERR_ALIGN, "qmm_pack: weights, scales, biases and the packed buffer must be 16-byte aligned");
  const PackedLayout L = packed_layout(N, K, bits);
  if (packed_bytes < L.bytes())
    return fail(DSPARK_ERR_WORKSPACE, "qmm_pack: packed buffer %zu < %zu bytes", packed_bytes, L.bytes());
  const long chunks = L.wchunks + L.schunks;
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), reinterpret_cast<const unsigned char*>(w),
                     static_cast<const u16*>(scales), static_cast<const u16*>(biases), nullptr, nullptr, nullptr,
                     (long)N, (int)K, bits, L.wchunks, L.schunks, static_cast<unsigned char*>(packed));
  return check_launch("dspark_qmm_pack");
}

// ---- packed expert weights for the fused MoE block: the weight part of the packed form over the
// E * N rows of [E, N, K*bits/32] (16-row tiles never straddle two experts: N % 16 == 0)
extern "C" size_t dspark_moe_packed_bytes(int64_t E, int64_t N, int64_t K, int bits, int group_size) {
  if (E < 1 || N % 16 || check_common(1, K, N, bits, group_size) || K % 128) return 0;
  return (size_t)packed_layout(E * N, K, bits).wchunks * 16;
}

extern "C" int dspark_moe_pack(const uint32_t* w, int64_t E, int64_t N, int64_t K, int bits, int group_size,
                               void* packed, size_t packed_bytes, dspark_stream stream) {
  int st = check_common(1, K, N, bits, group_size);
  if (st) return st;
  if (E < 1 || N % 16 || K % 128)
    return fail(DSPARK_ERR_SHAPE, "moe_pack: E=%lld N=%lld K=%lld (N %% 16 == 0, K %% 128 == 0)", (long long)E,
                (long long)N, (long long)K);
  if (!w || !packed) return fail(DSPARK_ERR_ARG, "moe_pack: null pointer");
  if (!aligned(w, 16) || !aligned(packed, 16)) return fail(DSPARK_ERR_ALIGN, "moe_pack: buffers must be 16-byte aligned");
  const PackedLayout L = packed_layout(E * N, K, bits);
  if (packed_bytes < (size_t)L.wchunks * 16)
    return fail(DSPARK_ERR_WORKSPACE, "moe_pack: packed buffer %zu < %zu bytes", packed_bytes, (size_t)L.wchunks * 16);
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((L.wchunks + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), reinterpret_cast<const unsigned char*>(w), nullptr, nullptr,
                     nullptr, nullptr, nullptr, (long)(E * N), (int)K, bits, L.wchunks, 0L,
                     static_cast<unsigned char*>(packed));
  return check_launch("dspark_moe_pack");
}

// ---- fused gate / up / SwiGLU over the pair form: rows of the pair buffer = 32 ceil(N / 16)
namespace {
long swiglu_rows(int64_t N) { return 32 * ((N + 15) / 16); }
}  // namespace

extern "C" size_t dspark_qmm_swiglu_packed_bytes(int64_t N, int64_t K, int bits, int group_size) {
  if (check_common(1, K, N, bits, group_size) || K % 512) return 0;
  return packed_layout(swiglu_rows(N), K, bits).bytes();
}

extern "C" int dspark_qmm_pack_swiglu(const uint32_t* gate_w, const void* gate_scales, const void* gate_biases,
                                      const uint32_t* up_w, const void* up_scales, const void* up_biases, int64_t N,
                                      int64_t K, int bits, int group_size, void* packed, size_t packed_bytes,
                                      dspark_stream stream) {
  int st = check_common(1, K, N, bits, group_size);
  if (st) return st;
  if (K % 512) return fail(DSPARK_ERR_SHAPE, "qmm_pack_swiglu: K=%lld is not a multiple of 512", (long long)K);
  if (!gate_w || !gate_scales || !gate_biases || !up_w || !up_scales || !up_biases || !packed)
    return fail(DSPARK_ERR_ARG, "qmm_pack_swiglu: null pointer");
  if (!aligned(gate_w, 16) || !aligned(gate_scales, 16) || !aligned(gate_biases, 16) || !aligned(up_w, 16) ||
      !aligned(up_scales, 16) || !aligned(up_biases, 16) || !aligned(packed, 16))
    return fail(DSPARK_ERR_ALIGN, "qmm_pack_swiglu: every buffer must be 16-byte aligned");
  const PackedLayout L = packed_layout(swiglu_rows(N), K, bits);
  if (packed_bytes < L.bytes())
    return fail(DSPARK_ERR_WORKSPACE, "qmm_pack_swiglu: packed buffer %zu < %zu bytes", packed_bytes, L.bytes());
  const long chunks = L.wchunks + L.schunks;
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), reinterpret_cast<const unsigned char*>(gate_w),
                     static_cast<const u16*>(gate_scales), static_cast<const u16*>(gate_biases),
                     reinterpret_cast<const unsigned char*>(up_w), static_cast<const u16*>(up_scales),
                     static_cast<const u16*>(up_biases), (long)N, (int)K, bits, L.wchunks, L.schunks,
                     static_cast<unsigned char*>(packed));
  return check_launch("dspark_qmm_pack_swiglu");
}

extern "C" size_t dspark_qmm_swiglu_packed_workspace(int64_t N, int64_t K, int64_t M, int bits, int group_size) {
  if (check_common(M, K, N, bits, group_size) || K % 512) return 0;
  long Ns[1] = {swiglu_rows(N)};
  const Plan p = make_plan(Ns, 1, K, M, bits);
  return p.ctr_bytes + p.part_bytes;
}

extern "C" int dspark_qmm_swiglu_packed(const void* x, int64_t ldx, const void* packed, void* h, int64_t ldh,
                                        int64_t N, int64_t K, int64_t M, int bits, int group_size, void* workspace,
                                        size_t workspace_bytes, dspark_stream stream) {
  int st = check_common(M, K, N, bits, group_size);
  if (st) return st;
  if (K % 512) return fail(DSPARK_ERR_SHAPE, "qmm_swiglu_packed: K=%lld is not a multiple of 512", (long long)K);
  if (!x || !packed || !h) return fail(DSPARK_ERR_ARG, "qmm_swiglu_packed: null pointer");
  if (!aligned(x, 16) || ldx % 8 || !aligned(packed, 16) || !aligned(h, 2))
    return fail(DSPARK_ERR_ALIGN, "qmm_swiglu_packed: x 16-byte aligned with ldx %% 8 == 0, packed 16-byte aligned");
  if (ldx < K || ldh < N)
    return fail(DSPARK_ERR_SHAPE, "qmm_swiglu_packed: ldx=%lld < K or ldh=%lld < N", (long long)ldx, (long long)ldh);
  long Ns[1] = {swiglu_rows(N)};
  const Plan p = make_plan(Ns, 1, K, M, bits);
  if (p.S == 0) return fail(DSPARK_ERR_SHAPE, "qmm_swiglu_packed: M=%lld needs too many split-K counters", (long long)M);
  const size_t need = p.ctr_bytes + p.part_bytes;
  if (need && (!workspace || workspace_bytes < need))
    return fail(DSPARK_ERR_WORKSPACE, "qmm_swiglu_packed: workspace %zu < %zu bytes", workspace_bytes, need);
  if (need && !aligned(workspace, 256))
    return fail(DSPARK_ERR_ALIGN, "qmm_swiglu_packed: workspace must be 256-byte aligned");
  const PackedLayout L = packed_layout(Ns[0], K, bits);
  QmmSkArgs a{};
  a.count = 1;
  a.M = (int)M;
  a.S = p.S;
  QmmSkProb& d = a.p[0];
  d.x = static_cast<const u16*>(x);
  d.w = static_cast<const u32*>(packed);
  d.s = reinterpret_cast<const u16*>(static_cast<const char*>(packed) + (size_t)L.wchunks * 16);
  d.b = d.s;
  d.y = static_cast<u16*>(h);
  d.ldx = ldx;
  d.ldy = ldh;
  d.N = (int)Ns[0];
  d.hN = (int)N;
  d.K = (int)K;
  d.strips = p.strips;
  d.strip0 = 0;
  if (need) {
    d.ctr = static_cast<int*>(workspace);
    d.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + p.ctr_bytes);
  }
  for (int i = 1; i < kQmmMaxProblems; ++i) {
    a.p[i] = a.p[0];
    a.p[i].strip0 = 1 << 30;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  return bits == 4 ? launch_packed<4, true>(a, p, s) : launch_packed<8, true>(a, p, s);
}

extern "C" int dspark_qmm_packed_multi(const dspark_qmm_packed_problem* problems, int count, int64_t M, int bits,
                                       int group_size, void* workspace, size_t workspace_bytes,
                                       dspark_stream stream) {
  dspark_qmm_problem views[kQmmMaxProblems];
  int st = packed_views(problems, count, bits, views);
  if (st) return st;
  return multi_impl(views, count, M, bits, group_size, true, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

extern "C" int dspark_qmm_packed_multi_plan(const dspark_qmm_packed_problem* problems, int count, int64_t M, int bits,
                                            int group_size, int32_t* out) {
  if (!out) return fail(DSPARK_ERR_ARG, "qmm_plan: null output");
  dspark_qmm_problem views[kQmmMaxProblems];
  long Ns[kQmmMaxProblems];
  int st = packed_views(problems, count, bits, views);
  if (st || (st = validate(views, count, M, bits, group_size, Ns, true))) return st;
  const Plan p = make_plan(Ns, count, views[0].K, M, bits, true);
  if (p.S == 0) return fail(DSPARK_ERR_SHAPE, "qmm_plan: shape refused");
  const CuShape c = cu_shape(views, count, Ns, views[0].K, bits, p);
  long tiles = 0;
  for (int i = 0; i < count; ++i) tiles += (Ns[i] + 15) / 16;
  out[0] = p.wholek ? 1 : c.tpw ? 2 : 0;
  out[1] = p.S;
  out[2] = c.tpw;
  out[3] = c.tpw ? (int)((tiles + c.tpw - 1) / c.tpw) * p.mtiles * c.kparts
                 : p.wholek ? p.tiles * p.mtiles : p.S * p.strips * p.mtiles;
  out[4] = c.tpw ? c.kparts : 0;
  return DSPARK_OK;
}

extern "C" size_t dspark_qmm_packed_multi_workspace(const dspark_qmm_packed_problem* problems, int count, int64_t M,
                                                    int bits, int group_size) {
  dspark_qmm_problem views[kQmmMaxProblems];
  if (packed_views(problems, count, bits, views)) return 0;
  return dspark_qmm_affine_multi_workspace(views, count, M, bits, group_size);
}

extern "C" int dspark_qmm_affine(const void* x, int64_t ldx, int64_t M, int64_t K, const uint32_t* w,
                                 const void* scales, const void* biases, int64_t N, int bits, int group_size,
                                 void* y, int64_t ldy, void* workspace, size_t workspace_bytes, dspark_stream stream) {
  dspark_qmm_problem p{x, ldx, w, scales, biases, y, ldy, N, K};
  return dspark_qmm_affine_multi(&p, 1, M, bits, group_size, workspace, workspace_bytes, stream);
}

// ---- dequantize once (the prefill wide path): w [N, K*bits/32] + scales/biases [N, K/64] ->
// out [N, K], out[n, j] = (scale * q) + bias in fp32 -- a product rounded, then a sum rounded,
// with no fma contraction, the arithmetic of an elementwise multiply followed by an add --
// stored as fp32 or rounded once more to bf16 / fp16. Thread = 8 consecutive values of a
// row (one word of 4-bit fields, two of 8-bit); grid-stride over N*K/8.
namespace dspark {
namespace {
template <int DT>
__device__ __forceinline__ float load_param(const void* p, long i) {
  if constexpr (DT == DSPARK_DTYPE_BF16) return bf2f(static_cast<const u16*>(p)[i]);
  else if constexpr (DT == DSPARK_DTYPE_F16) return (float)__builtin_bit_cast(_Float16, static_cast<const u16*>(p)[i]);
  else return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ float affine_value(float s, float q, float b) {
#pragma clang fp contract(off)
  const float p = s * q;
  return p + b;
}

template <int BITS, int SDT, int ODT>
__global__ __launch_bounds__(256) void dequant_kernel(const u32* __restrict__ w, const void* __restrict__ sc,
                                                      const void* __restrict__ bi, long N, int K,
                                                      void* __restrict__ out, long ldo) {
  const long per_row = K / 8;
  const long total = N * per_row;
  for (long c = (long)blockIdx.x * 256 + threadIdx.x; c < total; c += (long)gridDim.x * 256) {
    const long n = c / per_row;
    const int j0 = (int)(c - n * per_row) * 8;
    const long g = n * (K / 64) + j0 / 64;
    const float s = load_param<SDT>(sc, g), b = load_param<SDT>(bi, g);
    u32 f[8];
    if constexpr (BITS == 8) {
      const u32x2_t wv = ldg64(w + n * (K / 4) + j0 / 4);
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = (wv[i / 4] >> (8 * (i % 4))) & 0xFFu;
    } else {
      const u32 wv = w[n * (K / 8) + j0 / 8];
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = (wv >> (4 * i)) & 0xFu;
    }
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = affine_value(s, (float)f[i], b);
    if constexpr (ODT == DSPARK_DTYPE_F32) {
      float* o = static_cast<float*>(out) + n * ldo + j0;
      *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      u32x4_t o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (ODT == DSPARK_DTYPE_F16) {
          const _Float16 h0 = (_Float16)v[2 * i], h1 = (_Float16)v[2 * i + 1];
          o[i] = (u32)__builtin_bit_cast(u16, h0) | ((u32)__builtin_bit_cast(u16, h1) << 16);
        } else {
          o[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
        }
      }
      *reinterpret_cast<u32x4_t*>(static_cast<u16*>(out) + n * ldo + j0) = o;
    }
  }
}

template <int BITS, int SDT>
void launch_dequant(int odt, unsigned blocks, hipStream_t s, const u32* w, const void* sc, const void* bi, long N,
                    int K, void* out, long ldo) {
  if (odt == DSPARK_DTYPE_F32)
    hipLaunchKernelGGL((dequant_kernel<BITS, SDT, DSPARK_DTYPE_F32>), dim3(blocks), dim3(256), 0, s, w, sc, bi, N, K, out, ldo);
  else if (odt == DSPARK_DTYPE_F16)
    hipLaunchKernelGGL((dequant_kernel<BITS, SDT, DSPARK_DTYPE_F16>), dim3(blocks), dim3(256), 0, s, w, sc, bi, N, K, out, ldo);
  else
    hipLaunchKernelGGL((dequant_kernel<BITS, SDT, DSPARK_DTYPE_BF16>), dim3(blocks), dim3(256), 0, s, w, sc, bi, N, K, out, ldo);
}

template <int BITS>
void launch_dequant_bits(int sdt, int odt, unsigned blocks, hipStream_t s, const u32* w, const void* sc,
                         const void* bi, long N, int K, void* out, long ldo) {
  if (sdt == DSPARK_DTYPE_F32) launch_dequant<BITS, DSPARK_DTYPE_F32>(odt, blocks, s, w, sc, bi, N, K, out, ldo);
  else if (sdt == DSPARK_DTYPE_F16) launch_dequant<BITS, DSPARK_DTYPE_F16>(odt, blocks, s, w, sc, bi, N, K, out, ldo);
  else launch_dequant<BITS, DSPARK_DTYPE_BF16>(odt, blocks, s, w, sc, bi, N, K, out, ldo);
}

bool known_dtype(int dt) { return dt == DSPARK_DTYPE_BF16 || dt == DSPARK_DTYPE_F16 || dt == DSPARK_DTYPE_F32; }
}  // namespace
}  // namespace dspark

extern "C" int dspark_qmm_dequantize(const uint32_t* w, const void* scales, const void* biases, int scale_dtype,
                                     int64_t N, int64_t K, int bits, int group_size, int dtype, void* out,
                                     int64_t ldo, dspark_stream stream) {
  int st = check_common(1, K, N, bits, group_size);
  if (st) return st;
  if (!known_dtype(dtype) || !known_dtype(scale_dtype))
    return fail(DSPARK_ERR_UNSUPPORTED, "qmm_dequantize: dtype %d / scale dtype %d (bf16, fp16 or fp32)", dtype,
                scale_dtype);
  if (!w || !scales || !biases || !out) return fail(DSPARK_ERR_ARG, "qmm_dequantize: null pointer");
  const int pbytes = scale_dtype == DSPARK_DTYPE_F32 ? 4 : 2;
  if (!aligned(w, bits == 8 ? 8 : 4) || !aligned(scales, pbytes) || !aligned(biases, pbytes) || !aligned(out, 16) ||
      ldo % 8)
    return fail(DSPARK_ERR_ALIGN, "qmm_dequantize: w %d-byte aligned, out 16-byte aligned with ldo %% 8 == 0",
                bits == 8 ? 8 : 4);
  if (ldo < K) return fail(DSPARK_ERR_SHAPE, "qmm_dequantize: ldo=%lld < K=%lld", (long long)ldo, (long long)K);
  const long total = (long)N * (K / 8);
  const unsigned blocks = (unsigned)std::min<long>((total + 255) / 256, 1L << 20);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (bits == 8) launch_dequant_bits<8>(scale_dtype, dtype, blocks, s, w, scales, biases, (long)N, (int)K, out, (long)ldo);
  else launch_dequant_bits<4>(scale_dtype, dtype, blocks, s, w, scales, biases, (long)N, (int)K, out, (long)ldo);
  return check_launch("dspark_qmm_dequantize");
}

// ---- split-K counter reset: a fill kernel (not hipMemsetAsync, so the call may sit in a
// captured graph) over the counter region at the start of a qmm workspace.
namespace dspark {
namespace {
__global__ __launch_bounds__(256) void zero_words_kernel(u32* __restrict__ p, long n) {
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) p[i] = 0u;
}

int zero_counters(void* base, size_t bytes, hipStream_t s, const char* what) {
  const long words = (long)(bytes / sizeof(u32));
  hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s,
                     static_cast<u32*>(base), words);
  return check_launch(what);
}
}  // namespace
}  // namespace dspark

extern "C" int dspark_qmm_workspace_reset(void* workspace, size_t workspace_bytes, dspark_stream stream) {
  if (!workspace) return fail(DSPARK_ERR_ARG, "qmm_workspace_reset: null workspace");
  if (!aligned(workspace, 256)) return fail(DSPARK_ERR_ALIGN, "qmm_workspace_reset: workspace must be 256-byte aligned");
  const size_t n = workspace_bytes < kCtrRegionBytes ? workspace_bytes : kCtrRegionBytes;
  if (n < sizeof(int)) return DSPARK_OK;
  return zero_counters(workspace, n, static_cast<hipStream_t>(stream), "dspark_qmm_workspace_reset");
}

// ---- dspark_qmm_affine without a caller workspace: the split-K counters and partials live in
// a file-scope device array (one copy per GPU, held until the process ends). Host code never
// passes the array's name to a kernel: it stands in for the symbol on the host. The device
// address comes from hipGetSymbolAddress, once per device with that device current, and is
// kept per device.
namespace dspark {
namespace {
constexpr size_t kNoallocPartBytes = 32u << 20;  // fp32 split-K partials
constexpr size_t kNoallocBytes = kCtrRegionBytes + kNoallocPartBytes;
static __device__ __align__(256) unsigned char scratch[kNoallocBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The scratch address of the current device; its counter region is cleared (on `s`, before
// any use) the first time. Returns a dspark_status.
int scratch_for_current_device(hipStream_t s, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(DSPARK_ERR_LAUNCH, "qmm_affine_noalloc: no current HIP device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(DSPARK_ERR_LAUNCH, "qmm_affine_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                  hipGetErrorString(e));
    const int st = zero_counters(ptr, kCtrRegionBytes, s, "dspark_qmm_affine_noalloc(clear)");
    if (st) return st;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return DSPARK_OK;
}
}  // namespace
}  // namespace dspark

extern "C" int dspark_qmm_affine_noalloc(const void* x, int64_t ldx, int64_t M, int64_t K, const uint32_t* w,
                                         const void* scales, const void* biases, int64_t N, int bits,
                                         int group_size, void* y, int64_t ldy, dspark_stream stream) {
  dspark_qmm_problem p{x, ldx, w, scales, biases, y, ldy, N, K};
  long Ns[1];
  int st = validate(&p, 1, M, bits, group_size, Ns);
  if (st) return st;
  const Plan pl = make_plan(Ns, 1, K, M, bits, true);
  if (pl.S == 0)
    return fail(DSPARK_ERR_SHAPE, "qmm_affine_noalloc: M=%lld x N=%lld x K=%lld is not supported", (long long)M,
                (long long)N, (long long)K);
  const size_t need = pl.ctr_bytes + pl.part_bytes;
  if (need > kNoallocBytes)
    return fail(DSPARK_ERR_WORKSPACE,
                "qmm_affine_noalloc: M=%lld x N=%lld x K=%lld needs %zu bytes of split-K scratch, more than the "
                "%zu the library holds per GPU; call dspark_qmm_affine with a workspace",
                (long long)M, (long long)N, (long long)K, need, kNoallocBytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ptr = nullptr;
  if (need && (st = scratch_for_current_device(s, &ptr))) return st;
  return multi_impl(&p, 1, M, bits, group_size, false, ptr, need ? kNoallocBytes : 0, s);
}

extern "C" int dspark_qmm_noalloc_reset(dspark_stream stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ptr = nullptr;
  const int st = scratch_for_current_device(s, &ptr);
  if (st) return st;
  return zero_counters(ptr, kCtrRegionBytes, s, "dspark_qmm_noalloc_reset");
}

extern "C" int dspark_qmm_noalloc_scratch(void** ptr, size_t* bytes) {
  if (!ptr || !bytes) return fail(DSPARK_ERR_ARG, "qmm_noalloc_scratch: null pointer");
  *bytes = kNoallocBytes;
  return scratch_for_current_device(nullptr, ptr);
}
