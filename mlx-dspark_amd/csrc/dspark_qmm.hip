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
//   * K is split across the W waves of a workgroup; the W partial 16x16 tiles are summed in
//     LDS in a fixed wave order, so results are deterministic and independent of M.
#include "dspark_qmm_core.h"

namespace dspark {
namespace {

constexpr int kMaxProblems = DSPARK_QMM_MAX_PROBLEMS;

struct QmmProb {
  const u16* x;
  const u32* w;
  const u16* s;
  const u16* b;
  u16* y;
  long ldx;
  long ldy;
  int N;
  int K;
  int tile0;  // first workgroup (blockIdx.x) of this problem
  int pad_;
};

struct QmmArgs {
  QmmProb p[kMaxProblems];
  int count;
  int M;
};

// One workgroup: NT tiles of 16 output features x one 16-row tile of x, K split over W waves.
template <int BITS, int W, int NT, int CH>
__global__ __launch_bounds__(64 * W) void qmm_kernel(const QmmArgs args) {
  // -------- which problem / tile
  const int bx = blockIdx.x;
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxProblems; ++i)
    if (i < args.count && bx >= args.p[i].tile0) pi = i;
  const QmmProb& P = args.p[pi];
  const u16* __restrict__ x = P.x;
  const u32* __restrict__ w = P.w;
  const u16* __restrict__ sc = P.s;
  const u16* __restrict__ bi = P.b;
  u16* __restrict__ y = P.y;
  const long ldx = P.ldx;
  const long ldy = P.ldy;
  const int N = P.N;
  const int K = P.K;
  const int tile0 = P.tile0;

  const int G = K >> 6;
  const int n_base = (bx - tile0) * (16 * NT);
  const int m_base = blockIdx.y * 16;
  const int m_rows = min(16, args.M - m_base);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15;
  const int q = lane >> 4;
  const int g0 = (wave * G) / W;
  const int g1 = ((wave + 1) * G) / W;

  const u16* xr = x + (long)(m_base + min(c16, m_rows - 1)) * ldx + 16 * q;
  const u32* wr[NT];
  const u16* sr[NT];
  const u16* br[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int n = min(n_base + 16 * j + c16, N - 1);
    wr[j] = wrow_ptr<BITS>(w, n, K, q);
    sr[j] = sc + (long)n * G;
    br[j] = bi + (long)n * G;
  }
  f32x4_t acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  qmm_wave_partial<BITS, NT, CH>(xr, wr, sr, br, g0, g1, acc);

  // -------- split-K reduction over the W waves (fixed order)
  __shared__ float red[W][NT][256];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][j][(4 * q + r) * 16 + c16] = acc[j][r];
  __syncthreads();
  for (int t = threadIdx.x; t < NT * 256; t += 64 * W) {
    const int j = t >> 8, e = t & 255;
    const int m = e >> 4, nn = e & 15;
    float v = 0.f;
#pragma unroll
    for (int ww = 0; ww < W; ++ww) v += red[ww][j][e];
    const int n = n_base + 16 * j + nn;
    if (m < m_rows && n < N) y[(long)(m_base + m) * ldy + n] = f2bf(v);
  }
}

template <int BITS, int W, int NT, int CH>
int launch(const QmmArgs& a, int tiles, int mtiles, hipStream_t st) {
  hipLaunchKernelGGL((qmm_kernel<BITS, W, NT, CH>), dim3(tiles, mtiles, 1), dim3(64 * W, 1, 1), 0, st, a);
  return check_launch("dspark_qmm_affine");
}

// Launch geometry: workgroups of W waves split K; NT output tiles per workgroup. NT > 1 only
// when there are enough tiles to keep >= 2 workgroups per CU (256 CUs) busy.
struct Geometry {
  int W;
  int NT;
};

Geometry choose_geometry(long total_rows, long K) {
  Geometry g{8, 1};
  const long G = K / 64;
  if (G < 16) g.W = 4;
  if (total_rows >= 16L * 2 * 512) g.NT = 2;
  return g;
}

int qmm_dispatch(const QmmArgs& a, int bits, long total_rows, long K, hipStream_t st) {
  const Geometry geo = choose_geometry(total_rows, K);
  int tiles = 0;
  QmmArgs args = a;
  for (int i = 0; i < a.count; ++i) {
    args.p[i].tile0 = tiles;
    tiles += (int)((a.p[i].N + 16 * geo.NT - 1) / (16 * geo.NT));
  }
  for (int i = a.count; i < kMaxProblems; ++i) args.p[i] = args.p[0], args.p[i].tile0 = 1 << 30;
  const int mtiles = (a.M + 15) / 16;
  constexpr int CH = 4;
  if (bits == 4) {
    if (geo.W == 8) return geo.NT == 2 ? launch<4, 8, 2, CH>(args, tiles, mtiles, st) : launch<4, 8, 1, CH>(args, tiles, mtiles, st);
    return geo.NT == 2 ? launch<4, 4, 2, CH>(args, tiles, mtiles, st) : launch<4, 4, 1, CH>(args, tiles, mtiles, st);
  }
  if (geo.W == 8) return geo.NT == 2 ? launch<8, 8, 2, CH>(args, tiles, mtiles, st) : launch<8, 8, 1, CH>(args, tiles, mtiles, st);
  return geo.NT == 2 ? launch<8, 4, 2, CH>(args, tiles, mtiles, st) : launch<8, 4, 1, CH>(args, tiles, mtiles, st);
}

int check_common(int64_t M, int64_t K, int64_t N, int bits, int group_size) {
  if (bits != 4 && bits != 8) return fail(DSPARK_ERR_UNSUPPORTED, "qmm: bits=%d (4 or 8 supported)", bits);
  if (group_size != 64) return fail(DSPARK_ERR_UNSUPPORTED, "qmm: group_size=%d (64 supported)", group_size);
  if (M < 1 || N < 1 || K < 64) return fail(DSPARK_ERR_SHAPE, "qmm: M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  if (K % 64) return fail(DSPARK_ERR_SHAPE, "qmm: K=%lld is not a multiple of 64", (long long)K);
  if (M > (1 << 20) || N > (1L << 30) / 16 || K > (1L << 24))
    return fail(DSPARK_ERR_SHAPE, "qmm: shape too large (M=%lld N=%lld K=%lld)", (long long)M, (long long)N, (long long)K);
  return DSPARK_OK;
}

int check_problem(const dspark_qmm_problem& p, int64_t M, int bits) {
  if (!p.x || !p.w || !p.scales || !p.biases || !p.y) return fail(DSPARK_ERR_ARG, "qmm: null pointer");
  if (!aligned(p.x, 16) || (p.ldx % 8) != 0) return fail(DSPARK_ERR_ALIGN, "qmm: x must be 16-byte aligned with ldx %% 8 == 0 (ldx=%lld)", (long long)p.ldx);
  if (!aligned(p.w, 16)) return fail(DSPARK_ERR_ALIGN, "qmm: packed weights must be 16-byte aligned");
  if (!aligned(p.scales, 2) || !aligned(p.biases, 2) || !aligned(p.y, 2)) return fail(DSPARK_ERR_ALIGN, "qmm: bf16 buffers must be 2-byte aligned");
  if (p.ldx < p.K || p.ldy < p.N) return fail(DSPARK_ERR_SHAPE, "qmm: ldx=%lld < K=%lld or ldy=%lld < N=%lld", (long long)p.ldx, (long long)p.K, (long long)p.ldy, (long long)p.N);
  (void)M;
  (void)bits;
  return DSPARK_OK;
}

}  // namespace
}  // namespace dspark

using namespace dspark;

extern "C" int dspark_qmm_affine_supported(int64_t M, int64_t K, int64_t N, int bits, int group_size) {
  return check_common(M, K, N, bits, group_size);
}

extern "C" int dspark_qmm_affine_multi(const dspark_qmm_problem* problems, int count, int64_t M, int bits,
                                       int group_size, dspark_stream stream) {
  if (!problems || count < 1 || count > kMaxProblems)
    return fail(DSPARK_ERR_ARG, "qmm_multi: count=%d (1..%d)", count, kMaxProblems);
  QmmArgs a{};
  a.count = count;
  a.M = (int)M;
  long total_rows = 0, kmax = 0;
  for (int i = 0; i < count; ++i) {
    const dspark_qmm_problem& p = problems[i];
    int st = check_common(M, p.K, p.N, bits, group_size);
    if (st) return st;
    st = check_problem(p, M, bits);
    if (st) return st;
    if (p.K != problems[0].K) return fail(DSPARK_ERR_SHAPE, "qmm_multi: all problems must share K");
    a.p[i].x = static_cast<const u16*>(p.x);
    a.p[i].w = p.w;
    a.p[i].s = static_cast<const u16*>(p.scales);
    a.p[i].b = static_cast<const u16*>(p.biases);
    a.p[i].y = static_cast<u16*>(p.y);
    a.p[i].ldx = p.ldx;
    a.p[i].ldy = p.ldy;
    a.p[i].N = (int)p.N;
    a.p[i].K = (int)p.K;
    total_rows += p.N;
    kmax = p.K > kmax ? p.K : kmax;
  }
  return qmm_dispatch(a, bits, total_rows, kmax, static_cast<hipStream_t>(stream));
}

extern "C" int dspark_qmm_affine(const void* x, int64_t ldx, int64_t M, int64_t K, const uint32_t* w,
                                 const void* scales, const void* biases, int64_t N, int bits, int group_size,
                                 void* y, int64_t ldy, dspark_stream stream) {
  dspark_qmm_problem p{x, ldx, w, scales, biases, y, ldy, N, K};
  return dspark_qmm_affine_multi(&p, 1, M, bits, group_size, stream);
}
