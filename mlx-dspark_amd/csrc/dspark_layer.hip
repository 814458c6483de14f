// The small kernels a dense verify forward needs around the qmm and attention launches
// (gfx950): residual add + RMSNorm, per-head q/k RMSNorm + RoPE + KV-cache write, SwiGLU,
// row argmax and the greedy accept count.
//
// Semantics are mlx-lm's qwen3-style decoder layer as the reference runs it
// (target.py:187-221 -> mlx-lm DecoderLayer, third-party) with mlx's bf16 op rounding:
//   h  = bf16(x + r)                                     residual add
//   y  = bf16(bf16(h * rsqrt(mean(h^2) + eps)) * w)      RMSNorm (fp32 statistics)
//   RoPE (non-traditional, pairs (i, i + D/2)), angle a = pos * base^(-2i/D) in fp32:
//        y_i = bf16(x_i cos a - x_{i+D/2} sin a),  y_{i+D/2} = bf16(x_i sin a + x_{i+D/2} cos a)
//   h  = bf16(bf16(g * bf16(sigmoid(g))) * u)            SwiGLU (mlx's silu = x * sigmoid(x))
// and the greedy accept of the verify loop (generate.py:1544-1555):
//   tt = argmax(logits, -1) (first maximum); n = sum(cumprod(draft == tt[:len(draft)])).
#include "dspark_common.h"

namespace dspark {
namespace {

__device__ __forceinline__ float bf16r(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += shfl_xor(v, o);
  return v;
}

constexpr int kNormThreads = 256;

// one workgroup per row; 8 bf16 per 16-byte chunk
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(const u16* x, long ldx, const u16* __restrict__ r,
                                                                   long ldr, const u16* __restrict__ w, int H,
                                                                   float eps, u16* hout, long ldh,
                                                                   u16* __restrict__ y, long ldy) {
  __shared__ float red[kNormThreads / 64];
  const int m = blockIdx.x;
  const u16* xr = x + (long)m * ldx;
  const u16* rr = r ? r + (long)m * ldr : nullptr;
  u16* hr = hout ? hout + (long)m * ldh : nullptr;
  const int chunks = H >> 3;
  float ss = 0.f;
  for (int c = threadIdx.x; c < chunks; c += kNormThreads) {
    u32x4_t xv = ldg128(xr + 8 * c);
    if (rr) {
      const u32x4_t rv = ldg128(rr + 8 * c);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xv[i] = pack_bf16x2(bf2f(xv[i] & 0xFFFFu) + bf2f(rv[i] & 0xFFFFu), bf2f(xv[i] >> 16) + bf2f(rv[i] >> 16));
      if (hr) *reinterpret_cast<u32x4_t*>(hr + 8 * c) = xv;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = bf2f(xv[i] & 0xFFFFu), b = bf2f(xv[i] >> 16);
      ss += a * a + b * b;
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += red[i];
  const float inv = 1.0f / __builtin_sqrtf(tot / (float)H + eps);
  u16* yr = y + (long)m * ldy;
  for (int c = threadIdx.x; c < chunks; c += kNormThreads) {
    // the sum h: re-read from h_out when it was written (h_out may alias x: the residual is
    // then updated in place, and each thread re-reads only chunks it wrote itself)
    u32x4_t xv = ldg128((hr ? hr : xr) + 8 * c);
    if (rr && !hr) {
      const u32x4_t rv = ldg128(rr + 8 * c);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xv[i] = pack_bf16x2(bf2f(xv[i] & 0xFFFFu) + bf2f(rv[i] & 0xFFFFu), bf2f(xv[i] >> 16) + bf2f(rv[i] >> 16));
    }
    const u32x4_t wv = ldg128(w + 8 * c);
    u32x4_t out;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = bf16r(bf2f(xv[i] & 0xFFFFu) * inv) * bf2f(wv[i] & 0xFFFFu);
      const float b = bf16r(bf2f(xv[i] >> 16) * inv) * bf2f(wv[i] >> 16);
      out[i] = pack_bf16x2(a, b);
    }
    *reinterpret_cast<u32x4_t*>(yr + 8 * c) = out;
  }
}

// The same row op with every chunk of the row held in registers between the two phases: x, r
// and w are all requested in one memory round trip, h is written once and never re-read.
// Per-thread chunk order and the reductions match add_rmsnorm_kernel, so the results do too.
template <int MAXC>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_reg_kernel(const u16* x, long ldx, const u16* __restrict__ r,
                                                                       long ldr, const u16* __restrict__ w, int H,
                                                                       float eps, u16* hout, long ldh,
                                                                       u16* __restrict__ y, long ldy) {
  __shared__ float red[kNormThreads / 64];
  const int m = blockIdx.x;
  const u16* xr = x + (long)m * ldx;
  const u16* rr = r ? r + (long)m * ldr : nullptr;
  u16* hr = hout ? hout + (long)m * ldh : nullptr;
  const int chunks = H >> 3;
  u32x4_t hv[MAXC], rv[MAXC], wv[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = min((int)threadIdx.x + i * kNormThreads, chunks - 1);
    hv[i] = ldg128(xr + 8 * c);
    if (rr) rv[i] = ldg128(rr + 8 * c);
    wv[i] = ldg128(w + 8 * c);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = threadIdx.x + i * kNormThreads;
    if (c >= chunks) continue;
    if (rr) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        hv[i][j] = pack_bf16x2(bf2f(hv[i][j] & 0xFFFFu) + bf2f(rv[i][j] & 0xFFFFu),
                               bf2f(hv[i][j] >> 16) + bf2f(rv[i][j] >> 16));
      if (hr) *reinterpret_cast<u32x4_t*>(hr + 8 * c) = hv[i];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = bf2f(hv[i][j] & 0xFFFFu), b = bf2f(hv[i][j] >> 16);
      ss += a * a + b * b;
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += red[i];
  const float inv = 1.0f / __builtin_sqrtf(tot / (float)H + eps);
  u16* yr = y + (long)m * ldy;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = threadIdx.x + i * kNormThreads;
    if (c >= chunks) continue;
    u32x4_t out;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = bf16r(bf2f(hv[i][j] & 0xFFFFu) * inv) * bf2f(wv[i][j] & 0xFFFFu);
      const float b = bf16r(bf2f(hv[i][j] >> 16) * inv) * bf2f(wv[i][j] >> 16);
      out[j] = pack_bf16x2(a, b);
    }
    *reinterpret_cast<u32x4_t*>(yr + 8 * c) = out;
  }
}

struct QkArgs {
  const u16* q;
  const u16* k;
  const u16* v;
  const u16* qw;
  const u16* kw;
  u16* qout;
  u16* kc;
  u16* vc;
  long ldq, ldk, ldv;
  long kch, kcs, vch, vcs;  // cache strides (head, position) in elements (words when quantized)
  int M, Hq, Hk, pos0, D;
  float eps, log2_base;
  // quantized cache (mlx-lm QuantizedKVCache): scales and biases of K and V, strides (head,
  // position) in elements; the words are kc / vc
  u16* ks;
  u16* kb;
  u16* vs;
  u16* vb;
  long ksh, kss, vsh, vss;
};

// RMSNorm-scaled pair (x1, x2) = elements (i, i + D/2) of a head, rotated by RoPE at `pos`:
// the two results before their bf16 rounding (shared by the plain and quantized cache writes, so
// both round the same values)
__device__ __forceinline__ void norm_rope_pair(float x1, float x2, float w1, float w2, float inv, int i, int D,
                                               int pos, float log2_base, float& r1, float& r2) {
  const float n1 = bf16r(bf16r(x1 * inv) * w1);
  const float n2 = bf16r(bf16r(x2 * inv) * w2);
  const float inv_freq = exp2f(-(2.0f * (float)i / (float)D) * log2_base);
  const float ang = (float)pos * inv_freq;
  float sn, cs;
  sincosf(ang, &sn, &cs);
  r1 = n1 * cs - n2 * sn;
  r2 = n1 * sn + n2 * cs;
}

// One cache row (a head's D values, held as in qk_norm_rope_kv_kernel: lane l has d = l + 64 j
// in a[j] and d + D/2 in b[j]) quantized in groups of 64 with the rule of the build's quantizer
// (dspark_rocm.quant.quantize_rows): scale = bf16((max - min) / (2^QB - 1)), bias = bf16(min),
// q = clamp(round_half_even((x - bias) / scale), 0, 2^QB - 1) (scale 0 divides by 1), each an
// fp32 operation rounded to nearest. Fields are stored as bytes of the row's words (field j at
// bits QB*(j % (32/QB)) of word j / (32/QB), low bits first = byte-addressed little-endian).
template <int NP, int QB>
__device__ __forceinline__ void store_quant_row(const float (&a)[NP], const float (&b)[NP], int lane, int D,
                                                unsigned char* wrow, u16* srow, u16* brow) {
  const int HALF = D >> 1, G = D >> 6;
  constexpr float kLevels = (float)((1 << QB) - 1);
  float scale[4], bias[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    float lo = INFINITY, hi = -INFINITY;
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int d = lane + 64 * j;
      if (d < HALF) {
        if ((d >> 6) == g) {
          lo = fminf(lo, a[j]);
          hi = fmaxf(hi, a[j]);
        }
        if (((d + HALF) >> 6) == g) {
          lo = fminf(lo, b[j]);
          hi = fmaxf(hi, b[j]);
        }
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      lo = fminf(lo, shfl_xor(lo, o));
      hi = fmaxf(hi, shfl_xor(hi, o));
    }
    const u16 sbits = f2bf(__fdiv_rn(__fsub_rn(hi, lo), kLevels)), bbits = f2bf(lo);
    if (g < G && lane == 0) {
      srow[g] = sbits;
      brow[g] = bbits;
    }
    const float s32 = bf2f(sbits);
    scale[g] = s32 == 0.f ? 1.f : s32;
    bias[g] = bf2f(bbits);
  }
  auto field = [&](float x, int d) {
    const int g = d >> 6;
    const float q = rintf(__fdiv_rn(__fsub_rn(x, bias[g]), scale[g]));
    return (u32)fminf(fmaxf(q, 0.f), kLevels);
  };
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int d = lane + 64 * j;
    const bool on = d < HALF;
    const u32 qa = on ? field(a[j], d) : 0u, qb = on ? field(b[j], d + HALF) : 0u;
    if constexpr (QB == 8) {
      if (on) {
        wrow[d] = (unsigned char)qa;
        wrow[d + HALF] = (unsigned char)qb;
      }
    } else {
      // two fields per byte: the even lane takes its odd neighbour's (d + 1 sits in lane + 1)
      const u32 na = (u32)__builtin_amdgcn_ds_bpermute((lane ^ 1) << 2, (int)qa);
      const u32 nb = (u32)__builtin_amdgcn_ds_bpermute((lane ^ 1) << 2, (int)qb);
      if (on && !(lane & 1)) {
        wrow[d >> 1] = (unsigned char)(qa | (na << 4));
        wrow[(d + HALF) >> 1] = (unsigned char)(qb | (nb << 4));
      }
    }
  }
}

// qk_norm_rope_kv_kernel writing a quantized cache: the same q output and the same rotated k
// (rounded to bf16) and v values, quantized into the cache rows (store_quant_row)
template <int NP, int QB>
__global__ __launch_bounds__(64) void qk_norm_rope_qkv_kernel(const QkArgs a) {
  const int D = a.D, HALF = a.D >> 1;
  const int m = blockIdx.x, hh = blockIdx.y, lane = threadIdx.x;
  const int pos = a.pos0 + m;
  float o1[NP], o2[NP];
  if (hh >= a.Hq + a.Hk) {  // V head
    const int h = hh - a.Hq - a.Hk;
    const u16* src = a.v + (long)m * a.ldv + (long)h * D;
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int i = lane + 64 * j;
      o1[j] = i < HALF ? bf2f(src[i]) : 0.f;
      o2[j] = i < HALF ? bf2f(src[i + HALF]) : 0.f;
    }
    store_quant_row<NP, QB>(o1, o2, lane, D,
                            reinterpret_cast<unsigned char*>(a.vc + 2 * ((long)h * a.vch + (long)pos * a.vcs)),
                            a.vs + (long)h * a.vsh + (long)pos * a.vss, a.vb + (long)h * a.vsh + (long)pos * a.vss);
    return;
  }
  const bool isq = hh < a.Hq;
  const int h = isq ? hh : hh - a.Hq;
  const u16* src = isq ? a.q + (long)m * a.ldq + (long)h * D : a.k + (long)m * a.ldk + (long)h * D;
  const u16* w = isq ? a.qw : a.kw;
  float x1[NP], x2[NP];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int i = lane + 64 * j;
    const bool on = i < HALF;
    x1[j] = on ? bf2f(src[i]) : 0.f;
    x2[j] = on ? bf2f(src[i + HALF]) : 0.f;
    ss += x1[j] * x1[j] + x2[j] * x2[j];
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / __builtin_sqrtf(ss / (float)D + a.eps);
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int i = lane + 64 * j;
    o1[j] = o2[j] = 0.f;
    if (i < HALF) {
      float r1, r2;
      norm_rope_pair(x1[j], x2[j], bf2f(w[i]), bf2f(w[i + HALF]), inv, i, D, pos, a.log2_base, r1, r2);
      o1[j] = bf16r(r1);
      o2[j] = bf16r(r2);
    }
  }
  if (isq) {
    u16* dst = a.qout + ((long)h * a.M + m) * D;
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int i = lane + 64 * j;
      if (i < HALF) {
        dst[i] = f2bf(o1[j]);
        dst[i + HALF] = f2bf(o2[j]);
      }
    }
    return;
  }
  store_quant_row<NP, QB>(o1, o2, lane, D,
                          reinterpret_cast<unsigned char*>(a.kc + 2 * ((long)h * a.kch + (long)pos * a.kcs)),
                          a.ks + (long)h * a.ksh + (long)pos * a.kss, a.kb + (long)h * a.ksh + (long)pos * a.kss);
}

// one wave per (row, head); lane l owns the RoPE pairs (i, i + D/2) for i = l + 64 j, j < NP
// (NP = ceil(D / 128): head dims up to 128 take one pair per lane, up to 256 two)
template <int NP>
__global__ __launch_bounds__(64) void qk_norm_rope_kv_kernel(const QkArgs a) {
  const int D = a.D, HALF = a.D >> 1;
  const int m = blockIdx.x, hh = blockIdx.y, lane = threadIdx.x;
  if (hh >= a.Hq + a.Hk) {  // V head: copy into the cache
    const int h = hh - a.Hq - a.Hk;
    const u16* src = a.v + (long)m * a.ldv + (long)h * D;
    u16* dst = a.vc + (long)h * a.vch + (long)(a.pos0 + m) * a.vcs;
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int i = lane + 64 * j;
      if (i < HALF) {
        dst[i] = src[i];
        dst[i + HALF] = src[i + HALF];
      }
    }
    return;
  }
  const bool isq = hh < a.Hq;
  const int h = isq ? hh : hh - a.Hq;
  const u16* src = isq ? a.q + (long)m * a.ldq + (long)h * D : a.k + (long)m * a.ldk + (long)h * D;
  const u16* w = isq ? a.qw : a.kw;
  float x1[NP], x2[NP];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int i = lane + 64 * j;
    const bool on = i < HALF;
    x1[j] = on ? bf2f(src[i]) : 0.f;
    x2[j] = on ? bf2f(src[i + HALF]) : 0.f;
    ss += x1[j] * x1[j] + x2[j] * x2[j];
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / __builtin_sqrtf(ss / (float)D + a.eps);
  u16* dst = isq ? a.qout + ((long)h * a.M + m) * D : a.kc + (long)h * a.kch + (long)(a.pos0 + m) * a.kcs;
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int i = lane + 64 * j;
    if (i >= HALF) break;
    float r1, r2;
    norm_rope_pair(x1[j], x2[j], bf2f(w[i]), bf2f(w[i + HALF]), inv, i, D, a.pos0 + m, a.log2_base, r1, r2);
    dst[i] = f2bf(r1);
    dst[i + HALF] = f2bf(r2);
  }
}

__global__ __launch_bounds__(256) void swiglu_kernel(const u16* __restrict__ g, long ldg, const u16* __restrict__ u,
                                                     long ldu, u16* __restrict__ h, long ldh, int N) {
  const int m = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;  // 8-element chunk
  if (8 * c >= N) return;
  const u32x4_t gv = ldg128(g + (long)m * ldg + 8 * c);
  const u32x4_t uv = ldg128(u + (long)m * ldu + 8 * c);
  u32x4_t out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float r[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float gg = bf2f(j ? (gv[i] >> 16) : (gv[i] & 0xFFFFu));
      const float uu = bf2f(j ? (uv[i] >> 16) : (uv[i] & 0xFFFFu));
      const float sg = bf16r(1.0f / (1.0f + expf(-gg)));
      r[j] = bf16r(gg * sg) * uu;
    }
    out[i] = pack_bf16x2(r[0], r[1]);
  }
  *reinterpret_cast<u32x4_t*>(h + (long)m * ldh + 8 * c) = out;
}

constexpr int kArgmaxThreads = 1024;

// best by (value desc, index asc); NaN never wins
__device__ __forceinline__ void arg_better(float& v, int& id, float v2, int id2) {
  if (v2 > v || (v2 == v && id2 < id)) {
    v = v2;
    id = id2;
  }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const u16* __restrict__ x, long ld, int V,
                                                                     int32_t* __restrict__ out) {
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ int si[kArgmaxThreads / 64];
  const int m = blockIdx.x;
  const u16* row = x + (long)m * ld;
  float best = -INFINITY;
  int bid = 0x7FFFFFFF;
  const int chunks = V >> 3;
  // four chunks requested per round trip (the selection is order-independent: a strict order on
  // (value, -index), NaN never selected)
  auto take = [&](const u32x4_t v, int c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      arg_better(best, bid, bf2f(v[i] & 0xFFFFu), 8 * c + 2 * i);
      arg_better(best, bid, bf2f(v[i] >> 16), 8 * c + 2 * i + 1);
    }
  };
  int c = threadIdx.x;
  for (; c + 3 * kArgmaxThreads < chunks; c += 4 * kArgmaxThreads) {
    u32x4_t v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = ldg128(row + 8 * (c + u * kArgmaxThreads));
#pragma unroll
    for (int u = 0; u < 4; ++u) take(v[u], c + u * kArgmaxThreads);
  }
  for (; c < chunks; c += kArgmaxThreads) take(ldg128(row + 8 * c), c);
  for (int j = 8 * chunks + threadIdx.x; j < V; j += kArgmaxThreads) arg_better(best, bid, bf2f(row[j]), j);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float v2 = shfl_xor(best, o);
    const int i2 = __builtin_amdgcn_ds_bpermute((__lane_id() ^ o) << 2, bid);
    arg_better(best, bid, v2, i2);
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = best;
    si[threadIdx.x >> 6] = bid;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    int id = si[0];
    for (int w = 1; w < kArgmaxThreads / 64; ++w) arg_better(b, id, sv[w], si[w]);
    out[m] = (id == 0x7FFFFFFF) ? 0 : id;  // an all-NaN row reports token 0
  }
}

// Argmax of every row and the greedy accept count in one launch: workgroup (c, m) scans chunk c
// of row m (kAaValues values, every load of a thread issued before any is compared), stores its
// best (value, index) with device-coherent stores and arrives on a counter; the workgroup that
// arrives last reduces each row's chunk results (the same strict order, so the same index as
// argmax_rows_kernel), counts the accepted drafts and clears the counter.
constexpr int kAaThreads = 256;
constexpr int kAaLoads = 8;                                  // 16-byte chunks per thread
constexpr int kAaValues = kAaThreads * kAaLoads * 8;         // values per workgroup
constexpr int kAaLds = 2048;                                 // chunk results staged per round
constexpr int kAaDraft = 4;                                  // drafts per thread: m_draft <= 1024

__global__ __launch_bounds__(kAaThreads) void argmax_accept_kernel(const u16* __restrict__ x, long ld, int V,
                                                                   int M, const int32_t* __restrict__ draft,
                                                                   int m_draft, int32_t* __restrict__ tt,
                                                                   int32_t* __restrict__ n_out, int* ctr,
                                                                   float* pval, int* pidx) {
  __shared__ float sv[kAaThreads / 64];
  __shared__ int si[kAaThreads / 64];
  __shared__ int last;
  __shared__ float lv[kAaLds];
  __shared__ int li[kAaLds];
  __shared__ int ltt[kAaThreads * kAaDraft];
  const int C = gridDim.x, c = blockIdx.x, m = blockIdx.y;
  const u16* row = x + (long)m * ld;
  const int chunks = V >> 3;
  const int c0 = c * (kAaValues / 8);
  float best = -INFINITY;
  int bid = 0x7FFFFFFF;
  u32x4_t v[kAaLoads] = {};
  if (chunks > 0) {  // every load of the thread first (clamped to the row's last whole chunk)
#pragma unroll
    for (int u = 0; u < kAaLoads; ++u) v[u] = ldg128(row + 8 * min(c0 + (int)threadIdx.x + u * kAaThreads, chunks - 1));
  }
#pragma unroll
  for (int u = 0; u < kAaLoads; ++u) {
    const int cc = c0 + (int)threadIdx.x + u * kAaThreads;
    if (cc < chunks) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        arg_better(best, bid, bf2f(v[u][i] & 0xFFFFu), 8 * cc + 2 * i);
        arg_better(best, bid, bf2f(v[u][i] >> 16), 8 * cc + 2 * i + 1);
      }
    }
  }
  if (c == C - 1)
    for (int j = 8 * chunks + threadIdx.x; j < V; j += kAaThreads) arg_better(best, bid, bf2f(row[j]), j);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float v2 = shfl_xor(best, o);
    const int i2 = __builtin_amdgcn_ds_bpermute((__lane_id() ^ o) << 2, bid);
    arg_better(best, bid, v2, i2);
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = best;
    si[threadIdx.x >> 6] = bid;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    int id = si[0];
    for (int w = 1; w < kAaThreads / 64; ++w) arg_better(b, id, sv[w], si[w]);
    __hip_atomic_store(&pval[m * C + c], b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&pidx[m * C + c], id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // release: this chunk's result is visible before the arrival; acquire: the last arriver
    // sees every other chunk's (the workgroup barrier below extends it to the other threads)
    last = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == C * M - 1;
  }
  __syncthreads();
  if (!last) return;
  // the drafts are requested now, compared once the tokens are known
  __shared__ int first_miss;
  int dv[kAaDraft];
#pragma unroll
  for (int u = 0; u < kAaDraft; ++u) {
    const int i = threadIdx.x + u * kAaThreads;
    dv[u] = i < m_draft ? draft[i] : 0;
  }
  if (threadIdx.x == 0) first_miss = m_draft;
  // every chunk result of a run of rows into LDS at once (the whole workgroup's loads in flight
  // together), then one thread per row reduces its chunks in order
  const int rpc = kAaLds / C;  // >= 1 (C <= kAaLds, checked by the host)
  for (int r0 = 0; r0 < M; r0 += rpc) {
    const int ne = min(rpc, M - r0) * C;
    for (int e = threadIdx.x; e < ne; e += kAaThreads) {
      lv[e] = __hip_atomic_load(&pval[r0 * C + e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      li[e] = __hip_atomic_load(&pidx[r0 * C + e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    for (int r = threadIdx.x; r < min(rpc, M - r0); r += kAaThreads) {
      float b = -INFINITY;
      int id = 0x7FFFFFFF;
      for (int j = 0; j < C; ++j) arg_better(b, id, lv[r * C + j], li[r * C + j]);
      const int tok = (id == 0x7FFFFFFF) ? 0 : id;  // an all-NaN row reports token 0
      tt[r0 + r] = tok;
      if (r0 + r < m_draft) ltt[r0 + r] = tok;
    }
    __syncthreads();
  }
  // accepted = the first i < m_draft with draft[i] != tt[i] (m_draft when none)
#pragma unroll
  for (int u = 0; u < kAaDraft; ++u) {
    const int i = threadIdx.x + u * kAaThreads;
    if (i < m_draft && dv[u] != ltt[i]) atomicMin(&first_miss, i);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    n_out[0] = first_miss;
    __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__global__ void greedy_accept_kernel(const int32_t* __restrict__ draft, int m, const int32_t* __restrict__ tt,
                                     int32_t* __restrict__ n_out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int n = 0;
  while (n < m && draft[n] == tt[n]) ++n;
  n_out[0] = n;
}

}  // namespace
}  // namespace dspark

using namespace dspark;

extern "C" int dspark_rmsnorm(const void* x, int64_t ldx, const void* r, int64_t ldr, const void* w, int64_t M,
                              int64_t H, float eps, void* h_out, int64_t ldh, void* y, int64_t ldy,
                              dspark_stream stream) {
  if (!x || !w || !y) return fail(DSPARK_ERR_ARG, "rmsnorm: null pointer");
  if (M < 1 || H < 8 || H % 8 || M > 65535 || H > (1 << 20)) return fail(DSPARK_ERR_SHAPE, "rmsnorm: M=%lld H=%lld (H %% 8 == 0)", (long long)M, (long long)H);
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 16) || ldx % 8 || ldy % 8 || ldx < H || ldy < H ||
      (r && (!aligned(r, 16) || ldr % 8 || ldr < H)) || (h_out && (!aligned(h_out, 16) || ldh % 8 || ldh < H)))
    return fail(DSPARK_ERR_ALIGN, "rmsnorm: rows must be 16-byte aligned with strides %% 8 == 0 and >= H");
  if (h_out && !r) return fail(DSPARK_ERR_ARG, "rmsnorm: h_out needs a residual r");
  auto norm = H <= 8 * kNormThreads * 4 ? add_rmsnorm_reg_kernel<4> : add_rmsnorm_kernel;
  hipLaunchKernelGGL(norm, dim3((unsigned)M), dim3(kNormThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u16*>(x), (long)ldx, static_cast<const u16*>(r), (long)ldr,
                     static_cast<const u16*>(w), (int)H, eps, static_cast<u16*>(h_out), (long)ldh,
                     static_cast<u16*>(y), (long)ldy);
  return check_launch("rmsnorm");
}

namespace dspark {
namespace {
// The checks and arguments shared by the plain and quantized cache writes.
int qk_args(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv, int64_t M, int64_t Hq,
            int64_t Hk, int64_t D, const void* q_norm_w, const void* k_norm_w, float eps, float rope_base,
            int64_t pos0, void* q_out, void* k_cache, const int64_t* k_strides, void* v_cache,
            const int64_t* v_strides, const char* what, QkArgs& a) {
  if (!q || !k || !v || !q_norm_w || !k_norm_w || !q_out || !k_cache || !v_cache || !k_strides || !v_strides)
    return fail(DSPARK_ERR_ARG, "%s: null pointer", what);
  if (D < 8 || D > 256 || D % 8)
    return fail(DSPARK_ERR_SHAPE, "%s: head_dim %lld (a multiple of 8 up to 256)", what, (long long)D);
  if (M < 1 || M > 65535 || Hq < 1 || Hk < 1 || Hq + 2 * Hk > 65535 || pos0 < 0 || pos0 + M > (1L << 30))
    return fail(DSPARK_ERR_SHAPE, "%s: M=%lld Hq=%lld Hk=%lld pos0=%lld", what, (long long)M, (long long)Hq,
                (long long)Hk, (long long)pos0);
  if (ldq < Hq * D || ldk < Hk * D || ldv < Hk * D || !(rope_base > 0.f))
    return fail(DSPARK_ERR_SHAPE, "%s: row strides below the head widths or rope_base <= 0", what);
  a = QkArgs{};
  a.q = static_cast<const u16*>(q);
  a.k = static_cast<const u16*>(k);
  a.v = static_cast<const u16*>(v);
  a.qw = static_cast<const u16*>(q_norm_w);
  a.kw = static_cast<const u16*>(k_norm_w);
  a.qout = static_cast<u16*>(q_out);
  a.kc = static_cast<u16*>(k_cache);
  a.vc = static_cast<u16*>(v_cache);
  a.ldq = ldq;
  a.ldk = ldk;
  a.ldv = ldv;
  a.kch = k_strides[0];
  a.kcs = k_strides[1];
  a.vch = v_strides[0];
  a.vcs = v_strides[1];
  a.M = (int)M;
  a.Hq = (int)Hq;
  a.Hk = (int)Hk;
  a.pos0 = (int)pos0;
  a.D = (int)D;
  a.eps = eps;
  a.log2_base = log2f(rope_base);
  return DSPARK_OK;
}
}  // namespace
}  // namespace dspark

extern "C" int dspark_qk_norm_rope_kv(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                                      int64_t ldv, int64_t M, int64_t Hq, int64_t Hk, int64_t D, const void* q_norm_w,
                                      const void* k_norm_w, float eps, float rope_base, int64_t pos0, void* q_out,
                                      void* k_cache, const int64_t k_cache_strides[2], void* v_cache,
                                      const int64_t v_cache_strides[2], dspark_stream stream) {
  QkArgs a;
  const int st = qk_args(q, ldq, k, ldk, v, ldv, M, Hq, Hk, D, q_norm_w, k_norm_w, eps, rope_base, pos0, q_out,
                         k_cache, k_cache_strides, v_cache, v_cache_strides, "qk_norm_rope_kv", a);
  if (st) return st;
  const dim3 grid((unsigned)M, (unsigned)(Hq + 2 * Hk));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (D <= 128) hipLaunchKernelGGL(qk_norm_rope_kv_kernel<1>, grid, dim3(64), 0, s, a);
  else hipLaunchKernelGGL(qk_norm_rope_kv_kernel<2>, grid, dim3(64), 0, s, a);
  return check_launch("qk_norm_rope_kv");
}

extern "C" int dspark_qk_norm_rope_kv_quantized(
    const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv, int64_t M, int64_t Hq,
    int64_t Hk, int64_t D, const void* q_norm_w, const void* k_norm_w, float eps, float rope_base, int64_t pos0,
    void* q_out, uint32_t* k_words, void* k_scales, void* k_biases, const int64_t k_strides[2],
    const int64_t k_scale_strides[2], uint32_t* v_words, void* v_scales, void* v_biases, const int64_t v_strides[2],
    const int64_t v_scale_strides[2], int bits, int group_size, dspark_stream stream) {
  const char* what = "qk_norm_rope_kv_quantized";
  QkArgs a;
  int st = qk_args(q, ldq, k, ldk, v, ldv, M, Hq, Hk, D, q_norm_w, k_norm_w, eps, rope_base, pos0, q_out, k_words,
                   k_strides, v_words, v_strides, what, a);
  if (st) return st;
  if (bits != 4 && bits != 8) return fail(DSPARK_ERR_UNSUPPORTED, "%s: bits=%d (4 or 8)", what, bits);
  if (group_size != 64) return fail(DSPARK_ERR_UNSUPPORTED, "%s: group_size=%d (64)", what, group_size);
  if (D != 64 && D != 128 && D != 256) return fail(DSPARK_ERR_SHAPE, "%s: head_dim %lld (64, 128 or 256)", what, (long long)D);
  if (!k_scales || !k_biases || !v_scales || !v_biases || !k_scale_strides || !v_scale_strides)
    return fail(DSPARK_ERR_ARG, "%s: null pointer", what);
  a.ks = static_cast<u16*>(k_scales);
  a.kb = static_cast<u16*>(k_biases);
  a.vs = static_cast<u16*>(v_scales);
  a.vb = static_cast<u16*>(v_biases);
  a.ksh = k_scale_strides[0];
  a.kss = k_scale_strides[1];
  a.vsh = v_scale_strides[0];
  a.vss = v_scale_strides[1];
  const dim3 grid((unsigned)M, (unsigned)(Hq + 2 * Hk));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (bits == 8) {
    if (D <= 128) hipLaunchKernelGGL((qk_norm_rope_qkv_kernel<1, 8>), grid, dim3(64), 0, s, a);
    else hipLaunchKernelGGL((qk_norm_rope_qkv_kernel<2, 8>), grid, dim3(64), 0, s, a);
  } else {
    if (D <= 128) hipLaunchKernelGGL((qk_norm_rope_qkv_kernel<1, 4>), grid, dim3(64), 0, s, a);
    else hipLaunchKernelGGL((qk_norm_rope_qkv_kernel<2, 4>), grid, dim3(64), 0, s, a);
  }
  return check_launch(what);
}

extern "C" int dspark_swiglu(const void* g, int64_t ldg, const void* u, int64_t ldu, int64_t M, int64_t N, void* h,
                             int64_t ldh, dspark_stream stream) {
  if (!g || !u || !h) return fail(DSPARK_ERR_ARG, "swiglu: null pointer");
  if (M < 1 || M > 65535 || N < 8 || N % 8) return fail(DSPARK_ERR_SHAPE, "swiglu: M=%lld N=%lld (N %% 8 == 0)", (long long)M, (long long)N);
  if (!aligned(g, 16) || !aligned(u, 16) || !aligned(h, 16) || ldg % 8 || ldu % 8 || ldh % 8 || ldg < N || ldu < N || ldh < N)
    return fail(DSPARK_ERR_ALIGN, "swiglu: rows must be 16-byte aligned with strides %% 8 == 0 and >= N");
  const dim3 grid((unsigned)((N / 8 + 255) / 256), (unsigned)M);
  hipLaunchKernelGGL(swiglu_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), static_cast<const u16*>(g),
                     (long)ldg, static_cast<const u16*>(u), (long)ldu, static_cast<u16*>(h), (long)ldh, (int)N);
  return check_launch("swiglu");
}

extern "C" int dspark_argmax_rows(const void* logits, int64_t ld, int64_t M, int64_t V, int32_t* out,
                                  dspark_stream stream) {
  if (!logits || !out) return fail(DSPARK_ERR_ARG, "argmax_rows: null pointer");
  if (M < 1 || M > 65535 || V < 1 || V >= (1L << 30) || ld < V) return fail(DSPARK_ERR_SHAPE, "argmax_rows: M=%lld V=%lld", (long long)M, (long long)V);
  if (!aligned(logits, 16) || ld % 8) return fail(DSPARK_ERR_ALIGN, "argmax_rows: rows must be 16-byte aligned (ld %% 8 == 0)");
  hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)M), dim3(kArgmaxThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u16*>(logits), (long)ld, (int)V, out);
  return check_launch("argmax_rows");
}

namespace {
int aa_chunks(int64_t V) { return (int)((V + kAaValues - 1) / kAaValues); }
}  // namespace

extern "C" size_t dspark_argmax_accept_workspace(int64_t M, int64_t V) {
  if (M < 1 || M > 65535 || V < 1 || V > (int64_t)kAaLds * kAaValues) return 0;
  return 256 + (size_t)M * aa_chunks(V) * 8;
}

extern "C" int dspark_argmax_accept(const void* logits, int64_t ld, int64_t M, int64_t V, const int32_t* draft,
                                    int64_t m_draft, int32_t* target_tokens, int32_t* n_accepted, void* workspace,
                                    size_t workspace_bytes, dspark_stream stream) {
  if (!logits || !target_tokens || !n_accepted || (m_draft > 0 && !draft) || !workspace)
    return fail(DSPARK_ERR_ARG, "argmax_accept: null pointer");
  if (M < 1 || M > 65535 || V < 1 || V > (int64_t)kAaLds * kAaValues || ld < V || m_draft < 0 || m_draft > M ||
      m_draft > kAaThreads * kAaDraft)
    return fail(DSPARK_ERR_SHAPE, "argmax_accept: M=%lld V=%lld m_draft=%lld", (long long)M, (long long)V,
                (long long)m_draft);
  if (!aligned(logits, 16) || ld % 8) return fail(DSPARK_ERR_ALIGN, "argmax_accept: rows must be 16-byte aligned (ld %% 8 == 0)");
  const size_t need = dspark_argmax_accept_workspace(M, V);
  if (workspace_bytes < need)
    return fail(DSPARK_ERR_WORKSPACE, "argmax_accept: workspace %zu < %zu bytes", workspace_bytes, need);
  if (!aligned(workspace, 256)) return fail(DSPARK_ERR_ALIGN, "argmax_accept: workspace must be 256-byte aligned");
  const int C = aa_chunks(V);
  char* ws = static_cast<char*>(workspace);
  float* pval = reinterpret_cast<float*>(ws + 256);
  int* pidx = reinterpret_cast<int*>(ws + 256 + (size_t)M * C * 4);
  hipLaunchKernelGGL(argmax_accept_kernel, dim3((unsigned)C, (unsigned)M), dim3(kAaThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u16*>(logits), (long)ld, (int)V, (int)M,
                     draft, (int)m_draft, target_tokens, n_accepted, reinterpret_cast<int*>(ws), pval, pidx);
  return check_launch("argmax_accept");
}

extern "C" int dspark_greedy_accept(const int32_t* draft, int64_t m, const int32_t* target_tokens, int32_t* n_accepted,
                                    dspark_stream stream) {
  if (!target_tokens || !n_accepted || (m > 0 && !draft)) return fail(DSPARK_ERR_ARG, "greedy_accept: null pointer");
  if (m < 0 || m > (1 << 20)) return fail(DSPARK_ERR_SHAPE, "greedy_accept: m=%lld", (long long)m);
  hipLaunchKernelGGL(greedy_accept_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), draft, (int)m,
                     target_tokens, n_accepted);
  return check_launch("greedy_accept");
}
