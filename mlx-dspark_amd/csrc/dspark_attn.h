// Multi-row causal GQA verify attention for gfx950 (MI355X): kernels and launch plan.
//
// Semantics (multirow_attn.py:52-178, :223-259): q [B, Hq, Mq, D] is viewed per KV head as
// R = gqa * Mq rows (row r = g*Mq + i is query head hk*gqa + g at block position i). K/V hold
// L keys (prefix + the Mq verify rows, already written). Causal: row i sees keys
// 0 .. L - Mq + i. Softmax in the exp2 domain with fp32 running max m (init -1e30) and sum l;
// P is rounded to the input type for the P.V product (multirow_attn.py:131-140); partials of the
// split-KV blocks are merged as out = sum 2^(m_j - M) o_j / sum 2^(m_j - M) l_j
// (multirow_attn.py:162-178).
//
// MI355X mapping:
//   * grid = (B*Hk, NB key blocks, row groups); a workgroup owns one KV head's key block and up
//     to 4 or 8 row tiles of 16 rows (all gqa*Mq rows of the head when there are at most 128),
//     so each K/V byte is read from HBM once and shared by every query head of the GQA group.
//     On short caches (few blocks) the 4 row tiles are worked by 8 waves, two per tile
//     splitting its keys. Head dim 256 takes 32-key tiles so two K/V buffers still fit in
//     LDS, one wave per row tile over all 256 output columns with two tiles in flight (a
//     quantized cache: two waves per row tile, one per half of the output columns, both
//     computing the whole score tile, one tile in flight: its registers do not fit one wave).
//   * key tiles are staged through two alternating LDS buffers (one barrier per tile) from
//     registers loaded one (4-wave workgroups) or two (8-wave workgroups) tiles ahead: K
//     row-major (padded rows), V transposed (key-contiguous, 8-key blocks XOR-swizzled by d)
//     because the P.V MFMA reduces over keys.
//   * S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_16x16x32_{bf16,f16}. Computing the
//     transposed scores leaves each lane holding 8 keys of one query row, which is exactly the
//     B operand of the P.V MFMA: no shuffle of P.
//   * quantized K/V (mlx-lm QuantizedKVCache: uint32 words of 4- or 8-bit fields along D, low
//     bits first, one bf16/fp16 scale and bias per 64 values of a row) use the factored form of
//     the quantized matmul: the integer fields go to LDS as exact bf16/fp16 integers and each
//     (key, group) scale and bias to a small fp32 table, so
//       s[key, row] = sum_g scale_k[key, g] * (f_k[key, g] . q[row, g]) + bias_k[key, g] * sum q[row, g]
//       o[row, d]   = sum_key (p * scale_v[key, g(d)]) * f_v[key, d] + sum_key p * bias_v[key, g(d)]
//     with every product exact and the scales applied in fp32: no precision is lost against a
//     bf16/fp16 cache of the dequantized values.
#pragma once

#include "dspark_qmm_core.h"

namespace dspark {
namespace attn {

// ---------------------------------------------------------------- element types

struct BF16 {
  static constexpr bool kF16 = false;
};
struct F16 {
  static constexpr bool kF16 = true;
};

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <class T>
__device__ __forceinline__ float to_f32(u32 bits16) {
  if constexpr (T::kF16) return (float)__builtin_bit_cast(_Float16, (u16)bits16);
  else return __builtin_bit_cast(float, bits16 << 16);
}

template <class T>
__device__ __forceinline__ u32 pack2(float lo, float hi) {
  if constexpr (T::kF16) {
    f16x2_t p = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(u32, p);
  } else {
    return pack_bf16x2(lo, hi);
  }
}

template <class T>
__device__ __forceinline__ u16 from_f32(float f) {
  if constexpr (T::kF16) return __builtin_bit_cast(u16, (_Float16)f);
  else return f2bf(f);
}

// D = A(16 x 32) * B(32 x 16) + C for 8 bf16 / fp16 values per lane (layout: mfma16x16x32)
template <class T>
__device__ __forceinline__ f32x4_t mfma(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (T::kF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                   0, 0, 0);
  else
    return mfma16x16x32(a, b, c);
}

// ---------------------------------------------------------------- arguments and plan

struct AttnArgs {
  const u16* q;
  const void* k;  // bf16/fp16 [.., L, D] or, quantized, uint32 words [.., L, D*bits/32]
  const void* v;
  const u16* ks;  // quantized: scales of K / V [.., L, D/64] (biases at kb / vb, same strides)
  const u16* kb;
  const u16* vs;
  const u16* vb;
  const u32* anc;
  float* opart;  // split-KV partials, fp32: o [B*Hk][NB][RP][D], m and l [B*Hk][NB][RP]
  float* mpart;
  float* lpart;
  u16* out;
  long ksb, ksh, kss;     // K strides (batch, head, position) in elements (words when quantized)
  long vsb, vsh, vss;
  long qksb, qksh, qkss;  // quantized: scale/bias strides of K and V
  long qvsb, qvsh, qvss;
  long osb, osh, osi;     // output strides (batch, query head, position); head_dim contiguous
  int Hq, Hk, Mq, L;
  int dv;                 // the caller's head dim (a multiple of 8, <= the instance's D)
  int gqa, R, RT, RP;
  int chunk, NB;
  float scale_log2;
  int causal;
};

struct Plan {
  int R, RT, RP, WV, KS, PF, NRG, chunk, NB;
};

inline Plan make_plan(long B, long Hq, long Hk, long Mq, long D, long L) {
  Plan p{};
  p.R = (int)((Hq / Hk) * Mq);
  p.RT = (p.R + 15) / 16;
  p.RP = p.RT * 16;
  // head dim 256: up to 6 row tiles of one wave each (two waves per SIMD), so a 24/4-head
  // group's 96 rows share one pass over K/V
  p.WV = p.RT > 4 ? (D <= 128 ? 8 : 6) : 4;
  p.KS = 1;
  p.PF = p.WV == 8 ? 2 : 1;
  p.NRG = (p.RT + p.WV - 1) / p.WV;
  // Long caches: ~2 workgroups of 4 waves per CU (256 CUs), or one of 8 waves (twice the
  // rows per K/V tile: the fp32 partials, written here and read by the combine, double too),
  // which then keeps two tiles in flight. At least 256 keys per block from 4096 keys on; a
  // shorter cache, whose blocks that floor caps well below one workgroup per CU, takes blocks
  // of 128 keys (64 up to 1280): its time is a few tiles' latency per block, which shorter
  // blocks cut by more than the extra partials cost. When the blocks still stay below one
  // workgroup per CU, 4-row-tile heads of head dim <= 128 split each tile's keys over 8
  // waves. Row groups beyond one re-read the head's K/V.
  const long heads = B * Hk * p.NRG;
  const long target = (p.WV == 8 || D == 256) ? 256 : 512;
  long nb = (target + heads - 1) / heads;
  const long min_keys = L <= 1280 ? 64 : (L < 4096 ? 128 : 256);
  const long max_nb = (L + min_keys - 1) / min_keys;
  if (nb > max_nb) nb = max_nb;
  if (nb < 1) nb = 1;
  if (p.WV == 4 && D <= 128 && heads * nb < 256) p.KS = 2;
  long chunk = (L + nb - 1) / nb;
  chunk = ((chunk + 63) / 64) * 64;
  p.chunk = (int)chunk;
  p.NB = (int)((L + chunk - 1) / chunk);
  return p;
}

inline size_t partial_bytes(const Plan& p, long B, long Hk, long D) {
  if (p.NB <= 1) return 0;
  const size_t rows = (size_t)B * Hk * p.NB * p.RP;
  return rows * D * sizeof(float) + 2 * rows * sizeof(float);
}

// ---------------------------------------------------------------- LDS tile layout

// position of key (0..KT-1) inside a tile's transposed V row: the 8 keys one lane needs for one
// P.V MFMA (keys 32u + 4q + {0..3} and 32u + 16 + 4q + {0..3}) are made contiguous.
__device__ __forceinline__ int vt_pos(int key) {
  const int u = key >> 5, h = (key >> 4) & 1, qq = (key >> 2) & 3, i = key & 3;
  return (u << 5) | (qq << 3) | (h << 2) | i;
}
// 2^x with v_exp_f32 (results below 2^-126 flush to 0: negligible softmax weights)
__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }

// swizzled element offset of (d, pos) in the transposed V tile (row pitch KT): the 8-key block
// index is XORed with bits of d, a permutation of each row's blocks. The bits are the ones an
// LDS conflict probe found to keep both the staging stores and the P.V fragment reads free of
// bank conflicts: d >> 1 and d >> 3 for 64-key tiles, d >> 1 alone for 32-key tiles (with
// d >> 3 too, every 32-key fragment read took a 2-way conflict).
template <int KT>
__device__ __forceinline__ int vt_off(int d, int pos) {
  const int sw = KT == 64 ? ((d >> 1) ^ (d >> 3)) : (d >> 1);
  return d * KT + ((((pos >> 3) ^ sw) & (KT / 8 - 1)) << 3) + (pos & 7);
}

// 8 integer fields as 8 T values (exact: at most 255)
template <class T>
__device__ __forceinline__ u32x4_t fields_to_t(const u32* f) {
  u32x4_t o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = pack2<T>((float)f[2 * i], (float)f[2 * i + 1]);
  return o;
}

__device__ __forceinline__ float sum_t8(u32x4_t v, bool f16) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (f16) {
      s += (float)__builtin_bit_cast(_Float16, (u16)(v[i] & 0xFFFFu)) + (float)__builtin_bit_cast(_Float16, (u16)(v[i] >> 16));
    } else {
      s += bf2f(v[i] & 0xFFFFu) + bf2f(v[i] >> 16);
    }
  }
  return s;
}

// fields of quantized words: n = 8 values starting at field `first` of words w (BITS per field)
template <int BITS>
__device__ __forceinline__ void fields8(const u32* w, int first, u32* out) {
  constexpr u32 mask = (1u << BITS) - 1u;
  constexpr int per = 32 / BITS;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int f = first + i;
    out[i] = (w[f / per] >> (BITS * (f % per))) & mask;
  }
}

// 4-bit fields of word w as 8 T values, in the order (f0, f4, f1, f5, f2, f6, f3, f7), the
// matching x / q order being perm_x_u4's. One v_and_or_b32 per pair makes (off + f_t,
// off + f_{t+4}): bf16 off = 128 (0x43004300 is the pair (128, 128)), which the tables take
// back out (bias - 128 * scale); fp16 off = 1024 (0x6400), which one packed fp16 subtract per
// pair removes exactly here, so fp16 values are the fields themselves (no large offset term
// cancels in an fp32 sum: with 1024 in the tables, their rounding grew about 1024-fold)
template <class T>
__device__ __forceinline__ u32x4_t unpack4_off(u32 w) {
  if constexpr (T::kF16) {
    const u32 m = opaque_sgpr(0x000F000Fu), c = opaque_vgpr(0x64006400u);
    const f16x2_t off = {(_Float16)1024.0f, (_Float16)1024.0f};
    auto pair = [&](u32 x) { return __builtin_bit_cast(u32, __builtin_bit_cast(f16x2_t, and_or(x, m, c)) - off); };
    return u32x4_t{pair(w), pair(w >> 4), pair(w >> 8), pair(w >> 12)};
  } else {
    return unpack_u4(w);
  }
}
// offset left in the staged 4-bit fields (removed through the bias tables)
template <class T>
constexpr float kOff4 = T::kF16 ? 0.0f : 128.0f;

// ---------------------------------------------------------------- pass 1

// Template parameters: T element type; D head dim (64, 128, 256); TREE ancestry mask; WV row
// tiles per workgroup; KS waves splitting each tile's keys (1 or 2); PF tiles in flight (1 or
// 2); QB quantized K/V field width (0 = plain T, 4 or 8); PAD the caller's head dim is below D
// (its missing columns of q, K and V are zeros that are never read, nor written out); DSX waves
// per row tile, each taking D / DSX of the output columns (2 only for quantized head dim 256).
template <class T, int D, bool TREE, int WV, int KS, int PF, int QB, bool PAD = false, int DSX = (D == 256 ? 2 : 1)>
__global__ __launch_bounds__(64 * WV * KS * DSX) void p1_kernel(const AttnArgs a) {
  constexpr int DS = DSX;  // waves per row tile splitting the output columns
  constexpr int KT = D == 256 ? 32 : 64;  // keys per LDS tile
  static_assert(KS == 1 || KS == 2, "key split");
  static_assert(PF == 1 || PF == 2, "tiles in flight");
  static_assert(DS == 1 || KS == 1, "head dim 256 does not split keys");
  static_assert(QB == 0 || QB == 4 || QB == 8, "quantized field width");
  constexpr int THREADS = 64 * WV * KS * DS;
  constexpr int NKS = KT / 16 / KS;   // 16-key subtiles of a tile per wave
  constexpr int NU = KT / 32 / KS;    // 32-key halves of a tile per wave (P.V MFMA k-steps)
  static_assert(NU >= 1, "tile split");
  constexpr int DH = D / DS;          // output columns per wave
  constexpr int KP = D + 16;          // padded K row (elements): 32 bytes keep the score reads conflict-free
  constexpr int DC = D / 8;           // 16-byte chunks of a T row
  constexpr int LOADS = (KT * DC + THREADS - 1) / THREADS;  // 16-byte K chunks per thread per tile (plain)
  constexpr bool KPART = LOADS * THREADS != KT * DC;       // the last round covers part of the threads
  static_assert(THREADS % DC == 0, "K tile split");
  constexpr int NDC = D / 32;         // d-chunks of the S MFMA
  constexpr int NDT = DH / 16;        // d-tiles of the O MFMA per wave
  constexpr int VQ = KT / 4;          // 4-key quads of a V tile
  static_assert(VQ * DC <= THREADS, "V tile split");
  constexpr int VW = 4;               // V fragments requested ahead of their MFMAs
  // quantized K: a 16-byte word chunk holds 128 / QB values (16 or 32 = 2 or 4 T chunks)
  constexpr int QCH = QB ? D * QB / 128 : 1;           // word chunks per K row
  constexpr int QLOADS = QB ? (KT * QCH + THREADS - 1) / THREADS : 1;
  constexpr int QV = QB ? 128 / QB : 1;                // values per word chunk
  constexpr int G = D / 64;                            // scale groups per row
  // two tile buffers: tile i is staged into buffer i & 1 while the other buffer may still be in
  // use by waves finishing tile i - 1, so one barrier per tile suffices
  constexpr int TILE = KT * KP + D * KT;
  __shared__ __attribute__((aligned(16))) u16 smem[2 * TILE];
  // quantized: per buffer, fp32 scale_k, bias_k, scale_v, bias_v as [G groups][KT keys]
  __shared__ __attribute__((aligned(16))) float qsb[QB ? 2 : 1][4][QB ? G : 1][QB ? KT : 1];
  constexpr int GW = DH / 64;  // groups of this wave's output columns
  static_assert(KS == 1 || (WV * 64 * NDT * 4 + 2 * WV * 16) * 4 <= TILE * 2, "merge area");

  const int bh = blockIdx.x;
  const int b = bh / a.Hk, hk = bh % a.Hk;
  const int blk = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = uniform(tid >> 6);
  const int c16 = lane & 15, q4 = lane >> 4;
  const int rtw = wave % WV, kh = (wave / WV) % KS, dh = wave / (WV * KS);  // row tile, key half, d half
  const int dbase = dh * DH;
  const int rt = blockIdx.z * WV + rtw;
  const bool active = rt < a.RT;

  const int L = a.L;
  const int k0 = blk * a.chunk;
  const int k1 = min(L, k0 + a.chunk);

  // ---- this lane's query row (B operand of S^T = K Q^T), over the whole head dim
  const int rr = min(rt * 16 + c16, a.R - 1);
  const int qi = rr % a.Mq;
  const u16* qrow = a.q + ((long)(b * a.Hq + hk * a.gqa) * a.Mq + rr) * a.dv;
  u32x4_t qf[NDC];
  // head dims below the instance's D: the missing columns of q, K and V are zeros (never read)
#pragma unroll
  for (int c = 0; c < NDC; ++c)
    qf[c] = (!PAD || 32 * c + 8 * q4 < a.dv) ? ldg128(qrow + 32 * c + 8 * q4) : u32x4_t{0u, 0u, 0u, 0u};
  if constexpr (QB == 4) {
    // 4-bit K fields sit in LDS in unpack4_off's order: q follows (its row sums do not change)
#pragma unroll
    for (int c = 0; c < NDC; ++c) qf[c] = perm_x_u4(qf[c]);
  }
  // quantized: per group, the row's sum of q (the bias term of the factored score)
  float qsum[QB ? G : 1];
  if constexpr (QB != 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float t = sum_t8(qf[2 * g], T::kF16) + sum_t8(qf[2 * g + 1], T::kF16);
      t += shfl_xor(t, 16);
      qsum[g] = t + shfl_xor(t, 32);
    }
  }
  float bvs[QB ? GW : 1];  // quantized: lane-partial sum_key p * bias_v per output group
#pragma unroll
  for (int g = 0; g < (QB ? GW : 1); ++g) bvs[g] = 0.f;
  const int kmax = a.causal ? (L - a.Mq + qi) : (L - 1);
  const u32 anc = TREE ? a.anc[qi] : 0u;
  const int tail0 = L - a.Mq;  // first key of the verify block

  f32x4_t o[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) o[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -1e30f, l = 0.f;

  // ---- cooperative tile loads into registers.
  // K: 16-byte chunk c = tid + THREADS*j -> (key c / DC, d-chunk c % DC), stored row-major.
  // V: thread (key quad vkq = tid % VQ, d-chunk vdc = tid / VQ) loads keys 4vkq..4vkq+3 and
  //    writes the transposed tile as 8 ds_write_b64 (4 keys of one d each); odd d-chunks walk
  //    their 8 d-rows in pair-swapped order so each half-wave covers all 64 LDS banks.
  // Quantized: K word chunk c = tid + THREADS*j -> (key c / QCH, chunk c % QCH); V as above
  //    with the 8 (or 4) bytes of each key's d-chunk; thread tid < KT reads key tid's scales
  //    and biases of K and V into the tile's fp32 tables.
  const bool vthread = tid < VQ * DC;
  const int vkq = tid % VQ, vdc = tid / VQ;
  // a thread's K chunks all sit in column tid % DC (THREADS is a multiple of DC), its V chunks in
  // column vdc: columns at or past the head dim load nothing and stage zeros
  const bool kcol = !PAD || 8 * (tid % DC) < a.dv, vcol = !PAD || 8 * vdc < a.dv;
  const u32x4_t zero4 = {0u, 0u, 0u, 0u};
  const u16* kbase16 = static_cast<const u16*>(a.k) + b * a.ksb + hk * a.ksh;
  const u16* vbase16 = static_cast<const u16*>(a.v) + b * a.vsb + hk * a.vsh;
  const u32* kbase32 = static_cast<const u32*>(a.k) + b * a.ksb + hk * a.ksh;
  const u32* vbase32 = static_cast<const u32*>(a.v) + b * a.vsb + hk * a.vsh;
  struct TileRegs {
    u32x4_t k[QB ? QLOADS : LOADS];
    u32x4_t v[4];               // plain: 8 T of each key; quantized: words in .x (.y for 8-bit)
    u32 sb[QB ? 4 * G : 1];     // quantized, threads tid < KT: key tid's K scales, K biases, V
                                // scales, V biases (G each, T bits)
  };
  // A tile inside the cache is addressed as a uniform base (scalar) plus a loop-invariant
  // 32-bit lane offset; only a tile running past key L - 1 clamps each key.
  const unsigned koff = (unsigned)(((tid / DC) * a.kss + 8 * (tid % DC)) * 2);
  const unsigned voff = (unsigned)((4 * vkq * a.vss + 8 * vdc) * 2);
  const long kstep = (long)(THREADS / DC) * a.kss * 2;  // bytes between a thread's K chunks
  auto load_plain = [&](TileRegs& r, int kt) {
    if (kt + KT <= L) {
      const char* kb = reinterpret_cast<const char*>(kbase16 + (long)kt * a.kss);
      const char* vb = reinterpret_cast<const char*>(vbase16 + (long)kt * a.vss);
#pragma unroll
      for (int j = 0; j < LOADS; ++j)
        if (!KPART || tid + THREADS * j < KT * DC) r.k[j] = kcol ? ldg128((kb + j * kstep) + koff) : zero4;
      if (vthread) {
#pragma unroll
        for (int j = 0; j < 4; ++j) r.v[j] = vcol ? ldg128((vb + (long)j * a.vss * 2) + voff) : zero4;
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int c = min(tid + THREADS * j, KT * DC - 1);
      const int key = min(kt + c / DC, L - 1);
      r.k[j] = kcol ? ldg128(kbase16 + (long)key * a.kss + 8 * (c % DC)) : zero4;
    }
    if (vthread) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = min(kt + 4 * vkq + j, L - 1);
        r.v[j] = vcol ? ldg128(vbase16 + (long)key * a.vss + 8 * vdc) : zero4;
      }
    }
  };
  auto load_quant = [&](TileRegs& r, int kt) {
#pragma unroll
    for (int j = 0; j < QLOADS; ++j) {
      const int c = min(tid + THREADS * j, KT * QCH - 1);
      const int key = min(kt + c / QCH, L - 1), ch = c % QCH;
      r.k[j] = ldg128(kbase32 + (long)key * a.kss + 4 * ch);
    }
    if (vthread) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = min(kt + 4 * vkq + j, L - 1);
        const u32* w = vbase32 + (long)key * a.vss + (8 * vdc * QB) / 32;
        if constexpr (QB == 8) {
          const u32x2_t p = ldg64(w);
          r.v[j] = u32x4_t{p.x, p.y, 0u, 0u};
        } else {
          r.v[j] = u32x4_t{*w, 0u, 0u, 0u};
        }
      }
    }
    // the tile's scales and biases: one thread per key reads its 4 G values (a few gathers in
    // one wave instead of two per chunk in every thread)
    if (tid < KT) {
      const int key = min(kt + tid, L - 1);
      const long ko = b * a.qksb + hk * a.qksh + (long)key * a.qkss;
      const long vo = b * a.qvsb + hk * a.qvsh + (long)key * a.qvss;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        r.sb[g] = a.ks[ko + g];
        r.sb[G + g] = a.kb[ko + g];
        r.sb[2 * G + g] = a.vs[vo + g];
        r.sb[3 * G + g] = a.vb[vo + g];
      }
    }
  };
  auto load_tile = [&](TileRegs& r, int kt) {
    if constexpr (QB) load_quant(r, kt);
    else load_plain(r, kt);
  };
  // element (e ^ (vdc & 1)) of each 8-wide chunk: low half-word of word e >> 1 when that index
  // is even, high half-word when odd
  const u32 sel_lo = 0x05040100u, sel_hi = 0x07060302u;
  const u32 vsel_even = (vdc & 1) ? sel_hi : sel_lo;  // e even
  const u32 vsel_odd = (vdc & 1) ? sel_lo : sel_hi;   // e odd
  auto store_tile = [&](const TileRegs& r, int bsel) {
    u16* const ks_lds = smem + bsel * TILE;
    u16* const vt_lds = ks_lds + KT * KP;
    if constexpr (QB) {
#pragma unroll
      for (int j = 0; j < QLOADS; ++j) {
        const int c = tid + THREADS * j;
        if (c < KT * QCH) {
          const int key = c / QCH, ch = c % QCH;
          const u32 w[4] = {r.k[j].x, r.k[j].y, r.k[j].z, r.k[j].w};
#pragma unroll
          for (int e = 0; e < QV / 8; ++e) {
            u32x4_t val;
            if constexpr (QB == 4) {
              val = unpack4_off<T>(w[e]);
            } else {
              u32 f[8];
              fields8<QB>(w, 8 * e, f);
              val = fields_to_t<T>(f);
            }
            *reinterpret_cast<u32x4_t*>(&ks_lds[key * KP + ch * QV + 8 * e]) = val;
          }
        }
      }
      if (tid < KT) {
        // bf16 4-bit fields are staged as 128 + f: bias - 128 * scale takes the offset back out
#pragma unroll
        for (int t = 0; t < 4; t += 2)
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float sc = to_f32<T>(r.sb[t * G + g]), bi = to_f32<T>(r.sb[(t + 1) * G + g]);
            qsb[bsel][t][g][tid] = sc;
            qsb[bsel][t + 1][g][tid] = (QB == 4 && kOff4<T> != 0.f) ? __builtin_fmaf(-kOff4<T>, sc, bi) : bi;
          }
      }
    } else {
#pragma unroll
      for (int j = 0; j < LOADS; ++j) {
        const int c = tid + THREADS * j;
        if (!KPART || c < KT * DC) *reinterpret_cast<u32x4_t*>(&ks_lds[(c / DC) * KP + 8 * (c % DC)]) = r.k[j];
      }
    }
    if (vthread) {
      u32x4_t vv[4];
      if constexpr (QB == 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) vv[j] = unpack4_off<T>(r.v[j].x);
      } else if constexpr (QB == 8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u32 w[2] = {r.v[j].x, r.v[j].y};
          u32 f[8];
          fields8<QB>(w, 0, f);
          vv[j] = fields_to_t<T>(f);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) vv[j] = r.v[j];
      }
      const int pos = vt_pos(4 * vkq);
      if constexpr (QB == 4) {
        // word t of vv[j] holds the pair (t, t + 4): odd d-chunks walk their rows in the
        // half-swapped order e ^ 4, so the word is e & 3 in every lane and only the half differs
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int ep = e ^ (4 * (vdc & 1));
          const int d = 8 * vdc + ep;
          const int wd = e & 3;
          const u32 vsel = (ep >> 2) ? sel_hi : sel_lo;
          const u32x2_t pr = {__builtin_amdgcn_perm(vv[1][wd], vv[0][wd], vsel),
                              __builtin_amdgcn_perm(vv[3][wd], vv[2][wd], vsel)};
          *reinterpret_cast<u32x2_t*>(&vt_lds[vt_off<KT>(d, pos)]) = pr;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = 8 * vdc + (e ^ (vdc & 1));
          const int wd = e >> 1;
          const u32 vsel = (e & 1) ? vsel_odd : vsel_even;
          const u32x2_t pr = {__builtin_amdgcn_perm(vv[1][wd], vv[0][wd], vsel),
                              __builtin_amdgcn_perm(vv[3][wd], vv[2][wd], vsel)};
          *reinterpret_cast<u32x2_t*>(&vt_lds[vt_off<KT>(d, pos)]) = pr;
        }
      }
    }
  };

  auto compute_tile = [&](int kt, int bsel) {
    const u16* const ks_lds = smem + bsel * TILE;
    const u16* const vt_lds = ks_lds + KT * KP;
    // S^T[key][row] for this wave's NKS subtiles of 16 keys (keys 16 (ks0 + j) ..), whole D
    const int ks0 = kh * NKS;
    f32x4_t s[NKS];
#pragma unroll
    for (int j = 0; j < NKS; ++j) {
      s[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if constexpr (QB != 0) {
        // per group: the integer dot products, then scale and bias of the lane's 4 keys
#pragma unroll
        for (int g = 0; g < G; ++g) {
          f32x4_t t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 2 * g; c < 2 * g + 2; ++c) {
            const u32x4_t kf =
                *reinterpret_cast<const u32x4_t*>(&ks_lds[(16 * (ks0 + j) + c16) * KP + 32 * c + 8 * q4]);
            t = mfma<T>(kf, qf[c], t);
          }
          const int key0 = 16 * (ks0 + j) + 4 * q4;
          const f32x4_t sk = *reinterpret_cast<const f32x4_t*>(&qsb[bsel][0][g][key0]);
          const f32x4_t bk = *reinterpret_cast<const f32x4_t*>(&qsb[bsel][1][g][key0]);
#pragma unroll
          for (int i = 0; i < 4; ++i) s[j][i] = __builtin_fmaf(sk[i], t[i], __builtin_fmaf(bk[i], qsum[g], s[j][i]));
        }
      } else {
#pragma unroll
        for (int c = 0; c < NDC; ++c) {
          const u32x4_t kf =
              *reinterpret_cast<const u32x4_t*>(&ks_lds[(16 * (ks0 + j) + c16) * KP + 32 * c + 8 * q4]);
          s[j] = mfma<T>(kf, qf[c], s[j]);
        }
      }
    }
    // V fragments of the P.V product (fragment f = (d-tile f / NU, key half f % NU)): the first
    // VW are requested now, before the softmax, and each use requests the one VW further on,
    // so the LDS latency hides behind the softmax and the MFMAs instead of stalling each pair
    constexpr int NVF = NDT * NU;
    auto vfrag = [&](int f) {
      const int d = dbase + 16 * (f / NU) + c16, u = f % NU;
      return *reinterpret_cast<const u32x4_t*>(&vt_lds[vt_off<KT>(d, 32 * (kh * NU + u) + 8 * q4)]);
    };
    u32x4_t vwin[VW];
#pragma unroll
    for (int f = 0; f < VW; ++f) vwin[f] = vfrag(f);
    // row max of the raw scores (invisible keys -inf; only a chunk's last tile, the causal
    // diagonal and the tree block need the mask). The scale is applied in the exponent:
    // p = 2^(s * scale - m) with m the running max of the scaled scores.
    const bool edge = (kt + KT > k1) || (TREE ? (kt + KT > tail0) : (a.causal && kt + KT - 1 > L - a.Mq));
    float smax = -INFINITY;
    if (edge) {
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kt + 16 * (ks0 + ks) + 4 * q4 + i;
          bool vis = key < k1;
          if (TREE)
            vis = vis && (key < tail0 || ((anc >> ((unsigned)(key - tail0) & 31u)) & 1u));
          else
            vis = vis && key <= kmax;
          s[ks][i] = vis ? s[ks][i] : -INFINITY;
          smax = fmaxf(smax, s[ks][i]);
        }
    } else {
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int i = 0; i < 4; ++i) smax = fmaxf(smax, s[ks][i]);
    }
    smax = max_xor32(max_xor16(smax));
    const float mn = fmaxf(m, smax * a.scale_log2);
    const float alpha = exp2_raw(m - mn);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = exp2_raw(__builtin_fmaf(s[ks][i], a.scale_log2, -mn));
        s[ks][i] = p;
        ps += p;
      }
    l = l * alpha + ps;
    // P as a pair hi + lo (hi = T(p), lo = T(p - hi)): the P.V product keeps ~16 significant
    // bits of p, so the output rounding is the only error of note (a single bf16 P, as the
    // reference's kernel rounds it, leaves little margin on long flat rows).
    // Quantized V: per output group gg, P is scaled by the keys' scale_v (the integer fields
    // then multiply it exactly) and sum p * bias_v is accumulated per row.
    constexpr int NPG = QB ? GW : 1;  // P operands: one per output group when quantized
    u32x4_t ph[NPG][NU], pl[NPG][NU];
    float bt[NPG];                    // this tile's sum p * bias_v (added after the rescale)
#pragma unroll
    for (int gg = 0; gg < NPG; ++gg) {
      bt[gg] = 0.f;
      f32x4_t pv[NKS];
      if constexpr (QB != 0) {
        const int g = dbase / 64 + gg;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const int key0 = 16 * (ks0 + ks) + 4 * q4;
          const f32x4_t sv = *reinterpret_cast<const f32x4_t*>(&qsb[bsel][2][g][key0]);
          const f32x4_t bv = *reinterpret_cast<const f32x4_t*>(&qsb[bsel][3][g][key0]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pv[ks][i] = s[ks][i] * sv[i];
            bt[gg] = __builtin_fmaf(s[ks][i], bv[i], bt[gg]);
          }
        }
      } else {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) pv[ks] = s[ks];
      }
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const float a0 = pv[2 * u + h][2 * i], a1 = pv[2 * u + h][2 * i + 1];
            const u32 hi = pack2<T>(a0, a1);
            ph[gg][u][2 * h + i] = hi;
            pl[gg][u][2 * h + i] = pack2<T>(a0 - to_f32<T>(hi & 0xFFFFu), a1 - to_f32<T>(hi >> 16));
          }
    }
    // the running max rarely moves after the first tiles: rescale only when some row's did
    // (alpha == 1 exactly otherwise, so skipping the multiply changes no bit)
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int t = 0; t < NDT; ++t) o[t] *= alpha;
      if constexpr (QB != 0) {
#pragma unroll
        for (int gg = 0; gg < GW; ++gg) bvs[gg] *= alpha;
      }
    }
    if constexpr (QB != 0) {
#pragma unroll
      for (int gg = 0; gg < GW; ++gg) bvs[gg] += bt[gg];
    }
#pragma unroll
    for (int f = 0; f < NVF; ++f) {
      const int t = f / NU, u = f % NU;
      const int gg = QB ? (16 * t) / 64 : 0;
      const u32x4_t vf = vwin[f % VW];
      if (f + VW < NVF) vwin[f % VW] = vfrag(f + VW);
      o[t] = mfma<T>(vf, ph[gg][u], o[t]);
      o[t] = mfma<T>(vf, pl[gg][u], o[t]);
    }
  };

  // PF tiles in flight: tile kt is staged from the registers its load landed in, which then
  // take the load of tile kt + PF*KT while tile kt is computed.
  TileRegs r0, r1;
  auto step = [&](TileRegs& r, int kt, int bsel) {
    store_tile(r, bsel);
    __syncthreads();  // tile visible; every wave is done with the tile before (other buffer)
    if (kt + PF * KT < k1) load_tile(r, kt + PF * KT);
    if (active) compute_tile(kt, bsel);
  };
  if (k0 < k1) load_tile(r0, k0);
  if constexpr (PF == 1) {
    for (int kt = k0; kt < k1; kt += KT) step(r0, kt, ((kt - k0) / KT) & 1);
  } else {
    if (k0 + KT < k1) load_tile(r1, k0 + KT);
    for (int kt = k0; kt < k1; kt += 2 * KT) {
      step(r0, kt, 0);
      if (kt + KT < k1) step(r1, kt + KT, 1);
    }
  }
  // ---- finalize: lane (row c16, quarter q4) holds O^T[dbase + 16t + 4q4 + i][row]
  l += shfl_xor(l, 16);
  l += shfl_xor(l, 32);
  if constexpr (QB != 0) {
    // the bias term of each output group, summed over the row's lanes, joins every column
#pragma unroll
    for (int gg = 0; gg < GW; ++gg) {
      bvs[gg] += shfl_xor(bvs[gg], 16);
      bvs[gg] += shfl_xor(bvs[gg], 32);
    }
#pragma unroll
    for (int t = 0; t < NDT; ++t) o[t] += bvs[(16 * t) / 64];
  }
  if constexpr (KS == 2) {
    // key half 1 hands (m, l, O) to half 0 through LDS: M = max(m0, m1),
    // O = 2^(m0 - M) O0 + 2^(m1 - M) O1, l likewise
    float* mo = reinterpret_cast<float*>(smem);           // [WV][NDT][64 lanes][4]
    float* ml = mo + WV * NDT * 64 * 4;                   // [WV][16] m, then [WV][16] l
    __syncthreads();                                      // every wave is done with the last tile
    if (kh == 1 && active) {
#pragma unroll
      for (int t = 0; t < NDT; ++t) *reinterpret_cast<f32x4_t*>(&mo[((rtw * NDT + t) * 64 + lane) * 4]) = o[t];
      if (q4 == 0) {
        ml[rtw * 16 + c16] = m;
        ml[WV * 16 + rtw * 16 + c16] = l;
      }
    }
    __syncthreads();
    if (kh == 1 || !active) return;
    const float m1 = ml[rtw * 16 + c16], l1 = ml[WV * 16 + rtw * 16 + c16];
    const float mm = fmaxf(m, m1);
    const float a0 = exp2_raw(m - mm), a1 = exp2_raw(m1 - mm);
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const f32x4_t o1 = *reinterpret_cast<const f32x4_t*>(&mo[((rtw * NDT + t) * 64 + lane) * 4]);
#pragma unroll
      for (int i = 0; i < 4; ++i) o[t][i] = __builtin_fmaf(o[t][i], a0, o1[i] * a1);
    }
    l = __builtin_fmaf(l, a0, l1 * a1);
    m = mm;
  }
  if (!active) return;
  const int row = rt * 16 + c16;
  if (row >= a.R) return;
  if (a.NB == 1) {
    const float inv = 1.0f / l;
    u16* orow = a.out + b * a.osb + (long)(hk * a.gqa + row / a.Mq) * a.osh + (long)(row % a.Mq) * a.osi + dbase;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      u32x2_t pk2 = {pack2<T>(o[t][0] * inv, o[t][1] * inv), pack2<T>(o[t][2] * inv, o[t][3] * inv)};
      if (!PAD || dbase + 16 * t + 4 * q4 < a.dv) *reinterpret_cast<u32x2_t*>(orow + 16 * t + 4 * q4) = pk2;
    }
    return;
  }
  const long pbase = ((long)bh * a.NB + blk) * a.RP + row;
  float* op = a.opart + pbase * D + dbase;
#pragma unroll
  for (int t = 0; t < NDT; ++t) *reinterpret_cast<f32x4_t*>(op + 16 * t + 4 * q4) = o[t];
  if (q4 == 0 && dh == 0) {
    a.mpart[pbase] = m;
    a.lpart[pbase] = l;
  }
}

// Combine of the key blocks (multirow_attn.py:162-178): M = max_j m_j, out = sum_j 2^(m_j - M)
// o_j / sum_j 2^(m_j - M) l_j. One workgroup per (batch*kv-head, row): wave w folds blocks
// j = w, w+4, ... with an online max, issuing CB blocks' loads per memory round trip; the four
// wave results are merged in LDS in wave order.
template <class T, int D>
__global__ __launch_bounds__(256) void combine_kernel(const AttnArgs a) {
  constexpr int DPL = D / 64;  // d values per lane
  constexpr int CB = 8;        // blocks in flight per wave
  const int bh = blockIdx.x / a.R, row = blockIdx.x - bh * a.R;
  const int b = bh / a.Hk, hk = bh - b * a.Hk;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long base = (long)bh * a.NB * a.RP + row;
  float M = -1e30f, den = 0.f, num[DPL];
#pragma unroll
  for (int t = 0; t < DPL; ++t) num[t] = 0.f;
  for (int j0 = wave; j0 < a.NB; j0 += 4 * CB) {  // wave-uniform trip count
    float mj[CB], lj[CB], oj[CB][DPL];
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int j = min(j0 + 4 * i, a.NB - 1);
      const long pj = base + (long)j * a.RP;
      mj[i] = a.mpart[pj];
      lj[i] = a.lpart[pj];
      const float* src = a.opart + pj * D + DPL * lane;
      if constexpr (DPL == 4) {
        const float4 o4 = *reinterpret_cast<const float4*>(src);
        oj[i][0] = o4.x;
        oj[i][1] = o4.y;
        oj[i][2] = o4.z;
        oj[i][3] = o4.w;
      } else if constexpr (DPL == 2) {
        const float2 o2 = *reinterpret_cast<const float2*>(src);
        oj[i][0] = o2.x;
        oj[i][1] = o2.y;
      } else {
        oj[i][0] = *src;
      }
    }
    float mn = M;
#pragma unroll
    for (int i = 0; i < CB; ++i)
      if (j0 + 4 * i < a.NB) mn = fmaxf(mn, mj[i]);
    const float f = exp2f(M - mn);
    den *= f;
#pragma unroll
    for (int t = 0; t < DPL; ++t) num[t] *= f;
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      if (j0 + 4 * i < a.NB) {
        const float w = exp2f(mj[i] - mn);
        den += w * lj[i];
#pragma unroll
        for (int t = 0; t < DPL; ++t) num[t] += w * oj[i][t];
      }
    }
    M = mn;
  }
  __shared__ float sm[4], sd[4], so[4][D];
  if (lane == 0) {
    sm[wave] = M;
    sd[wave] = den;
  }
#pragma unroll
  for (int t = 0; t < DPL; ++t) so[wave][DPL * lane + t] = num[t];
  __syncthreads();
  for (int d = threadIdx.x; d < a.dv; d += 256) {
    const float Mx = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
    float nn = 0.f, dd = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = exp2f(sm[w] - Mx);
      nn += f * so[w][d];
      dd += f * sd[w];
    }
    a.out[b * a.osb + (long)(hk * a.gqa + row / a.Mq) * a.osh + (long)(row % a.Mq) * a.osi + d] =
        from_f32<T>(nn / dd);
  }
}

// Launch pass 1 (+ the combine when NB > 1) for element type T and head dim D; defined for
// each (T, D) in its own translation unit (dspark_attn_<type>_d<D>.hip).
template <class T, int D>
int launch(const AttnArgs& a, const Plan& p, long B, bool tree, int qbits, hipStream_t s);
#define DSPARK_ATTN_LAUNCH(T, D) \
  template <>                    \
  int launch<T, D>(const AttnArgs& a, const Plan& p, long B, bool tree, int qbits, hipStream_t s)
DSPARK_ATTN_LAUNCH(BF16, 64);
DSPARK_ATTN_LAUNCH(BF16, 128);
DSPARK_ATTN_LAUNCH(BF16, 256);
DSPARK_ATTN_LAUNCH(F16, 64);
DSPARK_ATTN_LAUNCH(F16, 128);
DSPARK_ATTN_LAUNCH(F16, 256);

template <class T, int D, bool PAD>
void launch_p1(const AttnArgs& a, const Plan& p, long B, bool tree, int qbits, hipStream_t s) {
  const dim3 grid1((unsigned)(B * a.Hk), (unsigned)p.NB, (unsigned)p.NRG);
  constexpr int DS = D == 256 ? 2 : 1;
#define DSPARK_P1(TR, W, K, F, Q) \
  hipLaunchKernelGGL((p1_kernel<T, D, TR, W, K, F, Q, PAD>), grid1, dim3(64 * W * K * DS), 0, s, a)
#define DSPARK_P1_W(TR, Q)              \
  if (p.WV == 8) DSPARK_P1(TR, 8, 1, 2, Q); \
  else if (p.KS == 2) DSPARK_P1(TR, 4, 2, 1, Q); \
  else DSPARK_P1(TR, 4, 1, 1, Q);
  if constexpr (D == 256) {
    // plain K/V: one wave per row tile over all 256 columns, two tiles in flight, 4 or 6 row
    // tiles. Quantized K/V: two waves per row tile, one per half of the columns (a wave's
    // registers do not hold all 256), always 4 row tiles; the same key blocks and partial
    // layout, so the workspace is the plan's, with one more row group when there are more
    // than 4 tiles.
    const dim3 grid4((unsigned)(B * a.Hk), (unsigned)p.NB, (unsigned)((a.RT + 3) / 4));
#define DSPARK_P1_4(TR, Q) \
  hipLaunchKernelGGL((p1_kernel<T, D, TR, 4, 1, 1, Q, PAD>), grid4, dim3(64 * 4 * DS), 0, s, a)
#define DSPARK_P1_S(TR, W, G) \
  hipLaunchKernelGGL((p1_kernel<T, D, TR, W, 1, 2, 0, PAD, 1>), G, dim3(64 * W), 0, s, a)
    if (!PAD && qbits == 8) DSPARK_P1_4(false, 8);
    else if (!PAD && qbits == 4) DSPARK_P1_4(false, 4);
    else if (p.WV == 6) { if (tree) DSPARK_P1_S(true, 6, grid1); else DSPARK_P1_S(false, 6, grid1); }
    else if (tree) DSPARK_P1_S(true, 4, grid4);
    else DSPARK_P1_S(false, 4, grid4);
#undef DSPARK_P1_S
#undef DSPARK_P1_4
  } else {
    if (!PAD && qbits == 8) { DSPARK_P1_W(false, 8) }
    else if (!PAD && qbits == 4) { DSPARK_P1_W(false, 4) }
    else if (tree) { DSPARK_P1_W(true, 0) }
    else { DSPARK_P1_W(false, 0) }
  }
#undef DSPARK_P1_W
#undef DSPARK_P1
}

template <class T, int D>
int launch_impl(const AttnArgs& a, const Plan& p, long B, bool tree, int qbits, hipStream_t s) {
  // quantized caches hold whole groups of 64 along D: never padded (the entry point checks)
  if (a.dv != D) launch_p1<T, D, true>(a, p, B, tree, 0, s);
  else launch_p1<T, D, false>(a, p, B, tree, qbits, s);
  int st = check_launch("verify_attention(p1)");
  if (st || p.NB == 1) return st;
  hipLaunchKernelGGL((combine_kernel<T, D>), dim3((unsigned)(B * a.Hk * a.R)), dim3(256), 0, s, a);
  return check_launch("verify_attention(combine)");
}

}  // namespace attn
}  // namespace dspark
