// Multi-row causal GQA verify attention for gfx950 (MI355X).
//
// Semantics (multirow_attn.py:52-178, :223-259): q [B, Hq, Mq, D] is viewed per KV head as
// R = gqa * Mq rows (row r = g*Mq + i is query head hk*gqa + g at block position i). K/V hold
// L keys (prefix + the Mq verify rows, already written). Causal: row i sees keys
// 0 .. L - Mq + i. Softmax in the exp2 domain with fp32 running max m (init -1e30) and sum l;
// P is rounded to bf16 for the P.V product (multirow_attn.py:131-140); partials of the
// split-KV blocks are merged as out = sum 2^(m_j - M) o_j / sum 2^(m_j - M) l_j
// (multirow_attn.py:162-178).
//
// MI355X mapping:
//   * grid = (B*Hk, NB key blocks, row groups); a workgroup of 4 or 8 waves owns one KV
//     head's key block and up to 4 or 8 row tiles of 16 rows (all gqa*Mq rows of the head
//     when there are at most 128), so each K/V byte is read from HBM once and shared by every
//     query head of the GQA group. On short caches (few blocks) the 4 row tiles are worked by
//     8 waves, two per tile splitting its keys.
//   * 64-key tiles are staged through two alternating LDS buffers (one barrier per tile) from
//     registers loaded one (4-wave workgroups) or two (8-wave workgroups) tiles ahead: K row-major (padded rows), V transposed (key-contiguous,
//     8-key blocks XOR-swizzled by d) because the P.V MFMA reduces over keys.
//   * S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_16x16x32_bf16. Computing the transposed
//     scores leaves each lane holding 8 keys of one query row, which is exactly the B operand
//     of the P.V MFMA — no shuffle of P.
//   * row max: 2 cross-lane xor-shuffles per tile; the row sum stays lane-partial until the end.
#include "dspark_common.h"

namespace dspark {
namespace {

constexpr int KT = 64;      // keys per LDS tile

struct AttnArgs {
  const u16* q;
  const u16* k;
  const u16* v;
  const u32* anc;
  float* opart;
  float* mpart;
  float* lpart;
  u16* out;
  long ksb, ksh, kss;
  long vsb, vsh, vss;
  long osb, osh, osi;  // output strides (batch, query head, position); head_dim contiguous
  int Hq, Hk, Mq, L;
  int gqa, R, RT, RP;
  int chunk, NB;
  float scale_log2;
  int causal;
};

// position of key (0..63) inside a tile's transposed V row: the 8 keys one lane needs for one
// P.V MFMA (keys 32u + 4q + {0..3} and 32u + 16 + 4q + {0..3}) are made contiguous.
__device__ __forceinline__ int vt_pos(int key) {
  const int u = key >> 5, h = (key >> 4) & 1, qq = (key >> 2) & 3, i = key & 3;
  return (u << 5) | (qq << 3) | (h << 2) | i;
}
// 2^x with v_exp_f32 (results below 2^-126 flush to 0: negligible softmax weights)
__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }

// swizzled element offset of (d, pos) in the transposed V tile (row pitch KT)
__device__ __forceinline__ int vt_off(int d, int pos) {
  return d * KT + ((((pos >> 3) ^ (d >> 1) ^ (d >> 3)) & 7) << 3) + (pos & 7);
}

// WV row tiles per workgroup (4, or 8 when a KV head has more than 4 row tiles, so every row
// of the head shares one read of each K/V tile), each worked by KS waves: with KS = 2 wave
// (tile r, half h) takes keys 32h..32h+31 of every 64-key tile, and the two halves' (m, l, O)
// are merged in LDS at the end (8 waves per workgroup either way).
template <int D, bool TREE, int WV, int KS, int PF>
__global__ __launch_bounds__(64 * WV * KS) void attn_p1_kernel(const AttnArgs a) {
  static_assert(KS == 1 || KS == 2, "key split");
  static_assert(PF == 1 || PF == 2, "tiles in flight");
  constexpr int THREADS = 64 * WV * KS;
  constexpr int NKS = 4 / KS;         // 16-key subtiles of a tile per wave
  constexpr int NU = 2 / KS;          // 32-key halves of a tile per wave (P.V MFMA k-steps)
  constexpr int KP = D + 8;           // padded K row (elements)
  constexpr int DC = D / 8;           // 16-byte chunks per key row
  constexpr int LOADS = KT * DC / THREADS;  // 16-byte K chunks per thread per tile
  constexpr int NDC = D / 32;         // d-chunks of the S MFMA
  constexpr int NDT = D / 16;         // d-tiles of the O MFMA
  constexpr int VW = 4;               // V fragments requested ahead of their MFMAs
  // K tile, then the transposed V tile; reused for the key-half merge after the last tile
  // two tile buffers: tile i is staged into buffer i & 1 while the other buffer may still be in
  // use by waves finishing tile i - 1, so one barrier per tile suffices
  constexpr int TILE = KT * KP + D * KT;
  __shared__ __attribute__((aligned(16))) u16 smem[2 * TILE];
  static_assert(KS == 1 || (WV * 64 * NDT * 4 + 2 * WV * 16) * 4 <= (KT * KP + D * KT) * 2, "merge area");

  const int bh = blockIdx.x;
  const int b = bh / a.Hk, hk = bh % a.Hk;
  const int blk = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = uniform(tid >> 6);
  const int c16 = lane & 15, q4 = lane >> 4;
  const int rtw = wave % WV, kh = wave / WV;  // row tile in the group, key half
  const int rt = blockIdx.z * WV + rtw;
  const bool active = rt < a.RT;

  const int L = a.L;
  const int k0 = blk * a.chunk;
  const int k1 = min(L, k0 + a.chunk);

  const u16* kbase = a.k + b * a.ksb + hk * a.ksh;
  const u16* vbase = a.v + b * a.vsb + hk * a.vsh;

  // ---- this lane's query row (B operand of S^T = K Q^T)
  const int rr = min(rt * 16 + c16, a.R - 1);
  const int qi = rr % a.Mq;
  const u16* qrow = a.q + ((long)(b * a.Hq + hk * a.gqa) * a.Mq + rr) * D;
  u32x4_t qf[NDC];
#pragma unroll
  for (int c = 0; c < NDC; ++c) qf[c] = ldg128(qrow + 32 * c + 8 * q4);
  const int kmax = a.causal ? (L - a.Mq + qi) : (L - 1);
  const u32 anc = TREE ? a.anc[qi] : 0u;
  const int tail0 = L - a.Mq;  // first key of the verify block

  f32x4_t o[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) o[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -1e30f, l = 0.f;

  // ---- cooperative tile loads into registers.
  // K: 16-byte chunk c = tid + THREADS*j -> (key c / DC, d-chunk c % DC), stored row-major.
  // V: thread (key quad vkq = tid & 15, d-chunk vdc = tid >> 4) loads keys 4vkq..4vkq+3 and
  //    writes the transposed tile as 8 ds_write_b64 (4 keys of one d each); odd d-chunks walk
  //    their 8 d-rows in pair-swapped order so each half-wave covers all 64 LDS banks.
  const bool vthread = tid < 16 * DC;
  const int vkq = tid & 15, vdc = tid >> 4;
  struct TileRegs {
    u32x4_t k[LOADS], v[4];
  };
  // A tile inside the cache is addressed as a uniform base (scalar) plus a loop-invariant
  // 32-bit byte offset per lane; only a tile running past key L - 1 clamps each key.
  static_assert(THREADS % DC == 0, "K chunks of one thread share their d-chunk");
  const unsigned koff = (unsigned)(((tid / DC) * a.kss + 8 * (tid % DC)) * 2);
  const unsigned voff = (unsigned)((4 * vkq * a.vss + 8 * vdc) * 2);
  const long kstep = (long)(THREADS / DC) * a.kss * 2;  // bytes between a thread's K chunks
  auto load_tile = [&](TileRegs& r, int kt) {
    if (kt + KT <= L) {
      const char* kb = reinterpret_cast<const char*>(kbase + (long)kt * a.kss);
      const char* vb = reinterpret_cast<const char*>(vbase + (long)kt * a.vss);
#pragma unroll
      for (int j = 0; j < LOADS; ++j) r.k[j] = ldg128((kb + j * kstep) + koff);
      if (vthread) {
#pragma unroll
        for (int j = 0; j < 4; ++j) r.v[j] = ldg128((vb + (long)j * a.vss * 2) + voff);
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int c = tid + THREADS * j;
      const int key = min(kt + c / DC, L - 1);
      r.k[j] = ldg128(kbase + (long)key * a.kss + 8 * (c % DC));
    }
    if (vthread) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = min(kt + 4 * vkq + j, L - 1);
        r.v[j] = ldg128(vbase + (long)key * a.vss + 8 * vdc);
      }
    }
  };
  // element (e ^ (vdc & 1)) of each 8-wide chunk: low half-word of word e >> 1 when that index
  // is even, high half-word when odd
  const u32 sel_lo = 0x05040100u, sel_hi = 0x07060302u;
  const u32 vsel_even = (vdc & 1) ? sel_hi : sel_lo;  // e even
  const u32 vsel_odd = (vdc & 1) ? sel_lo : sel_hi;   // e odd
  auto store_tile = [&](const TileRegs& r, int b) {
    u16* const ks_lds = smem + b * TILE;
    u16* const vt_lds = ks_lds + KT * KP;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int c = tid + THREADS * j;
      *reinterpret_cast<u32x4_t*>(&ks_lds[(c / DC) * KP + 8 * (c % DC)]) = r.k[j];
    }
    if (vthread) {
      const int pos = vt_pos(4 * vkq);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 8 * vdc + (e ^ (vdc & 1));
        const int wd = e >> 1;
        const u32 vsel = (e & 1) ? vsel_odd : vsel_even;
        const u32x2_t pr = {__builtin_amdgcn_perm(r.v[1][wd], r.v[0][wd], vsel),
                            __builtin_amdgcn_perm(r.v[3][wd], r.v[2][wd], vsel)};
        *reinterpret_cast<u32x2_t*>(&vt_lds[vt_off(d, pos)]) = pr;
      }
    }
  };

  auto compute_tile = [&](int kt, int b) {
    const u16* const ks_lds = smem + b * TILE;
    const u16* const vt_lds = ks_lds + KT * KP;
    // S^T[key][row] for this wave's NKS subtiles of 16 keys (keys 16 (ks0 + j) ..)
    const int ks0 = kh * NKS;
    f32x4_t s[NKS];
#pragma unroll
    for (int j = 0; j < NKS; ++j) {
      s[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NDC; ++c) {
        const u32x4_t kf =
            *reinterpret_cast<const u32x4_t*>(&ks_lds[(16 * (ks0 + j) + c16) * KP + 32 * c + 8 * q4]);
        s[j] = mfma16x16x32(kf, qf[c], s[j]);
      }
    }
    // V fragments of the P.V product (fragment f = (d-tile f / NU, key half f % NU)): the first
    // VW are requested now, before the softmax, and each use requests the one VW further on,
    // so the LDS latency hides behind the softmax and the MFMAs instead of stalling each pair
    constexpr int NVF = NDT * NU;
    auto vfrag = [&](int f) {
      const int d = 16 * (f / NU) + c16, u = f % NU;
      return *reinterpret_cast<const u32x4_t*>(&vt_lds[vt_off(d, 32 * (kh * NU + u) + 8 * q4)]);
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
    smax = fmaxf(smax, shfl_xor(smax, 16));
    smax = fmaxf(smax, shfl_xor(smax, 32));
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
    // P as a bf16 pair hi + lo (hi = bf16(p), lo = bf16(p - hi)): the P.V product keeps ~16
    // significant bits of p, so the bf16 output rounding is the only error of note (a single
    // bf16 P, as the reference's kernel rounds it, leaves little margin on long flat rows).
    u32x4_t ph[NU], pl[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const float a0 = s[2 * u + h][2 * i], a1 = s[2 * u + h][2 * i + 1];
          const u32 hi = pack_bf16x2(a0, a1);
          ph[u][2 * h + i] = hi;
          pl[u][2 * h + i] = pack_bf16x2(a0 - bf2f(hi & 0xFFFFu), a1 - bf2f(hi >> 16));
        }
    // the running max rarely moves after the first tiles: rescale only when some row's did
    // (alpha == 1 exactly otherwise, so skipping the multiply changes no bit)
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int t = 0; t < NDT; ++t) o[t] *= alpha;
    }
#pragma unroll
    for (int f = 0; f < NVF; ++f) {
      const int t = f / NU, u = f % NU;
      const u32x4_t vf = vwin[f % VW];
      if (f + VW < NVF) vwin[f % VW] = vfrag(f + VW);
      o[t] = mfma16x16x32(vf, ph[u], o[t]);
      o[t] = mfma16x16x32(vf, pl[u], o[t]);
    }
  };

  // PF tiles in flight: tile kt is staged from the registers its load landed in, which then
  // take the load of tile kt + PF*KT while tile kt is computed.
  TileRegs r0, r1;
  auto step = [&](TileRegs& r, int kt, int b) {
    store_tile(r, b);
    __syncthreads();  // tile visible; every wave is done with the tile before (other buffer)
    if (kt + PF * KT < k1) load_tile(r, kt + PF * KT);
    if (active) compute_tile(kt, b);
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
  // ---- finalize: lane (row c16, quarter q4) holds O^T[16t + 4q4 + i][row]
  l += shfl_xor(l, 16);
  l += shfl_xor(l, 32);
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
    u16* orow = a.out + b * a.osb + (long)(hk * a.gqa + row / a.Mq) * a.osh + (long)(row % a.Mq) * a.osi;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      u32x2_t pk2 = {pack_bf16x2(o[t][0] * inv, o[t][1] * inv), pack_bf16x2(o[t][2] * inv, o[t][3] * inv)};
      *reinterpret_cast<u32x2_t*>(orow + 16 * t + 4 * q4) = pk2;
    }
    return;
  }
  const long pbase = ((long)bh * a.NB + blk) * a.RP + row;
  float* op = a.opart + pbase * D;
#pragma unroll
  for (int t = 0; t < NDT; ++t) *reinterpret_cast<f32x4_t*>(op + 16 * t + 4 * q4) = o[t];
  if (q4 == 0) {
    a.mpart[pbase] = m;
    a.lpart[pbase] = l;
  }
}

// Combine of the key blocks (multirow_attn.py:162-178): M = max_j m_j, out = sum_j 2^(m_j - M)
// o_j / sum_j 2^(m_j - M) l_j. One workgroup per (batch*kv-head, row): wave w folds blocks
// j = w, w+4, ... with an online max, issuing CB blocks' loads per memory round trip; the four
// wave results are merged in LDS in wave order.
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs a) {
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
      if constexpr (DPL == 2) {
        const float2 o2 = *reinterpret_cast<const float2*>(&a.opart[pj * D + 2 * lane]);
        oj[i][0] = o2.x;
        oj[i][1] = o2.y;
      } else {
        oj[i][0] = a.opart[pj * D + lane];
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
  const int d = threadIdx.x;
  if (d < D) {
    const float Mx = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
    float nn = 0.f, dd = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = exp2f(sm[w] - Mx);
      nn += f * so[w][d];
      dd += f * sd[w];
    }
    a.out[b * a.osb + (long)(hk * a.gqa + row / a.Mq) * a.osh + (long)(row % a.Mq) * a.osi + d] = f2bf(nn / dd);
  }
}

struct Plan {
  int R, RT, RP, WV, KS, PF, NRG, chunk, NB;
};

Plan make_plan(long B, long Hq, long Hk, long Mq, long L) {
  Plan p{};
  p.R = (int)((Hq / Hk) * Mq);
  p.RT = (p.R + 15) / 16;
  p.RP = p.RT * 16;
  p.WV = p.RT > 4 ? 8 : 4;
  p.KS = 1;
  p.PF = p.WV == 8 ? 2 : 1;
  p.NRG = (p.RT + p.WV - 1) / p.WV;
  // Long caches: ~2 workgroups of 4 waves per CU (256 CUs), or one of 8 waves (twice the
  // rows per K/V tile: the fp32 partials, written here and read by the combine, double too),
  // which then keeps two tiles in flight. At least 4 tiles (256 keys) per block. When that
  // caps the blocks below one workgroup per CU, 4-row-tile heads split each tile's keys over
  // 8 waves. Row groups beyond one re-read the head's K/V (only when gqa * Mq > 128).
  const long heads = B * Hk * p.NRG;
  const long target = p.WV == 8 ? 256 : 512;
  long nb = (target + heads - 1) / heads;
  const long max_nb = (L + 4 * KT - 1) / (4 * KT);
  if (nb > max_nb) nb = max_nb;
  if (nb < 1) nb = 1;
  if (p.WV == 4 && heads * nb < 256) p.KS = 2;
  long chunk = (L + nb - 1) / nb;
  chunk = ((chunk + KT - 1) / KT) * KT;
  p.chunk = (int)chunk;
  p.NB = (int)((L + chunk - 1) / chunk);
  return p;
}

size_t workspace_bytes(const Plan& p, long B, long Hk, long D) {
  if (p.NB <= 1) return 0;
  const size_t rows = (size_t)B * Hk * p.NB * p.RP;
  return rows * D * sizeof(float) + 2 * rows * sizeof(float);
}

int check_shape(long B, long Hq, long Mq, long D, long Hk, long L) {
  if (B < 1 || Hq < 1 || Hk < 1 || Mq < 1 || L < 1)
    return fail(DSPARK_ERR_SHAPE, "verify_attention: B=%ld Hq=%ld Hk=%ld Mq=%ld L=%ld", B, Hq, Hk, Mq, L);
  if (Hq % Hk) return fail(DSPARK_ERR_SHAPE, "verify_attention: Hq=%ld not a multiple of Hk=%ld", Hq, Hk);
  if (D != 64 && D != 128) return fail(DSPARK_ERR_SHAPE, "verify_attention: head_dim %ld (64 or 128 supported)", D);
  if (Mq > L) return fail(DSPARK_ERR_SHAPE, "verify_attention: Mq=%ld > L=%ld", Mq, L);
  if ((Hq / Hk) * Mq > 256) return fail(DSPARK_ERR_SHAPE, "verify_attention: gqa*Mq=%ld > 256", (Hq / Hk) * Mq);
  if (L >= (1L << 30) || B * Hk >= (1L << 20)) return fail(DSPARK_ERR_SHAPE, "verify_attention: too large");
  return DSPARK_OK;
}

}  // namespace
}  // namespace dspark

using namespace dspark;

extern "C" size_t dspark_verify_attention_workspace(int64_t B, int64_t Hq, int64_t Hk, int64_t Mq, int64_t D,
                                                    int64_t L_total) {
  if (check_shape(B, Hq, Mq, D, Hk, L_total)) return 0;
  return workspace_bytes(make_plan(B, Hq, Hk, Mq, L_total), B, Hk, D);
}

extern "C" int dspark_verify_attention_plan(int64_t B, int64_t Hq, int64_t Hk, int64_t Mq, int64_t D,
                                            int64_t L_total, int32_t* out) {
  if (!out) return fail(DSPARK_ERR_ARG, "verify_attention_plan: null output");
  const int st = check_shape(B, Hq, Mq, D, Hk, L_total);
  if (st) return st;
  const Plan p = make_plan(B, Hq, Hk, Mq, L_total);
  out[0] = p.R;
  out[1] = p.RP;
  out[2] = p.NRG;
  out[3] = p.chunk;
  out[4] = p.NB;
  out[5] = (int32_t)(B * Hk * p.NB * p.NRG);
  return DSPARK_OK;
}

extern "C" int64_t dspark_verify_attention_blocks(int64_t B, int64_t Hq, int64_t Hk, int64_t Mq, int64_t D,
                                                  int64_t L_total) {
  if (check_shape(B, Hq, Mq, D, Hk, L_total)) return -1;
  return make_plan(B, Hq, Hk, Mq, L_total).NB;
}

namespace {
int verify_attention_impl(const void* q, int64_t B, int64_t Hq, int64_t Mq, int64_t D, const void* k, const void* v,
                          const int64_t k_strides[3], const int64_t v_strides[3], int64_t Hk, int64_t L_total,
                          float scale, int causal, const uint32_t* tree_anc, void* out, const int64_t out_strides[3],
                          void* workspace, size_t workspace_bytes_, dspark_stream stream) {
  if (!q || !k || !v || !k_strides || !v_strides || !out || !out_strides)
    return fail(DSPARK_ERR_ARG, "verify_attention: null pointer");
  for (int i = 0; i < 3; ++i)
    if ((out_strides[i] % 4) || out_strides[i] < 0)
      return fail(DSPARK_ERR_ALIGN, "verify_attention: output strides must be non-negative multiples of 4 elements");
  int st = check_shape(B, Hq, Mq, D, Hk, L_total);
  if (st) return st;
  if (tree_anc && Mq > 32) return fail(DSPARK_ERR_SHAPE, "verify_attention: tree mask needs Mq <= 32");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 8))
    return fail(DSPARK_ERR_ALIGN, "verify_attention: q/k/v must be 16-byte aligned, out 8-byte aligned");
  for (int i = 0; i < 3; ++i)
    if ((k_strides[i] % 8) || (v_strides[i] % 8) || k_strides[i] < 0 || v_strides[i] < 0)
      return fail(DSPARK_ERR_ALIGN, "verify_attention: K/V strides must be non-negative multiples of 8 elements");
  // the kernels address a 64-key tile with 32-bit byte offsets from its first key
  if (k_strides[2] >= (1L << 24) || v_strides[2] >= (1L << 24))
    return fail(DSPARK_ERR_SHAPE, "verify_attention: K/V position stride %ld/%ld too large", (long)k_strides[2],
                (long)v_strides[2]);
  const Plan p = make_plan(B, Hq, Hk, Mq, L_total);
  const size_t need = workspace_bytes(p, B, Hk, D);
  if (need && (!workspace || workspace_bytes_ < need))
    return fail(DSPARK_ERR_WORKSPACE, "verify_attention: workspace %zu < %zu bytes", workspace_bytes_, need);
  if (need && !aligned(workspace, 16)) return fail(DSPARK_ERR_ALIGN, "verify_attention: workspace must be 16-byte aligned");

  AttnArgs a{};
  a.q = static_cast<const u16*>(q);
  a.k = static_cast<const u16*>(k);
  a.v = static_cast<const u16*>(v);
  a.anc = tree_anc;
  a.out = static_cast<u16*>(out);
  a.ksb = k_strides[0];
  a.ksh = k_strides[1];
  a.kss = k_strides[2];
  a.vsb = v_strides[0];
  a.vsh = v_strides[1];
  a.vss = v_strides[2];
  a.osb = out_strides[0];
  a.osh = out_strides[1];
  a.osi = out_strides[2];
  a.Hq = (int)Hq;
  a.Hk = (int)Hk;
  a.Mq = (int)Mq;
  a.L = (int)L_total;
  a.gqa = (int)(Hq / Hk);
  a.R = p.R;
  a.RT = p.RT;
  a.RP = p.RP;
  a.chunk = p.chunk;
  a.NB = p.NB;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.causal = causal ? 1 : 0;
  if (need) {
    const size_t rows = (size_t)B * Hk * p.NB * p.RP;
    a.opart = static_cast<float*>(workspace);
    a.mpart = a.opart + rows * D;
    a.lpart = a.mpart + rows;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid1((unsigned)(B * Hk), (unsigned)p.NB, (unsigned)p.NRG);
  const bool tree = tree_anc != nullptr;
#define ATTN_P1(DD, TR, W, K, F) \
  hipLaunchKernelGGL((attn_p1_kernel<DD, TR, W, K, F>), grid1, dim3(64 * W * K), 0, s, a)
#define ATTN_P1_W(DD, TR) \
  if (p.WV == 8) ATTN_P1(DD, TR, 8, 1, 2); else if (p.KS == 2) ATTN_P1(DD, TR, 4, 2, 1); else ATTN_P1(DD, TR, 4, 1, 1);
  if (D == 128) {
    if (tree) { ATTN_P1_W(128, true) } else { ATTN_P1_W(128, false) }
  } else {
    if (tree) { ATTN_P1_W(64, true) } else { ATTN_P1_W(64, false) }
  }
#undef ATTN_P1_W
#undef ATTN_P1
  st = check_launch("verify_attention(p1)");
  if (st || p.NB == 1) return st;
  const dim3 grid2((unsigned)(B * Hk * p.R));
  if (D == 128) hipLaunchKernelGGL((attn_combine_kernel<128>), grid2, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((attn_combine_kernel<64>), grid2, dim3(256), 0, s, a);
  return check_launch("verify_attention(combine)");
}
}  // namespace

extern "C" int dspark_verify_attention(const void* q, int64_t B, int64_t Hq, int64_t Mq, int64_t D, const void* k,
                                       const void* v, const int64_t k_strides[3], const int64_t v_strides[3],
                                       int64_t Hk, int64_t L_total, float scale, int causal,
                                       const uint32_t* tree_anc, void* out, void* workspace, size_t workspace_bytes_,
                                       dspark_stream stream) {
  const int64_t os[3] = {Hq * Mq * D, Mq * D, D};
  return verify_attention_impl(q, B, Hq, Mq, D, k, v, k_strides, v_strides, Hk, L_total, scale, causal, tree_anc,
                               out, os, workspace, workspace_bytes_, stream);
}

extern "C" int dspark_verify_attention_strided(const void* q, int64_t B, int64_t Hq, int64_t Mq, int64_t D,
                                               const void* k, const void* v, const int64_t k_strides[3],
                                               const int64_t v_strides[3], int64_t Hk, int64_t L_total, float scale,
                                               int causal, const uint32_t* tree_anc, void* out,
                                               const int64_t out_strides[3], void* workspace, size_t workspace_bytes_,
                                               dspark_stream stream) {
  return verify_attention_impl(q, B, Hq, Mq, D, k, v, k_strides, v_strides, Hk, L_total, scale, causal, tree_anc,
                               out, out_strides, workspace, workspace_bytes_, stream);
}
