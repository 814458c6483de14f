// Multi-row verify attention: the C ABI (validation, plan queries, dispatch by element type and
// head dim). The kernels and the plan are in dspark_attn.h; each (type, head dim) is compiled in
// its own translation unit (dspark_attn_<type>_d<D>.hip).
#include "dspark_attn.h"

namespace dspark {
namespace attn {
namespace {

int check_shape(long B, long Hq, long Mq, long D, long Hk, long L) {
  if (B < 1 || Hq < 1 || Hk < 1 || Mq < 1 || L < 1)
    return fail(DSPARK_ERR_SHAPE, "verify_attention: B=%ld Hq=%ld Hk=%ld Mq=%ld L=%ld", B, Hq, Hk, Mq, L);
  if (Hq % Hk) return fail(DSPARK_ERR_SHAPE, "verify_attention: Hq=%ld not a multiple of Hk=%ld", Hq, Hk);
  if (D < 8 || D > 256 || D % 8)
    return fail(DSPARK_ERR_SHAPE, "verify_attention: head_dim %ld (a multiple of 8 up to 256)", D);
  if (Mq > L) return fail(DSPARK_ERR_SHAPE, "verify_attention: Mq=%ld > L=%ld", Mq, L);
  if ((Hq / Hk) * Mq > 256) return fail(DSPARK_ERR_SHAPE, "verify_attention: gqa*Mq=%ld > 256", (Hq / Hk) * Mq);
  if (L >= (1L << 30) || B * Hk >= (1L << 20)) return fail(DSPARK_ERR_SHAPE, "verify_attention: too large");
  return DSPARK_OK;
}

// the kernel instance serving head dim D: 64, 128 or 256 columns, the missing ones zero
long instance_d(long D) { return D <= 64 ? 64 : (D <= 128 ? 128 : 256); }

int check_strides(const int64_t* s, long mult, const char* what) {
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || s[i] % mult)
      return fail(DSPARK_ERR_ALIGN, "verify_attention: %s strides must be non-negative multiples of %ld", what, mult);
  return DSPARK_OK;
}

// The parts shared by the plain and the quantized entry points.
struct Common {
  const void* q;
  long B, Hq, Mq, D, Hk, L;
  float scale;
  int causal;
  const uint32_t* tree_anc;
  void* out;
  const int64_t* out_strides;
  void* workspace;
  size_t workspace_bytes;
};

int prepare(const Common& c, AttnArgs& a, Plan& p) {
  if (!c.q || !c.out || !c.out_strides) return fail(DSPARK_ERR_ARG, "verify_attention: null pointer");
  int st = check_shape(c.B, c.Hq, c.Mq, c.D, c.Hk, c.L);
  if (st) return st;
  if ((st = check_strides(c.out_strides, 4, "output"))) return st;
  if (c.tree_anc && c.Mq > 32) return fail(DSPARK_ERR_SHAPE, "verify_attention: tree mask needs Mq <= 32");
  if (!aligned(c.q, 16) || !aligned(c.out, 8))
    return fail(DSPARK_ERR_ALIGN, "verify_attention: q must be 16-byte aligned, out 8-byte aligned");
  const long DI = instance_d(c.D);
  p = make_plan(c.B, c.Hq, c.Hk, c.Mq, DI, c.L);
  const size_t need = partial_bytes(p, c.B, c.Hk, DI);
  if (need && (!c.workspace || c.workspace_bytes < need))
    return fail(DSPARK_ERR_WORKSPACE, "verify_attention: workspace %zu < %zu bytes", c.workspace_bytes, need);
  if (need && !aligned(c.workspace, 16))
    return fail(DSPARK_ERR_ALIGN, "verify_attention: workspace must be 16-byte aligned");
  a.q = static_cast<const u16*>(c.q);
  a.anc = c.tree_anc;
  a.out = static_cast<u16*>(c.out);
  a.osb = c.out_strides[0];
  a.osh = c.out_strides[1];
  a.osi = c.out_strides[2];
  a.Hq = (int)c.Hq;
  a.Hk = (int)c.Hk;
  a.Mq = (int)c.Mq;
  a.L = (int)c.L;
  a.dv = (int)c.D;
  a.gqa = (int)(c.Hq / c.Hk);
  a.R = p.R;
  a.RT = p.RT;
  a.RP = p.RP;
  a.chunk = p.chunk;
  a.NB = p.NB;
  a.scale_log2 = c.scale * 1.4426950408889634f;
  a.causal = c.causal ? 1 : 0;
  if (need) {
    const size_t rows = (size_t)c.B * c.Hk * p.NB * p.RP;
    a.opart = static_cast<float*>(c.workspace);
    a.mpart = a.opart + rows * DI;
    a.lpart = a.mpart + rows;
  }
  return DSPARK_OK;
}

template <class T>
int launch_d(const AttnArgs& a, const Plan& p, long B, long D, bool tree, int qbits, hipStream_t s) {
  const long DI = instance_d(D);
  if (DI == 64) return launch<T, 64>(a, p, B, tree, qbits, s);
  if (DI == 128) return launch<T, 128>(a, p, B, tree, qbits, s);
  return launch<T, 256>(a, p, B, tree, qbits, s);
}

int dispatch(int dtype, const AttnArgs& a, const Plan& p, long B, long D, bool tree, int qbits, hipStream_t s) {
  if (dtype == DSPARK_DTYPE_F16) return launch_d<F16>(a, p, B, D, tree, qbits, s);
  return launch_d<BF16>(a, p, B, D, tree, qbits, s);
}

int check_dtype(int dtype) {
  if (dtype != DSPARK_DTYPE_BF16 && dtype != DSPARK_DTYPE_F16)
    return fail(DSPARK_ERR_UNSUPPORTED, "verify_attention: dtype %d (bf16 or fp16)", dtype);
  return DSPARK_OK;
}

int plain_impl(int dtype, const Common& c, const void* k, const void* v, const int64_t* k_strides,
               const int64_t* v_strides, hipStream_t s) {
  int st = check_dtype(dtype);
  if (st) return st;
  if (!k || !v || !k_strides || !v_strides) return fail(DSPARK_ERR_ARG, "verify_attention: null pointer");
  AttnArgs a{};
  Plan p{};
  if ((st = prepare(c, a, p))) return st;
  if (!aligned(k, 16) || !aligned(v, 16)) return fail(DSPARK_ERR_ALIGN, "verify_attention: k/v must be 16-byte aligned");
  if ((st = check_strides(k_strides, 8, "K")) || (st = check_strides(v_strides, 8, "V"))) return st;
  // the kernels address a key tile with 32-bit byte offsets from its first key
  if (k_strides[2] >= (1L << 24) || v_strides[2] >= (1L << 24))
    return fail(DSPARK_ERR_SHAPE, "verify_attention: K/V position stride %ld/%ld too large", (long)k_strides[2],
                (long)v_strides[2]);
  a.k = k;
  a.v = v;
  a.ksb = k_strides[0];
  a.ksh = k_strides[1];
  a.kss = k_strides[2];
  a.vsb = v_strides[0];
  a.vsh = v_strides[1];
  a.vss = v_strides[2];
  return dispatch(dtype, a, p, c.B, c.D, c.tree_anc != nullptr, 0, s);
}

}  // namespace
}  // namespace attn
}  // namespace dspark

using namespace dspark;
using namespace dspark::attn;

extern "C" size_t dspark_verify_attention_workspace(int64_t B, int64_t Hq, int64_t Hk, int64_t Mq, int64_t D,
                                                    int64_t L_total) {
  if (check_shape(B, Hq, Mq, D, Hk, L_total)) return 0;
  const long DI = instance_d(D);
  return partial_bytes(make_plan(B, Hq, Hk, Mq, DI, L_total), B, Hk, DI);
}

extern "C" int dspark_verify_attention_plan(int64_t B, int64_t Hq, int64_t Hk, int64_t Mq, int64_t D,
                                            int64_t L_total, int32_t* out) {
  if (!out) return fail(DSPARK_ERR_ARG, "verify_attention_plan: null output");
  const int st = check_shape(B, Hq, Mq, D, Hk, L_total);
  if (st) return st;
  const Plan p = make_plan(B, Hq, Hk, Mq, instance_d(D), L_total);
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
  return make_plan(B, Hq, Hk, Mq, instance_d(D), L_total).NB;
}

extern "C" int dspark_verify_attention_typed(int dtype, const void* q, int64_t B, int64_t Hq, int64_t Mq, int64_t D,
                                             const void* k, const void* v, const int64_t k_strides[3],
                                             const int64_t v_strides[3], int64_t Hk, int64_t L_total, float scale,
                                             int causal, const uint32_t* tree_anc, void* out,
                                             const int64_t out_strides[3], void* workspace, size_t workspace_bytes,
                                             dspark_stream stream) {
  const Common c{q, B, Hq, Mq, D, Hk, L_total, scale, causal, tree_anc, out, out_strides, workspace, workspace_bytes};
  return plain_impl(dtype, c, k, v, k_strides, v_strides, static_cast<hipStream_t>(stream));
}

extern "C" int dspark_verify_attention(const void* q, int64_t B, int64_t Hq, int64_t Mq, int64_t D, const void* k,
                                       const void* v, const int64_t k_strides[3], const int64_t v_strides[3],
                                       int64_t Hk, int64_t L_total, float scale, int causal,
                                       const uint32_t* tree_anc, void* out, void* workspace, size_t workspace_bytes,
                                       dspark_stream stream) {
  const int64_t os[3] = {Hq * Mq * D, Mq * D, D};
  return dspark_verify_attention_typed(DSPARK_DTYPE_BF16, q, B, Hq, Mq, D, k, v, k_strides, v_strides, Hk, L_total,
                                       scale, causal, tree_anc, out, os, workspace, workspace_bytes, stream);
}

extern "C" int dspark_verify_attention_strided(const void* q, int64_t B, int64_t Hq, int64_t Mq, int64_t D,
                                               const void* k, const void* v, const int64_t k_strides[3],
                                               const int64_t v_strides[3], int64_t Hk, int64_t L_total, float scale,
                                               int causal, const uint32_t* tree_anc, void* out,
                                               const int64_t out_strides[3], void* workspace, size_t workspace_bytes,
                                               dspark_stream stream) {
  return dspark_verify_attention_typed(DSPARK_DTYPE_BF16, q, B, Hq, Mq, D, k, v, k_strides, v_strides, Hk, L_total,
                                       scale, causal, tree_anc, out, out_strides, workspace, workspace_bytes, stream);
}

extern "C" int dspark_verify_attention_quantized(
    int dtype, const void* q, int64_t B, int64_t Hq, int64_t Mq, int64_t D, const uint32_t* k_words,
    const void* k_scales, const void* k_biases, const int64_t k_strides[3], const int64_t k_scale_strides[3],
    const uint32_t* v_words, const void* v_scales, const void* v_biases, const int64_t v_strides[3],
    const int64_t v_scale_strides[3], int64_t Hk, int64_t L_total, float scale, int causal, int bits,
    int group_size, void* out, const int64_t out_strides[3], void* workspace, size_t workspace_bytes,
    dspark_stream stream) {
  int st = check_dtype(dtype);
  if (st) return st;
  if (bits != 4 && bits != 8) return fail(DSPARK_ERR_UNSUPPORTED, "verify_attention_quantized: bits=%d (4 or 8)", bits);
  if (group_size != 64)
    return fail(DSPARK_ERR_UNSUPPORTED, "verify_attention_quantized: group_size=%d (64 supported)", group_size);
  if (D != 64 && D != 128 && D != 256)
    return fail(DSPARK_ERR_SHAPE, "verify_attention_quantized: head_dim %ld (64, 128 or 256)", (long)D);
  if (!k_words || !k_scales || !k_biases || !v_words || !v_scales || !v_biases || !k_strides || !v_strides ||
      !k_scale_strides || !v_scale_strides)
    return fail(DSPARK_ERR_ARG, "verify_attention_quantized: null pointer");
  const Common c{q, B, Hq, Mq, D, Hk, L_total, scale, causal, nullptr, out, out_strides, workspace, workspace_bytes};
  AttnArgs a{};
  Plan p{};
  if ((st = prepare(c, a, p))) return st;
  // word rows are read as 16-byte chunks (K) and 8- or 4-byte pieces (V); scales and biases
  // as single values
  if (!aligned(k_words, 16) || !aligned(v_words, 16) || !aligned(k_scales, 2) || !aligned(k_biases, 2) ||
      !aligned(v_scales, 2) || !aligned(v_biases, 2))
    return fail(DSPARK_ERR_ALIGN, "verify_attention_quantized: words must be 16-byte aligned, scales/biases 2-byte");
  if ((st = check_strides(k_strides, 4, "K word")) || (st = check_strides(v_strides, 4, "V word"))) return st;
  if ((st = check_strides(k_scale_strides, 1, "K scale")) || (st = check_strides(v_scale_strides, 1, "V scale")))
    return st;
  a.k = k_words;
  a.v = v_words;
  a.ks = static_cast<const u16*>(k_scales);
  a.kb = static_cast<const u16*>(k_biases);
  a.vs = static_cast<const u16*>(v_scales);
  a.vb = static_cast<const u16*>(v_biases);
  a.ksb = k_strides[0];
  a.ksh = k_strides[1];
  a.kss = k_strides[2];
  a.vsb = v_strides[0];
  a.vsh = v_strides[1];
  a.vss = v_strides[2];
  a.qksb = k_scale_strides[0];
  a.qksh = k_scale_strides[1];
  a.qkss = k_scale_strides[2];
  a.qvsb = v_scale_strides[0];
  a.qvsh = v_scale_strides[1];
  a.qvss = v_scale_strides[2];
  return dispatch(dtype, a, p, B, D, false, bits, static_cast<hipStream_t>(stream));
}
