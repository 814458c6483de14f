/*
 * dspark.h — C ABI of the MI355X (gfx950) speculative-verify kernels.
 *
 * Three kernel families sit behind this boundary:
 *   1. the small-M affine-quantized matmul (4/8-bit, group 64, M = 1..16 verify rows);
 *   2. multi-row causal GQA verify attention over a strided KV cache (split-KV + combine);
 *   3. MoE top-k routing plus the grouped expert qmm (gather_qmm / SwitchGLU).
 * plus the small elementwise kernels a dense verify forward needs around them.
 *
 * Conventions (every entry point):
 *   - Plain pointers and sizes only; device pointers come from the caller (torch tensors).
 *     No entry point allocates, frees or synchronizes. Work is enqueued on `stream`
 *     (a hipStream_t; NULL = the legacy default stream).
 *   - Returns DSPARK_OK (0) or a negative dspark_status; the message for the last failure
 *     on the calling host thread is in dspark_last_error(). Nothing aborts.
 *   - bf16 tensors are passed as `const void*` / `void*` holding IEEE bfloat16 (uint16 bits).
 *   - Strides are in elements.
 *
 * Each declaration cites the reference interface it replaces (file:line in ARahim3/mlx-dspark
 * v0.20.4, src/mlx_dspark/ unless noted).
 */
#ifndef DSPARK_H_
#define DSPARK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* dspark_stream; /* hipStream_t */

/* Element type of an activation / KV tensor (verify attention). */
enum dspark_dtype {
  DSPARK_DTYPE_BF16 = 0,
  DSPARK_DTYPE_F16 = 1,
  DSPARK_DTYPE_F32 = 2   /* dspark_qmm_dequantize only */
};

enum dspark_status {
  DSPARK_OK = 0,
  DSPARK_ERR_ARG = -1,       /* null pointer or bad enum value */
  DSPARK_ERR_SHAPE = -2,     /* unsupported shape (K % 64, head_dim, M range, ...) */
  DSPARK_ERR_ALIGN = -3,     /* pointer / stride alignment the kernel's vector loads need */
  DSPARK_ERR_WORKSPACE = -4, /* workspace missing or too small */
  DSPARK_ERR_LAUNCH = -5,    /* hipLaunchKernel / hipGetLastError failure */
  DSPARK_ERR_UNSUPPORTED = -6 /* bits / group size / dtype the kernels do not implement */
};

/* Library version string and the gfx target the code objects were built for. */
const char* dspark_version(void);
/* Message of the last failed call on this host thread ("" if none). */
const char* dspark_last_error(void);

/* ------------------------------------------------------------------ small-M quantized matmul */

/*
 * y[m, n] = sum_g ( scale[n,g] * sum_{j in g} q[n,j] * x[m,j]  +  bias[n,g] * sum_{j in g} x[m,j] )
 * fp32 accumulation, bf16 output, for M = 1..16 rows (M > 16 is served in 16-row tiles).
 *
 * x       bf16 [M, K], row stride ldx (ldx % 8 == 0, 16-byte aligned base)
 * w       uint32 [N, K*bits/32] row-major, packed low bits first: element j of row n is field
 *         (j % (32/bits)) of word j / (32/bits)      (16-byte aligned base)
 * scales  bf16 [N, K/group_size]
 * biases  bf16 [N, K/group_size]
 * y       bf16 [M, N], row stride ldy
 * bits    4 or 8; group_size 64; K % 64 == 0, K <= 32768.
 * workspace  device buffer of at least dspark_qmm_affine_workspace(...) bytes, 256-byte
 *            aligned. Its first 256 KiB (arrival counters, the same bytes for every shape)
 *            must be ZERO before the first call that uses it; every call leaves them zero
 *            again, so one workspace serves calls of any shapes. NULL is allowed when the size
 *            is 0. Calls sharing one workspace must be ordered on one stream.
 *
 * Replaces skinny_qmm.qmm(x2, weight, scales, biases, bits) (skinny_qmm.py:239-246), i.e. the
 * `dspark_skinny_qmm` Metal kernel (skinny_qmm.py:56-171) and, outside its window, the stock
 * mx.quantized_matmul reached through QuantizedLinear.__call__ (small_m_qmm.py:53, :71-80).
 * Each output is computed independently of the other rows (row-count invariant, as the
 * reference tests at tests/test_small_m_qmm.py:107-119).
 */
int dspark_qmm_affine(const void* x, int64_t ldx, int64_t M, int64_t K,
                      const uint32_t* w, const void* scales, const void* biases,
                      int64_t N, int bits, int group_size,
                      void* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                      dspark_stream stream);

/* Workspace bytes dspark_qmm_affine needs for this shape (0 = none). */
size_t dspark_qmm_affine_workspace(int64_t M, int64_t K, int64_t N, int bits, int group_size);

/* Clears the split-K arrival counters of a qmm workspace (its first 256 KiB, or all of it when
 * smaller) with a fill kernel on `stream`, so the call may sit in a captured graph. Every qmm
 * call that completes leaves its counters at zero; this restores the invariant after a call
 * that did not complete, or for a workspace of unknown contents. No counterpart in the
 * reference, whose Metal kernel keeps no state between launches (skinny_qmm.py:56-159). */
int dspark_qmm_workspace_reset(void* workspace, size_t workspace_bytes, dspark_stream stream);

/* 0 if dspark_qmm_affine accepts this shape, else the dspark_status it would return.
 * Mirrors skinny_qmm.fits (skinny_qmm.py:174-181) without launching. */
int dspark_qmm_affine_supported(int64_t M, int64_t K, int64_t N, int bits, int group_size);

/* Launch geometry dspark_qmm_affine uses for this shape (host-only query, no GPU work):
 * out[0] K slices S, out[1] groups per slice the kernel is built for, out[2] 64-row strips,
 * out[3] workgroups. Mirrors skinny_qmm.plan / geometry (skinny_qmm.py:190-237), whose
 * (template, grid, threadgroup) the Python layer caches per module. Returns a dspark_status. */
int dspark_qmm_affine_plan(int64_t M, int64_t K, int64_t N, int bits, int group_size, int32_t out[4]);

/*
 * dspark_qmm_affine without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference. Same arguments (minus the workspace), kernels and results,
 * bit for bit, as dspark_qmm_affine. The split-K counters and partials live in a device array
 * inside the library, one per GPU, held until the process ends: 256 KiB of counters plus
 * 32 MiB of partials. A shape whose dspark_qmm_affine_workspace exceeds that is refused with
 * DSPARK_ERR_WORKSPACE: at M <= 16 that is ceil(N / 64) * S > 8192, with S the K slices
 * dspark_qmm_affine_plan reports (every projection of a hidden-5120, intermediate-25600 layer
 * fits; a 151936-row vocabulary head at K = 5120 does not). Nothing is
 * allocated: the first call on a device looks up the array's address and clears its
 * counters on `stream`. Every call on one GPU shares the array, so calls that overlap in time
 * on one GPU (other streams, other host threads) race; order them on one stream.
 */
int dspark_qmm_affine_noalloc(const void* x, int64_t ldx, int64_t M, int64_t K,
                              const uint32_t* w, const void* scales, const void* biases,
                              int64_t N, int bits, int group_size,
                              void* y, int64_t ldy, dspark_stream stream);

/* Clear the split-K arrival counters of dspark_qmm_affine_noalloc's array on the current GPU
 * (a fill kernel on `stream`, no allocation). Every completed call leaves them at zero; a call
 * that did not complete (a launch error or an aborted stream) can leave them stale, and every
 * later call on that GPU would then mis-sum. No counterpart in the reference: for the same
 * callers that cannot allocate, as the recovery step after such a failure. */
int dspark_qmm_noalloc_reset(dspark_stream stream);

/* Device address and size of dspark_qmm_affine_noalloc's array on the current GPU (looked up
 * and its counters cleared on first use, as the entry point does). No counterpart in the
 * reference: diagnostics and tests of the no-allocation entry point. */
int dspark_qmm_noalloc_scratch(void** ptr, size_t* bytes);

/*
 * Dequantize once, for the prefill wide path: out[n, j] = (scale[n, j/64] * q[n, j]) + bias[n, j/64]
 * for the reference-layout matrix of dspark_qmm_affine, each operation an fp32 operation rounded
 * to nearest (no fma), then stored as `dtype` (fp32, or rounded to bf16 / fp16). scales and
 * biases are `scale_dtype` (bf16, fp16 or fp32). out has row stride ldo (ldo % 8 == 0, 16-byte
 * aligned). A GEMM over `out` then serves wide (prefill) forwards. Replaces the
 * mx.dequantize(w, scales, biases) of the reference's wide path (wide_gemm.py:173-232).
 */
int dspark_qmm_dequantize(const uint32_t* w, const void* scales, const void* biases, int scale_dtype, int64_t N,
                          int64_t K, int bits, int group_size, int dtype, void* out, int64_t ldo,
                          dspark_stream stream);

/*
 * Streaming-read bandwidth probe: reads `bytes` (a positive multiple of 16, 16-byte aligned) once
 * with 16-byte non-temporal loads; sink[0] is written only in the (practically impossible) case
 * that the XOR of all words equals a sentinel. Timed by the caller, it gives the measured HBM
 * read rate the roofline fractions are also quoted against. Replaces the reference's
 * bandwidth probe (calibrate.py:871-894, an fp16 matvec over 512 MB).
 */
int dspark_stream_read(const void* p, size_t bytes, uint32_t* sink, dspark_stream stream);

/* One launch over up to DSPARK_QMM_MAX_PROBLEMS matrices that share bits, group size, M and K
 * (q/k/v of an attention block, gate/up of an MLP). Each problem has its own x, w, scales,
 * biases and y. Replaces the per-projection QuantizedLinear calls of one decoder layer
 * (target.py:208-221 -> mlx-lm DecoderLayer), which the reference launches one by one.
 * Results equal separate dspark_qmm_affine calls bit for bit, with one qualification: an 8-bit
 * [4096, 4096] matrix alone takes the whole-K kernel, whose per-group sums of x come from an MFMA
 * against ones, while in a launch with other matrices it takes split-K, whose sums are lane
 * sums. The two agree whenever those fp32 sums are exact (bf16 x of ordinary range); with x
 * spanning many binades in one group of 64 they can differ by an fp32 rounding of the bias
 * term, well inside the qmm tolerance. */
#define DSPARK_QMM_MAX_PROBLEMS 4
typedef struct dspark_qmm_problem {
  const void* x;
  int64_t ldx;
  const uint32_t* w;
  const void* scales;
  const void* biases;
  void* y;
  int64_t ldy;
  int64_t N;
  int64_t K;
} dspark_qmm_problem;

int dspark_qmm_affine_multi(const dspark_qmm_problem* problems, int count, int64_t M, int bits,
                            int group_size, void* workspace, size_t workspace_bytes,
                            dspark_stream stream);

size_t dspark_qmm_affine_multi_workspace(const dspark_qmm_problem* problems, int count, int64_t M,
                                         int bits, int group_size);

/*
 * MI355X packed form of one quantized matrix. This build's own format, with no counterpart in
 * the reference (whose checkpoints keep the layout above); callers that hold a matrix for many
 * calls (a loaded model) pack it once. Weights go in 16-row tiles in the lane order of the MFMA
 * loop, one 1 KB read per wave per group (8-bit) or group pair (4-bit), and scales/biases in
 * 16-row x 8-group tiles. Every product of dspark_qmm_packed_multi equals that of
 * dspark_qmm_affine_multi on the reference layout bit for bit.
 * Requires K % 512 == 0 (K <= 32768), bits 4 or 8, group_size 64; any N (rows are padded to
 * 16 with zeros).
 */
/* Bytes of the packed form (0 = shape not supported). */
size_t dspark_qmm_packed_bytes(int64_t N, int64_t K, int bits, int group_size);

/* Writes the packed form of (w, scales, biases) — the reference layout of dspark_qmm_affine,
 * all 16-byte aligned — into `packed` (16-byte aligned, >= dspark_qmm_packed_bytes). */
int dspark_qmm_pack(const uint32_t* w, const void* scales, const void* biases, int64_t N, int64_t K, int bits,
                    int group_size, void* packed, size_t packed_bytes, dspark_stream stream);

typedef struct dspark_qmm_packed_problem {
  const void* x;
  int64_t ldx;
  const void* packed;  /* dspark_qmm_pack output for [N, K] */
  void* y;
  int64_t ldy;
  int64_t N;
  int64_t K;
} dspark_qmm_packed_problem;

/* dspark_qmm_affine_multi over packed matrices (same x / y / M / workspace rules). */
int dspark_qmm_packed_multi(const dspark_qmm_packed_problem* problems, int count, int64_t M, int bits,
                            int group_size, void* workspace, size_t workspace_bytes, dspark_stream stream);

size_t dspark_qmm_packed_multi_workspace(const dspark_qmm_packed_problem* problems, int count, int64_t M,
                                         int bits, int group_size);

/* Which kernel dspark_qmm_packed_multi runs for these problems (host-only query, no GPU work):
 * out[0] 0 = split-K, 1 = one 16-row tile per workgroup over all of K, 2 = one workgroup per
 * CU (one x for every problem; K = 4096 with 3..6 row tiles per CU, or 2 at 8 bits, over all of
 * K; K = 12288 with 4 row tiles per CU over a quarter of K each); out[1] the K slices S whose
 * association the result follows (every kernel gives the split-K plan's bits for the same S,
 * the second one where the group sums of x are exact in fp32); out[2] row tiles per workgroup
 * (kind 2, else 0); out[3] workgroups; out[4] workgroups per row tile along K (kind 2, else 0).
 * Mirrors skinny_qmm.plan (skinny_qmm.py:190-237) for the packed form. Returns a
 * dspark_status. */
int dspark_qmm_packed_multi_plan(const dspark_qmm_packed_problem* problems, int count, int64_t M, int bits,
                                 int group_size, int32_t out[4]);

/*
 * Fused gate / up / SwiGLU for the MLP of a verify forward (no counterpart in the reference,
 * which runs the two quantized matmuls and silu(gate) * up as three ops (target.py:187-221 ->
 * mlx-lm's MLP); this replaces that sequence for packed weights):
 *   h[m, n] = bf16( bf16(g * bf16(sigmoid(g))) * u ),  g = bf16(x W_gate^T)[m, n],
 *                                                     u = bf16(x W_up^T)[m, n]
 * bit for bit what dspark_qmm_packed_multi over the two matrices followed by dspark_swiglu
 * gives when N is a multiple of 64 (same K slices; otherwise within the qmm tolerance).
 * dspark_qmm_pack_swiglu writes the pair form: the packed layout of 2 * ceil(N / 16) row
 * tiles, gate tile t then up tile t (K % 512 == 0); dspark_qmm_swiglu_packed_bytes sizes it.
 * x bf16 [M, K] (ldx), h bf16 [M, N] (ldh); workspace as for dspark_qmm_packed_multi.
 */
size_t dspark_qmm_swiglu_packed_bytes(int64_t N, int64_t K, int bits, int group_size);

int dspark_qmm_pack_swiglu(const uint32_t* gate_w, const void* gate_scales, const void* gate_biases,
                           const uint32_t* up_w, const void* up_scales, const void* up_biases, int64_t N, int64_t K,
                           int bits, int group_size, void* packed, size_t packed_bytes, dspark_stream stream);

int dspark_qmm_swiglu_packed(const void* x, int64_t ldx, const void* packed, void* h, int64_t ldh, int64_t N,
                             int64_t K, int64_t M, int bits, int group_size, void* workspace,
                             size_t workspace_bytes, dspark_stream stream);

size_t dspark_qmm_swiglu_packed_workspace(int64_t N, int64_t K, int64_t M, int bits, int group_size);

/* ------------------------------------------------------------------ verify attention */

/*
 * out = softmax(scale * q k^T + mask) v for a few verify rows over a long KV cache.
 *
 * q        bf16 [B, Hq, Mq, D] contiguous
 * k, v     bf16 [B, Hk, L_total, D] views with element strides k_strides = {batch, head, seq}
 *          (the last dim must be contiguous; the cache capacity may exceed L_total)
 * L_total  keys in the cache including the Mq rows being verified (already written)
 * causal   1: row i (0-based within the Mq block) sees keys 0 .. L_total - Mq + i
 *          0: every row sees every key
 * tree_anc nullable uint32 [Mq]: tree-verify visibility — every key < L_total - Mq is seen;
 *          key L_total - Mq + j is seen by row i iff bit j of tree_anc[i] is set (Mq <= 32).
 *          Overrides `causal`.
 * out      bf16 [B, Hq, Mq, D] contiguous
 * workspace  device buffer of at least dspark_verify_attention_workspace(...) bytes
 *            (fp32 split-KV partials); may be NULL when that size is 0.
 * D % 8 == 0, 8 <= D <= 256 (the reference's rule, multirow_attn.py:200; kernel instances at
 * 64, 128 and 256 columns, a smaller head dim's missing columns zero on chip and never read or
 * written in memory); Hq % Hk == 0; gqa * Mq <= 256.
 *
 * Replaces multirow_attn.multirow_sdpa(q, k, v, scale=, causal=, tree_anc=)
 * (multirow_attn.py:223-259): the dspark_mra_p1 / _p1_tree / _p2 Metal kernels
 * (multirow_attn.py:52-197).
 */
int dspark_verify_attention(const void* q, int64_t B, int64_t Hq, int64_t Mq, int64_t D,
                            const void* k, const void* v, const int64_t k_strides[3],
                            const int64_t v_strides[3], int64_t Hk, int64_t L_total, float scale,
                            int causal, const uint32_t* tree_anc, void* out, void* workspace,
                            size_t workspace_bytes, dspark_stream stream);

/* Workspace bytes dspark_verify_attention needs for this shape (0 = none). */
size_t dspark_verify_attention_workspace(int64_t B, int64_t Hq, int64_t Hk, int64_t Mq, int64_t D,
                                         int64_t L_total);

/* Number of split-KV blocks the launch plan uses for this shape (for tests and reports).
 * Mirrors multirow_attn.plan (multirow_attn.py:204-220) in spirit; the geometry is MI355X's. */
/* dspark_verify_attention with the output written through element strides
 * out_strides = {batch, query head, position} (head_dim contiguous; each a multiple of 4), so a
 * verify forward can write [B, Mq, Hq*D] rows directly as the o_proj input
 * ({Mq*Hq*D, D, Hq*D}). Same kernels and semantics as dspark_verify_attention. */
int dspark_verify_attention_strided(const void* q, int64_t B, int64_t Hq, int64_t Mq, int64_t D,
                                    const void* k, const void* v, const int64_t k_strides[3],
                                    const int64_t v_strides[3], int64_t Hk, int64_t L_total, float scale,
                                    int causal, const uint32_t* tree_anc, void* out,
                                    const int64_t out_strides[3], void* workspace, size_t workspace_bytes,
                                    dspark_stream stream);

/* dspark_verify_attention_strided for bf16 (dtype DSPARK_DTYPE_BF16) or fp16
 * (DSPARK_DTYPE_F16) q, K, V and output: the reference serves both (multirow_attn.py:294-307,
 * its kernel templated on the input type, :180-197). P is rounded to the input type for P.V;
 * accumulation is fp32 either way. */
int dspark_verify_attention_typed(int dtype, const void* q, int64_t B, int64_t Hq, int64_t Mq, int64_t D,
                                  const void* k, const void* v, const int64_t k_strides[3],
                                  const int64_t v_strides[3], int64_t Hk, int64_t L_total, float scale,
                                  int causal, const uint32_t* tree_anc, void* out,
                                  const int64_t out_strides[3], void* workspace, size_t workspace_bytes,
                                  dspark_stream stream);

/*
 * Verify attention over a quantized KV cache: the state of mlx-lm's QuantizedKVCache, which
 * the reference's targets build when kv_bits is set (target.py:166-184; its shape is read back
 * at calibrate.py:225-238). K and V are each
 *   words   uint32 [B, Hk, L, D*bits/32]: fields of `bits` (4 or 8) along D, low bits first
 *           (the affine layout of dspark_qmm_affine); strides k_strides / v_strides in words
 *           (each a multiple of 4; the last dim contiguous);
 *   scales, biases  [B, Hk, L, D/group_size] of the q dtype, one pair per 64 values of a row
 *           (strides k_scale_strides / v_scale_strides in elements, shared by scales and biases).
 * Each value is scale * field + bias (group_size 64). The reference's own multirow kernel does
 * not read this format (quantized caches fall through to mlx-lm's quantized SDPA,
 * multirow_attn.py:288-299); this entry point serves that fall-through on the same kernel in the
 * factored form of the quantized matmul: the integer fields go through the MFMA exactly, and the
 * per-(key, group) scales and biases are applied in fp32 (scores: scale_k * (f . q) + bias_k *
 * sum q; output: (p * scale_v) . f_v + sum p * bias_v). Mask, softmax and split-KV combine are
 * those of dspark_verify_attention_typed. D in {64, 128, 256}. No tree mask.
 */
int dspark_verify_attention_quantized(int dtype, const void* q, int64_t B, int64_t Hq, int64_t Mq, int64_t D,
                                      const uint32_t* k_words, const void* k_scales, const void* k_biases,
                                      const int64_t k_strides[3], const int64_t k_scale_strides[3],
                                      const uint32_t* v_words, const void* v_scales, const void* v_biases,
                                      const int64_t v_strides[3], const int64_t v_scale_strides[3], int64_t Hk,
                                      int64_t L_total, float scale, int causal, int bits, int group_size, void* out,
                                      const int64_t out_strides[3], void* workspace, size_t workspace_bytes,
                                      dspark_stream stream);

/* Launch geometry of dspark_verify_attention (host-only query): out[0] rows R = gqa * Mq,
 * out[1] padded rows RP, out[2] row groups NRG, out[3] keys per block CHUNK, out[4] key
 * blocks NB, out[5] pass-1 workgroups. Mirrors multirow_attn.plan (multirow_attn.py:204-220).
 * Returns a dspark_status. */
int dspark_verify_attention_plan(int64_t B, int64_t Hq, int64_t Hk, int64_t Mq, int64_t D, int64_t L_total,
                                 int32_t out[6]);

int64_t dspark_verify_attention_blocks(int64_t B, int64_t Hq, int64_t Hk, int64_t Mq, int64_t D,
                                       int64_t L_total);

/* ------------------------------------------------------------------ MoE */

/*
 * Router: gates = softmax(logits) computed in fp32 and rounded to bf16 (mlx
 * softmax(precise=True) keeps the input dtype); top-k by (gate desc, expert id asc);
 * scores = the selected gates, renormalized to sum 1 when renorm != 0 (norm_topk_prob),
 * rounded to bf16. Outputs:
 *   inds    int32 [M, k]    selected experts, in selection order (largest gate first)
 *   scores  bf16  [M, k]
 *   expert_offsets  int32 [E + 1] (nullable): bucket boundaries of the (token, slot) pairs
 *                   sorted by expert, then by pair id t*k + j
 *   sorted_pairs    int32 [M * k] (nullable): pair ids t*k + j in that sorted order
 *   pair_pos        int32 [M * k] (nullable): inverse of sorted_pairs
 * Requires 1 <= k <= 32, k <= E <= 1024.
 * Replaces mlx-lm's SparseMoeBlock routing (softmax → argpartition → take_along_axis →
 * renormalize; mlx-lm qwen3_moe, third-party, not vendored in the reference) and SwitchGLU's
 * sort of the (token, expert) pairs (mlx-lm switch_layers).
 */
int dspark_moe_route_topk(const void* logits, int64_t M, int64_t E, int64_t k, int renorm,
                          int32_t* inds, void* scores, int32_t* expert_offsets,
                          int32_t* sorted_pairs, int32_t* pair_pos, dspark_stream stream);

/*
 * Grouped affine qmm over expert-sorted rows (mx.gather_qmm(x, w, s, b, rhs_indices=...,
 * transpose=True, sorted_indices=True)):
 *   y[p, :] = x[row_index[p], :] @ dequant(w[e])^T   for expert_offsets[e] <= p < expert_offsets[e+1]
 * x       bf16 [*, K] (row stride ldx); row_index int32 [P] (nullable = identity)
 * w       uint32 [E, N, K*bits/32]; scales/biases bf16 [E, N, K/64]
 * y       bf16 [P, N] (row stride ldy), P = expert_offsets[E]
 * Rows are streamed per expert, so each selected expert's weights are read once.
 */
int dspark_gather_qmm(const void* x, int64_t ldx, int64_t K, const int32_t* row_index,
                      const int32_t* expert_offsets, int64_t E, int64_t P_max,
                      const uint32_t* w, const void* scales, const void* biases, int64_t N,
                      int bits, int group_size, void* y, int64_t ldy, dspark_stream stream);

/*
 * The whole routed-expert MLP of one MoE block for M tokens (SwitchGLU + score combine):
 *   route (dspark_moe_route_topk) → gate/up gather_qmm with h = silu(gate) * up (bf16)
 *   → down gather_qmm → out[t] = sum_j bf16(scores[t,j] * y[t,j]) (fp32 sum, slot order).
 * x bf16 [M, H]; logits bf16 [M, E]; w_gate/w_up uint32 [E, I, H*bits/32];
 * w_down uint32 [E, H, I*bits/32]; s_*, b_* bf16 [E, rows, cols/64]; out bf16 [M, H].
 * inds/scores (outputs, nullable) receive the routing.
 * workspace >= dspark_moe_workspace(M, H, I, E, k) bytes.
 * Replaces mlx-lm SwitchGLU.__call__ / QuantizedSwitchLinear (third-party; §3.3 of the
 * reference's call stack) for the A3B targets the reference routes (load.py:111-123).
 */
int dspark_moe_switch_glu(const void* x, const void* logits, int64_t M, int64_t H, int64_t I,
                          int64_t E, int64_t k, int renorm,
                          const uint32_t* w_gate, const void* s_gate, const void* b_gate,
                          const uint32_t* w_up, const void* s_up, const void* b_up,
                          const uint32_t* w_down, const void* s_down, const void* b_down,
                          int bits, int group_size, void* out, int32_t* inds, void* scores,
                          void* workspace, size_t workspace_bytes, dspark_stream stream);

size_t dspark_moe_workspace(int64_t M, int64_t H, int64_t I, int64_t E, int64_t k);

/*
 * Packed expert weights (no counterpart in the reference, whose experts stay in mlx-lm's
 * QuantizedSwitchLinear layout): each expert's [N, K] weights in 16-row tiles in the MFMA lane
 * order, one contiguous 1 KB read per wave per group (8-bit) or group pair (4-bit), experts one
 * after another (the same bytes as [E, N, K*bits/32]). Scales and biases keep their [E, N, K/64]
 * layout. Requires N % 16 == 0 and K % 128 == 0. dspark_moe_packed_bytes sizes the buffer (0 =
 * shape not supported); dspark_moe_pack writes it from the row-major weights (16-byte aligned).
 */
size_t dspark_moe_packed_bytes(int64_t E, int64_t N, int64_t K, int bits, int group_size);

int dspark_moe_pack(const uint32_t* w, int64_t E, int64_t N, int64_t K, int bits, int group_size, void* packed,
                    size_t packed_bytes, dspark_stream stream);

/* dspark_moe_switch_glu with w_gate / w_up / w_down in dspark_moe_pack's form (H and I multiples
 * of 16, K % 128 == 0 for both projections, 16-byte aligned scales and biases): the same
 * results, bit for bit. */
int dspark_moe_switch_glu_packed(const void* x, const void* logits, int64_t M, int64_t H, int64_t I, int64_t E,
                                 int64_t k, int renorm, const void* w_gate, const void* s_gate, const void* b_gate,
                                 const void* w_up, const void* s_up, const void* b_up, const void* w_down,
                                 const void* s_down, const void* b_down, int bits, int group_size, void* out,
                                 int32_t* inds, void* scores, void* workspace, size_t workspace_bytes,
                                 dspark_stream stream);

/* Which expert kernel dspark_moe_switch_glu_packed launches for a shape (no counterpart in the
 * reference; for tests and profiles): out[0] for gate/up, out[1] for down, 1 = one workgroup per
 * CU over a contiguous range of (live expert, 16-column strip) units (M <= 16 tokens, E <= 256,
 * M * k <= 512, gate/up K = H in {512, 2048}, down K = I in {256, 768}), 0 = one workgroup per
 * (expert, strip). */
int dspark_moe_packed_plan(int64_t M, int64_t H, int64_t I, int64_t E, int64_t k, int bits, int32_t* out);

/* ------------------------------------------------------------------ verify-forward layer kernels */

/*
 * The elementwise/normalisation steps of a dense verify forward around the qmm and attention
 * launches: mlx-lm's qwen3-style DecoderLayer as the reference runs it (target.py:187-221
 * _body_mlxlm -> layer(h, mask, cache), third-party), with mlx's bf16 op rounding.
 */

/* y[m] = bf16(bf16(h * rsqrt(mean(h^2) + eps)) * w) with h = x[m] (r NULL) or
 * h = bf16(x[m] + r[m]) (residual add; h is also written to h_out when non-NULL).
 * x, r, h_out, y, w bf16; rows 16-byte aligned, strides % 8 == 0, H % 8 == 0. Replaces
 * nn.RMSNorm (mx.fast.rms_norm) and the residual `h = x + r` of the decoder layer. */
int dspark_rmsnorm(const void* x, int64_t ldx, const void* r, int64_t ldr, const void* w, int64_t M, int64_t H,
                   float eps, void* h_out, int64_t ldh, void* y, int64_t ldy, dspark_stream stream);

/* Per verify row m and head: q/k RMSNorm over head_dim (weights q_norm_w / k_norm_w), RoPE
 * (non-traditional: pairs (i, i + D/2), angle (pos0 + m) * rope_base^(-2i/D), fp32), then
 *   q_out [Hq, M, D] (contiguous; the attention q input, batch 1),
 *   k_cache[h * k_cache_strides[0] + (pos0 + m) * k_cache_strides[1] + d] = rotated k,
 *   v_cache[...same with v strides...] = v.
 * q [M, ldq >= Hq*D], k/v [M, ld >= Hk*D] are the q/k/v projections; D % 8 == 0, D <= 256.
 * Replaces Attention.__call__'s q_norm/k_norm, rope(offset=cache.offset) and
 * cache.update_and_fetch (mlx-lm qwen3; the cache write of batch_engine.py:193-219). */
int dspark_qk_norm_rope_kv(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                           int64_t M, int64_t Hq, int64_t Hk, int64_t D, const void* q_norm_w,
                           const void* k_norm_w, float eps, float rope_base, int64_t pos0, void* q_out,
                           void* k_cache, const int64_t k_cache_strides[2], void* v_cache,
                           const int64_t v_cache_strides[2], dspark_stream stream);

/* dspark_qk_norm_rope_kv for a quantized KV cache (mlx-lm QuantizedKVCache, which the
 * reference's dense targets build for every layer when kv_bits is set, target.py:166-184): the
 * same q output, and the rotated k row and the v row (each as the bf16 values the plain entry
 * point would write) quantized into the cache row at position pos0 + m: `bits`-bit fields
 * along D (low bits first) in k_words / v_words [Hk, capacity, D*bits/32] (strides (head,
 * position) in words), one bf16 scale and bias per 64 values in k_scales / k_biases and
 * v_scales / v_biases [Hk, capacity, D/64] (strides (head, position) in elements). Per group:
 * scale = bf16((max - min) / (2^bits - 1)), bias = bf16(min), field = round-half-even((x - bias)
 * / scale) clamped to the range (scale 0 divides by 1), each step one fp32 operation: the rule
 * of this build's quantizer (dspark_rocm.quant.quantize_rows; mx.quantize's own choice is not
 * reproducible without MLX). Replaces QuantizedKVCache.update_and_fetch's mx.quantize of the
 * new rows. D in {64, 128, 256}, bits 4 or 8, group_size 64. */
int dspark_qk_norm_rope_kv_quantized(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                                     int64_t ldv, int64_t M, int64_t Hq, int64_t Hk, int64_t D,
                                     const void* q_norm_w, const void* k_norm_w, float eps, float rope_base,
                                     int64_t pos0, void* q_out, uint32_t* k_words, void* k_scales,
                                     void* k_biases, const int64_t k_strides[2], const int64_t k_scale_strides[2],
                                     uint32_t* v_words, void* v_scales, void* v_biases, const int64_t v_strides[2],
                                     const int64_t v_scale_strides[2], int bits, int group_size,
                                     dspark_stream stream);

/* h = bf16(bf16(g * bf16(sigmoid(g))) * u) over [M, N] (N % 8 == 0): MLP's silu(gate) * up. */
int dspark_swiglu(const void* g, int64_t ldg, const void* u, int64_t ldu, int64_t M, int64_t N, void* h,
                  int64_t ldh, dspark_stream stream);

/* out[m] = argmax over V of logits[m] (bf16; first index of the maximum). Replaces
 * mx.argmax(v_logits[0], -1) of the verify loop (generate.py:1548). */
int dspark_argmax_rows(const void* logits, int64_t ld, int64_t M, int64_t V, int32_t* out, dspark_stream stream);

/* n_accepted[0] = sum(cumprod(draft == target_tokens[:m])) (generate.py:1549-1550): the
 * accepted draft prefix length; device-side so the round needs one host read. */
int dspark_greedy_accept(const int32_t* draft, int64_t m, const int32_t* target_tokens, int32_t* n_accepted,
                         dspark_stream stream);

/* The greedy verify round's device part in one launch: target_tokens[m] = argmax over V of
 * logits[m] for m < M (exactly dspark_argmax_rows: first index of the maximum, NaN never chosen)
 * and n_accepted[0] = the number of leading i < m_draft with draft[i] == target_tokens[i]
 * (exactly dspark_greedy_accept). Each row is scanned by ceil(V / 16384) workgroups; the last
 * to finish reduces them and counts (V <= 33554432, m_draft <= 1024). Replaces
 * tt = mx.argmax(v_logits[0], -1) and
 * n = sum(cumprod(draft == tt)) of the verify loop (generate.py:1544-1555).
 * workspace >= dspark_argmax_accept_workspace(M, V) bytes, 256-byte aligned, its first 256 bytes
 * zero before the first call (an arrival counter; every call leaves it zero). */
size_t dspark_argmax_accept_workspace(int64_t M, int64_t V);

int dspark_argmax_accept(const void* logits, int64_t ld, int64_t M, int64_t V, const int32_t* draft, int64_t m_draft,
                         int32_t* target_tokens, int32_t* n_accepted, void* workspace, size_t workspace_bytes,
                         dspark_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* DSPARK_H_ */
