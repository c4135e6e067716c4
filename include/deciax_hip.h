/*
 * deciax_hip.h — C ABI of the MI355X (gfx950) decision-prefill kernels.
 *
 * Every entry point takes plain device pointers, int64 sizes and strides in
 * elements, fp32 scalars and a `hipStream_t` passed as `void *`. Calls are
 * stream-ordered and asynchronous: nothing allocates device memory and nothing
 * synchronises the host. The caller owns every buffer; entry points that need
 * scratch memory take a caller-provided workspace whose size comes from the
 * matching `*_workspace` query. Calls are thread-safe given distinct output
 * buffers; the library keeps no mutable device state, except the static
 * scratch array of dx_attn_prefill_noalloc.
 *
 * Return value: DX_OK, or a status code; `dx_last_error()` then holds a
 * message for the calling thread. DX_ERR_INVALID and DX_ERR_UNSUPPORTED mean
 * the arguments were rejected before any launch (the Python layer raises
 * ValueError, which the reference's HTTP layer maps to 422 —
 * src/deciax/serve/app.py:260-261); DX_ERR_RUNTIME is a HIP launch/runtime
 * failure (RuntimeError, mapped to 500 at src/deciax/serve/app.py:262-264).
 *
 * Reference interfaces replaced (paths relative to the deciax checkout):
 * each declaration names the function whose contract it takes over.
 */
#ifndef DECIAX_HIP_H
#define DECIAX_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum dx_status {
  DX_OK = 0,
  DX_ERR_INVALID = 1,     /* bad shape, stride, alignment, dtype or null pointer */
  DX_ERR_UNSUPPORTED = 2, /* well-formed but outside what the kernels implement */
  DX_ERR_RUNTIME = 3,     /* HIP runtime or launch failure */
};

enum dx_dtype { DX_BF16 = 0, DX_F32 = 1 };

enum dx_activation { DX_ACT_GELU_TANH = 0, DX_ACT_SILU = 1, DX_ACT_GELU_ERF = 2, DX_ACT_NONE = 3 };

/* Library identification and the calling thread's last error message. */
const char *dx_version(void);
const char *dx_last_error(void);

/* gfx architecture name of `device` (e.g. "gfx950") into buf; DX_OK or
 * DX_ERR_RUNTIME. Used by the impl resolver, which requires gfx950
 * (src/deciax/ops/backend.py:13-18 resolves impls; src/deciax/models/clef/model.py:46-50
 * rejects an impl whose device is missing). */
int dx_device_arch(int device, char *buf, int buf_len);

/* ------------------------------------------------------------------------ */
/* Attention                                                                 */
/* ------------------------------------------------------------------------ */

/* Causal (or bidirectional) GQA prefill attention over variable-length
 * sequences. Replaces `attention` in src/deciax/kernels/attention/blocked.py:9-32
 * (causal GQA, fp32 scores, softmax, P.V) and the masked forms of
 * src/deciax/kernels/attention/reference.py:20-42 and
 * src/deciax/kernels/attention/pallas.py:52-135, extended with Gemma-2 logit
 * soft-capping and the causal sliding window.
 *
 * Sequence s occupies rows [seq_start[s], seq_start[s] + seq_len[s]) of q, k,
 * v and out (device int32 arrays). Row r, head h lives at
 * base + r * row_stride + h * head_dim. The padded [B, S, H, D] layout with a
 * right-padded key mask is the case seq_start[s] = s * S.
 *
 * scores = scale * q.k; if softcap > 0, scores = softcap * tanh(scores / softcap);
 * causal: key j is visible to query i iff j <= i and (window == 0 or j > i - window);
 * bidirectional (causal == 0): iff window == 0 or |i - j| <= window.
 * Softmax in fp32; bf16 P.V with fp32 accumulation (dtype DX_BF16), or fp32
 * throughout (DX_F32). Rows past seq_len are never written.
 *
 * bf16 requires head_dim in {64, 128, 256} and num_q_heads / num_kv_heads in
 * {1, 2, 4}; fp32 requires head_dim in {64, 128, 256}. The bf16 path stages V
 * transposed in `workspace` (size from dx_attn_prefill_workspace with the
 * same num_seqs and max_seq_len; the fp32 path needs none). Every seq_len must
 * be <= max_seq_len (longer ones are cut to max_seq_len). The bf16 kernel
 * addresses one sequence's K rows and one KV head's V^T rows with 32-bit byte
 * offsets: max_seq_len * k_row_stride * 2 and ((head_dim - 1) * vt_ld +
 * max_seq_len rounded up to 64) * 2 must stay below 2^31 (DX_ERR_UNSUPPORTED
 * otherwise; vt_ld is the V^T leading dimension, here max_seq_len rounded up
 * to 64 times num_seqs). At head_dim 64 and 128 the fp32 path reads 32-key
 * blocks with 32-bit byte offsets: k_row_stride and v_row_stride must stay
 * below 2^24 elements there (head_dim 256 has no such limit). */
int dx_attn_prefill(const void *q, const void *k, const void *v, void *out,
                    const int32_t *seq_start, const int32_t *seq_len,
                    int32_t num_seqs, int32_t max_seq_len, int32_t num_q_heads,
                    int32_t num_kv_heads, int32_t head_dim, int64_t q_row_stride,
                    int64_t k_row_stride, int64_t v_row_stride,
                    int64_t out_row_stride, float scale, float softcap,
                    int32_t window, int32_t causal, int32_t dtype,
                    void *workspace, int64_t workspace_bytes, void *stream);

int64_t dx_attn_prefill_workspace(int32_t num_seqs, int32_t max_seq_len,
                                  int32_t num_kv_heads, int32_t head_dim,
                                  int32_t dtype);

/* dx_attn_prefill without a workspace: no counterpart in the reference. For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops that forbid hipMalloc). The bf16 path stages V^T in a static
 * device array of DX_NOALLOC_SCRATCH_BYTES that the library holds on each GPU
 * it runs on until the process ends; calls whose V^T staging,
 * dx_attn_prefill_workspace(...) bytes, exceeds it return DX_ERR_UNSUPPORTED.
 * Nothing is allocated and nothing needs clearing: the transpose writes every
 * V^T column the attention kernel reads. Every call on one GPU shares that
 * GPU's array, so calls that overlap on one GPU (concurrent streams or
 * threads) race; serialise them. Results are identical to dx_attn_prefill's.
 * The array's device address is looked up once per device, by
 * dx_noalloc_init or else by the first call on that device; that lookup is
 * not allowed under graph capture, so a first call on a capturing stream
 * returns DX_ERR_UNSUPPORTED: call dx_noalloc_init on each device before
 * capturing. The address is kept for the life of the process; a device reset
 * is not supported. */
#define DX_NOALLOC_SCRATCH_BYTES (64LL << 20)

/* Look up the current device's static scratch of dx_attn_prefill_noalloc
 * (idempotent; call outside graph capture). No counterpart in the reference:
 * for the callers that cannot allocate. Returns DX_OK or DX_ERR_RUNTIME. */
int dx_noalloc_init(void);

int dx_attn_prefill_noalloc(const void *q, const void *k, const void *v,
                            void *out, const int32_t *seq_start,
                            const int32_t *seq_len, int32_t num_seqs,
                            int32_t max_seq_len, int32_t num_q_heads,
                            int32_t num_kv_heads, int32_t head_dim,
                            int64_t q_row_stride, int64_t k_row_stride,
                            int64_t v_row_stride, int64_t out_row_stride,
                            float scale, float softcap, int32_t window,
                            int32_t causal, int32_t dtype, void *stream);

/* dx_attn_prefill with an arbitrary key mask: key j of sequence s is visible
 * only where key_mask[seq_start[s] + j] != 0 (uint8 per row), in addition to
 * the causal / window rule. Replaces `attention` in
 * src/deciax/kernels/attention/blocked.py:9-32 with its [B, K] key mask
 * (`where(valid, scores, MASK_FILL)`, blocked.py:23-27) and the masked dense
 * attention of src/deciax/kernels/attention/reference.py:11-42. Every query
 * row below seq_len is computed; a row that sees no key is written as zeros
 * (the reference returns the uniform average of all values there, an
 * artefact of the finite MASK_FILL; the Python layer restores it). Workspace
 * size from dx_attn_prefill_masked_workspace (V^T plus the mask as bits). */
int dx_attn_prefill_masked(const void *q, const void *k, const void *v,
                           const uint8_t *key_mask, void *out,
                           const int32_t *seq_start, const int32_t *seq_len,
                           int32_t num_seqs, int32_t max_seq_len,
                           int32_t num_q_heads, int32_t num_kv_heads,
                           int32_t head_dim, int64_t q_row_stride,
                           int64_t k_row_stride, int64_t v_row_stride,
                           int64_t out_row_stride, float scale, float softcap,
                           int32_t window, int32_t causal, int32_t dtype,
                           void *workspace, int64_t workspace_bytes,
                           void *stream);

int64_t dx_attn_prefill_masked_workspace(int32_t num_seqs, int32_t max_seq_len,
                                         int32_t num_kv_heads, int32_t head_dim,
                                         int32_t dtype);

/* Same as dx_attn_prefill (bf16 only), with V already transposed: position
 * p of sequence s, kv head g, dim d at vt[(g * head_dim + d) * vt_ld +
 * vt_start[s] + p]. This is the layout dx_transpose_v writes; the model
 * driver produces it once per layer. Each vt_start[s] is a multiple of 8 and
 * columns [vt_start[s], vt_start[s] + seq_len[s] rounded up to 64) lie inside
 * vt_ld and hold zeros past seq_len[s] (dx_transpose_v writes them). The
 * sequences may be listed in any order and are launched in that order;
 * listing the longest first starts the heaviest work first. */
int dx_attn_prefill_vt(const void *q, const void *k, const void *vt, void *out,
                       const int32_t *seq_start, const int32_t *seq_len,
                       const int32_t *vt_start, int32_t num_seqs,
                       int32_t max_seq_len,
                       int32_t num_q_heads, int32_t num_kv_heads,
                       int32_t head_dim, int64_t q_row_stride,
                       int64_t k_row_stride, int64_t vt_ld,
                       int64_t out_row_stride, float scale, float softcap,
                       int32_t window, int32_t causal, void *stream);

/* V of every sequence (rows seq_start[s] + p, kv head g at g * head_dim) into
 * vt[(g * head_dim + d) * vt_ld + vt_start[s] + p] (bf16), writing zeros for
 * p in [seq_len[s], seq_len[s] rounded up to 64). head_dim % 64 == 0. Layout
 * helper for dx_attn_prefill_vt; no reference counterpart (the reference
 * repeats K/V to every query head instead, blocked.py:12-13). */
int dx_transpose_v(const void *v, void *vt, const int32_t *seq_start,
                   const int32_t *seq_len, const int32_t *vt_start,
                   int32_t num_seqs, int32_t max_seq_len, int32_t num_kv_heads,
                   int32_t head_dim, int64_t v_row_stride, int64_t vt_ld,
                   void *stream);


/* Zero the V^T columns [vt_start[s] + seq_len[s], vt_start[s] + seq_len[s]
 * rounded up to 64) of rows [0, vt_rows), for every sequence s: the tail
 * dx_attn_prefill_vt reads as zero keys' values. dx_transpose_v writes these
 * itself; a caller that fills V^T through dx_qkv_rope calls this once per
 * batch layout (the projection writes only columns below seq_len). Layout
 * helper, no reference counterpart. */
int dx_vt_zero_tails(void *vt, const int32_t *seq_len, const int32_t *vt_start,
                     int32_t num_seqs, int32_t vt_rows, int64_t vt_ld,
                     void *stream);

/* ------------------------------------------------------------------------ */
/* Projections and MLP                                                       */
/* ------------------------------------------------------------------------ */

/* y[m, n] = x[m, k] @ w[n, k]^T with bf16 operands and fp32 accumulation;
 * y is bf16 (rounded once) or fp32. Replaces `linear` in src/deciax/nn.py:11-19
 * (PyTorch [out, in] weight layout, fp32 accumulation) followed by the
 * `.astype(x.dtype)` of `dense`, src/deciax/models/qwen3_5/text.py:21-22.
 * Requires n % 256 == 0, k % 64 == 0, 16-byte aligned rows. */
int dx_linear(const void *x, const void *w, void *y, int64_t m, int64_t n,
              int64_t k, int64_t ldx, int64_t ldw, int64_t ldy,
              int32_t out_dtype, void *stream);

/* Gated projection: for a packed gate|up weight (dx_pack_gate_up layout,
 * [2f, k]), act[m, f] = bf16(bf16(act(bf16(x @ gate^T))) * bf16(x @ up^T)).
 * The rounding points are those of src/deciax/kernels/swiglu.py:100-101
 * (`gu.astype(bf16)`, activation, product rounded to bf16). Requires
 * f % 128 == 0, k % 64 == 0. */
int dx_gated_linear(const void *x, const void *gate_up, void *act, int64_t m,
                    int64_t f, int64_t k, int64_t ldx, int64_t ld_act,
                    int32_t activation, void *stream);

/* Fused QKV projection. With w_qkv the packed [(Hq + 2 Hkv) D, hidden]
 * weight (rows q | k | v), t = bf16(x @ w_qkv^T) (fp32 accumulation), and:
 *   q | k heads (columns [0, (Hq + Hkv) D)): rotate-half RoPE at
 *     positions[row] with the formula and rounding of dx_rope, into
 *     qk[row * ld_qk + col];
 *   v (columns (Hq + Hkv) D + g D + d): into
 *     vt[(g D + d) * vt_ld + vt_col[row]], the V^T layout of
 *     dx_attn_prefill_vt (vt_col[row] = vt_start[s] + p for row
 *     seq_start[s] + p). Columns past each seq_len are not written
 *     (dx_vt_zero_tails).
 * Replaces the packed projection with RoPE in the epilogue of
 * src/deciax/kernels/fused.py:93-99,120-122 (and the per-layer `apply_rope`
 * of src/deciax/nn.py:35-44 on the q / k split of
 * src/deciax/models/qwen3_5/text.py:75-91). Requires (Hq + 2 Hkv) D % 256
 * == 0, hidden % 64 == 0, head_dim in {64, 128, 256}; cos/sin are bf16
 * [max_pos, D / 2]. */
int dx_qkv_rope(const void *x, const void *w_qkv, void *qk, void *vt,
                const int32_t *positions, const int32_t *vt_col,
                const void *cos, const void *sin, int64_t rows,
                int64_t hidden, int32_t num_q_heads, int32_t num_kv_heads,
                int32_t head_dim, int64_t ldx, int64_t ld_qk, int64_t vt_ld,
                int32_t max_pos, void *stream);

/* Pack gate[f, k] and up[f, k] (PyTorch layout) into the [2f, k] layout of
 * dx_gated_linear: rows [128 b, 128 b + 64) are gate rows [64 b, 64 b + 64)
 * and rows [128 b + 64, 128 b + 128) are the matching up rows. Replaces `pack`
 * in src/deciax/kernels/swiglu.py:45-51 (gate|up per intermediate tile). */
int dx_pack_gate_up(const void *gate, const void *up, void *packed, int64_t f,
                    int64_t k, void *stream);

/* Fused RMSNorm + packed projection: h = bf16(x * rsqrt(mean(x^2) + eps) * (1 + norm_w)),
 * optionally h *= row_mask (uint8, nullable), y[rows, n] = bf16(h @ w[n, d]^T).
 * Replaces `norm_project` in src/deciax/kernels/projection.py:13-53 (the
 * packed weight is [n, d] here, K-contiguous for the MFMA operand loads).
 * Workspace holds h; size from dx_norm_project_workspace. */
int dx_norm_project(const void *x, const void *norm_w, const uint8_t *row_mask,
                    const void *w, void *y, int64_t rows, int64_t d, int64_t n,
                    float eps, void *workspace, int64_t workspace_bytes,
                    void *stream);

int64_t dx_norm_project_workspace(int64_t rows, int64_t d);

/* Fused RMSNorm + gated MLP: h = rms(x)(1 + norm_w) in bf16, a = gated(h), y =
 * a @ down[d, f]^T with fp32 accumulation over all of f; y is fp32 (the
 * partial the reference reduces across shards) or bf16. Replaces
 * `fused_mlp_partial` in src/deciax/kernels/swiglu.py:166-208. gate_up is the
 * dx_pack_gate_up layout; down is [d, f] (PyTorch layout). */
int dx_mlp(const void *x, const void *norm_w, const void *gate_up,
           const void *down, void *y, int64_t rows, int64_t d, int64_t f,
           float eps, int32_t activation, int32_t out_dtype, void *workspace,
           int64_t workspace_bytes, void *stream);

int64_t dx_mlp_workspace(int64_t rows, int64_t d, int64_t f);

/* Output projection with the sandwich-norm residual update fused behind it:
 *   y = bf16(a @ w^T)                            ([m, d], d = hidden width)
 *   x = bf16(x + bf16(rms(y) * (1 + post_w)))
 *   if next_w: h = bf16(rms(x) * (1 + next_w))
 * with x, h [m, d] contiguous and y a caller-provided [m, d] scratch (its
 * contents are undefined afterwards). The results are bit-identical to
 * dx_linear followed by dx_add_rmsnorm. Replaces the o / down projection plus
 * the fp32-partial -> bf16 residual step of src/deciax/models/qwen3_5/pallas.py:64-70
 * (post-norm and residual of the Gemma-2 sandwich layer,
 * TF/models/gemma2/modeling_gemma2.py:313-333), in the spirit of the fused
 * o-projection + residual + norm of src/deciax/kernels/fused.py:216-247.
 * The last workgroup to finish a row block's column tiles applies the update to
 * the block's rows; `counters` holds dx_linear_residual_norm_counters(m) int32
 * values that must be zero before the first call and are left zero by every
 * completed call (calls sharing one counter array must not overlap). Requires
 * d % 256 == 0 and d <= 6144, k % 64 == 0, 16-byte aligned operands. */
int dx_linear_residual_norm(const void *a, const void *w, void *y, void *x,
                            const void *post_w, const void *next_w, void *h,
                            int32_t *counters, int64_t m, int64_t d, int64_t k,
                            int64_t lda, int64_t ldw, float eps, void *stream);

int64_t dx_linear_residual_norm_counters(int64_t m);

/* ------------------------------------------------------------------------ */
/* Norms, embedding, RoPE                                                    */
/* ------------------------------------------------------------------------ */

/* y = bf16(x * rsqrt(mean(x^2) + eps) * (1 + w)) per row, fp32 inside.
 * Replaces `rms` in src/deciax/models/qwen3_5/text.py:25-28. */
int dx_rmsnorm(const void *x, const void *w, void *y, int64_t rows, int64_t d,
               int64_t ldx, int64_t ldy, float eps, void *stream);

/* Residual update of one layer half, in place on x:
 *   t = post_w ? bf16(rms(y) * (1 + post_w)) : y;   x = bf16(x + t);
 *   if h: h = bf16(rms(x) * (1 + next_w)).
 * With post_w == NULL this is the pre-norm residual of
 * src/deciax/models/qwen3_5/text.py:96-102 (`x + attn`, then the next rms);
 * with post_w it is the Gemma-2 sandwich (post-norm before the add). */
int dx_add_rmsnorm(const void *y, const void *post_w, void *x,
                   const void *next_w, void *h, int64_t rows, int64_t d,
                   float eps, void *stream);

/* x[t] = bf16(table[ids[t]] * scale) for t < tokens (scale is applied to the
 * bf16 value; pass 1 for a plain gather); if h: h = bf16(rms(x) * (1 + norm_w)).
 * Replaces `_embed` in src/deciax/models/clef/model.py:81,95. Ids outside
 * [0, vocab) are clamped into range by the kernel; the Python layer rejects
 * them before the call. */
int dx_embed(const int32_t *ids, const void *table, void *x, int64_t tokens,
             int64_t d, int64_t vocab, float scale, const void *norm_w,
             void *h, float eps, void *stream);

/* In-place rotate-half RoPE on heads [0, num_heads) of each row:
 * x[j] <- bf16(bf16(x[j] cos[p, j']) + bf16(rot(x)[j] sin[p, j'])), j' = j mod D/2,
 * rot(x)[j] = -x[j + D/2] (j < D/2), x[j - D/2] (j >= D/2), p = positions[row].
 * cos/sin are bf16 tables [max_pos, D/2]. Replaces `apply_rope` in
 * src/deciax/nn.py:35-44 (positions are per row, so packed sequences restart
 * at 0). */
int dx_rope(void *x, const int32_t *positions, const void *cos,
            const void *sin, int64_t rows, int32_t num_heads, int32_t head_dim,
            int64_t row_stride, int32_t max_pos, void *stream);

/* ------------------------------------------------------------------------ */
/* Option readout                                                            */
/* ------------------------------------------------------------------------ */

/* For option o (question q owns options [q_offsets[q], q_offsets[q + 1])):
 *   g = bf16(rms(hidden[opt_pos[o]]) * (1 + norm_w))
 *   z = <g, table[opt_label[o]]>            (fp32 accumulation)
 *   logits[o] = softcap > 0 ? softcap * tanh(z / softcap) : z
 *   probs[o]  = softmax over the options of its question (fp32).
 * Positions are clamped into [0, hidden_rows) and labels into [0, vocab) by
 * the kernel, and each question's range [q_offsets[q], q_offsets[q + 1]) into
 * [0, num_options), so a malformed device array can give wrong answers but
 * never touches memory outside the option arrays; callers validate the
 * offsets first (they must rise from 0 to num_options). num_options above
 * INT32_MAX is refused with DX_ERR_INVALID.
 * Replaces the marker gather + score + per-question softmax of `_scorer`,
 * src/deciax/models/laya/heads.py:74-91 (gather at marker_pos, masked
 * softmax) and the softmax of `decode`, src/deciax/models/clef/input.py:185-194
 * (per-field softmax of the option logits). */
int dx_readout(const void *hidden, const void *norm_w, const void *table,
               const int32_t *opt_pos, const int32_t *opt_label,
               const int32_t *q_offsets, int32_t num_questions,
               int64_t num_options, int64_t hidden_rows, int64_t d,
               int64_t ld_hidden, int64_t vocab, float eps, float softcap,
               float *logits, float *probs, void *stream);

/* ------------------------------------------------------------------------ */
/* Clef joint schema head (fp32), the steps of                               */
/* src/deciax/models/clef/head.py:54-111; deciax_amd/clef_head.py chains    */
/* them in that order. Batched tensors are rows: row b * n + i of a         */
/* [batch, n, d] tensor, each row ld* floats apart.                          */
/* ------------------------------------------------------------------------ */

/* y = (x - mean) * rsqrt(mean((x - mean)^2) + eps) * w + b per row, fp32
 * (b nullable). Replaces `layer_norm` in src/deciax/nn.py:22-29 as the head's
 * `norm` uses it (eps 1e-5, head.py:20-21). */
int dx_layer_norm_f32(const float *x, const float *w, const float *b, float *y,
                      int64_t rows, int64_t d, int64_t ldx, int64_t ldy,
                      float eps, void *stream);

/* y[m, n] = (accumulate ? y[m, n] : 0) + act(x @ w[n, k]^T + bias), fp32,
 * act DX_ACT_NONE or DX_ACT_GELU_ERF (exact GELU, jax.nn.gelu with
 * approximate=False). Replaces `linear` (src/deciax/nn.py:11-19) / `dense`
 * (src/deciax/models/qwen3_5/text.py:21-22) with the head's residual adds
 * (head.py:71-74,92-95) folded in. bias nullable. */
int dx_linear_f32(const float *x, const float *w, const float *bias, float *y,
                  int64_t m, int64_t n, int64_t k, int64_t ldx, int64_t ldw,
                  int64_t ldy, int32_t activation, int32_t accumulate,
                  void *stream);

/* out[b, o] = mean of x[b, s] over s in [spans[b, o, 0], spans[b, o, 1])
 * clipped to [0, seq); 0 for an empty span. Replaces `means`,
 * src/deciax/models/clef/head.py:24-29. */
int dx_span_means_f32(const float *x, const int32_t *spans, float *out,
                      int32_t batch, int32_t seq, int32_t spans_per_row,
                      int64_t d, int64_t ldx, int64_t ld_out, void *stream);

/* Per batch row b, query i, head h: softmax over keys j (masked where
 * key_mask[b, j] == 0, at MASK_FILL) of q_i . k_j / sqrt(head_dim), times v.
 * The attention core of `mha`, src/deciax/models/clef/head.py:41-51, with the
 * masking of src/deciax/kernels/attention/blocked.py:21-28 (non-causal). q,
 * k, v, out hold heads * head_dim columns per row; num_keys <= 32768. */
int dx_mha_f32(const float *q, const float *k, const float *v,
               const uint8_t *key_mask, float *out, int32_t batch,
               int32_t num_queries, int32_t num_keys, int32_t heads,
               int32_t head_dim, int64_t ldq, int64_t ldk, int64_t ldv,
               int64_t ld_out, void *stream);

/* y[b, i] = (accumulate ? y[b, i] : 0) + x[b, index[b, i]] (index clamped to
 * [0, rows_per_batch)). Replaces `gather`, src/deciax/models/clef/head.py:32-33. */
int dx_gather_rows_f32(const float *x, const int32_t *index, float *y,
                       int32_t batch, int32_t rows_per_batch,
                       int32_t picks_per_batch, int64_t d, int64_t ldx,
                       int64_t ldy, int32_t accumulate, void *stream);

/* For field q of batch row b: routing = softmax over options o of
 * options[b, o] . base[b, q] / sqrt(width), restricted to options with
 * option_field[b, o] == q and option_mask[b, o]; summary[b, q] =
 * sum_o routing[o] options[b, o]. Replaces head.py:77-85. Rows are dense
 * ([batch, n, width] contiguous). */
int dx_head_routing_f32(const float *options, const float *base,
                        const int32_t *option_field, const uint8_t *option_mask,
                        float *summary, int32_t batch, int32_t num_options,
                        int32_t num_fields, int32_t width, void *stream);

/* fields[b, q] = base[b, q] + summary_norm[b, q] + global_proj[b] +
 * type_embedding[types[b, q]] (head.py:86-88). Dense rows. */
int dx_head_fields_init_f32(const float *base, const float *summary_norm,
                            const float *global_proj,
                            const float *type_embedding, const int32_t *types,
                            float *fields, int32_t batch, int32_t num_fields,
                            int32_t width, int32_t num_types, void *stream);

/* Per option (b, o) (head.py:98-106): prior = normalize(lexical[b, o]) .
 * normalize(questions[b, f] + global_vector[b]) * prior_scale with
 * f = option_field[b, o]; cosine = normalize(fields[b, o], 1e-8) .
 * normalize(options[b, o], 1e-8); features[b, o] = [f, o, f * o, |f - o|]
 * (4 width columns). fields / options have width columns, questions /
 * global_vector / lexical hidden. Dense rows. */
int dx_head_features_f32(const float *fields, const float *options,
                         const float *questions, const float *global_vector,
                         const float *lexical, const int32_t *option_field,
                         float *features, float *prior, float *cosine,
                         int32_t batch, int32_t num_options, int32_t num_fields,
                         int32_t width, int32_t hidden, float prior_scale,
                         void *stream);

/* logits[i] = option_mask[i] ? prior[i] + gate * (joint_scale * cosine[i] +
 * residual[i]) : -1e9 (head.py:107-111; gate = sigmoid(residual_gate),
 * joint_scale = exp(min(joint_logit_scale, ln 100))). */
int dx_head_combine_f32(const float *prior, const float *cosine,
                        const float *residual, const uint8_t *option_mask,
                        float *logits, int64_t n, float gate,
                        float joint_scale, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* DECIAX_HIP_H */
