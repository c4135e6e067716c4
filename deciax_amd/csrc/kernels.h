// Internal launchers shared between the kernel files and the C ABI layer.
// Shapes are validated by the ABI layer before any of these is called.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// GEMM operands are addressed through buffer resources based at the tile origin with 32-bit byte
// offsets: 256 rows of a leading dimension up to this many elements stay below 2^31 bytes.
#define DX_MAX_LD (1 << 22)

hipError_t dx_gemm_bf16(const uint16_t *A, const uint16_t *B, uint16_t *C, long M, long N, long K, long lda,
                        long ldb, long ldc, hipStream_t s);
hipError_t dx_gemm_f32(const uint16_t *A, const uint16_t *B, float *C, long M, long N, long K, long lda, long ldb,
                       long ldc, hipStream_t s);
hipError_t dx_gemm_gated(const uint16_t *A, const uint16_t *B, uint16_t *C, long M, long F, long K, long lda,
                         long ldc, int act, hipStream_t s);

// QKV epilogue parameters: columns [0, qk_cols) of the packed projection are q | k heads of size d
// (RoPE with bf16 cos/sin tables [max_pos, d / 2] at pos[row]); columns [qk_cols, N) are v, written to
// vt[(col - qk_cols) * vt_ld + vt_col[row]].
struct QkvEpilogue {
  uint16_t *vt = nullptr;
  const int32_t *vt_col = nullptr;
  const int32_t *pos = nullptr;
  const uint16_t *cos = nullptr, *sin = nullptr;
  long vt_ld = 0;
  int qk_cols = 0, d = 0, max_pos = 0;
};
hipError_t dx_gemm_qkv(const uint16_t *A, const uint16_t *B, uint16_t *QK, long M, long N, long K, long lda, long ldb,
                       long ld_qk, const QkvEpilogue &qe, hipStream_t s);

// Residual-norm epilogue of an output projection whose N is the hidden width d: y = bf16(A @ B^T) is
// stored (system-coherent) to C, and the last workgroup to finish a row block's column tiles applies
//   x = bf16(x + bf16(rms(y) (1 + post_w)));  if next_w: h = bf16(rms(x) (1 + next_w))
// to the block's rows (x, h: [M, N] contiguous). counters: one int per row block of the launch's tile
// height, zero before the call and left zero after it.
struct NormEpilogue {
  uint16_t *x = nullptr;
  const uint16_t *post_w = nullptr, *next_w = nullptr;
  uint16_t *h = nullptr;
  int *counters = nullptr;
  float eps = 0.f;
};
hipError_t dx_gemm_norm(const uint16_t *A, const uint16_t *B, uint16_t *C, long M, long N, long K, long lda,
                        long ldb, const NormEpilogue &ne, hipStream_t s);
// Row blocks (counters) dx_gemm_norm uses for M rows.
long dx_gemm_norm_row_blocks(long M);
hipError_t dx_vt_zero_tails_launch(uint16_t *vt, const int32_t *seq_len, const int32_t *vt_start, int num_seqs,
                                   int vt_rows, long vt_ld, hipStream_t s);

struct AttnArgs {
  const void *q, *k, *v;  // v: token-major (fp32 path) or transposed (bf16 path)
  void *out;
  const int32_t *seq_start, *seq_len, *vt_start;
  int num_seqs, max_seq_len, hq, hkv, d;
  long q_stride, k_stride, v_stride, out_stride;  // v_stride = vt_ld on the bf16 path
  long vt_seq_stride;                              // used when vt_start == nullptr
  float scale, softcap;
  int window, causal;
  const uint8_t *key_mask = nullptr;   // fp32 path: per key row, nullable
  const uint32_t *key_bits = nullptr;  // bf16 path: key_words bits-words per sequence, nullable
  int key_words = 0;
};

hipError_t dx_attn_bf16(const AttnArgs &a, hipStream_t s);
hipError_t dx_attn_f32(const AttnArgs &a, hipStream_t s);
hipError_t dx_pack_key_bits_launch(const uint8_t *key_mask, const int32_t *seq_start, const int32_t *seq_len,
                                   int num_seqs, int max_seq_len, int words, uint32_t *bits, hipStream_t s);
hipError_t dx_transpose_v_launch(const uint16_t *v, uint16_t *vt, const int32_t *seq_start, const int32_t *seq_len,
                                 const int32_t *vt_start, long vt_seq_stride, int num_seqs, int max_seq_len, int hkv,
                                 int d, long v_stride, long vt_ld, hipStream_t s);

hipError_t dx_rmsnorm_launch(const uint16_t *x, const uint16_t *w, uint16_t *y, const uint8_t *mask, long rows,
                             int d, long ldx, long ldy, float eps, hipStream_t s);
hipError_t dx_add_rmsnorm_launch(const uint16_t *y, const uint16_t *post_w, uint16_t *x, const uint16_t *next_w,
                                 uint16_t *h, long rows, int d, float eps, hipStream_t s);
hipError_t dx_embed_launch(const int32_t *ids, const uint16_t *table, uint16_t *x, long tokens, int d, long vocab,
                           float scale, const uint16_t *norm_w, uint16_t *h, float eps, hipStream_t s);
hipError_t dx_rope_launch(uint16_t *x, const int32_t *pos, const uint16_t *cos, const uint16_t *sin, long rows,
                          int heads, int d, long stride, int max_pos, hipStream_t s);
hipError_t dx_readout_launch(const uint16_t *hidden, const uint16_t *norm_w, const uint16_t *table,
                             const int32_t *opt_pos, const int32_t *opt_label, const int32_t *q_off, int nq,
                             int num_options, long hidden_rows, int d, long ld_hidden, long vocab, float eps,
                             float softcap, float *logits, float *probs, hipStream_t s);
hipError_t dx_pack_gate_up_launch(const uint16_t *gate, const uint16_t *up, uint16_t *packed, long f, long k,
                                  hipStream_t s);

// Clef joint-head operations (head.hip), fp32.
hipError_t dx_layer_norm_f32_launch(const float *x, const float *w, const float *b, float *y, long rows, int d,
                                    long ldx, long ldy, float eps, hipStream_t s);
hipError_t dx_linear_f32_launch(const float *x, const float *w, const float *bias, float *y, long m, int n, int k,
                                long ldx, long ldw, long ldy, int act, int acc, hipStream_t s);
hipError_t dx_span_means_f32_launch(const float *x, const int32_t *spans, float *out, int B, int S, int O, int d,
                                    long ldx, long ldo, hipStream_t s);
hipError_t dx_mha_f32_launch(const float *q, const float *k, const float *v, const uint8_t *key_mask, float *out,
                             int B, int Q, int K, int H, int dh, long ldq, long ldk, long ldv, long ldo, hipStream_t s);
hipError_t dx_gather_rows_f32_launch(const float *x, const int32_t *idx, float *y, int B, int R, int I, int d,
                                     long ldx, long ldy, int acc, hipStream_t s);
hipError_t dx_routing_f32_launch(const float *options, const float *base, const int32_t *owner,
                                 const uint8_t *option_mask, float *summary, int B, int O, int NQ, int W,
                                 hipStream_t s);
hipError_t dx_fields_init_f32_launch(const float *base, const float *sn, const float *glob, const float *type_emb,
                                     const int32_t *types, float *fields, int B, int NQ, int W, int num_types,
                                     hipStream_t s);
hipError_t dx_features_f32_launch(const float *fields, const float *opts, const float *questions, const float *glob,
                                  const float *lexical, const int32_t *owner, float *features, float *prior,
                                  float *cosine, int B, int O, int NQ, int W, int Hd, float prior_scale,
                                  hipStream_t s);
hipError_t dx_combine_f32_launch(const float *prior, const float *cosine, const float *residual,
                                 const uint8_t *option_mask, float *out, long n, float gate, float joint_scale,
                                 hipStream_t s);
