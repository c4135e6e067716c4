// extern "C" entry points declared in include/deciax_hip.h: argument
// validation, then dispatch to the kernel launchers. Nothing here allocates
// or synchronises.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "common.h"
#include "kernels.h"

namespace {

thread_local char g_err[512];

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(hipError_t e, const char *what) {
  if (e != hipSuccess) return fail(DX_ERR_RUNTIME, "%s: %s", what, hipGetErrorString(e));
  g_err[0] = 0;
  return DX_OK;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

#define REQUIRE(cond, ...)                                   \
  do {                                                       \
    if (!(cond)) return fail(DX_ERR_INVALID, __VA_ARGS__);   \
  } while (0)
#define SUPPORTED(cond, ...)                                    \
  do {                                                          \
    if (!(cond)) return fail(DX_ERR_UNSUPPORTED, __VA_ARGS__);  \
  } while (0)

int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// Key-mask words per sequence: whole 64-key tiles, since a tile's second 32-key block may start past the
// sequence's last key.
int32_t key_mask_words(int64_t max_seq_len) { return (int32_t)(align_up(max_seq_len, 64) / 32); }

int validate_attn(const void *q, const void *k, const void *v, const void *out, const int32_t *seq_start,
                  const int32_t *seq_len, int32_t num_seqs, int32_t max_seq_len, int32_t hq, int32_t hkv,
                  int32_t d, int64_t qs, int64_t ks, int64_t os, float scale, float softcap, int32_t window,
                  int32_t dtype) {
  REQUIRE(q && k && v && out && seq_start && seq_len, "attention: null pointer argument");
  REQUIRE(num_seqs >= 0 && max_seq_len >= 0, "attention: negative sequence count or length");
  REQUIRE(hq > 0 && hkv > 0 && hq % hkv == 0, "attention: num_q_heads %d must be a positive multiple of num_kv_heads %d",
          hq, hkv);
  REQUIRE(window >= 0, "attention: window must be >= 0, got %d", window);
  REQUIRE(softcap >= 0.f && scale > 0.f, "attention: need scale > 0 and softcap >= 0");
  REQUIRE(dtype == DX_BF16 || dtype == DX_F32, "attention: unknown dtype %d", dtype);
  SUPPORTED(d == 64 || d == 128 || d == 256, "attention: head_dim %d not in {64, 128, 256}", d);
  if (dtype == DX_BF16) SUPPORTED(hq / hkv == 1 || hq / hkv == 2 || hq / hkv == 4,
                                  "attention: bf16 GQA group %d not in {1, 2, 4}", hq / hkv);
  // launch grids: bf16 (query tiles, KV heads, sequences) and its V^T transpose (64-row tiles,
  // sequences, KV heads x D / 64); fp32 (query tiles, sequences, heads). y and z stop at 65535.
  SUPPORTED(num_seqs <= 65535 && hq <= 65535, "attention: %d sequences or %d heads beyond the launch grid",
            num_seqs, hq);
  const int64_t vec = dtype == DX_BF16 ? 8 : 4;
  REQUIRE(qs % vec == 0 && ks % vec == 0 && os % vec == 0, "attention: row strides must be multiples of %ld elements",
          (long)vec);
  REQUIRE(qs >= (int64_t)hq * d && ks >= (int64_t)hkv * d && os >= (int64_t)hq * d,
          "attention: row stride smaller than heads * head_dim");
  REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out), "attention: pointers must be 16-byte aligned");
  return DX_OK;
}

// The bf16 kernel reads one sequence's K rows and one KV head's V^T block through buffer resources whose
// byte ranges and per-lane offsets are 32-bit: len * k_stride * 2 bytes of K, and
// ((D - 1) * vt_ld + len rounded up to 64) * 2 bytes of V^T. Larger spans would wrap.
int check_bf16_ranges(int64_t max_seq_len, int64_t k_stride, int64_t d, int64_t vt_ld) {
  const int64_t lim = INT64_C(1) << 31;
  SUPPORTED(max_seq_len * k_stride * 2 < lim,
            "attention: %ld keys x k row stride %ld exceed the kernel's 2 GiB K range", (long)max_seq_len,
            (long)k_stride);
  SUPPORTED(((d - 1) * vt_ld + align_up(max_seq_len, 64)) * 2 < lim,
            "attention: V^T leading dimension %ld x head_dim %ld exceeds the kernel's 2 GiB V^T range", (long)vt_ld,
            (long)d);
  return DX_OK;
}

}  // namespace

extern "C" {

const char *dx_version(void) { return "deciax-mi355x 0.1.0 gfx950"; }

const char *dx_last_error(void) { return g_err; }

int dx_device_arch(int device, char *buf, int buf_len) {
  if (!buf || buf_len <= 0) return fail(DX_ERR_INVALID, "dx_device_arch: empty buffer");
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return fail(DX_ERR_RUNTIME, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  int n = 0;
  while (prop.gcnArchName[n] && prop.gcnArchName[n] != ':' && n < buf_len - 1) {
    buf[n] = prop.gcnArchName[n];
    ++n;
  }
  buf[n] = 0;
  return DX_OK;
}

int64_t dx_attn_prefill_workspace(int32_t num_seqs, int32_t max_seq_len, int32_t num_kv_heads, int32_t head_dim,
                                  int32_t dtype) {
  if (dtype != DX_BF16 || num_seqs <= 0 || max_seq_len <= 0) return 0;
  // V^T with one 64-aligned column block per sequence.
  return align_up(max_seq_len, 64) * num_seqs * num_kv_heads * head_dim * 2;
}

int64_t dx_attn_prefill_masked_workspace(int32_t num_seqs, int32_t max_seq_len, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t dtype) {
  if (dtype != DX_BF16 || num_seqs <= 0 || max_seq_len <= 0) return 0;
  // V^T, then the key mask as bits: two 32-bit words per 64 keys (whole key tiles) per sequence.
  return align_up(dx_attn_prefill_workspace(num_seqs, max_seq_len, num_kv_heads, head_dim, dtype), 256) +
         (int64_t)num_seqs * key_mask_words(max_seq_len) * 4;
}

}  // extern "C"

// V^T staging of dx_attn_prefill_noalloc, for callers that cannot allocate. Each GPU holds its own copy
// from the library's first use on it until the process ends. In host code `scratch` only names the
// array: its device address comes from hipGetSymbolAddress, once per device (scratch_on_current_device).
static __device__ __align__(256) unsigned char scratch[DX_NOALLOC_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mu;
constexpr int MAX_DEVICES = 64;
void *g_scratch[MAX_DEVICES] = {};

// Device address of the current device's `scratch`, looked up once per device (by dx_noalloc_init or the
// first allocation-free call). The lookup may load the library's code object on that device, which graph
// capture does not allow: a call on a capturing `stream` that would need it is refused instead.
int scratch_on_current_device(void **out, hipStream_t stream, bool from_init) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(DX_ERR_RUNTIME, "hipGetDevice: %s", hipGetErrorString(e));
  SUPPORTED(dev >= 0 && dev < MAX_DEVICES, "attention: device %d beyond the %d the static scratch tracks", dev,
            MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev] && !from_init) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &capture);
    if (e != hipSuccess) return fail(DX_ERR_RUNTIME, "hipStreamIsCapturing: %s", hipGetErrorString(e));
    SUPPORTED(capture == hipStreamCaptureStatusNone,
              "attention_noalloc: device %d's static scratch is looked up outside graph capture; call "
              "dx_noalloc_init() on this device before capturing",
              dev);
  }
  if (!g_scratch[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(DX_ERR_RUNTIME, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return DX_OK;
}

// static_scratch: stage V^T in the current device's `scratch` instead of `workspace` (which is ignored).
int attn_prefill(const void *q, const void *k, const void *v, const uint8_t *key_mask, void *out,
                 const int32_t *seq_start, const int32_t *seq_len, int32_t num_seqs, int32_t max_seq_len,
                 int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int64_t q_row_stride,
                 int64_t k_row_stride, int64_t v_row_stride, int64_t out_row_stride, float scale, float softcap,
                 int32_t window, int32_t causal, int32_t dtype, void *workspace, int64_t workspace_bytes,
                 void *stream, bool static_scratch = false) {
  int st = validate_attn(q, k, v, out, seq_start, seq_len, num_seqs, max_seq_len, num_q_heads, num_kv_heads,
                         head_dim, q_row_stride, k_row_stride, out_row_stride, scale, softcap, window, dtype);
  if (st) return st;
  const int64_t vec = dtype == DX_BF16 ? 8 : 4;
  REQUIRE(v_row_stride % vec == 0 && v_row_stride >= (int64_t)num_kv_heads * head_dim,
          "attention: bad v row stride %ld", (long)v_row_stride);
  // the matrix-core fp32 kernel (head_dim 64 and 128) reads a 32-key block of K or V through a buffer
  // resource with 32-bit byte offsets; the head_dim 256 kernel addresses with 64-bit pointers
  if (dtype == DX_F32)
    SUPPORTED(head_dim > 128 || (k_row_stride < (INT64_C(1) << 24) && v_row_stride < (INT64_C(1) << 24)),
              "attention: fp32 k / v row strides of 2^24 elements or more are not supported at head_dim %d",
              head_dim);
  if (num_seqs == 0 || max_seq_len == 0) return DX_OK;
  AttnArgs a{q, k, v, out, seq_start, seq_len, nullptr, num_seqs, max_seq_len, num_q_heads, num_kv_heads, head_dim,
             q_row_stride, k_row_stride, v_row_stride, out_row_stride, 0, scale, softcap, window, causal ? 1 : 0};
  a.key_mask = key_mask;
  if (dtype == DX_F32) return check_launch(dx_attn_f32(a, as_stream(stream)), "attention fp32 launch");

  const int64_t seq_stride = align_up(max_seq_len, 64);
  const int64_t vt_ld = seq_stride * num_seqs;
  st = check_bf16_ranges(max_seq_len, k_row_stride, head_dim, vt_ld);
  if (st) return st;
  const int64_t vt_bytes = dx_attn_prefill_workspace(num_seqs, max_seq_len, num_kv_heads, head_dim, DX_BF16);
  const int64_t need = key_mask ? dx_attn_prefill_masked_workspace(num_seqs, max_seq_len, num_kv_heads, head_dim,
                                                                   DX_BF16)
                                : vt_bytes;
  if (static_scratch) {
    SUPPORTED(need <= DX_NOALLOC_SCRATCH_BYTES,
              "attention_noalloc: V^T staging of %ld bytes exceeds the %ld-byte static scratch", (long)need,
              (long)DX_NOALLOC_SCRATCH_BYTES);
    st = scratch_on_current_device(&workspace, as_stream(stream), false);
    if (st) return st;
    workspace_bytes = DX_NOALLOC_SCRATCH_BYTES;
  }
  REQUIRE(workspace && aligned16(workspace), "attention: bf16 needs a 16-byte aligned workspace");
  REQUIRE(workspace_bytes >= need, "attention: workspace of %ld bytes, need %ld", (long)workspace_bytes, (long)need);
  uint16_t *vt = static_cast<uint16_t *>(workspace);
  hipError_t e = dx_transpose_v_launch(static_cast<const uint16_t *>(v), vt, seq_start, seq_len, nullptr, seq_stride,
                                       num_seqs, max_seq_len, num_kv_heads, head_dim, v_row_stride, vt_ld,
                                       as_stream(stream));
  if (e != hipSuccess) return check_launch(e, "transpose_v launch");
  if (key_mask) {
    uint32_t *bits = reinterpret_cast<uint32_t *>(static_cast<char *>(workspace) + align_up(vt_bytes, 256));
    a.key_words = key_mask_words(max_seq_len);
    e = dx_pack_key_bits_launch(key_mask, seq_start, seq_len, num_seqs, max_seq_len, a.key_words, bits,
                                as_stream(stream));
    if (e != hipSuccess) return check_launch(e, "key mask launch");
    a.key_bits = bits;
  }
  a.v = vt;
  a.v_stride = vt_ld;
  a.vt_seq_stride = seq_stride;
  return check_launch(dx_attn_bf16(a, as_stream(stream)), "attention bf16 launch");
}

}  // namespace

extern "C" {

int dx_attn_prefill(const void *q, const void *k, const void *v, void *out, const int32_t *seq_start,
                    const int32_t *seq_len, int32_t num_seqs, int32_t max_seq_len, int32_t num_q_heads,
                    int32_t num_kv_heads, int32_t head_dim, int64_t q_row_stride, int64_t k_row_stride,
                    int64_t v_row_stride, int64_t out_row_stride, float scale, float softcap, int32_t window,
                    int32_t causal, int32_t dtype, void *workspace, int64_t workspace_bytes, void *stream) {
  return attn_prefill(q, k, v, nullptr, out, seq_start, seq_len, num_seqs, max_seq_len, num_q_heads, num_kv_heads,
                      head_dim, q_row_stride, k_row_stride, v_row_stride, out_row_stride, scale, softcap, window,
                      causal, dtype, workspace, workspace_bytes, stream);
}

int dx_noalloc_init(void) {
  void *p = nullptr;
  return scratch_on_current_device(&p, nullptr, true);
}

int dx_attn_prefill_noalloc(const void *q, const void *k, const void *v, void *out, const int32_t *seq_start,
                            const int32_t *seq_len, int32_t num_seqs, int32_t max_seq_len, int32_t num_q_heads,
                            int32_t num_kv_heads, int32_t head_dim, int64_t q_row_stride, int64_t k_row_stride,
                            int64_t v_row_stride, int64_t out_row_stride, float scale, float softcap,
                            int32_t window, int32_t causal, int32_t dtype, void *stream) {
  return attn_prefill(q, k, v, nullptr, out, seq_start, seq_len, num_seqs, max_seq_len, num_q_heads, num_kv_heads,
                      head_dim, q_row_stride, k_row_stride, v_row_stride, out_row_stride, scale, softcap, window,
                      causal, dtype, nullptr, 0, stream, /*static_scratch=*/true);
}

int dx_attn_prefill_masked(const void *q, const void *k, const void *v, const uint8_t *key_mask, void *out,
                           const int32_t *seq_start, const int32_t *seq_len, int32_t num_seqs, int32_t max_seq_len,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int64_t q_row_stride,
                           int64_t k_row_stride, int64_t v_row_stride, int64_t out_row_stride, float scale,
                           float softcap, int32_t window, int32_t causal, int32_t dtype, void *workspace,
                           int64_t workspace_bytes, void *stream) {
  REQUIRE(key_mask, "attention: key_mask must not be null");
  return attn_prefill(q, k, v, key_mask, out, seq_start, seq_len, num_seqs, max_seq_len, num_q_heads, num_kv_heads,
                      head_dim, q_row_stride, k_row_stride, v_row_stride, out_row_stride, scale, softcap, window,
                      causal, dtype, workspace, workspace_bytes, stream);
}

int dx_attn_prefill_vt(const void *q, const void *k, const void *vt, void *out, const int32_t *seq_start,
                       const int32_t *seq_len, const int32_t *vt_start, int32_t num_seqs, int32_t max_seq_len,
                       int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int64_t q_row_stride,
                       int64_t k_row_stride, int64_t vt_ld, int64_t out_row_stride, float scale, float softcap,
                       int32_t window, int32_t causal, void *stream) {
  int st = validate_attn(q, k, vt, out, seq_start, seq_len, num_seqs, max_seq_len, num_q_heads, num_kv_heads,
                         head_dim, q_row_stride, k_row_stride, out_row_stride, scale, softcap, window, DX_BF16);
  if (st) return st;
  REQUIRE(vt_start, "attention: vt_start must not be null");
  REQUIRE(vt_ld % 8 == 0 && vt_ld > 0, "attention: vt_ld must be a positive multiple of 8");
  st = check_bf16_ranges(max_seq_len, k_row_stride, head_dim, vt_ld);
  if (st) return st;
  if (num_seqs == 0 || max_seq_len == 0) return DX_OK;
  AttnArgs a{q, k, vt, out, seq_start, seq_len, vt_start, num_seqs, max_seq_len, num_q_heads, num_kv_heads,
             head_dim, q_row_stride, k_row_stride, vt_ld, out_row_stride, 0, scale, softcap, window, causal ? 1 : 0};
  return check_launch(dx_attn_bf16(a, as_stream(stream)), "attention bf16 launch");
}

int dx_transpose_v(const void *v, void *vt, const int32_t *seq_start, const int32_t *seq_len,
                   const int32_t *vt_start, int32_t num_seqs, int32_t max_seq_len, int32_t num_kv_heads,
                   int32_t head_dim, int64_t v_row_stride, int64_t vt_ld, void *stream) {
  REQUIRE(v && vt && seq_start && seq_len && vt_start, "transpose_v: null pointer argument");
  REQUIRE(aligned16(v) && aligned16(vt), "transpose_v: pointers must be 16-byte aligned");
  SUPPORTED(head_dim % 64 == 0, "transpose_v: head_dim %d not a multiple of 64", head_dim);
  REQUIRE(v_row_stride % 8 == 0 && vt_ld % 8 == 0, "transpose_v: strides must be multiples of 8");
  REQUIRE(num_seqs >= 0 && max_seq_len >= 0 && num_kv_heads > 0, "transpose_v: bad sizes");
  SUPPORTED(num_seqs <= 65535 && (int64_t)num_kv_heads * (head_dim / 64) <= 65535,
            "transpose_v: %d sequences or %d heads beyond the launch grid", num_seqs, num_kv_heads);
  if (num_seqs == 0 || max_seq_len == 0) return DX_OK;
  return check_launch(dx_transpose_v_launch(static_cast<const uint16_t *>(v), static_cast<uint16_t *>(vt), seq_start,
                                            seq_len, vt_start, 0, num_seqs, max_seq_len, num_kv_heads, head_dim,
                                            v_row_stride, vt_ld, as_stream(stream)),
                      "transpose_v launch");
}

int dx_vt_zero_tails(void *vt, const int32_t *seq_len, const int32_t *vt_start, int32_t num_seqs, int32_t vt_rows,
                     int64_t vt_ld, void *stream) {
  REQUIRE(vt && seq_len && vt_start, "vt_zero_tails: null pointer argument");
  REQUIRE(num_seqs >= 0 && vt_rows >= 0 && vt_ld > 0 && vt_ld % 8 == 0, "vt_zero_tails: bad sizes");
  if (num_seqs == 0 || vt_rows == 0) return DX_OK;
  return check_launch(dx_vt_zero_tails_launch(static_cast<uint16_t *>(vt), seq_len, vt_start, num_seqs, vt_rows,
                                              vt_ld, as_stream(stream)),
                      "vt_zero_tails launch");
}

int dx_qkv_rope(const void *x, const void *w_qkv, void *qk, void *vt, const int32_t *positions, const int32_t *vt_col,
                const void *cos, const void *sin, int64_t rows, int64_t hidden, int32_t num_q_heads,
                int32_t num_kv_heads, int32_t head_dim, int64_t ldx, int64_t ld_qk, int64_t vt_ld, int32_t max_pos,
                void *stream) {
  REQUIRE(x && w_qkv && qk && vt && positions && vt_col && cos && sin, "qkv_rope: null pointer argument");
  REQUIRE(rows >= 0 && hidden > 0 && num_q_heads > 0 && num_kv_heads > 0 && max_pos > 0, "qkv_rope: bad sizes");
  SUPPORTED(head_dim == 64 || head_dim == 128 || head_dim == 256, "qkv_rope: head_dim %d not in {64, 128, 256}",
            head_dim);
  const int64_t qk_cols = (int64_t)(num_q_heads + num_kv_heads) * head_dim;
  const int64_t n = qk_cols + (int64_t)num_kv_heads * head_dim;
  SUPPORTED(n % 256 == 0, "qkv_rope: packed width %ld must be a multiple of 256", (long)n);
  SUPPORTED(hidden % 64 == 0, "qkv_rope: hidden=%ld must be a multiple of 64", (long)hidden);
  REQUIRE(ldx >= hidden && ldx % 8 == 0 && ld_qk >= qk_cols && ld_qk % 8 == 0 && vt_ld > 0,
          "qkv_rope: leading dimensions must cover the row and be multiples of 8");
  SUPPORTED(ldx <= DX_MAX_LD && hidden <= DX_MAX_LD, "qkv_rope: leading dimensions above %d", DX_MAX_LD);
  REQUIRE(aligned16(x) && aligned16(w_qkv) && aligned16(qk) && aligned16(cos) && aligned16(sin),
          "qkv_rope: pointers must be 16-byte aligned");
  if (rows == 0) return DX_OK;
  QkvEpilogue qe;
  qe.vt = static_cast<uint16_t *>(vt);
  qe.vt_col = vt_col;
  qe.pos = positions;
  qe.cos = static_cast<const uint16_t *>(cos);
  qe.sin = static_cast<const uint16_t *>(sin);
  qe.vt_ld = vt_ld;
  qe.qk_cols = (int)qk_cols;
  qe.d = head_dim;
  qe.max_pos = max_pos;
  return check_launch(dx_gemm_qkv(static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(w_qkv),
                                  static_cast<uint16_t *>(qk), rows, n, hidden, ldx, hidden, ld_qk, qe,
                                  as_stream(stream)),
                      "qkv_rope launch");
}

int dx_linear(const void *x, const void *w, void *y, int64_t m, int64_t n, int64_t k, int64_t ldx, int64_t ldw,
              int64_t ldy, int32_t out_dtype, void *stream) {
  REQUIRE(x && w && y, "linear: null pointer argument");
  REQUIRE(m >= 0 && n > 0 && k > 0, "linear: bad sizes m=%ld n=%ld k=%ld", (long)m, (long)n, (long)k);
  SUPPORTED(n % 256 == 0, "linear: n=%ld must be a multiple of 256", (long)n);
  SUPPORTED(k % 64 == 0, "linear: k=%ld must be a multiple of 64", (long)k);
  REQUIRE(ldx >= k && ldw >= k && ldy >= n && ldx % 8 == 0 && ldw % 8 == 0 && ldy % 8 == 0,
          "linear: leading dimensions must cover the row and be multiples of 8");
  SUPPORTED(ldx <= DX_MAX_LD && ldw <= DX_MAX_LD, "linear: leading dimensions above %d", DX_MAX_LD);
  REQUIRE(aligned16(x) && aligned16(w) && aligned16(y), "linear: pointers must be 16-byte aligned");
  REQUIRE(out_dtype == DX_BF16 || out_dtype == DX_F32, "linear: unknown out dtype %d", out_dtype);
  if (m == 0) return DX_OK;
  const auto *X = static_cast<const uint16_t *>(x);
  const auto *W = static_cast<const uint16_t *>(w);
  hipError_t e = out_dtype == DX_BF16
                     ? dx_gemm_bf16(X, W, static_cast<uint16_t *>(y), m, n, k, ldx, ldw, ldy, as_stream(stream))
                     : dx_gemm_f32(X, W, static_cast<float *>(y), m, n, k, ldx, ldw, ldy, as_stream(stream));
  return check_launch(e, "linear launch");
}

int dx_gated_linear(const void *x, const void *gate_up, void *act, int64_t m, int64_t f, int64_t k, int64_t ldx,
                    int64_t ld_act, int32_t activation, void *stream) {
  REQUIRE(x && gate_up && act, "gated_linear: null pointer argument");
  REQUIRE(m >= 0 && f > 0 && k > 0, "gated_linear: bad sizes");
  SUPPORTED(f % 128 == 0, "gated_linear: f=%ld must be a multiple of 128", (long)f);
  SUPPORTED(k % 64 == 0, "gated_linear: k=%ld must be a multiple of 64", (long)k);
  REQUIRE(ldx >= k && ld_act >= f && ldx % 8 == 0 && ld_act % 8 == 0, "gated_linear: bad leading dimensions");
  SUPPORTED(ldx <= DX_MAX_LD && k <= DX_MAX_LD, "gated_linear: leading dimensions above %d", DX_MAX_LD);
  REQUIRE(aligned16(x) && aligned16(gate_up) && aligned16(act), "gated_linear: pointers must be 16-byte aligned");
  REQUIRE(activation == DX_ACT_GELU_TANH || activation == DX_ACT_SILU, "gated_linear: unknown activation %d",
          activation);
  if (m == 0) return DX_OK;
  return check_launch(dx_gemm_gated(static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(gate_up),
                                    static_cast<uint16_t *>(act), m, f, k, ldx, ld_act, activation,
                                    as_stream(stream)),
                      "gated_linear launch");
}

int dx_pack_gate_up(const void *gate, const void *up, void *packed, int64_t f, int64_t k, void *stream) {
  REQUIRE(gate && up && packed, "pack_gate_up: null pointer argument");
  SUPPORTED(f % 64 == 0 && f > 0, "pack_gate_up: f=%ld must be a positive multiple of 64", (long)f);
  REQUIRE(k % 8 == 0 && k > 0, "pack_gate_up: k must be a positive multiple of 8");
  REQUIRE(aligned16(gate) && aligned16(up) && aligned16(packed), "pack_gate_up: pointers must be 16-byte aligned");
  return check_launch(dx_pack_gate_up_launch(static_cast<const uint16_t *>(gate), static_cast<const uint16_t *>(up),
                                             static_cast<uint16_t *>(packed), f, k, as_stream(stream)),
                      "pack_gate_up launch");
}

int64_t dx_linear_residual_norm_counters(int64_t m) { return m > 0 ? dx_gemm_norm_row_blocks(m) : 0; }

int dx_linear_residual_norm(const void *a, const void *w, void *y, void *x, const void *post_w, const void *next_w,
                            void *h, int32_t *counters, int64_t m, int64_t d, int64_t k, int64_t lda, int64_t ldw,
                            float eps, void *stream) {
  REQUIRE(a && w && y && x && post_w && counters, "linear_residual_norm: null pointer argument");
  REQUIRE((h == nullptr) == (next_w == nullptr), "linear_residual_norm: h and next_w must both be set or both be null");
  REQUIRE(m >= 0 && d > 0 && k > 0, "linear_residual_norm: bad sizes");
  SUPPORTED(d % 256 == 0 && d <= 6144, "linear_residual_norm: d=%ld must be a multiple of 256 and <= 6144", (long)d);
  SUPPORTED(k % 64 == 0, "linear_residual_norm: k=%ld must be a multiple of 64", (long)k);
  REQUIRE(lda >= k && ldw >= k && lda % 8 == 0 && ldw % 8 == 0,
          "linear_residual_norm: leading dimensions must cover the row and be multiples of 8");
  SUPPORTED(lda <= DX_MAX_LD && ldw <= DX_MAX_LD && d <= DX_MAX_LD,
            "linear_residual_norm: leading dimensions above %d", DX_MAX_LD);
  REQUIRE(aligned16(a) && aligned16(w) && aligned16(y) && aligned16(x) && aligned16(post_w) &&
              (!h || (aligned16(h) && aligned16(next_w))) && (reinterpret_cast<uintptr_t>(counters) & 3) == 0,
          "linear_residual_norm: pointers must be 16-byte aligned (counters 4-byte)");
  if (m == 0) return DX_OK;
  NormEpilogue ne;
  ne.x = static_cast<uint16_t *>(x);
  ne.post_w = static_cast<const uint16_t *>(post_w);
  ne.next_w = static_cast<const uint16_t *>(next_w);
  ne.h = static_cast<uint16_t *>(h);
  ne.counters = counters;
  ne.eps = eps;
  return check_launch(dx_gemm_norm(static_cast<const uint16_t *>(a), static_cast<const uint16_t *>(w),
                                   static_cast<uint16_t *>(y), m, d, k, lda, ldw, ne, as_stream(stream)),
                      "linear_residual_norm launch");
}

int64_t dx_norm_project_workspace(int64_t rows, int64_t d) { return align_up(rows * d * 2, 256); }

int dx_norm_project(const void *x, const void *norm_w, const uint8_t *row_mask, const void *w, void *y, int64_t rows,
                    int64_t d, int64_t n, float eps, void *workspace, int64_t workspace_bytes, void *stream) {
  REQUIRE(x && norm_w && w && y && workspace, "norm_project: null pointer argument");
  REQUIRE(rows >= 0 && d > 0 && n > 0, "norm_project: bad sizes");
  SUPPORTED(d % 64 == 0 && d <= 8192, "norm_project: d=%ld must be a multiple of 64 and <= 8192", (long)d);
  SUPPORTED(n % 256 == 0, "norm_project: n=%ld must be a multiple of 256", (long)n);
  REQUIRE(workspace_bytes >= dx_norm_project_workspace(rows, d), "norm_project: workspace too small");
  REQUIRE(aligned16(x) && aligned16(norm_w) && aligned16(w) && aligned16(y) && aligned16(workspace),
          "norm_project: pointers must be 16-byte aligned");
  if (rows == 0) return DX_OK;
  uint16_t *h = static_cast<uint16_t *>(workspace);
  hipError_t e = dx_rmsnorm_launch(static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(norm_w), h,
                                   row_mask, rows, (int)d, d, d, eps, as_stream(stream));
  if (e != hipSuccess) return check_launch(e, "norm_project rmsnorm launch");
  return check_launch(dx_gemm_bf16(h, static_cast<const uint16_t *>(w), static_cast<uint16_t *>(y), rows, n, d, d, d,
                                   n, as_stream(stream)),
                      "norm_project gemm launch");
}

int64_t dx_mlp_workspace(int64_t rows, int64_t d, int64_t f) {
  return align_up(rows * d * 2, 256) + align_up(rows * f * 2, 256);
}

int dx_mlp(const void *x, const void *norm_w, const void *gate_up, const void *down, void *y, int64_t rows, int64_t d,
           int64_t f, float eps, int32_t activation, int32_t out_dtype, void *workspace, int64_t workspace_bytes,
           void *stream) {
  REQUIRE(x && norm_w && gate_up && down && y && workspace, "mlp: null pointer argument");
  REQUIRE(rows >= 0 && d > 0 && f > 0, "mlp: bad sizes");
  SUPPORTED(d % 256 == 0 && d <= 8192, "mlp: d=%ld must be a multiple of 256 and <= 8192", (long)d);
  SUPPORTED(f % 128 == 0, "mlp: f=%ld must be a multiple of 128", (long)f);
  REQUIRE(activation == DX_ACT_GELU_TANH || activation == DX_ACT_SILU, "mlp: unknown activation %d", activation);
  REQUIRE(out_dtype == DX_BF16 || out_dtype == DX_F32, "mlp: unknown out dtype %d", out_dtype);
  REQUIRE(workspace_bytes >= dx_mlp_workspace(rows, d, f), "mlp: workspace too small");
  REQUIRE(aligned16(x) && aligned16(norm_w) && aligned16(gate_up) && aligned16(down) && aligned16(y) &&
              aligned16(workspace),
          "mlp: pointers must be 16-byte aligned");
  if (rows == 0) return DX_OK;
  hipStream_t s = as_stream(stream);
  uint16_t *h = static_cast<uint16_t *>(workspace);
  uint16_t *a = h + align_up(rows * d * 2, 256) / 2;
  hipError_t e = dx_rmsnorm_launch(static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(norm_w), h,
                                   nullptr, rows, (int)d, d, d, eps, s);
  if (e != hipSuccess) return check_launch(e, "mlp rmsnorm launch");
  e = dx_gemm_gated(h, static_cast<const uint16_t *>(gate_up), a, rows, f, d, d, f, activation, s);
  if (e != hipSuccess) return check_launch(e, "mlp gate/up launch");
  const auto *D = static_cast<const uint16_t *>(down);
  e = out_dtype == DX_BF16 ? dx_gemm_bf16(a, D, static_cast<uint16_t *>(y), rows, d, f, f, f, d, s)
                           : dx_gemm_f32(a, D, static_cast<float *>(y), rows, d, f, f, f, d, s);
  return check_launch(e, "mlp down launch");
}

int dx_rmsnorm(const void *x, const void *w, void *y, int64_t rows, int64_t d, int64_t ldx, int64_t ldy, float eps,
               void *stream) {
  REQUIRE(x && w && y, "rmsnorm: null pointer argument");
  REQUIRE(rows >= 0 && d > 0 && ldx >= d && ldy >= d, "rmsnorm: bad sizes");
  SUPPORTED(d % 8 == 0 && d <= 8192, "rmsnorm: d=%ld must be a multiple of 8 and <= 8192", (long)d);
  REQUIRE(ldx % 8 == 0 && ldy % 8 == 0, "rmsnorm: leading dimensions must be multiples of 8");
  REQUIRE(aligned16(x) && aligned16(w) && aligned16(y), "rmsnorm: pointers must be 16-byte aligned");
  if (rows == 0) return DX_OK;
  return check_launch(dx_rmsnorm_launch(static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(w),
                                        static_cast<uint16_t *>(y), nullptr, rows, (int)d, ldx, ldy, eps,
                                        as_stream(stream)),
                      "rmsnorm launch");
}

int dx_add_rmsnorm(const void *y, const void *post_w, void *x, const void *next_w, void *h, int64_t rows, int64_t d,
                   float eps, void *stream) {
  REQUIRE(y && x, "add_rmsnorm: null pointer argument");
  REQUIRE((h == nullptr) == (next_w == nullptr), "add_rmsnorm: h and next_w must both be set or both be null");
  REQUIRE(rows >= 0 && d > 0, "add_rmsnorm: bad sizes");
  SUPPORTED(d % 8 == 0 && d <= 8192, "add_rmsnorm: d=%ld must be a multiple of 8 and <= 8192", (long)d);
  REQUIRE(aligned16(y) && aligned16(x) && (!post_w || aligned16(post_w)) && (!h || (aligned16(h) && aligned16(next_w))),
          "add_rmsnorm: pointers must be 16-byte aligned");
  if (rows == 0) return DX_OK;
  return check_launch(dx_add_rmsnorm_launch(static_cast<const uint16_t *>(y), static_cast<const uint16_t *>(post_w),
                                            static_cast<uint16_t *>(x), static_cast<const uint16_t *>(next_w),
                                            static_cast<uint16_t *>(h), rows, (int)d, eps, as_stream(stream)),
                      "add_rmsnorm launch");
}

int dx_embed(const int32_t *ids, const void *table, void *x, int64_t tokens, int64_t d, int64_t vocab, float scale,
             const void *norm_w, void *h, float eps, void *stream) {
  REQUIRE(ids && table && x, "embed: null pointer argument");
  REQUIRE((h == nullptr) == (norm_w == nullptr), "embed: h and norm_w must both be set or both be null");
  REQUIRE(tokens >= 0 && d > 0 && vocab > 0, "embed: bad sizes");
  SUPPORTED(d % 8 == 0 && d <= 8192, "embed: d=%ld must be a multiple of 8 and <= 8192", (long)d);
  REQUIRE(aligned16(table) && aligned16(x) && (!h || (aligned16(h) && aligned16(norm_w))),
          "embed: pointers must be 16-byte aligned");
  if (tokens == 0) return DX_OK;
  return check_launch(dx_embed_launch(ids, static_cast<const uint16_t *>(table), static_cast<uint16_t *>(x), tokens,
                                      (int)d, vocab, scale, static_cast<const uint16_t *>(norm_w),
                                      static_cast<uint16_t *>(h), eps, as_stream(stream)),
                      "embed launch");
}

int dx_rope(void *x, const int32_t *positions, const void *cos, const void *sin, int64_t rows, int32_t num_heads,
            int32_t head_dim, int64_t row_stride, int32_t max_pos, void *stream) {
  REQUIRE(x && positions && cos && sin, "rope: null pointer argument");
  REQUIRE(rows >= 0 && num_heads > 0 && max_pos > 0, "rope: bad sizes");
  SUPPORTED(head_dim % 16 == 0 && head_dim > 0, "rope: head_dim %d must be a multiple of 16", head_dim);
  REQUIRE(row_stride % 8 == 0 && row_stride >= (int64_t)num_heads * head_dim, "rope: bad row stride");
  REQUIRE(aligned16(x) && aligned16(cos) && aligned16(sin), "rope: pointers must be 16-byte aligned");
  if (rows == 0) return DX_OK;
  return check_launch(dx_rope_launch(static_cast<uint16_t *>(x), positions, static_cast<const uint16_t *>(cos),
                                     static_cast<const uint16_t *>(sin), rows, num_heads, head_dim, row_stride,
                                     max_pos, as_stream(stream)),
                      "rope launch");
}

int dx_readout(const void *hidden, const void *norm_w, const void *table, const int32_t *opt_pos,
               const int32_t *opt_label, const int32_t *q_offsets, int32_t num_questions, int64_t num_options,
               int64_t hidden_rows, int64_t d, int64_t ld_hidden, int64_t vocab, float eps, float softcap,
               float *logits, float *probs, void *stream) {
  REQUIRE(hidden && norm_w && table && opt_pos && opt_label && q_offsets && logits && probs,
          "readout: null pointer argument");
  REQUIRE(num_questions >= 0 && num_options >= 0 && hidden_rows > 0 && d > 0 && vocab > 0 && ld_hidden >= d,
          "readout: bad sizes");
  REQUIRE(num_options <= INT32_MAX, "readout: num_options=%lld exceeds the int32 range of the offsets",
          (long long)num_options);
  SUPPORTED(d % 8 == 0 && d <= 8192, "readout: d=%ld must be a multiple of 8 and <= 8192", (long)d);
  REQUIRE(ld_hidden % 8 == 0, "readout: ld_hidden must be a multiple of 8");
  REQUIRE(softcap >= 0.f, "readout: softcap must be >= 0");
  REQUIRE(aligned16(hidden) && aligned16(norm_w) && aligned16(table), "readout: pointers must be 16-byte aligned");
  if (num_questions == 0) return DX_OK;
  return check_launch(dx_readout_launch(static_cast<const uint16_t *>(hidden), static_cast<const uint16_t *>(norm_w),
                                        static_cast<const uint16_t *>(table), opt_pos, opt_label, q_offsets,
                                        num_questions, (int)num_options, hidden_rows, (int)d, ld_hidden, vocab, eps,
                                        softcap, logits, probs, as_stream(stream)),
                      "readout launch");
}

}  // extern "C"

/* ------------------------------------------------------------------------ */
/* Clef joint schema head (fp32)                                             */
/* ------------------------------------------------------------------------ */

int dx_layer_norm_f32(const float *x, const float *w, const float *b, float *y, int64_t rows, int64_t d, int64_t ldx,
                      int64_t ldy, float eps, void *stream) {
  REQUIRE(x && w && y, "layer_norm: null pointer argument");
  REQUIRE(rows >= 0 && d > 0 && ldx >= d && ldy >= d && eps >= 0.f, "layer_norm: bad sizes");
  if (rows == 0) return DX_OK;
  return check_launch(dx_layer_norm_f32_launch(x, w, b, y, rows, (int)d, ldx, ldy, eps, as_stream(stream)),
                      "layer_norm launch");
}

int dx_linear_f32(const float *x, const float *w, const float *bias, float *y, int64_t m, int64_t n, int64_t k,
                  int64_t ldx, int64_t ldw, int64_t ldy, int32_t activation, int32_t accumulate, void *stream) {
  REQUIRE(x && w && y, "linear_f32: null pointer argument");
  REQUIRE(m >= 0 && n > 0 && k > 0 && ldx >= k && ldw >= k && ldy >= n, "linear_f32: bad sizes");
  REQUIRE(activation == DX_ACT_NONE || activation == DX_ACT_GELU_ERF,
          "linear_f32: activation %d not in {DX_ACT_NONE, DX_ACT_GELU_ERF}", activation);
  SUPPORTED(n < (1L << 30) && k < (1L << 30), "linear_f32: n, k must fit 30 bits");
  if (m == 0) return DX_OK;
  return check_launch(dx_linear_f32_launch(x, w, bias, y, m, (int)n, (int)k, ldx, ldw, ldy,
                                           activation == DX_ACT_GELU_ERF ? 1 : 0,
                                           accumulate ? 1 : 0, as_stream(stream)),
                      "linear_f32 launch");
}

int dx_span_means_f32(const float *x, const int32_t *spans, float *out, int32_t batch, int32_t seq, int32_t spans_per_row,
                      int64_t d, int64_t ldx, int64_t ld_out, void *stream) {
  REQUIRE(x && spans && out, "span_means: null pointer argument");
  REQUIRE(batch >= 0 && seq > 0 && spans_per_row >= 0 && d > 0 && ldx >= d && ld_out >= d, "span_means: bad sizes");
  if (batch == 0 || spans_per_row == 0) return DX_OK;
  return check_launch(dx_span_means_f32_launch(x, spans, out, batch, seq, spans_per_row, (int)d, ldx, ld_out,
                                               as_stream(stream)),
                      "span_means launch");
}

int dx_mha_f32(const float *q, const float *k, const float *v, const uint8_t *key_mask, float *out, int32_t batch,
               int32_t num_queries, int32_t num_keys, int32_t heads, int32_t head_dim, int64_t ldq, int64_t ldk,
               int64_t ldv, int64_t ld_out, void *stream) {
  REQUIRE(q && k && v && key_mask && out, "mha_f32: null pointer argument");
  REQUIRE(batch >= 0 && num_queries >= 0 && num_keys > 0 && heads > 0 && head_dim > 0, "mha_f32: bad sizes");
  const int64_t width = (int64_t)heads * head_dim;
  REQUIRE(ldq >= width && ldk >= width && ldv >= width && ld_out >= width, "mha_f32: row strides below heads * head_dim");
  SUPPORTED(num_keys <= 32768, "mha_f32: %d keys above 32768", num_keys);
  if (batch == 0 || num_queries == 0) return DX_OK;
  return check_launch(dx_mha_f32_launch(q, k, v, key_mask, out, batch, num_queries, num_keys, heads, head_dim, ldq, ldk,
                                        ldv, ld_out, as_stream(stream)),
                      "mha_f32 launch");
}

int dx_gather_rows_f32(const float *x, const int32_t *index, float *y, int32_t batch, int32_t rows_per_batch,
                       int32_t picks_per_batch, int64_t d, int64_t ldx, int64_t ldy, int32_t accumulate, void *stream) {
  REQUIRE(x && index && y, "gather_rows: null pointer argument");
  REQUIRE(batch >= 0 && rows_per_batch > 0 && picks_per_batch >= 0 && d > 0 && ldx >= d && ldy >= d,
          "gather_rows: bad sizes");
  if (batch == 0 || picks_per_batch == 0) return DX_OK;
  return check_launch(dx_gather_rows_f32_launch(x, index, y, batch, rows_per_batch, picks_per_batch, (int)d, ldx, ldy,
                                                accumulate ? 1 : 0, as_stream(stream)),
                      "gather_rows launch");
}

int dx_head_routing_f32(const float *options, const float *base, const int32_t *option_field,
                        const uint8_t *option_mask, float *summary, int32_t batch, int32_t num_options,
                        int32_t num_fields, int32_t width, void *stream) {
  REQUIRE(options && base && option_field && option_mask && summary, "head_routing: null pointer argument");
  REQUIRE(batch >= 0 && num_options > 0 && num_fields >= 0 && width > 0, "head_routing: bad sizes");
  SUPPORTED(num_options <= 16384, "head_routing: %d options above 16384", num_options);
  if (batch == 0 || num_fields == 0) return DX_OK;
  return check_launch(dx_routing_f32_launch(options, base, option_field, option_mask, summary, batch, num_options,
                                            num_fields, width, as_stream(stream)),
                      "head_routing launch");
}

int dx_head_fields_init_f32(const float *base, const float *summary_norm, const float *global_proj,
                            const float *type_embedding, const int32_t *types, float *fields, int32_t batch,
                            int32_t num_fields, int32_t width, int32_t num_types, void *stream) {
  REQUIRE(base && summary_norm && global_proj && type_embedding && types && fields,
          "head_fields_init: null pointer argument");
  REQUIRE(batch >= 0 && num_fields >= 0 && width > 0 && num_types > 0, "head_fields_init: bad sizes");
  if (batch == 0 || num_fields == 0) return DX_OK;
  return check_launch(dx_fields_init_f32_launch(base, summary_norm, global_proj, type_embedding, types, fields, batch,
                                                num_fields, width, num_types, as_stream(stream)),
                      "head_fields_init launch");
}

int dx_head_features_f32(const float *fields, const float *options, const float *questions, const float *global_vector,
                         const float *lexical, const int32_t *option_field, float *features, float *prior,
                         float *cosine, int32_t batch, int32_t num_options, int32_t num_fields, int32_t width,
                         int32_t hidden, float prior_scale, void *stream) {
  REQUIRE(fields && options && questions && global_vector && lexical && option_field && features && prior && cosine,
          "head_features: null pointer argument");
  REQUIRE(batch >= 0 && num_options >= 0 && num_fields > 0 && width > 0 && hidden > 0, "head_features: bad sizes");
  if (batch == 0 || num_options == 0) return DX_OK;
  return check_launch(dx_features_f32_launch(fields, options, questions, global_vector, lexical, option_field, features,
                                             prior, cosine, batch, num_options, num_fields, width, hidden, prior_scale,
                                             as_stream(stream)),
                      "head_features launch");
}

int dx_head_combine_f32(const float *prior, const float *cosine, const float *residual, const uint8_t *option_mask,
                        float *logits, int64_t n, float gate, float joint_scale, void *stream) {
  REQUIRE(prior && cosine && residual && option_mask && logits, "head_combine: null pointer argument");
  REQUIRE(n >= 0, "head_combine: bad size");
  if (n == 0) return DX_OK;
  return check_launch(dx_combine_f32_launch(prior, cosine, residual, option_mask, logits, n, gate, joint_scale,
                                            as_stream(stream)),
                      "head_combine launch");
}

