// Memory-bound row kernels: RMSNorm family, embedding gather, RoPE, gate|up
// packing and the option readout. One wavefront per row; rows are read as
// 16-byte chunks (8 bf16) held in registers between the two passes that an
// RMSNorm needs (sum of squares, then scale).
//
// RMSNorm follows the reference exactly in fp32
// (src/deciax/models/qwen3_5/text.py:25-28, src/deciax/kernels/projection.py:31-33):
//   v = x * rsqrt(mean(x^2) + eps);  v = v * (1 + w);  round to bf16.
#include "common.h"
#include "kernels.h"
#include "rownorm.h"

namespace {

constexpr int THREADS = 256;
constexpr int ROWS_PER_BLOCK = THREADS / 64;

template <int MAXC>
__global__ void __launch_bounds__(THREADS)
rmsnorm_kernel(const uint16_t *__restrict__ x, const uint16_t *__restrict__ w, uint16_t *__restrict__ y,
               const uint8_t *__restrict__ mask, long rows, int d, long ldx, long ldy, float eps) {
  const long row = (long)blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int nch = d / 8;
  Row<MAXC> xr, out;
  load_row(xr, x + row * ldx, nch, lane);
  const float inv = rms_inv(row_sumsq(xr, nch, lane), d, eps);
  row_scale(out, xr, w, inv, nch, lane);
  if (mask && !mask[row]) {
#pragma unroll
    for (int i = 0; i < MAXC; ++i) out.c[i] = u32x4{0, 0, 0, 0};
  }
  store_row(out, y + row * ldy, nch, lane);
}

template <int MAXC, bool POST, bool NEXT>
__global__ void __launch_bounds__(THREADS)
add_rmsnorm_kernel(const uint16_t *__restrict__ y, const uint16_t *__restrict__ post_w, uint16_t *__restrict__ x,
                   const uint16_t *__restrict__ next_w, uint16_t *__restrict__ h, long rows, int d, float eps) {
  const long row = (long)blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  add_rmsnorm_row<MAXC, POST, NEXT, false>(y + row * d, post_w, x + row * d, next_w, h + row * d, d, eps, lane);
}

template <int MAXC, bool NORM>
__global__ void __launch_bounds__(THREADS)
embed_kernel(const int32_t *__restrict__ ids, const uint16_t *__restrict__ table, uint16_t *__restrict__ x,
             long tokens, int d, long vocab, float scale, const uint16_t *__restrict__ norm_w,
             uint16_t *__restrict__ h, float eps) {
  const long row = (long)blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= tokens) return;
  const int nch = d / 8;
  const long id = min(max((long)ids[row], 0L), vocab - 1);
  Row<MAXC> xr;
  load_row(xr, table + id * d, nch, lane);
  if (scale != 1.f) {
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
#pragma unroll
        for (int j = 0; j < 4; ++j) xr.c[i][j] = pack_bf2(lo_bf(xr.c[i][j]) * scale, hi_bf(xr.c[i][j]) * scale);
      }
    }
  }
  store_row(xr, x + row * d, nch, lane);
  if constexpr (NORM) {
    Row<MAXC> hr;
    const float inv = rms_inv(row_sumsq(xr, nch, lane), d, eps);
    row_scale(hr, xr, norm_w, inv, nch, lane);
    store_row(hr, h + row * d, nch, lane);
  }
}

// One thread per (row, head, 8 consecutive rotary pairs).
__global__ void __launch_bounds__(THREADS)
rope_kernel(uint16_t *__restrict__ x, const int32_t *__restrict__ pos, const uint16_t *__restrict__ cos_t,
            const uint16_t *__restrict__ sin_t, long rows, int heads, int d, long stride, int max_pos) {
  const int per_head = d / 16;
  const long gid = (long)blockIdx.x * THREADS + threadIdx.x;
  if (gid >= rows * heads * per_head) return;
  const long row = gid / (heads * per_head);
  const int rem = (int)(gid % (heads * per_head));
  const int head = rem / per_head, j0 = (rem % per_head) * 8;
  const int p = min(max(pos[row], 0), max_pos - 1);
  uint16_t *x1 = x + row * stride + (long)head * d + j0;
  uint16_t *x2 = x1 + d / 2;
  const u32x4 a = *reinterpret_cast<const u32x4 *>(x1);
  const u32x4 b = *reinterpret_cast<const u32x4 *>(x2);
  const u32x4 c = *reinterpret_cast<const u32x4 *>(cos_t + (long)p * (d / 2) + j0);
  const u32x4 s = *reinterpret_cast<const u32x4 *>(sin_t + (long)p * (d / 2) + j0);
  u32x4 o1, o2;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float r1[2], r2[2];
    const float av[2] = {lo_bf(a[j]), hi_bf(a[j])}, bv[2] = {lo_bf(b[j]), hi_bf(b[j])};
    const float cv[2] = {lo_bf(c[j]), hi_bf(c[j])}, sv[2] = {lo_bf(s[j]), hi_bf(s[j])};
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      r1[e] = round_bf(av[e] * cv[e]) - round_bf(bv[e] * sv[e]);
      r2[e] = round_bf(bv[e] * cv[e]) + round_bf(av[e] * sv[e]);
    }
    o1[j] = pack_bf2(r1[0], r1[1]);
    o2[j] = pack_bf2(r2[0], r2[1]);
  }
  *reinterpret_cast<u32x4 *>(x1) = o1;
  *reinterpret_cast<u32x4 *>(x2) = o2;
}

// packed row 128 b + i: gate row 64 b + i (i < 64), else up row 64 b + i - 64.
__global__ void __launch_bounds__(THREADS)
pack_gate_up_kernel(const uint16_t *__restrict__ gate, const uint16_t *__restrict__ up,
                    uint16_t *__restrict__ packed, long f, long k) {
  const long nch = k / 8;
  const long gid = (long)blockIdx.x * THREADS + threadIdx.x;
  if (gid >= 2 * f * nch) return;
  const long prow = gid / nch, c = gid % nch;
  const long blk = prow / 128, i = prow % 128;
  const uint16_t *src = i < 64 ? gate + (blk * 64 + i) * k : up + (blk * 64 + i - 64) * k;
  *reinterpret_cast<u32x4 *>(packed + prow * k + c * 8) = *reinterpret_cast<const u32x4 *>(src + c * 8);
}

// One workgroup per question; each wave scores options in turn, then the
// workgroup takes the softmax over the question's options.
// Readout: one workgroup per question, RO_WAVES waves, one option per wave at a time. Each wave requests
// its option's hidden row and label row together, so an option costs one memory round trip (the norm
// weights, shared by every option, come from L2); the products and the summation order are those of
// row_scale.
constexpr int RO_WAVES = 8;
constexpr int RO_MAX_LDS = 512;  // the most options one request may hold

template <int MAXC>
__global__ void __launch_bounds__(64 * RO_WAVES)
readout_kernel(const uint16_t *__restrict__ hidden, const uint16_t *__restrict__ norm_w,
               const uint16_t *__restrict__ table, const int32_t *__restrict__ opt_pos,
               const int32_t *__restrict__ opt_label, const int32_t *__restrict__ q_off, int num_options,
               long hidden_rows, int d, long ld_hidden,
               long vocab, float eps, float softcap, float *__restrict__ logits, float *__restrict__ probs) {
  __shared__ float red[RO_WAVES];
  __shared__ float zs[RO_MAX_LDS];  // the question's logits, when it has at most RO_MAX_LDS options
  __shared__ u32x4 wsh[MAXC * 64];  // the final norm's weights, 16-byte chunks
  const int q = blockIdx.x;
  // The offsets come from device memory: clamp the question's range into [0, num_options) so that a
  // malformed offset array can give wrong answers but never reads or writes outside the option arrays.
  const int o0 = min(max(q_off[q], 0), num_options);
  const int o1 = min(max(q_off[q + 1], o0), num_options);
  const bool in_lds = o1 - o0 <= RO_MAX_LDS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = d / 8;
  // The norm weights, shared by every option, are staged in LDS once per workgroup while the offsets
  // resolve: read from global memory inside the dot loop they cost one dependent round trip per 16-byte
  // chunk, and held in registers beside both rows they spill at H 4608.
  for (int c = threadIdx.x; c < nch; c += 64 * RO_WAVES) wsh[c] = *reinterpret_cast<const u32x4 *>(norm_w + c * 8);
  __syncthreads();
  for (int o = o0 + wave; o < o1; o += RO_WAVES) {
    Row<MAXC> xr, er;
    const long prow = min(max((long)opt_pos[o], 0L), hidden_rows - 1);
    const long lab = min(max((long)opt_label[o], 0L), vocab - 1);
    load_row(xr, hidden + prow * ld_hidden, nch, lane);
    load_row(er, table + lab * d, nch, lane);
    const float inv = rms_inv(row_sumsq(xr, nch, lane), d, eps);
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
        const u32x4 wc = wsh[c];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t g = pack_bf2((lo_bf(xr.c[i][j]) * inv) * (1.f + lo_bf(wc[j])),
                                      (hi_bf(xr.c[i][j]) * inv) * (1.f + hi_bf(wc[j])));
          dot = fmaf(lo_bf(g), lo_bf(er.c[i][j]), dot);
          dot = fmaf(hi_bf(g), hi_bf(er.c[i][j]), dot);
        }
      }
    }
    dot = wave_sum(dot);
    const float z = softcap > 0.f ? softcap * tanhf(dot / softcap) : dot;
    if (lane == 0) {
      logits[o] = z;
      if (in_lds) zs[o - o0] = z;
    }
  }
  __threadfence_block();
  __syncthreads();
  auto logit = [&](int o) { return in_lds ? zs[o - o0] : logits[o]; };
  float m = -INFINITY;
  for (int o = o0 + (int)threadIdx.x; o < o1; o += 64 * RO_WAVES) m = fmaxf(m, logit(o));
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = red[0];
#pragma unroll
  for (int w = 1; w < RO_WAVES; ++w) m = fmaxf(m, red[w]);
  __syncthreads();
  float s = 0.f;
  for (int o = o0 + (int)threadIdx.x; o < o1; o += 64 * RO_WAVES) s += expf(logit(o) - m);
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  s = 0.f;
#pragma unroll
  for (int w = 0; w < RO_WAVES; ++w) s += red[w];
  for (int o = o0 + (int)threadIdx.x; o < o1; o += 64 * RO_WAVES) probs[o] = expf(logit(o) - m) / s;
}

// TWELVE: rows of 9-12 chunks per lane take 12-chunk register rows instead of 16 (H 4608, the 27B width,
// is 9 chunks per lane).
template <template <int> class F, bool TWELVE = false, typename... Args>
hipError_t by_chunks(int d, Args... args) {
  const int per_lane = (d / 8 + 63) / 64;
  if (per_lane <= 1) return F<1>::run(args...);
  if (per_lane <= 2) return F<2>::run(args...);
  if (per_lane <= 4) return F<4>::run(args...);
  if (per_lane <= 8) return F<8>::run(args...);
  if constexpr (TWELVE)
    if (per_lane <= 12) return F<12>::run(args...);
  return F<16>::run(args...);
}

inline dim3 row_grid(long rows) { return dim3((unsigned)((rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK)); }

template <int MAXC>
struct RmsRun {
  static hipError_t run(const uint16_t *x, const uint16_t *w, uint16_t *y, const uint8_t *mask, long rows, int d,
                        long ldx, long ldy, float eps, hipStream_t s) {
    rmsnorm_kernel<MAXC><<<row_grid(rows), dim3(THREADS), 0, s>>>(x, w, y, mask, rows, d, ldx, ldy, eps);
    return hipGetLastError();
  }
};

template <int MAXC>
struct AddRmsRun {
  static hipError_t run(const uint16_t *y, const uint16_t *pw, uint16_t *x, const uint16_t *nw, uint16_t *h,
                        long rows, int d, float eps, hipStream_t s) {
    const dim3 grid = row_grid(rows), block(THREADS);
    if (pw && h)
      add_rmsnorm_kernel<MAXC, true, true><<<grid, block, 0, s>>>(y, pw, x, nw, h, rows, d, eps);
    else if (pw)
      add_rmsnorm_kernel<MAXC, true, false><<<grid, block, 0, s>>>(y, pw, x, nw, h, rows, d, eps);
    else if (h)
      add_rmsnorm_kernel<MAXC, false, true><<<grid, block, 0, s>>>(y, pw, x, nw, h, rows, d, eps);
    else
      add_rmsnorm_kernel<MAXC, false, false><<<grid, block, 0, s>>>(y, pw, x, nw, h, rows, d, eps);
    return hipGetLastError();
  }
};

template <int MAXC>
struct EmbedRun {
  static hipError_t run(const int32_t *ids, const uint16_t *table, uint16_t *x, long tokens, int d, long vocab,
                        float scale, const uint16_t *nw, uint16_t *h, float eps, hipStream_t s) {
    if (h)
      embed_kernel<MAXC, true><<<row_grid(tokens), dim3(THREADS), 0, s>>>(ids, table, x, tokens, d, vocab, scale, nw,
                                                                         h, eps);
    else
      embed_kernel<MAXC, false><<<row_grid(tokens), dim3(THREADS), 0, s>>>(ids, table, x, tokens, d, vocab, scale,
                                                                          nw, h, eps);
    return hipGetLastError();
  }
};

template <int MAXC>
struct ReadoutRun {
  static hipError_t run(const uint16_t *hidden, const uint16_t *nw, const uint16_t *table, const int32_t *pos,
                        const int32_t *lab, const int32_t *q_off, int nq, int nopt, long hrows, int d, long ldh,
                        long vocab, float eps, float softcap, float *logits, float *probs, hipStream_t s) {
    readout_kernel<MAXC><<<dim3(nq), dim3(64 * RO_WAVES), 0, s>>>(hidden, nw, table, pos, lab, q_off, nopt, hrows, d,
                                                                  ldh, vocab, eps, softcap, logits, probs);
    return hipGetLastError();
  }
};

}  // namespace

hipError_t dx_rmsnorm_launch(const uint16_t *x, const uint16_t *w, uint16_t *y, const uint8_t *mask, long rows,
                             int d, long ldx, long ldy, float eps, hipStream_t s) {
  return by_chunks<RmsRun>(d, x, w, y, mask, rows, d, ldx, ldy, eps, s);
}

hipError_t dx_add_rmsnorm_launch(const uint16_t *y, const uint16_t *post_w, uint16_t *x, const uint16_t *next_w,
                                 uint16_t *h, long rows, int d, float eps, hipStream_t s) {
  // 12-chunk rows at H 4608 leave room for the prefetched norm weights (add_rmsnorm_row): 65536 x 4608
  // 520 -> 454 us, bit-identical; rmsnorm and embed measured 2-3% slower with them and keep 16
  return by_chunks<AddRmsRun, true>(d, y, post_w, x, next_w, h, rows, d, eps, s);
}

hipError_t dx_embed_launch(const int32_t *ids, const uint16_t *table, uint16_t *x, long tokens, int d, long vocab,
                           float scale, const uint16_t *norm_w, uint16_t *h, float eps, hipStream_t s) {
  return by_chunks<EmbedRun>(d, ids, table, x, tokens, d, vocab, scale, norm_w, h, eps, s);
}

hipError_t dx_rope_launch(uint16_t *x, const int32_t *pos, const uint16_t *cos, const uint16_t *sin, long rows,
                          int heads, int d, long stride, int max_pos, hipStream_t s) {
  const long total = rows * heads * (d / 16);
  rope_kernel<<<dim3((unsigned)((total + THREADS - 1) / THREADS)), dim3(THREADS), 0, s>>>(x, pos, cos, sin, rows,
                                                                                          heads, d, stride, max_pos);
  return hipGetLastError();
}

hipError_t dx_readout_launch(const uint16_t *hidden, const uint16_t *norm_w, const uint16_t *table,
                             const int32_t *opt_pos, const int32_t *opt_label, const int32_t *q_off, int nq,
                             int num_options, long hidden_rows, int d, long ld_hidden, long vocab, float eps,
                             float softcap, float *logits, float *probs, hipStream_t s) {
  return by_chunks<ReadoutRun>(d, hidden, norm_w, table, opt_pos, opt_label, q_off, nq, num_options, hidden_rows, d,
                               ld_hidden, vocab, eps, softcap, logits, probs, s);
}

hipError_t dx_pack_gate_up_launch(const uint16_t *gate, const uint16_t *up, uint16_t *packed, long f, long k,
                                  hipStream_t s) {
  const long total = 2 * f * (k / 8);
  pack_gate_up_kernel<<<dim3((unsigned)((total + THREADS - 1) / THREADS)), dim3(THREADS), 0, s>>>(gate, up, packed,
                                                                                                 f, k);
  return hipGetLastError();
}
