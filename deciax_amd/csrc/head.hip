// Clef joint schema head on gfx950, fp32 (the reference's head runs in the model dtype; its
// fixture and this path are fp32). The steps of src/deciax/models/clef/head.py:54-111 map onto a
// few kernels that the host driver (deciax_amd/clef_head.py) chains:
//   layer_norm_f32   nn.py:22-29 / head.py:20-21            one wave per row
//   linear_f32       nn.py:11-19 + text.py:21-22, + exact GELU and residual accumulate
//   span_means_f32   head.py:24-29                          one workgroup per span
//   mha_f32          head.py:41-51 core: masked softmax(q k^T / sqrt(dh)) v, blocked.py:9-32
//   gather_rows_f32  head.py:32-33                          (optionally accumulating)
//   routing_f32      head.py:76-85: per-question softmax over owned options and the summary
//   fields_init_f32  head.py:86-88
//   features_f32     head.py:97-106: anchor / prior, cosine, [f, o, f*o, |f-o|]
//   combine_f32      head.py:107-111
// The head's work is small next to the backbone (options <= 512, fields <= 64); the kernels favour
// plain, exactly-ordered fp32 arithmetic over throughput.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int THREADS = 256;
constexpr float MASK_FILL = -1e30f;  // src/deciax/kernels/attention/reference.py:8

DX_DEVICE float wave_reduce_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
DX_DEVICE float wave_reduce_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Sum / max over the 256 threads of a workgroup (every thread gets the result).
DX_DEVICE float block_sum(float v, float *red) {
  v = wave_reduce_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}
DX_DEVICE float block_max(float v, float *red) {
  v = wave_reduce_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

DX_DEVICE float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

// y = (x - mean) / sqrt(mean((x - mean)^2) + eps) * w + b, one wave per row.
__global__ void __launch_bounds__(THREADS)
layer_norm_f32_kernel(const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ b,
                      float *__restrict__ y, long rows, int d, long ldx, long ldy, float eps) {
  const long row = (long)blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const float *xr = x + row * ldx;
  float s = 0.f;
  for (int i = lane; i < d; i += 64) s += xr[i];
  const float mean = wave_reduce_sum(s) / (float)d;
  float q = 0.f;
  for (int i = lane; i < d; i += 64) {
    const float z = xr[i] - mean;
    q += z * z;
  }
  const float r = 1.0f / sqrtf(wave_reduce_sum(q) / (float)d + eps);
  float *yr = y + row * ldy;
  for (int i = lane; i < d; i += 64) yr[i] = (xr[i] - mean) * r * w[i] + (b ? b[i] : 0.f);
}

// y[m, n] = (acc ? y[m, n] : 0) + act(x[m, :] . w[n, :] + bias[n]); 64 x 64 output tile, 4 x 4 per
// thread, k in chunks of 16 through LDS. act: 0 identity, 1 exact GELU.
__global__ void __launch_bounds__(THREADS)
linear_f32_kernel(const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ bias,
                  float *__restrict__ y, long m, int n, int k, long ldx, long ldw, long ldy, int act, int acc) {
  __shared__ float xs[16][65];
  __shared__ float ws[16][65];
  const long m0 = (long)blockIdx.y * 64;
  const int n0 = blockIdx.x * 64;
  const int tid = threadIdx.x, tr = tid / 16, tc = tid % 16;
  float c[4][4] = {};
  for (int k0 = 0; k0 < k; k0 += 16) {
    for (int idx = tid; idx < 64 * 16; idx += THREADS) {
      const int r = idx / 16, kk = idx % 16;
      const long gm = m0 + r;
      const int gn = n0 + r, gk = k0 + kk;
      xs[kk][r] = (gm < m && gk < k) ? x[gm * ldx + gk] : 0.f;
      ws[kk][r] = (gn < n && gk < k) ? w[(long)gn * ldw + gk] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], bb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = xs[kk][tr * 4 + i];
        bb[i] = ws[kk][tc * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) c[i][j] = fmaf(a[i], bb[j], c[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const long gm = m0 + tr * 4 + i;
    if (gm >= m) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gn = n0 + tc * 4 + j;
      if (gn >= n) continue;
      float v = c[i][j] + (bias ? bias[gn] : 0.f);
      if (act == 1) v = gelu_erf(v);
      float *dst = y + gm * ldy + gn;
      *dst = acc ? *dst + v : v;
    }
  }
}

// out[b * O + o, :] = mean of x[b * S + s, :] over s in [spans[b, o, 0], spans[b, o, 1]) (within
// [0, S)); an empty span gives 0 (head.py:28 divides by max(count, 1)).
__global__ void __launch_bounds__(THREADS)
span_means_f32_kernel(const float *__restrict__ x, const int32_t *__restrict__ spans, float *__restrict__ out, int S,
                      int O, int d, long ldx, long ldo) {
  const int bo = blockIdx.x, b = bo / O;
  const int lo = max(spans[2 * bo], 0), hi = min(spans[2 * bo + 1], S);
  const float inv = 1.0f / (float)max(hi - lo, 1);
  for (int i = threadIdx.x; i < d; i += THREADS) {
    float s = 0.f;
    for (int t = lo; t < hi; ++t) s += x[((long)b * S + t) * ldx + i];
    out[(long)bo * ldo + i] = hi > lo ? s * inv : 0.f;
  }
}

// One workgroup per (b, query, head): scores over the K keys of batch row b into LDS, masked keys at
// MASK_FILL, softmax in fp32, then out = sum_k p_k v_k. q, k, v, out: rows of ld* floats, head h at
// columns [h dh, h dh + dh). key_mask: [B, K] bytes (nonzero = visible).
__global__ void __launch_bounds__(THREADS)
mha_f32_kernel(const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
               const uint8_t *__restrict__ key_mask, float *__restrict__ out, int Q, int K, int H, int dh, long ldq,
               long ldk, long ldv, long ldo) {
  extern __shared__ float smem[];  // K scores, then THREADS partial sums
  __shared__ float red[4];
  const int h = blockIdx.x % H, qi = (blockIdx.x / H) % Q, b = blockIdx.x / (H * Q);
  const float *qr = q + ((long)b * Q + qi) * ldq + (long)h * dh;
  const float scale = 1.0f / sqrtf((float)dh);
  float mx = MASK_FILL;
  for (int j = threadIdx.x; j < K; j += THREADS) {
    const float *kr = k + ((long)b * K + j) * ldk + (long)h * dh;
    float s = 0.f;
    for (int i = 0; i < dh; ++i) s = fmaf(qr[i], kr[i], s);
    s = key_mask[(long)b * K + j] ? s * scale : MASK_FILL;
    smem[j] = s;
    mx = fmaxf(mx, s);
  }
  mx = block_max(mx, red);
  float sum = 0.f;
  for (int j = threadIdx.x; j < K; j += THREADS) {
    const float p = expf(smem[j] - mx);
    smem[j] = p;
    sum += p;
  }
  sum = block_sum(sum, red);  // its barriers also publish the probabilities
  // dimensions [d0, d0 + dsub) per pass; thread t takes dimension d0 + t % dsub and keys t / dsub,
  // t / dsub + slices, ...; the slices' partial sums meet in LDS
  const int dsub = min(dh, THREADS), slices = THREADS / dsub;
  float *part = smem + K;
  for (int d0 = 0; d0 < dh; d0 += dsub) {
    const int i = d0 + (int)threadIdx.x % dsub, sl = (int)threadIdx.x / dsub;
    float acc = 0.f;
    if (i < dh && sl < slices)
      for (int j = sl; j < K; j += slices) acc = fmaf(smem[j], v[((long)b * K + j) * ldv + (long)h * dh + i], acc);
    part[threadIdx.x] = acc;
    __syncthreads();
    if ((int)threadIdx.x < min(dsub, dh - d0)) {
      float t = 0.f;
      for (int s2 = 0; s2 < slices; ++s2) t += part[s2 * dsub + threadIdx.x];
      out[((long)b * Q + qi) * ldo + (long)h * dh + d0 + threadIdx.x] = t / sum;
    }
    __syncthreads();
  }
}

// y[b * I + i, :] = (acc ? y : 0) + x[b * R + idx[b * I + i], :]
__global__ void __launch_bounds__(THREADS)
gather_rows_f32_kernel(const float *__restrict__ x, const int32_t *__restrict__ idx, float *__restrict__ y, int R,
                       int I, int d, long ldx, long ldy, int acc) {
  const int bi = blockIdx.x, b = bi / I;
  const int r = min(max(idx[bi], 0), R - 1);
  const float *src = x + ((long)b * R + r) * ldx;
  float *dst = y + (long)bi * ldy;
  for (int i = threadIdx.x; i < d; i += THREADS) dst[i] = acc ? dst[i] + src[i] : src[i];
}

// One workgroup per (b, question qi): logits[o] = options[b, o] . base[b, qi] / sqrt(W) over options
// this question owns (owner == qi and option_mask), MASK_FILL elsewhere; routing = softmax over o;
// summary[b, qi] = sum_o routing[o] * options[b, o] (head.py:76-85).
__global__ void __launch_bounds__(THREADS)
routing_f32_kernel(const float *__restrict__ options, const float *__restrict__ base, const int32_t *__restrict__ owner,
                   const uint8_t *__restrict__ option_mask, float *__restrict__ summary, int O, int NQ, int W) {
  extern __shared__ float p[];  // O routing weights
  __shared__ float red[4];
  const int qi = blockIdx.x % NQ, b = blockIdx.x / NQ;
  const float *br = base + ((long)b * NQ + qi) * W;
  const float inv = 1.0f / sqrtf((float)W);
  float mx = MASK_FILL;
  for (int o = threadIdx.x; o < O; o += THREADS) {
    const float *orow = options + ((long)b * O + o) * W;
    float s = 0.f;
    for (int i = 0; i < W; ++i) s = fmaf(orow[i], br[i], s);
    const bool owns = owner[(long)b * O + o] == qi && option_mask[(long)b * O + o];
    s = owns ? s * inv : MASK_FILL;
    p[o] = s;
    mx = fmaxf(mx, s);
  }
  mx = block_max(mx, red);
  float sum = 0.f;
  for (int o = threadIdx.x; o < O; o += THREADS) {
    const float e = expf(p[o] - mx);
    p[o] = e;
    sum += e;
  }
  sum = block_sum(sum, red);
  for (int i = threadIdx.x; i < W; i += THREADS) {
    float s = 0.f;
    for (int o = 0; o < O; ++o) s += (p[o] / sum) * options[((long)b * O + o) * W + i];
    summary[((long)b * NQ + qi) * W + i] = s;
  }
}

// fields[b, qi] = base[b, qi] + summary_norm[b, qi] + glob[b] + type_emb[types[b, qi]]
__global__ void __launch_bounds__(THREADS)
fields_init_f32_kernel(const float *__restrict__ base, const float *__restrict__ sn, const float *__restrict__ glob,
                       const float *__restrict__ type_emb, const int32_t *__restrict__ types, float *__restrict__ fields,
                       int NQ, int W, int num_types) {
  const int bq = blockIdx.x, b = bq / NQ;
  const int t = min(max(types[bq], 0), num_types - 1);
  for (int i = threadIdx.x; i < W; i += THREADS)
    fields[(long)bq * W + i] = ((base[(long)bq * W + i] + sn[(long)bq * W + i]) + glob[(long)b * W + i]) +
                               type_emb[(long)t * W + i];
}

DX_DEVICE float inv_length(float sumsq, float eps) { return 1.0f / fmaxf(sqrtf(sumsq), eps); }

// One workgroup per (b, o) (head.py:97-106): anchor = normalize(questions[b, owner] + glob[b]),
// prior = normalize(lexical[b, o]) . anchor * prior_scale, cosine of normalize(fields, 1e-8) and
// normalize(opts, 1e-8), features = [f, o, f * o, |f - o|]. questions / glob / lexical have H
// columns, fields / opts W.
__global__ void __launch_bounds__(THREADS)
features_f32_kernel(const float *__restrict__ fields, const float *__restrict__ opts, const float *__restrict__ questions,
                    const float *__restrict__ glob, const float *__restrict__ lexical, const int32_t *__restrict__ owner,
                    float *__restrict__ features, float *__restrict__ prior, float *__restrict__ cosine, int O, int NQ,
                    int W, int Hd, float prior_scale) {
  __shared__ float red[4];
  const int bo = blockIdx.x, b = bo / O;
  const int qi = min(max(owner[bo], 0), NQ - 1);
  const float *qr = questions + ((long)b * NQ + qi) * Hd, *gr = glob + (long)b * Hd, *lr = lexical + (long)bo * Hd;
  float sa = 0.f, sl = 0.f;
  for (int i = threadIdx.x; i < Hd; i += THREADS) {
    const float a = qr[i] + gr[i];
    sa += a * a;
    sl += lr[i] * lr[i];
  }
  const float ia = inv_length(block_sum(sa, red), 1e-12f), il = inv_length(block_sum(sl, red), 1e-12f);
  float dp = 0.f;
  for (int i = threadIdx.x; i < Hd; i += THREADS) dp += (lr[i] * il) * ((qr[i] + gr[i]) * ia);
  dp = block_sum(dp, red);
  const float *fr = fields + (long)bo * W, *orow = opts + (long)bo * W;
  float sf = 0.f, so = 0.f;
  for (int i = threadIdx.x; i < W; i += THREADS) {
    sf += fr[i] * fr[i];
    so += orow[i] * orow[i];
  }
  const float jf = inv_length(block_sum(sf, red), 1e-8f), jo = inv_length(block_sum(so, red), 1e-8f);
  float cs = 0.f;
  float *ft = features + (long)bo * 4 * W;
  for (int i = threadIdx.x; i < W; i += THREADS) {
    const float f = fr[i], o = orow[i];
    cs += (f * jf) * (o * jo);
    ft[i] = f;
    ft[W + i] = o;
    ft[2 * W + i] = f * o;
    ft[3 * W + i] = fabsf(f - o);
  }
  cs = block_sum(cs, red);
  if (threadIdx.x == 0) {
    prior[bo] = dp * prior_scale;
    cosine[bo] = cs;
  }
}

// out[b, o] = option_mask ? prior + gate * (joint_scale * cosine + residual) : -1e9
__global__ void __launch_bounds__(THREADS)
combine_f32_kernel(const float *__restrict__ prior, const float *__restrict__ cosine, const float *__restrict__ residual,
                   const uint8_t *__restrict__ option_mask, float *__restrict__ out, long n, float gate,
                   float joint_scale) {
  const long i = (long)blockIdx.x * THREADS + threadIdx.x;
  if (i >= n) return;
  out[i] = option_mask[i] ? prior[i] + gate * (joint_scale * cosine[i] + residual[i]) : -1e9f;
}

unsigned blocks(long n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

hipError_t dx_layer_norm_f32_launch(const float *x, const float *w, const float *b, float *y, long rows, int d,
                                    long ldx, long ldy, float eps, hipStream_t s) {
  layer_norm_f32_kernel<<<blocks(rows, THREADS / 64), THREADS, 0, s>>>(x, w, b, y, rows, d, ldx, ldy, eps);
  return hipGetLastError();
}

hipError_t dx_linear_f32_launch(const float *x, const float *w, const float *bias, float *y, long m, int n, int k,
                                long ldx, long ldw, long ldy, int act, int acc, hipStream_t s) {
  const dim3 grid(blocks(n, 64), blocks(m, 64));
  linear_f32_kernel<<<grid, THREADS, 0, s>>>(x, w, bias, y, m, n, k, ldx, ldw, ldy, act, acc);
  return hipGetLastError();
}

hipError_t dx_span_means_f32_launch(const float *x, const int32_t *spans, float *out, int B, int S, int O, int d,
                                    long ldx, long ldo, hipStream_t s) {
  span_means_f32_kernel<<<(unsigned)(B * O), THREADS, 0, s>>>(x, spans, out, S, O, d, ldx, ldo);
  return hipGetLastError();
}

hipError_t dx_mha_f32_launch(const float *q, const float *k, const float *v, const uint8_t *key_mask, float *out,
                             int B, int Q, int K, int H, int dh, long ldq, long ldk, long ldv, long ldo, hipStream_t s) {
  const size_t shm = ((size_t)K + THREADS) * sizeof(float);
  mha_f32_kernel<<<(unsigned)(B * Q * H), THREADS, shm, s>>>(q, k, v, key_mask, out, Q, K, H, dh, ldq, ldk, ldv, ldo);
  return hipGetLastError();
}

hipError_t dx_gather_rows_f32_launch(const float *x, const int32_t *idx, float *y, int B, int R, int I, int d,
                                     long ldx, long ldy, int acc, hipStream_t s) {
  gather_rows_f32_kernel<<<(unsigned)(B * I), THREADS, 0, s>>>(x, idx, y, R, I, d, ldx, ldy, acc);
  return hipGetLastError();
}

hipError_t dx_routing_f32_launch(const float *options, const float *base, const int32_t *owner,
                                 const uint8_t *option_mask, float *summary, int B, int O, int NQ, int W,
                                 hipStream_t s) {
  routing_f32_kernel<<<(unsigned)(B * NQ), THREADS, (size_t)O * sizeof(float), s>>>(options, base, owner, option_mask,
                                                                                    summary, O, NQ, W);
  return hipGetLastError();
}

hipError_t dx_fields_init_f32_launch(const float *base, const float *sn, const float *glob, const float *type_emb,
                                     const int32_t *types, float *fields, int B, int NQ, int W, int num_types,
                                     hipStream_t s) {
  fields_init_f32_kernel<<<(unsigned)(B * NQ), THREADS, 0, s>>>(base, sn, glob, type_emb, types, fields, NQ, W,
                                                                num_types);
  return hipGetLastError();
}

hipError_t dx_features_f32_launch(const float *fields, const float *opts, const float *questions, const float *glob,
                                  const float *lexical, const int32_t *owner, float *features, float *prior,
                                  float *cosine, int B, int O, int NQ, int W, int Hd, float prior_scale,
                                  hipStream_t s) {
  features_f32_kernel<<<(unsigned)(B * O), THREADS, 0, s>>>(fields, opts, questions, glob, lexical, owner, features,
                                                            prior, cosine, O, NQ, W, Hd, prior_scale);
  return hipGetLastError();
}

hipError_t dx_combine_f32_launch(const float *prior, const float *cosine, const float *residual,
                                 const uint8_t *option_mask, float *out, long n, float gate, float joint_scale,
                                 hipStream_t s) {
  combine_f32_kernel<<<blocks(n, THREADS), THREADS, 0, s>>>(prior, cosine, residual, option_mask, out, n, gate,
                                                            joint_scale);
  return hipGetLastError();
}
