// Row helpers shared by the row kernels (rowwise.hip) and the GEMM's residual-norm epilogue (gemm.hip):
// one wavefront per row, the row held in registers as 16-byte chunks (8 bf16), chunk c = lane + 64 i.
// Both callers run these same functions, so their results are bit-identical.
//
// RMSNorm follows the reference exactly in fp32
// (src/deciax/models/qwen3_5/text.py:25-28, src/deciax/kernels/projection.py:31-33):
//   v = x * rsqrt(mean(x^2) + eps);  v = v * (1 + w);  round to bf16.
#pragma once

#include "common.h"

namespace {

template <int MAXC>
struct Row {
  u32x4 c[MAXC];
};

template <int MAXC>
DX_DEVICE void load_row(Row<MAXC> &r, const uint16_t *p, int nch, int lane) {
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) r.c[i] = *reinterpret_cast<const u32x4 *>(p + c * 8);
  }
}

template <int MAXC>
DX_DEVICE void store_row(const Row<MAXC> &r, uint16_t *p, int nch, int lane) {
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) *reinterpret_cast<u32x4 *>(p + c * 8) = r.c[i];
  }
}

template <int MAXC>
DX_DEVICE float row_sumsq(const Row<MAXC> &r, int nch, int lane) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = lo_bf(r.c[i][j]), b = hi_bf(r.c[i][j]);
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
    }
  }
  return wave_sum(ss);
}

// out = bf16((x * inv) * (1 + w)) with w already loaded (the same products as row_scale).
template <int MAXC>
DX_DEVICE void row_scale_w(Row<MAXC> &out, const Row<MAXC> &x, const Row<MAXC> &w, float inv, int nch, int lane) {
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = (lo_bf(x.c[i][j]) * inv) * (1.f + lo_bf(w.c[i][j]));
        const float b = (hi_bf(x.c[i][j]) * inv) * (1.f + hi_bf(w.c[i][j]));
        out.c[i][j] = pack_bf2(a, b);
      }
    }
  }
}

// out = bf16((x * inv) * (1 + w)), elementwise over the row.
template <int MAXC>
DX_DEVICE void row_scale(Row<MAXC> &out, const Row<MAXC> &x, const uint16_t *w, float inv, int nch, int lane) {
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      const u32x4 wc = *reinterpret_cast<const u32x4 *>(w + c * 8);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = (lo_bf(x.c[i][j]) * inv) * (1.f + lo_bf(wc[j]));
        const float b = (hi_bf(x.c[i][j]) * inv) * (1.f + hi_bf(wc[j]));
        out.c[i][j] = pack_bf2(a, b);
      }
    }
  }
}

DX_DEVICE float rms_inv(float ss, int d, float eps) { return rsqrtf(ss / (float)d + eps); }

// y with system-coherent loads (sc0 sc1: served from memory, not from a possibly stale cache), for rows
// that other workgroups wrote in the same kernel with system-coherent stores.
template <int MAXC>
DX_DEVICE void load_row_coherent(Row<MAXC> &r, const uint16_t *p, int nch, int lane) {
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, nch * 16, 0x00020000);
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) r.c[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, c * 16, 0, 17));
  }
}

// The residual update's arithmetic on rows already in registers (y, x), storing x and h; the weights are
// read where used. Its products and sums are those of add_rmsnorm_row below.
template <int MAXC, bool NEXT>
DX_DEVICE void add_rmsnorm_regs(Row<MAXC> &yr, Row<MAXC> &xr, const uint16_t *post_w, uint16_t *x,
                                const uint16_t *next_w, uint16_t *h, int d, float eps, int lane) {
  const int nch = d / 8;
  const float inv = rms_inv(row_sumsq(yr, nch, lane), d, eps);
  row_scale(yr, yr, post_w, inv, nch, lane);
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        xr.c[i][j] = pack_bf2(lo_bf(xr.c[i][j]) + lo_bf(yr.c[i][j]), hi_bf(xr.c[i][j]) + hi_bf(yr.c[i][j]));
    }
  }
  store_row(xr, x, nch, lane);
  if constexpr (NEXT) {
    const float inv2 = rms_inv(row_sumsq(xr, nch, lane), d, eps);
    row_scale(yr, xr, next_w, inv2, nch, lane);
    store_row(yr, h, nch, lane);
  }
}

// Residual update of one row (the Gemma-2 sandwich half-layer):
//   t = POST ? bf16(rms(y) (1 + post_w)) : y;  x = bf16(x + t);  if NEXT: h = bf16(rms(x) (1 + next_w)).
// COHERENT reads y with load_row_coherent.
template <int MAXC, bool POST, bool NEXT, bool COHERENT>
DX_DEVICE void add_rmsnorm_row(const uint16_t *y, const uint16_t *post_w, uint16_t *x, const uint16_t *next_w,
                               uint16_t *h, int d, float eps, int lane) {
  const int nch = d / 8;
  // Rows of up to 12 chunks per lane request the norm weights with the rows (the next norm's once the
  // first is used), so their latency hides behind the row loads and the sums (H 3584: -3.8%; H 4608 in
  // 12-chunk rows: -12.9%). 16-chunk rows read them where used: a third 64-register row costs them
  // occupancy (H 4608 in 16-chunk rows: +14%).
  constexpr bool PREFETCH = MAXC <= 12;
  Row<MAXC> yr, xr, wr;
  if constexpr (COHERENT) load_row_coherent(yr, y, nch, lane);
  else load_row(yr, y, nch, lane);
  load_row(xr, x, nch, lane);
  if constexpr (PREFETCH && POST) load_row(wr, post_w, nch, lane);
  else if constexpr (PREFETCH && NEXT) load_row(wr, next_w, nch, lane);
  if constexpr (POST) {
    const float inv = rms_inv(row_sumsq(yr, nch, lane), d, eps);
    if constexpr (PREFETCH) {
      row_scale_w(yr, yr, wr, inv, nch, lane);
      if constexpr (NEXT) load_row(wr, next_w, nch, lane);
    } else {
      row_scale(yr, yr, post_w, inv, nch, lane);
    }
  }
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        xr.c[i][j] = pack_bf2(lo_bf(xr.c[i][j]) + lo_bf(yr.c[i][j]), hi_bf(xr.c[i][j]) + hi_bf(yr.c[i][j]));
    }
  }
  store_row(xr, x, nch, lane);
  if constexpr (NEXT) {
    const float inv = rms_inv(row_sumsq(xr, nch, lane), d, eps);
    if constexpr (PREFETCH) row_scale_w(yr, xr, wr, inv, nch, lane);
    else row_scale(yr, xr, next_w, inv, nch, lane);
    store_row(yr, h, nch, lane);
  }
}

}  // namespace
