// Shared device helpers for the gfx950 decision-prefill kernels.
//
// Storage type for bf16 is uint16_t (raw bits); arithmetic happens in fp32 and
// every rounding back to bf16 is round-to-nearest-even, the rounding JAX and
// PyTorch apply on `astype(bfloat16)`.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "deciax_hip.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

#define DX_DEVICE __device__ __forceinline__

DX_DEVICE float bf2f(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }

DX_DEVICE uint16_t f2bf(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(uint16_t, b);
}

// Two fp32 values -> one dword of two bf16 (lo in the low half).
DX_DEVICE uint32_t pack_bf2(float lo, float hi) {
  typedef float floatx2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const floatx2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));  // one v_cvt_pk_bf16_f32
}

// Round an fp32 value to the nearest bf16 and return it as fp32: the bf16 in the high half over a zero low
// half is that value's fp32 bit pattern, so this is one conversion and no shift.
DX_DEVICE float round_bf(float f) { return __uint_as_float(pack_bf2(0.f, f)); }

DX_DEVICE float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
DX_DEVICE float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

DX_DEVICE bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// 32x32x16 bf16 MFMA: D[32x32] += A[32x16] * B[16x32].
// Lane l supplies A row (l % 32) and B column (l % 32), eight k-values each;
// D is returned with lane l holding column (l % 32), rows
// (r / 4) * 8 + (l / 32) * 4 + (r % 4) for r = 0..15.
DX_DEVICE floatx16 mfma32(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

DX_DEVICE float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
DX_DEVICE float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// Sum over the 64 lanes of a wavefront.
DX_DEVICE float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

DX_DEVICE float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// GELU with the tanh approximation, 0.5 x (1 + tanh(y)), y = sqrt(2/pi) (x + 0.044715 x^3).
// Since 1 + tanh(y) = 2 / (1 + e^{-2y}) this is x / (1 + 2^{-x (c1 + c2 x^2)}) with
// c1 = 2 sqrt(2/pi) log2(e) and c2 = 0.044715 c1: one exp2 and one reciprocal, and no
// cancellation for negative x (relative error about 1e-6 against the exact formula).
DX_DEVICE float gelu_tanh(float x) {
  const float e = fast_exp2(x * __builtin_fmaf(x * x, -0.1029432395800235f, -2.302208198144325f));
  return x * fast_rcp(1.0f + e);
}

// SiLU x * sigmoid(x).
DX_DEVICE float silu(float x) { return x * fast_rcp(1.0f + fast_exp2(-1.4426950408889634f * x)); }

static inline int dx_ceil_div(long a, long b) { return (int)((a + b - 1) / b); }
