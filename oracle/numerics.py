"""bf16 rounding and the elementwise functions of the path (test infrastructure only)."""

from __future__ import annotations

from collections.abc import Iterator
from contextlib import contextmanager

import numpy as np

F32 = np.float32
ORDERS = ("blas", "k_tiles", "k_tiles_reversed")
K_TILE = 64
_ACC = [(np.dtype(np.float32), "blas")]


def acc_dtype() -> np.dtype:
    """Accumulation dtype of the oracle's contractions (fp32 unless inside `accumulation`)."""
    return _ACC[-1][0]


@contextmanager
def accumulation(dtype: type, order: str = "blas") -> Iterator[None]:
    """Run the oracle's matrix products in `dtype` (np.float64 gives the exactly-summed value of
    every contraction, up to the bf16 rounding points, to measure fp32 summation-order noise).

    `order` picks one of three valid summation orders of a contraction: "blas" is numpy's BLAS
    blocking; "k_tiles" sums K in tiles of 64, each tile's partial product added to the running
    sum in turn, as a tiled GEMM walks K; "k_tiles_reversed" walks the same tiles from the last.
    In fp64 they agree to fp64 rounding."""
    if order not in ORDERS:
        raise ValueError(f"order must be one of {ORDERS}, got {order!r}")
    _ACC.append((np.dtype(dtype), order))
    try:
        yield
    finally:
        _ACC.pop()


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """a @ b accumulated in `acc_dtype()` in the current summation order, returned as fp32."""
    d, order = _ACC[-1]
    a, b = np.asarray(a, d), np.asarray(b, d)
    if order == "blas" or a.shape[-1] <= K_TILE:
        return (a @ b).astype(F32)
    starts = list(range(0, a.shape[-1], K_TILE))
    if order == "k_tiles_reversed":
        starts.reverse()
    acc = a[..., starts[0]:starts[0] + K_TILE] @ b[starts[0]:starts[0] + K_TILE]
    for k0 in starts[1:]:
        acc += a[..., k0:k0 + K_TILE] @ b[k0:k0 + K_TILE]
    return acc.astype(F32)


def bf16(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to the nearest bf16 (ties to even); result kept as fp32.

    This is the rounding of `astype(jnp.bfloat16)` in the reference (e.g.
    src/deciax/kernels/swiglu.py:100-101) and of torch's `.to(torch.bfloat16)`."""
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32)
    rounded = (u + (((u >> 16) & 1) + np.uint32(0x7FFF))) & np.uint32(0xFFFF0000)
    out = rounded.view(F32).copy()
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.nan
    return out


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """uint16 bit patterns of bf16(x)."""
    return (bf16(x).view(np.uint32) >> 16).astype(np.uint16)


def from_bits(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> fp32 values."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(F32)


def maybe(x: np.ndarray, on: bool) -> np.ndarray:
    return bf16(x) if on else np.asarray(x, F32)


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) — TF/activations.py:31-45
    (`gelu_pytorch_tanh`, the Gemma-2 hidden activation)."""
    x = np.asarray(x, F32)
    inner = F32(0.7978845608028654) * (x + F32(0.044715) * x * x * x)
    return (F32(0.5) * x * (F32(1.0) + np.tanh(inner))).astype(F32)


def silu(x: np.ndarray) -> np.ndarray:
    """x * sigmoid(x) — the reference's SwiGLU activation (src/deciax/kernels/swiglu.py:101)."""
    x = np.asarray(x, F32)
    return (x / (F32(1.0) + np.exp(-x))).astype(F32)


ACTIVATIONS = {"gelu_tanh": gelu_tanh, "silu": silu}


def softcap(x: np.ndarray, cap: float) -> np.ndarray:
    """cap * tanh(x / cap) — TF/models/gemma2/modeling_gemma2.py:203-206 (attention) and
    :527-530 (final logits); identity for cap <= 0."""
    if cap <= 0:
        return np.asarray(x, F32)
    c = F32(cap)
    return (c * np.tanh(np.asarray(x, F32) / c)).astype(F32)


def softmax(z: np.ndarray) -> np.ndarray:
    """max-subtracted softmax in fp32 — src/deciax/protocol/answers.py:44-46."""
    z = np.asarray(z, F32)
    e = np.exp(z - z.max())
    return (e / e.sum()).astype(F32)
