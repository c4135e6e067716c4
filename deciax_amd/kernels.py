"""Typed host wrappers over the C ABI, on torch device tensors.

torch provides device memory and the current HIP stream; every computation
runs in the gfx950 kernels of `libdeciax_hip.so`. Wrappers validate shapes,
dtypes and devices on the host (raising ValueError, like the reference's
kernel wrappers, e.g. src/deciax/kernels/projection.py:22-26) and then launch
asynchronously on `torch.cuda.current_stream()`.
"""

from __future__ import annotations

import ctypes
import weakref
from collections.abc import Sequence

import torch

from deciax_amd import _lib
from deciax_amd._lib import DX_ACT_GELU_ERF, DX_ACT_GELU_TANH, DX_ACT_NONE, DX_ACT_SILU, DX_BF16, DX_F32, call

BF16 = torch.bfloat16
F32 = torch.float32
ACTIVATIONS = {"gelu_tanh": DX_ACT_GELU_TANH, "gelu_pytorch_tanh": DX_ACT_GELU_TANH, "silu": DX_ACT_SILU}


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, ndim: int | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a device (HIP) tensor, got {t.device}")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims, got shape {tuple(t.shape)}")


def _rows(t: torch.Tensor, name: str) -> int:
    """Row stride of a 2-D view whose rows are contiguous."""
    if t.stride(-1) != 1:
        raise ValueError(f"{name} rows must be contiguous")
    return t.stride(0)


def _check_heads(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, hq: int, hkv: int, d: int) -> None:
    if q.shape[1] < hq * d or k.shape[1] < hkv * d or v.shape[1] < hkv * d:
        raise ValueError("attention: q / k / v rows narrower than heads * head_dim")
    if not q.shape[0] == k.shape[0] == v.shape[0]:
        raise ValueError("attention: q, k and v need the same number of rows")


def _check_out(out: torch.Tensor, q: torch.Tensor, width: int) -> None:
    if out.shape[0] < q.shape[0] or out.shape[1] < width:
        raise ValueError(f"attention: out must hold [{q.shape[0]}, {width}], got {tuple(out.shape)}")


def _activation(act: str) -> int:
    try:
        return ACTIVATIONS[act]
    except KeyError:
        raise ValueError(f"activation must be one of {sorted(ACTIVATIONS)}, got {act!r}") from None


# ---------------------------------------------------------------------------- projections


def linear(x: torch.Tensor, w: torch.Tensor, *, out: torch.Tensor | None = None,
           out_dtype: torch.dtype = BF16) -> torch.Tensor:
    """`x @ w.T` for a PyTorch-layout [out, in] weight (src/deciax/nn.py:11-19), bf16 operands,
    fp32 accumulation, result rounded once to `out_dtype`."""
    _need(x, "x", BF16, 2)
    _need(w, "w", BF16, 2)
    m, k = x.shape
    n = w.shape[0]
    if w.shape[1] != k:
        raise ValueError(f"linear: x {tuple(x.shape)} and w {tuple(w.shape)} disagree on k")
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=x.device)
    _need(out, "out", out_dtype, 2)
    if tuple(out.shape) != (m, n):
        raise ValueError(f"linear: out must be {(m, n)}, got {tuple(out.shape)}")
    code = {BF16: DX_BF16, F32: DX_F32}.get(out_dtype)
    if code is None:
        raise ValueError(f"linear: out_dtype must be bf16 or fp32, got {out_dtype}")
    call("dx_linear", _ptr(x), _ptr(w), _ptr(out), m, n, k, _rows(x, "x"), _rows(w, "w"), _rows(out, "out"), code,
         _stream())
    return out


def qkv_rope(x: torch.Tensor, w_qkv: torch.Tensor, qk: torch.Tensor, vt: torch.Tensor, positions: torch.Tensor,
             vt_col: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *, num_q_heads: int, num_kv_heads: int,
             head_dim: int) -> torch.Tensor:
    """Packed q | k | v projection with RoPE on q and k in the epilogue (`fused.py:93-99,120-122`):
    qk [rows, >= (Hq + Hkv) D] receives rotated q | k; V goes transposed into vt at column vt_col[row]
    (the layout of `attention_vt`; columns past each sequence's length are left to `vt_zero_tails`)."""
    for t, n in ((x, "x"), (w_qkv, "w_qkv"), (qk, "qk"), (vt, "vt"), (cos, "cos"), (sin, "sin")):
        _need(t, n, BF16, 2)
    _need(positions, "positions", torch.int32, 1)
    _need(vt_col, "vt_col", torch.int32, 1)
    rows, hidden = x.shape
    width = (num_q_heads + 2 * num_kv_heads) * head_dim
    if w_qkv.shape != (width, hidden):
        raise ValueError(f"qkv_rope: weight must be [{width}, {hidden}], got {tuple(w_qkv.shape)}")
    if qk.shape[0] < rows or vt.shape[0] != num_kv_heads * head_dim:
        raise ValueError("qkv_rope: qk needs a row per token and vt one row per (kv head, dim)")
    if positions.shape[0] != rows or vt_col.shape[0] != rows:
        raise ValueError("qkv_rope: one position and one V^T column per row")
    if cos.shape != sin.shape or cos.shape[1] != head_dim // 2:
        raise ValueError("qkv_rope: cos/sin tables must be [max_pos, head_dim / 2]")
    call("dx_qkv_rope", _ptr(x), _ptr(w_qkv), _ptr(qk), _ptr(vt), _ptr(positions), _ptr(vt_col), _ptr(cos), _ptr(sin),
         rows, hidden, num_q_heads, num_kv_heads, head_dim, _rows(x, "x"), _rows(qk, "qk"), _rows(vt, "vt"),
         cos.shape[0], _stream())
    return qk


def residual_norm_counters(rows: int, device: torch.device | str) -> torch.Tensor:
    """Zeroed row-block counters for `linear_residual_norm` on up to `rows` rows (each completed call
    leaves them zero, so one array serves a whole forward)."""
    n = max(int(_lib.lib().dx_linear_residual_norm_counters(max(rows, 1))),
            int(_lib.lib().dx_linear_residual_norm_counters(min(max(rows, 1), 1024))))
    return torch.zeros(n, dtype=torch.int32, device=device)


def linear_residual_norm(a: torch.Tensor, w: torch.Tensor, y: torch.Tensor, x: torch.Tensor, post_w: torch.Tensor,
                         *, eps: float, counters: torch.Tensor, next_w: torch.Tensor | None = None,
                         h: torch.Tensor | None = None) -> torch.Tensor | None:
    """y = a @ w.T (bf16), then in place x = bf16(x + bf16(rms(y)(1 + post_w))) and, with `next_w`,
    h = bf16(rms(x)(1 + next_w)): `linear` followed by `add_rmsnorm`, bit-identically, in one kernel
    (dx_linear_residual_norm). y is scratch; `counters` comes from `residual_norm_counters`."""
    for t, n in ((a, "a"), (w, "w"), (y, "y"), (x, "x")):
        _need(t, n, BF16, 2)
    m, k = a.shape
    d = w.shape[0]
    if w.shape[1] != k:
        raise ValueError(f"linear_residual_norm: a {tuple(a.shape)} and w {tuple(w.shape)} disagree on k")
    for t, n in ((y, "y"), (x, "x")):
        if tuple(t.shape) != (m, d) or not t.is_contiguous():
            raise ValueError(f"linear_residual_norm: {n} must be a contiguous [{m}, {d}] tensor")
    for t, n in ((post_w, "post_w"), (next_w, "next_w")):
        if t is not None:
            _need(t, n, BF16, 1)
            if t.shape[0] != d or not t.is_contiguous():
                raise ValueError(f"linear_residual_norm: {n} must be a contiguous [{d}] tensor")
    if (h is None) != (next_w is None):
        raise ValueError("linear_residual_norm: h and next_w go together")
    if h is not None:
        _need(h, "h", BF16, 2)
        if tuple(h.shape) != (m, d) or not h.is_contiguous():
            raise ValueError(f"linear_residual_norm: h must be a contiguous [{m}, {d}] tensor")
    _need(counters, "counters", torch.int32, 1)
    if counters.shape[0] < _lib.lib().dx_linear_residual_norm_counters(m) or not counters.is_contiguous():
        raise ValueError("linear_residual_norm: counters too short; use residual_norm_counters")
    call("dx_linear_residual_norm", _ptr(a), _ptr(w), _ptr(y), _ptr(x), _ptr(post_w), _ptr(next_w), _ptr(h),
         _ptr(counters), m, d, k, _rows(a, "a"), _rows(w, "w"), float(eps), _stream())
    return h


def pack_gate_up(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """[f, k] gate and up weights -> the [2f, k] packed layout of `gated_linear`
    (the role of `pack`, src/deciax/kernels/swiglu.py:45-51)."""
    _need(gate, "gate", BF16, 2)
    _need(up, "up", BF16, 2)
    if gate.shape != up.shape:
        raise ValueError("gate and up must have the same shape")
    f, k = gate.shape
    gate, up = gate.contiguous(), up.contiguous()
    packed = torch.empty((2 * f, k), dtype=BF16, device=gate.device)
    call("dx_pack_gate_up", _ptr(gate), _ptr(up), _ptr(packed), f, k, _stream())
    return packed


def gated_linear(x: torch.Tensor, gate_up: torch.Tensor, activation: str = "gelu_tanh", *,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """act(x @ gate.T) * (x @ up.T) with the reference's bf16 rounding points
    (src/deciax/kernels/swiglu.py:100-101)."""
    _need(x, "x", BF16, 2)
    _need(gate_up, "gate_up", BF16, 2)
    m, k = x.shape
    f2, kw = gate_up.shape
    if kw != k or f2 % 2:
        raise ValueError(f"gated_linear: x {tuple(x.shape)} and gate_up {tuple(gate_up.shape)} disagree")
    f = f2 // 2
    if out is None:
        out = torch.empty((m, f), dtype=BF16, device=x.device)
    _need(out, "out", BF16, 2)
    if out.shape[0] < m or out.shape[1] < f:
        raise ValueError(f"gated_linear: out must hold [{m}, {f}], got {tuple(out.shape)}")
    call("dx_gated_linear", _ptr(x), _ptr(gate_up), _ptr(out), m, f, k, _rows(x, "x"), _rows(out, "out"),
         _activation(activation), _stream())
    return out


def norm_project(x: torch.Tensor, norm: torch.Tensor, weight: torch.Tensor, *, eps: float,
                 row_mask: torch.Tensor | None = None) -> torch.Tensor:
    """RMSNorm(1 + w) -> optional row mask -> packed projection [n, d]
    (`norm_project`, src/deciax/kernels/projection.py:13-53)."""
    _need(x, "x", BF16, 2)
    _need(norm, "norm", BF16, 1)
    _need(weight, "weight", BF16, 2)
    rows, d = x.shape
    n = weight.shape[0]
    if weight.shape[1] != d or norm.shape[0] != d:
        raise ValueError("norm_project: hidden sizes disagree")
    x = x.contiguous()
    mask_u8 = None
    if row_mask is not None:
        if row_mask.shape != (rows,):
            raise ValueError("norm_project: row_mask must be [rows]")
        mask_u8 = row_mask.to(device=x.device, dtype=torch.uint8).contiguous()
    ws_bytes = _lib.lib().dx_norm_project_workspace(rows, d)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=x.device)
    y = torch.empty((rows, n), dtype=BF16, device=x.device)
    call("dx_norm_project", _ptr(x), _ptr(norm.contiguous()), _ptr(mask_u8), _ptr(weight.contiguous()), _ptr(y), rows,
         d, n, float(eps), _ptr(ws), ws.numel(), _stream())
    return y


def mlp(x: torch.Tensor, norm: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor, *, eps: float,
        activation: str = "gelu_tanh", out_dtype: torch.dtype = F32) -> torch.Tensor:
    """RMSNorm(1 + w) -> gated gate|up -> down with fp32 accumulation over all of f
    (`fused_mlp_partial`, src/deciax/kernels/swiglu.py:166-208). `down` is [d, f]."""
    _need(x, "x", BF16, 2)
    _need(norm, "norm", BF16, 1)
    _need(gate_up, "gate_up", BF16, 2)
    _need(down, "down", BF16, 2)
    rows, d = x.shape
    f = gate_up.shape[0] // 2
    if gate_up.shape != (2 * f, d) or down.shape != (d, f) or norm.shape != (d,):
        raise ValueError("mlp: inconsistent packed MLP shapes")
    code = {BF16: DX_BF16, F32: DX_F32}.get(out_dtype)
    if code is None:
        raise ValueError("mlp: out_dtype must be bf16 or fp32")
    x = x.contiguous()
    ws_bytes = _lib.lib().dx_mlp_workspace(rows, d, f)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=x.device)
    y = torch.empty((rows, d), dtype=out_dtype, device=x.device)
    call("dx_mlp", _ptr(x), _ptr(norm.contiguous()), _ptr(gate_up.contiguous()), _ptr(down.contiguous()), _ptr(y),
         rows, d, f, float(eps), _activation(activation), code, _ptr(ws), ws.numel(), _stream())
    return y


# ---------------------------------------------------------------------------- norms, embedding, rope


def rmsnorm(x: torch.Tensor, w: torch.Tensor, *, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """`rms` of src/deciax/models/qwen3_5/text.py:25-28 over the last dim of a 2-D tensor."""
    _need(x, "x", BF16, 2)
    _need(w, "w", BF16, 1)
    rows, d = x.shape
    if w.shape[0] != d:
        raise ValueError(f"rmsnorm: w must be [{d}], got {tuple(w.shape)}")
    if out is None:
        out = torch.empty_like(x)
    _need(out, "out", BF16, 2)
    if tuple(out.shape) != (rows, d):
        raise ValueError(f"rmsnorm: out must be [{rows}, {d}], got {tuple(out.shape)}")
    call("dx_rmsnorm", _ptr(x), _ptr(w), _ptr(out), rows, d, _rows(x, "x"), _rows(out, "out"), float(eps), _stream())
    return out


def add_rmsnorm(y: torch.Tensor, x: torch.Tensor, *, eps: float, post_w: torch.Tensor | None = None,
                next_w: torch.Tensor | None = None, h: torch.Tensor | None = None) -> torch.Tensor | None:
    """In place x = x + (post-normed) y; returns h = rms(x)(1 + next_w) when next_w is given."""
    _need(y, "y", BF16, 2)
    _need(x, "x", BF16, 2)
    if y.shape != x.shape or not (x.is_contiguous() and y.is_contiguous()):
        raise ValueError("add_rmsnorm: y and x must be contiguous and of one shape")
    rows, d = x.shape
    for t, n in ((post_w, "post_w"), (next_w, "next_w")):
        if t is not None:
            _need(t, n, BF16, 1)
            if t.shape[0] != d or not t.is_contiguous():
                raise ValueError(f"add_rmsnorm: {n} must be a contiguous [{d}] tensor")
    if next_w is not None and h is None:
        h = torch.empty_like(x)
    if next_w is not None:
        _need(h, "h", BF16, 2)
        if h.shape != x.shape or not h.is_contiguous():
            raise ValueError("add_rmsnorm: h must be contiguous and of x's shape")
    call("dx_add_rmsnorm", _ptr(y), _ptr(post_w), _ptr(x), _ptr(next_w), _ptr(h if next_w is not None else None),
         rows, d, float(eps), _stream())
    return h if next_w is not None else None


def embed(ids: torch.Tensor, table: torch.Tensor, *, scale: float = 1.0, norm_w: torch.Tensor | None = None,
          eps: float = 1e-6, x: torch.Tensor | None = None,
          h: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Embedding gather times a bf16 scale (`_embed`, src/deciax/models/clef/model.py:81), plus the
    first layer's input norm when `norm_w` is given."""
    _need(ids, "ids", torch.int32, 1)
    _need(table, "table", BF16, 2)
    vocab, d = table.shape
    if x is None:
        x = torch.empty((ids.shape[0], d), dtype=BF16, device=table.device)
    if norm_w is not None and h is None:
        h = torch.empty_like(x)
    for t, n in ((x, "x"), (h, "h")):
        if t is not None:
            _need(t, n, BF16, 2)
            if tuple(t.shape) != (ids.shape[0], d) or not t.is_contiguous():
                raise ValueError(f"embed: {n} must be a contiguous [tokens, d] tensor")
    if norm_w is not None:
        _need(norm_w, "norm_w", BF16, 1)
        if norm_w.shape[0] != d or not norm_w.is_contiguous():
            raise ValueError(f"embed: norm_w must be a contiguous [{d}] tensor")
    h = h if norm_w is not None else None
    call("dx_embed", _ptr(ids.contiguous()), _ptr(table), _ptr(x), ids.shape[0], d, vocab, float(scale),
         _ptr(norm_w), _ptr(h), float(eps), _stream())
    return x, h


def rope(x: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *, num_heads: int,
         head_dim: int) -> torch.Tensor:
    """In-place rotate-half RoPE on the first `num_heads` heads of each row of a 2-D
    [rows, >= num_heads * head_dim] tensor (`apply_rope`, src/deciax/nn.py:35-44)."""
    _need(x, "x", BF16, 2)
    _need(positions, "positions", torch.int32, 1)
    _need(cos, "cos", BF16, 2)
    _need(sin, "sin", BF16, 2)
    if cos.shape != sin.shape or cos.shape[1] != head_dim // 2:
        raise ValueError("rope: cos/sin tables must be [max_pos, head_dim / 2]")
    if positions.shape[0] != x.shape[0]:
        raise ValueError("rope: one position per row")
    call("dx_rope", _ptr(x), _ptr(positions), _ptr(cos), _ptr(sin), x.shape[0], num_heads, head_dim,
         _rows(x, "x"), cos.shape[0], _stream())
    return x


# ---------------------------------------------------------------------------- attention


def attention_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, seq_start: torch.Tensor,
                     seq_len: torch.Tensor, max_seq_len: int, *, num_q_heads: int, num_kv_heads: int, head_dim: int,
                     scale: float, softcap: float = 0.0, window: int = 0, causal: bool = True,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """Prefill attention over packed rows: q [rows, >= Hq*D], k/v [rows, >= Hkv*D] (2-D views with
    contiguous rows, possibly column slices of one packed qkv buffer). bf16 or fp32."""
    dtype = q.dtype
    if dtype not in (BF16, F32):
        raise ValueError(f"attention: dtype must be bf16 or fp32, got {dtype}")
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _need(t, n, dtype, 2)
    _need(seq_start, "seq_start", torch.int32, 1)
    _need(seq_len, "seq_len", torch.int32, 1)
    if seq_start.shape != seq_len.shape:
        raise ValueError("attention: one seq_start per seq_len")
    _check_heads(q, k, v, num_q_heads, num_kv_heads, head_dim)
    if out is None:
        out = torch.empty((q.shape[0], num_q_heads * head_dim), dtype=dtype, device=q.device)
    _need(out, "out", dtype, 2)
    _check_out(out, q, num_q_heads * head_dim)
    nseq = seq_start.shape[0]
    code = DX_BF16 if dtype == BF16 else DX_F32
    ws_bytes = _lib.lib().dx_attn_prefill_workspace(nseq, max_seq_len, num_kv_heads, head_dim, code)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    call("dx_attn_prefill", _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(seq_start), _ptr(seq_len), nseq, max_seq_len,
         num_q_heads, num_kv_heads, head_dim, _rows(q, "q"), _rows(k, "k"), _rows(v, "v"), _rows(out, "out"),
         float(scale), float(softcap), int(window), int(bool(causal)), code, _ptr(ws), ws.numel(), _stream())
    return out


def transpose_v(v: torch.Tensor, vt: torch.Tensor, seq_start: torch.Tensor, seq_len: torch.Tensor,
                vt_start: torch.Tensor, max_seq_len: int, *, num_kv_heads: int, head_dim: int) -> torch.Tensor:
    _need(v, "v", BF16, 2)
    _need(vt, "vt", BF16, 2)
    for t, n in ((seq_start, "seq_start"), (seq_len, "seq_len"), (vt_start, "vt_start")):
        _need(t, n, torch.int32, 1)
    if not seq_start.shape[0] == seq_len.shape[0] == vt_start.shape[0]:
        raise ValueError("transpose_v: seq_start, seq_len and vt_start need one entry per sequence")
    call("dx_transpose_v", _ptr(v), _ptr(vt), _ptr(seq_start), _ptr(seq_len), _ptr(vt_start), seq_start.shape[0],
         max_seq_len, num_kv_heads, head_dim, _rows(v, "v"), _rows(vt, "vt"), _stream())
    return vt


def vt_zero_tails(vt: torch.Tensor, seq_len: torch.Tensor, vt_start: torch.Tensor) -> torch.Tensor:
    """Zero each sequence's V^T columns past its length, up to the next multiple of 64."""
    _need(vt, "vt", BF16, 2)
    _need(seq_len, "seq_len", torch.int32, 1)
    _need(vt_start, "vt_start", torch.int32, 1)
    if seq_len.shape != vt_start.shape:
        raise ValueError("vt_zero_tails: one vt_start per sequence")
    call("dx_vt_zero_tails", _ptr(vt), _ptr(seq_len), _ptr(vt_start), seq_len.shape[0], vt.shape[0],
         _rows(vt, "vt"), _stream())
    return vt


def attention_vt(q: torch.Tensor, k: torch.Tensor, vt: torch.Tensor, seq_start: torch.Tensor, seq_len: torch.Tensor,
                 vt_start: torch.Tensor, max_seq_len: int, *, num_q_heads: int, num_kv_heads: int, head_dim: int,
                 scale: float, softcap: float = 0.0, window: int = 0, causal: bool = True,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 attention with V pre-transposed by `transpose_v` (the model driver's form). The sequence
    descriptors (int32 seq_start, seq_len, vt_start) may come in any order; the kernel launches them
    in that order, so listing the longest first starts the heaviest work first."""
    for t, n in ((q, "q"), (k, "k"), (vt, "vt")):
        _need(t, n, BF16, 2)
    for t, n in ((seq_start, "seq_start"), (seq_len, "seq_len"), (vt_start, "vt_start")):
        _need(t, n, torch.int32, 1)
    if not seq_start.shape[0] == seq_len.shape[0] == vt_start.shape[0]:
        raise ValueError("attention_vt: seq_start, seq_len and vt_start need one entry per sequence")
    if q.shape[1] < num_q_heads * head_dim or k.shape[1] < num_kv_heads * head_dim or k.shape[0] < q.shape[0]:
        raise ValueError("attention_vt: q / k rows narrower than heads * head_dim or fewer key rows than queries")
    if vt.shape[0] != num_kv_heads * head_dim:
        raise ValueError(f"attention_vt: vt must have {num_kv_heads * head_dim} rows, got {vt.shape[0]}")
    if out is None:
        out = torch.empty((q.shape[0], num_q_heads * head_dim), dtype=BF16, device=q.device)
    _need(out, "out", BF16, 2)
    _check_out(out, q, num_q_heads * head_dim)
    call("dx_attn_prefill_vt", _ptr(q), _ptr(k), _ptr(vt), _ptr(out), _ptr(seq_start), _ptr(seq_len),
         _ptr(vt_start), seq_start.shape[0], max_seq_len, num_q_heads, num_kv_heads, head_dim, _rows(q, "q"),
         _rows(k, "k"), _rows(vt, "vt"), _rows(out, "out"), float(scale), float(softcap), int(window),
         int(bool(causal)), _stream())
    return out


def noalloc_init() -> None:
    """Look up the current device's static scratch of the allocation-free attention (outside graph
    capture; idempotent)."""
    call("dx_noalloc_init")


def attention_varlen_noalloc(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, seq_start: torch.Tensor,
                             seq_len: torch.Tensor, max_seq_len: int, *, num_q_heads: int, num_kv_heads: int,
                             head_dim: int, scale: float, softcap: float = 0.0, window: int = 0, causal: bool = True,
                             out: torch.Tensor) -> torch.Tensor:
    """`attention_varlen` through dx_attn_prefill_noalloc: nothing is allocated (the caller passes
    `out`; the bf16 path stages V^T in the library's static per-GPU scratch of
    DX_NOALLOC_SCRATCH_BYTES). Calls that overlap on one GPU race on that scratch. Outside graph
    capture the scratch's address is looked up first (dx_noalloc_init); a first call on a device made
    under capture, without `noalloc_init()` beforehand, raises ValueError."""
    if not torch.cuda.is_current_stream_capturing():
        noalloc_init()
    dtype = q.dtype
    if dtype not in (BF16, F32):
        raise ValueError(f"attention: dtype must be bf16 or fp32, got {dtype}")
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _need(t, n, dtype, 2)
    _need(seq_start, "seq_start", torch.int32, 1)
    _need(seq_len, "seq_len", torch.int32, 1)
    if seq_start.shape != seq_len.shape:
        raise ValueError("attention: one seq_start per seq_len")
    _check_heads(q, k, v, num_q_heads, num_kv_heads, head_dim)
    _need(out, "out", dtype, 2)
    _check_out(out, q, num_q_heads * head_dim)
    call("dx_attn_prefill_noalloc", _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(seq_start), _ptr(seq_len),
         seq_start.shape[0], max_seq_len, num_q_heads, num_kv_heads, head_dim, _rows(q, "q"), _rows(k, "k"),
         _rows(v, "v"), _rows(out, "out"), float(scale), float(softcap), int(window), int(bool(causal)),
         DX_BF16 if dtype == BF16 else DX_F32, _stream())
    return out


def attention_masked(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, key_mask: torch.Tensor,
                     seq_start: torch.Tensor, seq_len: torch.Tensor, max_seq_len: int, *, num_q_heads: int,
                     num_kv_heads: int, head_dim: int, scale: float, softcap: float = 0.0, window: int = 0,
                     causal: bool = True, out: torch.Tensor | None = None) -> torch.Tensor:
    """`attention_varlen` with a per-row key mask (uint8 or bool [rows]): key j of sequence s is
    visible only where key_mask[seq_start[s] + j] is set. Query rows that see no key are written as
    zeros (dx_attn_prefill_masked)."""
    dtype = q.dtype
    if dtype not in (BF16, F32):
        raise ValueError(f"attention: dtype must be bf16 or fp32, got {dtype}")
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _need(t, n, dtype, 2)
    _need(seq_start, "seq_start", torch.int32, 1)
    _need(seq_len, "seq_len", torch.int32, 1)
    if seq_start.shape != seq_len.shape:
        raise ValueError("attention: one seq_start per seq_len")
    if key_mask.dim() != 1 or key_mask.shape[0] != k.shape[0] or key_mask.device != k.device:
        raise ValueError("attention: key_mask must be a device tensor with one entry per key row")
    mask_u8 = key_mask.to(torch.uint8).contiguous()
    _check_heads(q, k, v, num_q_heads, num_kv_heads, head_dim)
    if out is None:
        out = torch.empty((q.shape[0], num_q_heads * head_dim), dtype=dtype, device=q.device)
    _need(out, "out", dtype, 2)
    _check_out(out, q, num_q_heads * head_dim)
    nseq = seq_start.shape[0]
    code = DX_BF16 if dtype == BF16 else DX_F32
    ws_bytes = _lib.lib().dx_attn_prefill_masked_workspace(nseq, max_seq_len, num_kv_heads, head_dim, code)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    call("dx_attn_prefill_masked", _ptr(q), _ptr(k), _ptr(v), _ptr(mask_u8), _ptr(out), _ptr(seq_start),
         _ptr(seq_len), nseq, max_seq_len, num_q_heads, num_kv_heads, head_dim, _rows(q, "q"), _rows(k, "k"),
         _rows(v, "v"), _rows(out, "out"), float(scale), float(softcap), int(window), int(bool(causal)), code,
         _ptr(ws), ws.numel(), _stream())
    return out


def _visible_counts(mask: torch.Tensor, nq: int, causal: bool, window: int) -> torch.Tensor:
    """[B, K] key mask -> [B, nq] number of keys each query row sees (index bookkeeping for the rows
    that see none)."""
    b, nk = mask.shape
    cs = torch.nn.functional.pad(torch.cumsum(mask.to(torch.int32), dim=1), (1, 0))  # cs[:, j] = keys < j
    i = torch.arange(nq, device=mask.device)
    if causal:
        hi = torch.clamp(i + 1, max=nk)
        lo = torch.clamp(i - window + 1, min=0) if window > 0 else torch.zeros_like(i)
    elif window > 0:
        hi = torch.clamp(i + window + 1, max=nk)
        lo = torch.clamp(i - window, min=0)
    else:
        hi = torch.full_like(i, nk)
        lo = torch.zeros_like(i)
    lo = torch.minimum(lo, hi)
    return cs[:, hi] - cs[:, lo]


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, key_mask: torch.Tensor, *, causal: bool = False,
              window: int = 0, softcap: float = 0.0, scale: float | None = None) -> torch.Tensor:
    """[B, Q, H, D] queries against [B, K, Hkv, D] keys and values with a [B, K] key mask ->
    [B, Q, H, D]: the interface of `blocked.attention` (src/deciax/kernels/attention/blocked.py:9-32)
    and, with `causal=False` and a symmetric `window`, of `ops.attention`
    (src/deciax/ops/__init__.py:10-26, src/deciax/kernels/attention/reference.py:11-42).

    Any mask is accepted (blocked.py:23-27): masked keys get no weight. Causal visibility compares
    row indices, key j <= query i, as blocked.py:25 does. Every query row is computed, padded ones
    included. A row that sees no key at all gets what the reference's finite MASK_FILL gives it:
    the uniform average of all K values (softmax of K equal scores)."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("attention: q must be [B, Q, H, D] and k, v [B, K, Hkv, D]")
    b, nq, hq, d = q.shape
    nk, hkv = k.shape[1], k.shape[2]
    if k.shape != (b, nk, hkv, d) or v.shape != k.shape or tuple(key_mask.shape) != (b, nk):
        raise ValueError("attention: inconsistent q/k/v/mask shapes")
    if q.dtype not in (BF16, F32) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("attention: q, k, v must share one dtype, bf16 or fp32")
    if window < 0:
        raise ValueError("attention: window must be >= 0")
    scale = d ** -0.5 if scale is None else scale
    mask = key_mask.to(device=q.device, dtype=torch.bool)
    length = max(nq, nk)
    if nk == 0:
        raise ValueError("attention: need at least one key")

    def rows_view(t: torch.Tensor, h: int) -> torch.Tensor | None:
        # [B, L, h, D] as [B L, h D] rows without a copy (row-strided views, such as slices of a packed
        # q | k | v, included); None when the strides do not allow it
        try:
            return t.view(b * length, h * d)
        except RuntimeError:
            return None

    flat = [rows_view(q, hq), rows_view(k, hkv), rows_view(v, hkv)] if nq == nk else [None]
    if all(x is not None for x in flat):
        # already one sequence of `length` rows per batch row: the kernels read the tensors in place
        qp, kp, vp = flat
        mp = mask
    else:
        # One sequence per batch row of `length` rows: queries padded past Q (dropped afterwards), keys
        # padded past K (masked out).
        qp = torch.zeros((b, length, hq, d), dtype=q.dtype, device=q.device)
        kp = torch.zeros((b, length, hkv, d), dtype=q.dtype, device=q.device)
        vp = torch.zeros_like(kp)
        mp = torch.zeros((b, length), dtype=torch.bool, device=q.device)
        qp[:, :nq], kp[:, :nk], vp[:, :nk], mp[:, :nk] = q, k, v, mask
    starts = torch.arange(b, device=q.device, dtype=torch.int32) * length
    lengths = torch.full((b,), length, device=q.device, dtype=torch.int32)
    rows = b * length
    kw = dict(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, scale=scale, softcap=softcap, window=window,
              causal=causal)
    args = (qp.reshape(rows, hq * d), kp.reshape(rows, hkv * d), vp.reshape(rows, hkv * d))
    # Always the key-mask kernel: tiles whose keys the mask keeps run its unmasked body, so a full mask
    # costs about what the maskless kernel does, bit for bit the same output, and asking whether the mask
    # is full would stall the stream for a host round trip.
    out = attention_masked(*args, mp.reshape(rows), starts, lengths, length, **kw)
    out = out.reshape(b, length, hq, d)[:, :nq]
    empty = _visible_counts(mask, nq, causal, window) == 0
    if bool(empty.any()):
        # softmax over K equal scores: the average of every value row, which the kernel computes for a
        # zero query attending all K keys
        kz = torch.zeros((b * nk, hq * d), dtype=q.dtype, device=q.device)
        uniform = attention_varlen(kz, k.reshape(b * nk, hkv * d).contiguous(), v.reshape(b * nk, hkv * d).contiguous(),
                                   torch.arange(b, device=q.device, dtype=torch.int32) * nk,
                                   torch.full((b,), nk, device=q.device, dtype=torch.int32), nk, num_q_heads=hq,
                                   num_kv_heads=hkv, head_dim=d, scale=scale, causal=False)
        uniform = uniform.reshape(b, nk, hq, d)[:, :1].expand(b, nq, hq, d)
        out = torch.where(empty[:, :, None, None], uniform, out)
    return out.contiguous()


FLASH_HEAD_DIM = 64  # the reference TPU kernel's fixed head size (pallas.py:18)


def flash_attention(qkv: torch.Tensor, mask: torch.Tensor, *, heads: int, window: int = 0,
                    out_dtype: torch.dtype = BF16) -> torch.Tensor:
    """Packed [B, S, 3 H 64] q | k | v and a [B, S] key mask (1 = real token) -> [B, S, H 64]: the
    interface of the reference's TPU flash kernel (`flash_attention`,
    src/deciax/kernels/attention/pallas.py:52-135). Bidirectional, one key head per query head,
    head_dim 64, queries scaled by 64^-0.5 (exact: a power of two), keys with |q - k| <= window when
    window > 0 (mask_bias, :31-39); online softmax in fp32 with P rounded to the value dtype for P.V
    (pv_t, :47-49).

    Differences from the reference, stated rather than copied: S need not be a multiple of its
    256 / 512 blocks (it asserts that), shape errors raise ValueError (it asserts), and the output
    takes the input's dtype (`out_dtype` must equal it)."""
    if not isinstance(qkv, torch.Tensor) or qkv.dim() != 3:
        raise ValueError("flash_attention: qkv must be [B, S, 3 * heads * 64]")
    b, s, width = qkv.shape
    if heads < 1 or width != 3 * heads * FLASH_HEAD_DIM:
        raise ValueError(f"flash_attention: qkv width {width} is not 3 * {heads} heads * {FLASH_HEAD_DIM}")
    if tuple(mask.shape) != (b, s):
        raise ValueError(f"flash_attention: mask must be [{b}, {s}], got {tuple(mask.shape)}")
    if window < 0:
        raise ValueError("flash_attention: window must be >= 0")
    if out_dtype != qkv.dtype:
        raise ValueError(f"flash_attention: out_dtype must be the input dtype {qkv.dtype}, got {out_dtype}")
    d = heads * FLASH_HEAD_DIM
    q, k, v = (qkv[..., i * d:(i + 1) * d].reshape(b, s, heads, FLASH_HEAD_DIM) for i in range(3))
    out = attention(q, k, v, mask, causal=False, window=window, scale=FLASH_HEAD_DIM ** -0.5)
    return out.reshape(b, s, d)


# ---------------------------------------------------------------------------- readout


# Device offset arrays built by `offsets_tensor`, with the host values they were built from: the
# readout validates those without reading the device tensor back (which would synchronise the stream).
# Keyed by id(); the weak reference confirms the entry still belongs to that tensor, and a finalizer
# drops it with the tensor.
_OFFSETS: dict[int, tuple[weakref.ref, tuple[int, ...]]] = {}


def offsets_tensor(values: Sequence[int], device: torch.device | str) -> torch.Tensor:
    """An int32 device copy of question offsets, remembered together with its host values."""
    host = tuple(int(v) for v in values)
    t = torch.as_tensor(host, dtype=torch.int32).to(device)
    key = id(t)
    _OFFSETS[key] = (weakref.ref(t), host)
    weakref.finalize(t, _OFFSETS.pop, key, None)
    return t


def known_offsets(t: torch.Tensor) -> tuple[int, ...] | None:
    """The host values `t` was built from by `offsets_tensor`, or None for any other tensor."""
    entry = _OFFSETS.get(id(t))
    if entry is None or entry[0]() is not t or len(entry[1]) != t.shape[0]:
        return None
    return entry[1]


def readout(hidden: torch.Tensor, norm_w: torch.Tensor, table: torch.Tensor, opt_pos: torch.Tensor,
            opt_label: torch.Tensor, q_offsets: torch.Tensor, *, eps: float, softcap: float = 0.0,
            q_offsets_host: Sequence[int] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Option logits and per-question probabilities (see dx_readout).

    `q_offsets` is validated on the host before the launch. For a tensor made by `offsets_tensor` the
    values it was built from are used, with no device read; any other tensor is read back (which
    synchronises the stream). `q_offsets_host`, when given, must equal those values, else ValueError.
    The kernel also clamps every question's range into the option arrays."""
    _need(hidden, "hidden", BF16, 2)
    _need(norm_w, "norm_w", BF16, 1)
    _need(table, "table", BF16, 2)
    for t, n in ((opt_pos, "opt_pos"), (opt_label, "opt_label"), (q_offsets, "q_offsets")):
        _need(t, n, torch.int32, 1)
    nopt = opt_pos.shape[0]
    d = hidden.shape[1]
    if opt_label.shape[0] != nopt:
        raise ValueError("readout: one label per option position")
    if norm_w.shape[0] != d or table.shape[1] != d:
        raise ValueError(f"readout: norm_w and table rows must have {d} entries")
    if q_offsets.shape[0] < 1:
        raise ValueError("readout: q_offsets needs at least one entry")
    known = known_offsets(q_offsets)
    if known is None:
        known = tuple(int(v) for v in q_offsets.cpu().tolist())
    if q_offsets_host is not None and tuple(int(v) for v in q_offsets_host) != known:
        raise ValueError("readout: q_offsets_host differs from the values of q_offsets")
    offs = torch.as_tensor(known, dtype=torch.int64)
    if int(offs[0]) != 0 or int(offs[-1]) != nopt or bool((offs[1:] < offs[:-1]).any()):
        raise ValueError("readout: q_offsets must rise monotonically from 0 to the number of options")
    logits = torch.empty(nopt, dtype=F32, device=hidden.device)
    probs = torch.empty(nopt, dtype=F32, device=hidden.device)
    nq = q_offsets.shape[0] - 1
    call("dx_readout", _ptr(hidden), _ptr(norm_w), _ptr(table), _ptr(opt_pos), _ptr(opt_label), _ptr(q_offsets),
         nq, nopt, hidden.shape[0], hidden.shape[1], _rows(hidden, "hidden"), table.shape[0], float(eps),
         float(softcap),
         _ptr(logits), _ptr(probs), _stream())
    return logits, probs


# ---------------------------------------------------------------------------- Clef joint head (fp32)


def _f32(t: torch.Tensor, name: str, ndim: int = 2) -> None:
    _need(t, name, F32, ndim)


def layer_norm_f32(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, *, eps: float,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """Row LayerNorm in fp32 (`layer_norm`, src/deciax/nn.py:22-29)."""
    _f32(x, "x")
    d = x.shape[1]
    for t, n in ((w, "w"), (b, "b")):
        if t is not None:
            _f32(t, n, 1)
            if t.shape[0] != d:
                raise ValueError(f"layer_norm_f32: {n} must be [{d}]")
    if w is None:
        raise ValueError("layer_norm_f32: w is required")
    out = torch.empty_like(x) if out is None else out
    _f32(out, "out")
    if out.shape[0] < x.shape[0] or out.shape[1] < d:
        raise ValueError(f"layer_norm_f32: out must hold {tuple(x.shape)}")
    call("dx_layer_norm_f32", _ptr(x), _ptr(w), _ptr(b), _ptr(out), x.shape[0], x.shape[1], _rows(x, "x"),
         _rows(out, "out"), float(eps), _stream())
    return out


def linear_f32(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None, *, gelu: bool = False,
               out: torch.Tensor | None = None, accumulate: bool = False) -> torch.Tensor:
    """out (+)= act(x @ w^T + bias) in fp32; act = exact GELU when `gelu` (`dense`,
    src/deciax/models/qwen3_5/text.py:21-22, with the head's residual adds)."""
    _f32(x, "x")
    _f32(w, "w")
    if out is None:
        if accumulate:
            raise ValueError("linear_f32: accumulate needs out")
        out = torch.empty((x.shape[0], w.shape[0]), dtype=F32, device=x.device)
    _f32(out, "out")
    if x.shape[1] != w.shape[1] or out.shape != (x.shape[0], w.shape[0]):
        raise ValueError(f"linear_f32: shapes {tuple(x.shape)} x {tuple(w.shape)}^T -> {tuple(out.shape)}")
    call("dx_linear_f32", _ptr(x), _ptr(w), _ptr(bias), _ptr(out), x.shape[0], w.shape[0], x.shape[1], _rows(x, "x"),
         _rows(w, "w"), _rows(out, "out"), DX_ACT_GELU_ERF if gelu else DX_ACT_NONE, int(accumulate), _stream())
    return out


def span_means_f32(x: torch.Tensor, spans: torch.Tensor, *, batch: int) -> torch.Tensor:
    """x [batch * S, d] rows, spans [batch, n, 2] -> [batch * n, d] (`means`, head.py:24-29)."""
    _f32(x, "x")
    _need(spans, "spans", torch.int32, 3)
    n = spans.shape[1]
    out = torch.empty((batch * n, x.shape[1]), dtype=F32, device=x.device)
    call("dx_span_means_f32", _ptr(x), _ptr(spans), _ptr(out), batch, x.shape[0] // batch, n, x.shape[1],
         _rows(x, "x"), _rows(out, "out"), _stream())
    return out


def mha_f32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, key_mask: torch.Tensor, *, batch: int,
            heads: int) -> torch.Tensor:
    """Masked multi-head attention core over [batch * n, heads * dh] rows (head.py:41-51)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _f32(t, n)
    _need(key_mask, "key_mask", torch.uint8, 2)
    width = q.shape[1]
    nq, nk = q.shape[0] // batch, k.shape[0] // batch
    if key_mask.shape != (batch, nk):
        raise ValueError("mha_f32: key_mask must be [batch, num_keys]")
    out = torch.empty((q.shape[0], width), dtype=F32, device=q.device)
    call("dx_mha_f32", _ptr(q), _ptr(k), _ptr(v), _ptr(key_mask), _ptr(out), batch, nq, nk, heads, width // heads,
         _rows(q, "q"), _rows(k, "k"), _rows(v, "v"), _rows(out, "out"), _stream())
    return out


def gather_rows_f32(x: torch.Tensor, index: torch.Tensor, *, batch: int, out: torch.Tensor | None = None,
                    accumulate: bool = False) -> torch.Tensor:
    """out[b * I + i] (+)= x[b * R + index[b, i]] (`gather`, head.py:32-33)."""
    _f32(x, "x")
    _need(index, "index", torch.int32, 2)
    picks = index.shape[1]
    if index.shape[0] != batch or x.shape[0] % max(batch, 1):
        raise ValueError("gather_rows_f32: index must be [batch, picks] and x hold batch equal row blocks")
    if out is None:
        out = torch.empty((batch * picks, x.shape[1]), dtype=F32, device=x.device)
    _f32(out, "out")
    if out.shape[0] < batch * picks or out.shape[1] < x.shape[1]:
        raise ValueError(f"gather_rows_f32: out must hold [{batch * picks}, {x.shape[1]}]")
    call("dx_gather_rows_f32", _ptr(x), _ptr(index), _ptr(out), batch, x.shape[0] // batch, picks, x.shape[1],
         _rows(x, "x"), _rows(out, "out"), int(accumulate), _stream())
    return out


def head_routing_f32(options: torch.Tensor, base: torch.Tensor, option_field: torch.Tensor,
                     option_mask: torch.Tensor, *, batch: int) -> torch.Tensor:
    """Per-field softmax over the owned options and the routed summary (head.py:77-85)."""
    _f32(options, "options")
    _f32(base, "base")
    _need(option_field, "option_field", torch.int32)
    _need(option_mask, "option_mask", torch.uint8)
    if options.shape[0] % batch or base.shape[0] % batch or options.shape[1] != base.shape[1]:
        raise ValueError("head_routing_f32: options and base must be batch row blocks of one width")
    if option_field.numel() != options.shape[0] or option_mask.numel() != options.shape[0]:
        raise ValueError("head_routing_f32: one field index and one mask entry per option")
    out = torch.empty_like(base)
    call("dx_head_routing_f32", _ptr(options), _ptr(base), _ptr(option_field), _ptr(option_mask), _ptr(out), batch,
         options.shape[0] // batch, base.shape[0] // batch, base.shape[1], _stream())
    return out


def head_fields_init_f32(base: torch.Tensor, summary_norm: torch.Tensor, global_proj: torch.Tensor,
                         type_embedding: torch.Tensor, types: torch.Tensor, *, batch: int) -> torch.Tensor:
    for t, n in ((base, "base"), (summary_norm, "summary_norm"), (global_proj, "global_proj"),
                 (type_embedding, "type_embedding")):
        _f32(t, n)
    _need(types, "types", torch.int32)
    if base.shape[0] % batch or summary_norm.shape != base.shape or types.numel() != base.shape[0]:
        raise ValueError("head_fields_init_f32: base, summary_norm and types must cover batch x fields rows")
    if global_proj.shape != (batch, base.shape[1]) or type_embedding.shape[1] != base.shape[1]:
        raise ValueError("head_fields_init_f32: global_proj must be [batch, width] and type_embedding [types, width]")
    out = torch.empty_like(base)
    call("dx_head_fields_init_f32", _ptr(base), _ptr(summary_norm), _ptr(global_proj), _ptr(type_embedding),
         _ptr(types), _ptr(out), batch, base.shape[0] // batch, base.shape[1], type_embedding.shape[0], _stream())
    return out


def head_features_f32(fields: torch.Tensor, options: torch.Tensor, questions: torch.Tensor,
                      global_vector: torch.Tensor, lexical: torch.Tensor, option_field: torch.Tensor, *, batch: int,
                      prior_scale: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    for t, nm in ((fields, "fields"), (options, "options"), (questions, "questions"), (global_vector, "global_vector"),
                  (lexical, "lexical")):
        _f32(t, nm)
    _need(option_field, "option_field", torch.int32)
    n, width = fields.shape
    if options.shape != fields.shape or lexical.shape[0] != n or option_field.numel() != n or n % batch:
        raise ValueError("head_features_f32: fields, options, lexical and option_field need one row per option")
    if questions.shape[0] % batch or global_vector.shape != (batch, questions.shape[1]) or \
            lexical.shape[1] != questions.shape[1]:
        raise ValueError("head_features_f32: questions [batch x fields, hidden], global_vector [batch, hidden]")
    features = torch.empty((n, 4 * width), dtype=F32, device=fields.device)
    prior = torch.empty(n, dtype=F32, device=fields.device)
    cosine = torch.empty(n, dtype=F32, device=fields.device)
    call("dx_head_features_f32", _ptr(fields), _ptr(options), _ptr(questions), _ptr(global_vector), _ptr(lexical),
         _ptr(option_field), _ptr(features), _ptr(prior), _ptr(cosine), batch, n // batch,
         questions.shape[0] // batch, width, questions.shape[1], float(prior_scale), _stream())
    return features, prior, cosine


def head_combine_f32(prior: torch.Tensor, cosine: torch.Tensor, residual: torch.Tensor, option_mask: torch.Tensor, *,
                     gate: float, joint_scale: float) -> torch.Tensor:
    for t, n in ((prior, "prior"), (cosine, "cosine"), (residual, "residual")):
        _need(t, n, F32, 1)
    _need(option_mask, "option_mask", torch.uint8, 1)
    if not prior.numel() == cosine.numel() == residual.numel() == option_mask.numel():
        raise ValueError("head_combine_f32: one prior, cosine, residual and mask entry per option")
    out = torch.empty_like(prior)
    call("dx_head_combine_f32", _ptr(prior), _ptr(cosine), _ptr(residual), _ptr(option_mask), _ptr(out),
         prior.numel(), float(gate), float(joint_scale), _stream())
    return out


def int32_device(values: Sequence[int] | torch.Tensor, device: torch.device | str) -> torch.Tensor:
    return torch.as_tensor(values, dtype=torch.int32).to(device)
