"""ctypes binding of `libdeciax_hip.so` (the C ABI in `include/deciax_hip.h`).

Status codes map onto the reference's error conventions: argument errors raise
`ValueError` (the reference raises ValueError for bad shapes/dtypes,
src/deciax/kernels/projection.py:22-26, src/deciax/kernels/swiglu.py:183-186;
its HTTP layer maps them to 422, src/deciax/serve/app.py:260-261) and HIP
runtime failures raise `RuntimeError` (500, src/deciax/serve/app.py:262-264).

There is no fallback: if the library is missing, loading raises.
"""

from __future__ import annotations

import ctypes
import re
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_void_p
from pathlib import Path
from typing import Any

LIB_PATH = Path(__file__).resolve().parent / "libdeciax_hip.so"
HEADER = Path(__file__).resolve().parent.parent / "include" / "deciax_hip.h"

DX_OK, DX_ERR_INVALID, DX_ERR_UNSUPPORTED, DX_ERR_RUNTIME = 0, 1, 2, 3
DX_BF16, DX_F32 = 0, 1
DX_ACT_GELU_TANH, DX_ACT_SILU, DX_ACT_GELU_ERF, DX_ACT_NONE = 0, 1, 2, 3
DX_NOALLOC_SCRATCH_BYTES = 64 << 20

_p = c_void_p
_i32p = POINTER(c_int32)

# Argument types of every entry point, in header order.
SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "dx_version": (c_char_p, []),
    "dx_noalloc_init": (c_int, []),
    "dx_last_error": (c_char_p, []),
    "dx_device_arch": (c_int, [c_int, c_char_p, c_int]),
    "dx_attn_prefill": (
        c_int,
        [_p, _p, _p, _p, _p, _p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64, c_int64,
         c_float, c_float, c_int32, c_int32, c_int32, _p, c_int64, _p],
    ),
    "dx_attn_prefill_workspace": (c_int64, [c_int32, c_int32, c_int32, c_int32, c_int32]),
    "dx_attn_prefill_noalloc": (
        c_int,
        [_p, _p, _p, _p, _p, _p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64, c_int64,
         c_float, c_float, c_int32, c_int32, c_int32, _p],
    ),
    "dx_attn_prefill_masked": (
        c_int,
        [_p, _p, _p, _p, _p, _p, _p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64,
         c_int64, c_float, c_float, c_int32, c_int32, c_int32, _p, c_int64, _p],
    ),
    "dx_attn_prefill_masked_workspace": (c_int64, [c_int32, c_int32, c_int32, c_int32, c_int32]),
    "dx_attn_prefill_vt": (
        c_int,
        [_p, _p, _p, _p, _p, _p, _p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64, c_int64,
         c_float, c_float, c_int32, c_int32, _p],
    ),
    "dx_transpose_v": (c_int, [_p, _p, _p, _p, _p, c_int32, c_int32, c_int32, c_int32, c_int64, c_int64, _p]),
    "dx_vt_zero_tails": (c_int, [_p, _p, _p, c_int32, c_int32, c_int64, _p]),
    "dx_linear": (c_int, [_p, _p, _p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int32, _p]),
    "dx_gated_linear": (c_int, [_p, _p, _p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int32, _p]),
    "dx_qkv_rope": (
        c_int,
        [_p, _p, _p, _p, _p, _p, _p, _p, c_int64, c_int64, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64,
         c_int32, _p],
    ),
    "dx_linear_residual_norm": (
        c_int,
        [_p, _p, _p, _p, _p, _p, _p, _p, c_int64, c_int64, c_int64, c_int64, c_int64, c_float, _p],
    ),
    "dx_linear_residual_norm_counters": (c_int64, [c_int64]),
    "dx_pack_gate_up": (c_int, [_p, _p, _p, c_int64, c_int64, _p]),
    "dx_norm_project": (
        c_int, [_p, _p, _p, _p, _p, c_int64, c_int64, c_int64, c_float, _p, c_int64, _p]),
    "dx_norm_project_workspace": (c_int64, [c_int64, c_int64]),
    "dx_mlp": (
        c_int,
        [_p, _p, _p, _p, _p, c_int64, c_int64, c_int64, c_float, c_int32, c_int32, _p, c_int64, _p],
    ),
    "dx_mlp_workspace": (c_int64, [c_int64, c_int64, c_int64]),
    "dx_rmsnorm": (c_int, [_p, _p, _p, c_int64, c_int64, c_int64, c_int64, c_float, _p]),
    "dx_add_rmsnorm": (c_int, [_p, _p, _p, _p, _p, c_int64, c_int64, c_float, _p]),
    "dx_embed": (c_int, [_p, _p, _p, c_int64, c_int64, c_int64, c_float, _p, _p, c_float, _p]),
    "dx_rope": (c_int, [_p, _p, _p, _p, c_int64, c_int32, c_int32, c_int64, c_int32, _p]),
    "dx_readout": (
        c_int,
        [_p, _p, _p, _p, _p, _p, c_int32, c_int64, c_int64, c_int64, c_int64, c_int64, c_float, c_float, _p, _p, _p],
    ),
    "dx_layer_norm_f32": (c_int, [_p, _p, _p, _p, c_int64, c_int64, c_int64, c_int64, c_float, _p]),
    "dx_linear_f32": (
        c_int, [_p, _p, _p, _p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int32, c_int32, _p]),
    "dx_span_means_f32": (c_int, [_p, _p, _p, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64, _p]),
    "dx_mha_f32": (
        c_int,
        [_p, _p, _p, _p, _p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64, c_int64, _p],
    ),
    "dx_gather_rows_f32": (
        c_int, [_p, _p, _p, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64, c_int32, _p]),
    "dx_head_routing_f32": (c_int, [_p, _p, _p, _p, _p, c_int32, c_int32, c_int32, c_int32, _p]),
    "dx_head_fields_init_f32": (c_int, [_p, _p, _p, _p, _p, _p, c_int32, c_int32, c_int32, c_int32, _p]),
    "dx_head_features_f32": (
        c_int,
        [_p, _p, _p, _p, _p, _p, _p, _p, _p, c_int32, c_int32, c_int32, c_int32, c_int32, c_float, _p],
    ),
    "dx_head_combine_f32": (c_int, [_p, _p, _p, _p, _p, c_int64, c_float, c_float, _p]),
}

_LIB: ctypes.CDLL | None = None


def header_symbols() -> list[str]:
    """Names of every function the public header declares."""
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:const\s+char\s*\*|int64_t|int)\s*\**\s*(dx_\w+)\s*\(", text, re.M)


def lib() -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing; build it with `python -m deciax_amd.build`")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def check(status: int, what: str) -> None:
    if status == DX_OK:
        return
    msg = lib().dx_last_error().decode(errors="replace")
    if status in (DX_ERR_INVALID, DX_ERR_UNSUPPORTED):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def call(name: str, *args: Any) -> None:
    check(getattr(lib(), name)(*args), name)


def device_arch(device: int = 0) -> str:
    buf = ctypes.create_string_buffer(64)
    check(lib().dx_device_arch(device, buf, len(buf)), "dx_device_arch")
    return buf.value.decode()
