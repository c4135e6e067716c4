"""Implementation selection for the decision path (the role of src/deciax/ops/backend.py:9-18).

The reference's `ImplChoice` is `auto | jax | pallas`; this package adds the
value `"hip"` — the gfx950 kernels of `libdeciax_hip.so`. `resolve` raises
ValueError for anything it cannot serve, as the reference does for unknown
values (backend.py:18) and for an impl whose hardware is missing
(src/deciax/models/clef/model.py:46-50).
"""

from __future__ import annotations

from typing import Literal

Impl = Literal["hip"]
ImplChoice = Literal["auto", "jax", "pallas", "hip"]
REQUIRED_ARCH = "gfx950"


def hip_device_arch(device: int = 0) -> str | None:
    """gfx name of the visible device, or None when no HIP device is present."""
    import torch

    if not torch.cuda.is_available():
        return None
    from deciax_amd import _lib

    return _lib.device_arch(device)


def resolve(impl: ImplChoice) -> Impl:
    """`auto` and `hip` resolve to `hip` when a gfx950 device is visible; `jax` and `pallas` are the
    reference package's own backends and are not provided here."""
    if impl in ("jax", "pallas"):
        raise ValueError(f"impl={impl!r} is provided by the reference deciax package; deciax_amd serves 'hip'")
    if impl not in ("auto", "hip"):
        raise ValueError(f"impl must be 'auto', 'jax', 'pallas' or 'hip', got {impl!r}")
    arch = hip_device_arch()
    if arch is None:
        raise ValueError("impl='hip' requires a visible MI355X (gfx950) GPU; none was found")
    if arch != REQUIRED_ARCH:
        raise ValueError(f"impl='hip' requires a {REQUIRED_ARCH} GPU, found {arch}")
    return "hip"
