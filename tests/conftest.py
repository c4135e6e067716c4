"""Shared fixtures: the `gpu` marker, device round-trips and seeded inputs.

GPU tests call the C ABI through `deciax_amd`; the oracle is the checker.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    if not any("gpu" in item.keywords for item in items):
        return
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter, exitstatus: int, config: pytest.Config) -> None:
    """Print the measured decision-forward parity numbers (tests/forward_parity.py) after the run, so
    that they appear in the log of a quiet (-q) run as well."""
    records = getattr(sys.modules.get("tests.forward_parity"), "RECORDS", None)
    if records:
        terminalreporter.write_sep("-", "decision-forward parity, measured")
        for line in records:
            terminalreporter.write_line(line)


def rng(seed: int = 0) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def bf16_np(x: np.ndarray) -> np.ndarray:
    from oracle.numerics import bf16

    return bf16(np.asarray(x, np.float32))


def to_dev(x: np.ndarray, dtype: str = "bf16"):
    """numpy fp32 -> device tensor (bf16 values rounded to nearest even, or fp32)."""
    import torch

    from oracle.numerics import bf16_bits

    if dtype == "bf16":
        bits = bf16_bits(np.asarray(x, np.float32))
        return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).cuda()
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


def to_np(t) -> np.ndarray:
    import torch

    return t.detach().to("cpu", torch.float32).numpy()


def i32(values) -> "object":
    import torch

    return torch.as_tensor(np.asarray(values, np.int64).astype(np.int32)).cuda()


def say(msg: str) -> None:
    """Name the case on stdout before a GPU step (so a crash log shows what ran)."""
    print(msg, flush=True)
