"""The oracle reproduces the committed golden fixtures (tests/golden/, written by
tests/golden/make_golden.py): a regression guard on the checker itself."""

from __future__ import annotations

from pathlib import Path

import numpy as np

from oracle.numerics import from_bits
from tests.golden import make_golden as mg

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_attention_fixture_reproduces() -> None:
    g = np.load(GOLDEN / "attention_packed.npz")
    case = mg.attention_case()
    for key in ("q_bits", "k_bits", "v_bits", "seq_start", "seq_len"):
        np.testing.assert_array_equal(case[key], g[key])
    np.testing.assert_allclose(case["out_bf16"], g["out_bf16"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(case["out_f32"], g["out_f32"], rtol=1e-6, atol=1e-6)
    # the fixture's inputs are bf16 values and its sequences never see each other
    q = from_bits(g["q_bits"])
    assert q.shape == (122, 4, 64) and np.isfinite(g["out_bf16"]).all()
    # bf16 and fp32 forms within the attention tolerance, 2e-2 of the output's largest magnitude
    assert np.abs(g["out_bf16"] - g["out_f32"]).max() < 2e-2 * np.abs(g["out_f32"]).max()


def test_forward_fixture_reproduces() -> None:
    g = np.load(GOLDEN / "forward_micro.npz")
    b = mg.micro_batch()
    for key, value in b.items():
        np.testing.assert_array_equal(value, g[key])
    z, p = mg.micro_reference(np.float64)
    np.testing.assert_allclose(z, g["logits"], rtol=0, atol=1e-5)
    np.testing.assert_allclose(p, g["probs"], rtol=0, atol=1e-6)
    # per-question softmax sums to one; exact and fp32 sums stay within fp32 noise of each other
    q_off = g["q_offsets"]
    for a, c in zip(q_off[:-1], q_off[1:]):
        assert abs(g["probs"][a:c].sum() - 1) < 1e-5
    assert np.abs(g["probs"] - g["probs_f32"]).max() < 1e-3
