"""Pins the oracle's attention (oracle/attention.py) on the CPU.

Three independent checks, each able to catch a dropped term, a wrong sign, an
off-by-one window or a transposed operand:
  * a brute-force per-(sequence, head, query) loop in float64, the reference's
    `_naive` (tests/kernels/test_attention.py:17-32) extended with GQA, the
    causal window and soft-capping;
  * the dense causal-GQA closed form of tests/test_qwen3_5.py:27-40 (repeat
    K/V, einsum, where(-1e30), softmax) at s=139 (over one 128-query block)
    with a key mask of length 97;
  * transformers' Gemma-2 eager attention (TF/models/gemma2/modeling_gemma2.py:
    eager_attention_forward, with TF/masking_utils.py sliding-window masks) on
    torch CPU in fp32.
Plus closed-form special cases: a window of 1 returns V of the same position,
a uniform query returns the running mean of V, and the flash rounding form
equals the normalized form in fp32.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle.attention import attention_flops, attention_packed, attention_seq, visible
from tests.conftest import rng


def brute(q, k, v, *, scale, cap, window, causal):
    """float64 loops: out[i, h] = sum_j softmax_j(cap-tanh(scale q.k)) v_j over visible keys."""
    length, hq, d = q.shape
    group = hq // k.shape[1]
    out = np.zeros((length, hq, d))
    for h in range(hq):
        g = h // group
        for i in range(length):
            keys = [j for j in range(length)
                    if (j <= i and (window <= 0 or j > i - window)) if causal] if causal else \
                [j for j in range(length) if window <= 0 or abs(i - j) <= window]
            s = np.array([float(np.dot(q[i, h].astype(np.float64), k[j, g].astype(np.float64))) for j in keys])
            s = s * scale
            if cap > 0:
                s = cap * np.tanh(s / cap)
            w = np.exp(s - s.max())
            out[i, h] = (w / w.sum()) @ v[keys, g].astype(np.float64)
    return out


@pytest.mark.parametrize("causal,window,cap,hq,hkv", [
    (True, 0, 0.0, 4, 2), (True, 5, 0.0, 4, 2), (True, 7, 50.0, 4, 1), (True, 0, 50.0, 2, 2),
    (False, 0, 0.0, 2, 1), (False, 3, 30.0, 4, 2),
])
def test_oracle_matches_brute_force(causal, window, cap, hq, hkv) -> None:
    r = rng(11)
    length, d = 23, 16
    q = r.normal(size=(length, hq, d)).astype(np.float32) * 2
    k = r.normal(size=(length, hkv, d)).astype(np.float32) * 2
    v = r.normal(size=(length, hkv, d)).astype(np.float32)
    scale = d ** -0.5
    got = attention_seq(q, k, v, scale=scale, softcap_value=cap, window=window, causal=causal, bf16=False)
    want = brute(q, k, v, scale=scale, cap=cap, window=window, causal=causal)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_blocked_causal_gqa_matches_dense_closed_form() -> None:
    """tests/test_qwen3_5.py:27-40: s=139 spans two 128-query blocks; the second sequence's keys
    are masked past 97 (rows past 97 are padding and not compared, as the reference's valid-row
    comparison at tests/kernels/test_attention.py:42)."""
    r = rng(3)
    s, d = 139, 8
    q = r.normal(size=(2, s, 4, d)).astype(np.float32)
    k = r.normal(size=(2, s, 2, d)).astype(np.float32)
    v = r.normal(size=(2, s, 2, d)).astype(np.float32)
    lengths = [s, 97]
    keys, values = np.repeat(k, 2, axis=2), np.repeat(v, 2, axis=2)
    logits = np.einsum("bqhd,bkhd->bhqk", q, keys).astype(np.float32) * np.float32(d ** -0.5)
    mask = np.arange(s)[None] < np.array(lengths)[:, None]
    causal = np.arange(s)[:, None] >= np.arange(s)[None, :]
    logits = np.where(mask[:, None, None, :] & causal, logits, np.float32(-1e30))
    e = np.exp(logits - logits.max(-1, keepdims=True))
    expected = np.einsum("bhqk,bkhd->bqhd", e / e.sum(-1, keepdims=True), values)

    packed = attention_packed(q.reshape(2 * s, 4, d), k.reshape(2 * s, 2, d), v.reshape(2 * s, 2, d),
                              [0, s], lengths, scale=d ** -0.5, causal=True, bf16=False).reshape(2, s, 4, d)
    for b, n in enumerate(lengths):
        np.testing.assert_allclose(packed[b, :n], expected[b, :n], atol=1e-6, rtol=1e-5)
    assert not packed[1, 97:].any(), "rows past a sequence's length must stay untouched"


@pytest.mark.parametrize("window", [0, 6])
def test_oracle_matches_transformers_gemma2_eager(window: int) -> None:
    torch = pytest.importorskip("torch")
    pytest.importorskip("transformers")
    from transformers.models.gemma2.modeling_gemma2 import eager_attention_forward

    r = rng(5)
    length, hq, hkv, d, cap = 37, 4, 2, 32, 50.0
    scale = 24.0 ** -0.5
    q = r.normal(size=(length, hq, d)).astype(np.float32) * 3
    k = r.normal(size=(length, hkv, d)).astype(np.float32) * 3
    v = r.normal(size=(length, hkv, d)).astype(np.float32)

    class Module:
        num_key_value_groups = hq // hkv
        training = False
        head_dim = d

    i = np.arange(length)[:, None]
    j = np.arange(length)[None, :]
    allowed = (j <= i) & ((j > i - window) if window else True)
    mask = torch.from_numpy(np.where(allowed, 0.0, np.finfo(np.float32).min).astype(np.float32))[None, None]
    tq, tk, tv = (torch.from_numpy(a).permute(1, 0, 2)[None] for a in (q, k, v))
    want, _ = eager_attention_forward(Module(), tq, tk, tv, mask, scaling=scale, softcap=cap)
    got = attention_seq(q, k, v, scale=scale, softcap_value=cap, window=window, causal=True, bf16=False)
    np.testing.assert_allclose(got, want[0].numpy(), rtol=2e-5, atol=2e-5)


def test_window_one_returns_own_value_and_uniform_query_gives_running_mean() -> None:
    r = rng(2)
    length, d = 20, 8
    q = r.normal(size=(length, 2, d)).astype(np.float32)
    k = r.normal(size=(length, 1, d)).astype(np.float32)
    v = r.normal(size=(length, 1, d)).astype(np.float32)
    own = attention_seq(q, k, v, scale=0.3, window=1, causal=True, bf16=False)
    np.testing.assert_allclose(own, np.repeat(v, 2, axis=1), rtol=1e-6, atol=1e-6)
    zero_q = np.zeros_like(q)
    mean = attention_seq(zero_q, k, v, scale=0.3, softcap_value=50.0, causal=True, bf16=False)
    running = np.cumsum(v[:, 0].astype(np.float64), axis=0) / np.arange(1, length + 1)[:, None]
    np.testing.assert_allclose(mean[:, 0], running, rtol=1e-5, atol=1e-6)
    w3 = attention_seq(zero_q, k, v, scale=0.3, window=3, causal=True, bf16=False)
    for i in range(length):
        lo = max(0, i - 2)
        np.testing.assert_allclose(w3[i, 1], v[lo:i + 1, 0].mean(0), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("cap", [0.0, 50.0])
def test_flash_and_normalized_rounding_agree_in_fp32_and_differ_by_bf16_noise(cap: float) -> None:
    r = rng(9)
    q, k, v = (r.normal(size=(150, 2, 32)).astype(np.float32) for _ in range(3))
    kw = dict(scale=32 ** -0.5, softcap_value=cap, causal=True)
    a = attention_seq(q, k, v, bf16=False, rounding="flash", **kw)
    b = attention_seq(q, k, v, bf16=False, rounding="normalized", **kw)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)
    c = attention_seq(q, k, v, bf16=True, rounding="flash", **kw)
    e = attention_seq(q, k, v, bf16=True, rounding="normalized", **kw)
    assert np.abs(c - e).max() < 2e-2 and np.abs(c - a).max() < 2e-2
    assert np.abs(c - a).max() > 0, "bf16 mode must actually round"


def test_visible_matches_gemma_causal_window() -> None:
    """q - W < k <= q (TF/masking_utils.py: sliding_window_overlay and causal_mask_function)."""
    ok = visible(np.arange(10), np.arange(10), 10, 4, True)
    for i in range(10):
        for j in range(10):
            assert ok[i, j] == (j <= i and j > i - 4)
    assert not visible(np.arange(10), np.arange(10), 7, 0, True)[:, 7:].any()


def test_attention_flops_counts_visible_pairs() -> None:
    for n, w in [(50, 0), (50, 8), (7, 20), (4096, 4096), (5000, 4096)]:
        pairs = int(visible(np.arange(n), np.arange(n), n, w, True).sum()) if n <= 64 else None
        flops = attention_flops([n], num_q_heads=3, head_dim=16, window=w)
        if pairs is not None:
            assert flops == 4 * 16 * 3 * pairs
        if w == 0 or w >= n:
            assert flops == 4 * 16 * 3 * n * (n + 1) // 2
        else:
            assert flops == 4 * 16 * 3 * (w * (w + 1) // 2 + (n - w) * w)
    assert math.isclose(attention_flops([2048] * 8, num_q_heads=16, head_dim=256), 2.750e11, rel_tol=1e-3)


def brute_masked(q, k, v, key_mask, *, scale, window, causal):
    """float64 loops with an arbitrary key mask and separate query / key lengths: the reference's
    `_naive` (tests/kernels/test_attention.py:17-32: keys j with mask[j] and |i - j| <= window)
    extended with the causal rule of blocked.py:25 (j <= i) and GQA. Rows with no key are left out
    (None), as `_naive` leaves them."""
    nq, hq, d = q.shape
    nk, hkv = k.shape[0], k.shape[1]
    out = np.zeros((nq, hq, d))
    empty = []
    for i in range(nq):
        if causal:
            keys = [j for j in range(nk) if key_mask[j] and j <= i and (window <= 0 or j > i - window)]
        else:
            keys = [j for j in range(nk) if key_mask[j] and (window <= 0 or abs(i - j) <= window)]
        if not keys:
            empty.append(i)
            continue
        for h in range(hq):
            g = h // (hq // hkv)
            s = np.array([float(np.dot(q[i, h].astype(np.float64), k[j, g].astype(np.float64))) for j in keys])
            w = np.exp(s * scale - (s * scale).max())
            out[i, h] = (w / w.sum()) @ v[keys, g].astype(np.float64)
    return out, empty


@pytest.mark.parametrize("nq,nk,causal,window", [(23, 23, True, 0), (17, 29, True, 0), (29, 17, True, 6),
                                                 (20, 26, False, 0), (26, 20, False, 4)])
def test_oracle_key_mask_matches_brute_force(nq, nk, causal, window) -> None:
    r = rng(nq * 31 + nk)
    hq, hkv, d = 4, 2, 16
    q = r.normal(size=(nq, hq, d)).astype(np.float32)
    k = r.normal(size=(nk, hkv, d)).astype(np.float32)
    v = r.normal(size=(nk, hkv, d)).astype(np.float32)
    key_mask = r.random(nk) < 0.6
    key_mask[0] = False  # causal row 0 then sees no key
    for rounding in ("flash", "normalized"):
        got = attention_seq(q, k, v, scale=0.25, window=window, causal=causal, bf16=False, key_mask=key_mask,
                            rounding=rounding)
        want, empty = brute_masked(q, k, v, key_mask, scale=0.25, window=window, causal=causal)
        keep = np.setdiff1d(np.arange(nq), empty)
        np.testing.assert_allclose(got[keep], want[keep], rtol=1e-5, atol=1e-5)
        if empty:  # softmax over nk equal MASK_FILL scores: the mean of all value rows
            mean = np.repeat(v.astype(np.float64).mean(axis=0), hq // hkv, axis=0)
            np.testing.assert_allclose(got[empty], np.broadcast_to(mean, (len(empty), hq, d)), rtol=1e-5, atol=1e-5)


def test_oracle_non_prefix_mask_matches_dense_closed_form() -> None:
    """The dense form of tests/test_qwen3_5.py:27-40 (repeat K/V, einsum, where(-1e30), softmax) with
    a non-prefix key mask whose first keys are hidden, so the first causal rows see no key and take
    the uniform softmax the finite MASK_FILL gives them; every row is compared."""
    r = rng(8)
    s, d = 139, 8
    q = r.normal(size=(s, 4, d)).astype(np.float32)
    k = r.normal(size=(s, 2, d)).astype(np.float32)
    v = r.normal(size=(s, 2, d)).astype(np.float32)
    mask = r.random(s) < 0.5
    mask[:3] = False
    keys, values = np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1)
    logits = np.einsum("qhd,khd->hqk", q, keys).astype(np.float32) * np.float32(d ** -0.5)
    causal = np.arange(s)[:, None] >= np.arange(s)[None, :]
    logits = np.where(mask[None, None, :] & causal[None], logits, np.float32(-1e30))
    e = np.exp(logits - logits.max(axis=-1, keepdims=True))
    want = np.einsum("hqk,khd->qhd", e / e.sum(axis=-1, keepdims=True), values)
    got = attention_seq(q, k, v, scale=d ** -0.5, bf16=False, key_mask=mask)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
