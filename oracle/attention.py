"""Causal GQA prefill attention, restated in numpy (test infrastructure only).

Follows `attention` in src/deciax/kernels/attention/blocked.py:9-32: K/V
repeated to every query head (:12-13), queries in blocks of 128 (:15-17),
fp32 scores times the scale (:21), masked scores set to MASK_FILL = -1e30
(src/deciax/kernels/attention/reference.py:8, blocked.py:23-27), softmax in
fp32, weights rounded to the input dtype (:27), P.V accumulated in fp32 and
rounded (:28-29).

bf16 rounding of the probabilities has two forms in the reference:
  * "normalized" — blocked.py:27-29 rounds the normalised softmax weights;
  * "flash" (default) — the online-softmax kernel, pallas.py:104-116, rounds
    the unnormalised p = exp(s - m) to the value dtype for P.V (pv_t, :47-49),
    sums l from the unrounded p and divides at the end (:113-116).
The two differ by bf16 noise (about 2^-9 relative per weight), which after a
few layers is of the order of 1e-3 in option probabilities, so the oracle
restates the flash form exactly as the GPU path evaluates it: the reference
point m is the row maximum, except for soft-capped scores, where every score
lies in (-cap, cap) and m is the fixed bound cap / 2 (the kernel needs no
running max then). With that fixed shift the bf16 kernel also multiplies the
query by c1 = 2 log2(e) scale / cap as it loads it, one more bf16 rounding, so
that its QK^T products are already the exponent's argument; the flash form in
bf16 mode scores with bf16(c1 q) as well. In fp32 the two forms coincide up to
fp32 rounding.

Gemma-2 additions the reference has no code for:
  * logit soft-capping after scaling and before the mask,
    TF/models/gemma2/modeling_gemma2.py:203-211;
  * the causal sliding window `q - W < k <= q`, TF/masking_utils.py:92-99,134-138
    (the reference's own window is symmetric, reference.py:14-16, and is what
    `causal=False` with a window gives here).
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np

from oracle.numerics import F32, acc_dtype, matmul, maybe, softcap

MASK_FILL = F32(-1e30)
BLOCK = 128
LOG2E = 1.4426950408889634


def visible(qpos: np.ndarray, kpos: np.ndarray, length: int, window: int, causal: bool) -> np.ndarray:
    """[nq, nk] boolean: may query qpos[i] attend to key kpos[j]."""
    qp = np.asarray(qpos)[:, None]
    kp = np.asarray(kpos)[None, :]
    ok = kp < length
    if causal:
        ok = ok & (kp <= qp)
        if window > 0:
            ok = ok & (kp > qp - window)
    elif window > 0:
        ok = ok & (np.abs(qp - kp) <= window)
    return ok


FIXED_SHIFT_MAX_CAP = 56.0  # p = exp(t - cap/2) stays a normal fp32 / bf16 number for cap <= 56


def attention_seq(q: np.ndarray, k: np.ndarray, v: np.ndarray, *, scale: float, softcap_value: float = 0.0,
                  window: int = 0, causal: bool = True, bf16: bool = True,
                  query_pos: Sequence[int] | None = None, rounding: str = "flash",
                  key_mask: np.ndarray | None = None) -> np.ndarray:
    """One sequence: q [Lq, Hq, D], k/v [Lk, Hkv, D] (values already in the input dtype) ->
    out [nq, Hq, D] for the query positions `query_pos` (default: all Lq).

    `key_mask` [Lk] (bool, default all true) hides keys as blocked.py:23-27 does; causal visibility
    compares indices, key j <= query i (blocked.py:25), also when Lq != Lk. A query that sees no
    key at all gets softmax over Lk equal MASK_FILL scores: the uniform average of every value row."""
    if rounding not in ("flash", "normalized"):
        raise ValueError(f"rounding must be 'flash' or 'normalized', got {rounding!r}")
    length, hq, d = q.shape
    nk, hkv = k.shape[0], k.shape[1]
    group = hq // hkv
    qpos = np.arange(length) if query_pos is None else np.asarray(query_pos)
    out = np.zeros((len(qpos), hq, d), F32)
    kpos = np.arange(nk)
    kmask = np.ones(nk, bool) if key_mask is None else np.asarray(key_mask, bool)
    fixed = 0.0 < softcap_value <= FIXED_SHIFT_MAX_CAP
    fold = fixed and bf16 and rounding == "flash"
    c1 = F32(2.0 * LOG2E * scale / softcap_value) if fold else F32(1.0)
    for b0 in range(0, len(qpos), BLOCK):
        rows = qpos[b0:b0 + BLOCK]
        ok = visible(rows, kpos, nk, window, causal) & kmask[None, :]
        empty = ~ok.any(axis=1, keepdims=True)  # every score MASK_FILL: softmax is uniform over all keys
        for h in range(hq):
            g = h // group
            if fold:  # the kernel's pre-scaled query: scores from bf16(c1 q), then back to scale units
                scores = matmul(maybe(q[rows, h, :] * c1, True), k[:, g, :].T) * F32(scale / c1)
            else:
                scores = matmul(q[rows, h, :], k[:, g, :].T) * F32(scale)
            scores = softcap(scores, softcap_value)
            scores = np.where(ok, scores, MASK_FILL)
            vg = v[:, g, :].astype(F32)
            if rounding == "normalized":
                m = scores.max(axis=1, keepdims=True)
                e = np.exp(scores - m)
                w = maybe((e / e.sum(axis=1, keepdims=True)).astype(F32), bf16)
                res = matmul(w, vg)
            else:
                m = F32(0.5 * softcap_value) if fixed else scores.max(axis=1, keepdims=True)
                p = np.where(ok, np.exp(scores - m), F32(0.0)).astype(F32)
                p = np.where(empty, F32(1.0), p).astype(F32)
                res = matmul(maybe(p, bf16), vg) / p.sum(axis=1, keepdims=True, dtype=acc_dtype()).astype(F32)
            out[b0:b0 + len(rows), h, :] = maybe(res.astype(F32), bf16)
    return out


def attention_packed(q: np.ndarray, k: np.ndarray, v: np.ndarray, seq_start: Sequence[int], seq_len: Sequence[int],
                     *, scale: float, softcap_value: float = 0.0, window: int = 0, causal: bool = True,
                     bf16: bool = True, rounding: str = "flash") -> np.ndarray:
    """Packed rows: q [R, Hq, D], k/v [R, Hkv, D]; sequence s is rows [start_s, start_s + len_s).
    Rows outside every sequence stay zero."""
    out = np.zeros(q.shape, F32)
    for start, length in zip(seq_start, seq_len):
        sl = slice(start, start + length)
        out[sl] = attention_seq(q[sl], k[sl], v[sl], scale=scale, softcap_value=softcap_value, window=window,
                                causal=causal, bf16=bf16, rounding=rounding)
    return out


def attention_flops(lengths: Sequence[int], *, num_q_heads: int, head_dim: int, window: int = 0,
                    causal: bool = True) -> int:
    """4 * D * Hq * (number of visible (query, key) pairs): the algorithmic work of one layer."""
    pairs = 0
    for n in lengths:
        if causal and window <= 0:
            pairs += n * (n + 1) // 2
        elif causal:
            w = min(window, n)
            pairs += w * (w + 1) // 2 + (n - w) * w
        else:
            pairs += n * n if window <= 0 else int(visible(np.arange(n), np.arange(n), n, window, False).sum())
    return 4 * head_dim * num_q_heads * pairs
