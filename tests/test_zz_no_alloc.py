"""dx_attn_prefill_noalloc against dx_attn_prefill on the GPU: the allocation-free entry point stages V^T
in the library's static per-GPU scratch and must give exactly the allocating entry point's output, on
two calls in a row, the second with a smaller input (the scratch keeps the first call's contents)."""

from __future__ import annotations

import numpy as np
import pytest

from tests.conftest import bf16_np, i32, rng, say, to_dev, to_np

pytestmark = pytest.mark.gpu


def _case(seed: int, lengths: list[int], hq: int, hkv: int, d: int):
    r = rng(seed)
    rows = int(sum(lengths))
    q, k, v = (bf16_np(r.normal(size=(rows, h * d)).astype(np.float32) * 0.5) for h in (hq, hkv, hkv))
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])
    return to_dev(q), to_dev(k), to_dev(v), i32(starts), i32(lengths)


def test_noalloc_attention_matches_allocating_entry_point() -> None:
    import torch

    from deciax_amd import _lib
    from deciax_amd import kernels as K

    calls = [  # (lengths, hq, hkv, d, window, softcap): the second is smaller than the first
        ([2048, 2048, 2048, 2048, 1500, 2048, 977, 2048], 16, 8, 256, 0, 50.0),
        ([300, 45, 129], 8, 4, 128, 64, 0.0),
    ]
    for lengths, hq, hkv, d, window, softcap in calls:
        say(f"noalloc attention lengths={lengths} hq={hq} hkv={hkv} d={d} window={window} softcap={softcap}")
        need = _lib.lib().dx_attn_prefill_workspace(len(lengths), max(lengths), hkv, d, _lib.DX_BF16)
        assert 0 < need <= _lib.DX_NOALLOC_SCRATCH_BYTES
        q, k, v, starts, lens = _case(len(lengths) + d, lengths, hq, hkv, d)
        kw = dict(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, scale=d ** -0.5, softcap=softcap, window=window)
        want = K.attention_varlen(q, k, v, starts, lens, max(lengths), **kw)
        got = torch.full_like(want, float("nan"))
        K.attention_varlen_noalloc(q, k, v, starts, lens, max(lengths), out=got, **kw)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_np(got), to_np(want))
    with pytest.raises(ValueError, match="static scratch"):
        q, k, v, starts, lens = _case(1, [4096] * 9, 16, 8, 256)
        K.attention_varlen_noalloc(q, k, v, starts, lens, 4096, num_q_heads=16, num_kv_heads=8, head_dim=256,
                                   scale=1 / 16, out=torch.empty((9 * 4096, 16 * 256), dtype=torch.bfloat16,
                                                                 device="cuda"))
