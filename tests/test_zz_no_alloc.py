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


_FIRST_CALL_UNDER_CAPTURE = r'''
import sys
sys.path.insert(0, sys.argv[1])
import numpy as np
import torch
from deciax_amd import kernels as K
from tests.conftest import bf16_np, i32, rng, to_dev

r = rng(3)
lengths, hq, hkv, d = [700, 129], 16, 8, 256
rows = sum(lengths)
q, k, v = (to_dev(bf16_np(r.normal(size=(rows, h * d)).astype(np.float32) * 0.5)) for h in (hq, hkv, hkv))
starts, lens = i32([0, lengths[0]]), i32(lengths)
kw = dict(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, scale=1 / 16, softcap=50.0, window=0)
want = K.attention_varlen(q, k, v, starts, lens, max(lengths), **kw)   # the allocating entry point
out = torch.empty_like(want)
torch.cuda.synchronize()
refused = False
try:
    with torch.cuda.graph(torch.cuda.CUDAGraph()):
        K.attention_varlen_noalloc(q, k, v, starts, lens, max(lengths), out=out, **kw)  # first call, captured
except ValueError as e:
    refused = "dx_noalloc_init" in str(e)
torch.cuda.synchronize()
print("first call under capture refused:", refused, flush=True)
assert refused
K.noalloc_init()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    K.attention_varlen_noalloc(q, k, v, starts, lens, max(lengths), out=out, **kw)
for i in range(3):
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), f"replay {i} differs"
print("ok: replays after dx_noalloc_init equal the allocating entry point", flush=True)
'''


def test_noalloc_first_call_under_graph_capture_is_refused_then_works_after_init() -> None:
    """In a fresh process (no earlier lookup of the static scratch), the first allocation-free call made
    under HIP graph capture is refused with DX_ERR_UNSUPPORTED (the lookup is not allowed there) instead
    of being attempted; after dx_noalloc_init the same call captures, and every replay equals the
    allocating entry point's output."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parent.parent)
    say("noalloc: first call under graph capture, in a fresh process")
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE, root], capture_output=True, text=True,
                         timeout=240, cwd=root)
    print(res.stdout[-2000:], res.stderr[-3000:], flush=True)
    assert res.returncode == 0, res.stderr[-3000:]
    assert "ok: replays" in res.stdout
