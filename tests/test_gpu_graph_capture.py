"""HIP graph capture of C-ABI calls: the allocation-free attention entry point (for callers under graph
capture) and a GEMM, captured once and replayed. Every replay must equal the eager result, with other
eager work, including an allocation-free attention call on another input that rewrites the shared
static scratch, run and synchronised between the replays."""

from __future__ import annotations

import numpy as np
import pytest

from tests.conftest import bf16_np, i32, rng, say, to_dev

pytestmark = pytest.mark.gpu


def _attn_case(seed: int, lengths: list[int], hq: int, hkv: int, d: int):
    r = rng(seed)
    rows = int(sum(lengths))
    q, k, v = (bf16_np(r.normal(size=(rows, h * d)).astype(np.float32) * 0.5) for h in (hq, hkv, hkv))
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])
    return to_dev(q), to_dev(k), to_dev(v), i32(starts), i32(lengths)


def test_graph_replays_of_noalloc_attention_and_gemm_match_eager() -> None:
    import torch

    from deciax_amd import kernels as K

    hq, hkv, d = 16, 8, 256
    lengths = [1200, 700, 333]
    kw = dict(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, scale=1 / 16, softcap=50.0, window=512)
    q, k, v, starts, lens = _attn_case(5, lengths, hq, hkv, d)
    r = rng(6)
    x = to_dev(bf16_np(r.normal(size=(sum(lengths), 2048)).astype(np.float32)))
    w = to_dev(bf16_np(r.normal(size=(1024, 2048)).astype(np.float32) * 0.02))

    # another input for the eager calls between replays: it rewrites the static scratch
    q2, k2, v2, starts2, lens2 = _attn_case(7, [900, 64], hq, hkv, d)
    out2 = torch.empty((q2.shape[0], hq * d), dtype=torch.bfloat16, device="cuda")

    att_want = torch.empty((q.shape[0], hq * d), dtype=torch.bfloat16, device="cuda")
    K.attention_varlen_noalloc(q, k, v, starts, lens, max(lengths), out=att_want, **kw)
    y_want = K.linear(x, w)
    torch.cuda.synchronize()

    att = torch.empty_like(att_want)
    y = torch.empty_like(y_want)

    def step() -> None:
        K.attention_varlen_noalloc(q, k, v, starts, lens, max(lengths), out=att, **kw)
        K.linear(x, w, out=y)

    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()

    for i in range(4):
        att.fill_(float("nan"))
        y.fill_(float("nan"))
        K.attention_varlen_noalloc(q2, k2, v2, starts2, lens2, 900, out=out2, **kw)  # eager, same scratch
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(att, att_want), f"replay {i}: attention differs from the eager result"
        assert torch.equal(y, y_want), f"replay {i}: GEMM differs from the eager result"
    say("graph capture: 4 replays of noalloc attention + GEMM equal the eager results")
