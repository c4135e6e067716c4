"""Concurrent C-ABI calls: two host threads, each with its own stream and buffers, must get exactly
the results one thread gets alone.

The boundary promises that entry points are asynchronous on the caller's stream and thread-safe
given distinct output buffers (include/deciax_hip.h; the reference's engine serialises its
device forward with a lock, src/deciax/runtime/clef.py:21,36, so this is a property of the C ABI
that the engine itself does not rely on). ctypes releases the GIL for the foreign call, so the
host sides of the calls overlap too.
"""

from __future__ import annotations

import threading

import numpy as np
import pytest

from tests.conftest import say

pytestmark = pytest.mark.gpu

LENGTHS = [700, 333, 64]  # ragged packed batch: window, tile and length edges
HQ, HKV, D, HIDDEN, N = 8, 4, 128, 1024, 1536
ROUNDS = 6


def _inputs(torch, seed: int):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    t = sum(LENGTHS)
    x = torch.randn(t, HIDDEN, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(N, HIDDEN, device="cuda", generator=g) * 0.03).to(torch.bfloat16)
    qkv = (torch.randn(t, (HQ + 2 * HKV) * D, device="cuda", generator=g) * 0.5).to(torch.bfloat16)
    return x, w, qkv


def _run(torch, kernels, inputs, starts, lens, out_y, out_a):
    x, w, qkv = inputs
    kernels.linear(x, w, out=out_y)
    q, k, v = qkv[:, :HQ * D], qkv[:, HQ * D:(HQ + HKV) * D], qkv[:, (HQ + HKV) * D:]
    kernels.attention_varlen(q, k, v, starts, lens, max(LENGTHS), num_q_heads=HQ, num_kv_heads=HKV, head_dim=D,
                             scale=D ** -0.5, softcap=50.0, window=256, causal=True, out=out_a)


def test_two_threads_on_two_streams_match_one_thread() -> None:
    import torch
    from deciax_amd import kernels

    starts = torch.tensor(np.concatenate([[0], np.cumsum(LENGTHS)[:-1]]), dtype=torch.int32, device="cuda")
    lens = torch.tensor(LENGTHS, dtype=torch.int32, device="cuda")
    t = sum(LENGTHS)
    inputs = [_inputs(torch, 11 + i) for i in range(2)]

    # one thread, the default stream
    want = []
    for inp in inputs:
        y = torch.empty(t, N, device="cuda", dtype=torch.bfloat16)
        a = torch.empty(t, HQ * D, device="cuda", dtype=torch.bfloat16)
        _run(torch, kernels, inp, starts, lens, y, a)
        want.append((y, a))
    torch.cuda.synchronize()

    # two threads, a stream each (default priority), every round into fresh buffers
    results: list[list] = [[], []]
    errors: list[BaseException] = []
    barrier = threading.Barrier(2)

    def worker(i: int) -> None:
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                barrier.wait()
                for _ in range(ROUNDS):
                    y = torch.empty(t, N, device="cuda", dtype=torch.bfloat16)
                    a = torch.empty(t, HQ * D, device="cuda", dtype=torch.bfloat16)
                    _run(torch, kernels, inputs[i], starts, lens, y, a)
                    results[i].append((y, a))
            stream.synchronize()
        except BaseException as e:  # reported below, on the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors[0]
    torch.cuda.synchronize()
    for i in range(2):
        assert len(results[i]) == ROUNDS
        for y, a in results[i]:
            assert torch.equal(y, want[i][0]), f"thread {i}: GEMM output differs from the single-thread run"
            assert torch.equal(a, want[i][1]), f"thread {i}: attention output differs from the single-thread run"
    say(f"concurrency: 2 threads x {ROUNDS} rounds of linear + attention on 2 streams, bit-identical")
