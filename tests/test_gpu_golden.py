"""The HIP path against the committed golden fixtures (tests/golden/): attention within 2e-2 of the
oracle's bf16 output, and the micro-model decision forward checked layer by layer and at the readout
(tests/forward_parity.py), with the same argmax as the fixture's exactly summed probabilities
wherever their top-2 gap exceeds twice the fp32 oracle's drift from them."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from tests.conftest import i32, say, to_np
from tests.forward_parity import check_forward

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _bits_dev(bits: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def test_attention_matches_golden() -> None:
    from deciax_amd import kernels as K
    from tests.golden.make_golden import ATTN

    say("golden attention fixture")
    g = np.load(GOLDEN / "attention_packed.npz")
    rows = g["q_bits"].shape[0]
    q, k, v = (_bits_dev(g[n].reshape(rows, -1)) for n in ("q_bits", "k_bits", "v_bits"))
    out = K.attention_varlen(q, k, v, i32(g["seq_start"]), i32(g["seq_len"]), int(g["seq_len"].max()),
                             num_q_heads=ATTN["hq"], num_kv_heads=ATTN["hkv"], head_dim=ATTN["d"],
                             scale=ATTN["scale"], softcap=ATTN["softcap"], window=ATTN["window"], causal=True)
    got = to_np(out).reshape(g["out_bf16"].shape)
    want = g["out_bf16"]
    err = np.abs(got - want).max()
    assert err <= 2e-2 * np.abs(want).max(), err


def test_micro_forward_matches_golden() -> None:
    import torch

    from deciax_amd import gemma
    from tests.golden.make_golden import MICRO, micro_weights

    say("golden micro decision forward")
    g = np.load(GOLDEN / "forward_micro.npz")
    cfg = gemma.GemmaConfig("micro", MICRO.layers, MICRO.hidden, MICRO.heads, MICRO.kv_heads, MICRO.head_dim,
                            MICRO.intermediate, MICRO.vocab, window=MICRO.window, query_pre_attn_scalar=128.0,
                            max_position=256)
    assert cfg.query_scale == MICRO.query_scale
    w = gemma.weights_from_host(cfg, micro_weights(int(g["seed"])), keep_unpacked=True)
    lengths = g["lengths"].tolist()
    starts = g["seq_start"].tolist()
    ids = [g["ids"][s:s + n].tolist() for s, n in zip(starts, lengths)]
    # rebuild per-request option lists (request, position-in-request, label) from the flat layout
    opt_req = np.searchsorted(np.array(starts), g["opt_pos"], side="right") - 1
    options: list[list[list[tuple[int, int]]]] = [[] for _ in lengths]
    q_off = g["q_offsets"]
    for a, c in zip(q_off[:-1], q_off[1:]):
        req = int(opt_req[a])
        options[req].append([(int(g["opt_pos"][o] - starts[req]), int(g["opt_label"][o])) for o in range(a, c)])
    batch = gemma.pack_batch(ids, options)
    np.testing.assert_array_equal(batch.opt_pos.cpu().numpy(), g["opt_pos"])
    check_forward("micro fixture, 2 layers", w, batch)
    logits, probs = gemma.forward(w, batch)
    torch.cuda.synchronize()
    p = probs.cpu().numpy()
    floor = float(np.abs(g["probs_f32"] - g["probs"]).max())
    say(f"micro forward: max |p - fixture truth| = {float(np.abs(p - g['probs']).max()):.2e} "
        f"(fp32 oracle {floor:.2e})")
    for a, c in zip(q_off[:-1], q_off[1:]):
        top = np.sort(g["probs"][a:c])[::-1]
        if c - a > 1 and top[0] - top[1] > 2 * floor:
            assert np.argmax(p[a:c]) == np.argmax(g["probs"][a:c])
    np.testing.assert_allclose(logits.cpu().numpy(), g["logits"], atol=5e-2, rtol=0)
