"""The Clef joint head on the GPU (deciax_amd/clef_head.py + csrc/head.hip).

Truth is the reference's own golden vectors (tests/golden/clef_head.npz =
tests/fixtures/clef_head.npz, Cloudflare's torch head), checked as tests/clef/test_head.py:11-29
checks the reference: the expected logits at atol 3e-6 / rtol 3e-5 and no leakage from padded
positions. Larger random shapes, with ragged spans and odd sizes, are checked against the oracle
(oracle/clef_head.py, itself pinned to the fixture)."""

from __future__ import annotations

import numpy as np
import pytest

from tests.conftest import rng, say
from tests.test_oracle_clef_head import load_fixture

pytestmark = pytest.mark.gpu


def _dev_params(params: dict) -> dict:
    import torch

    return {k: torch.as_tensor(np.ascontiguousarray(v, np.float32)).cuda() for k, v in params.items()}


def test_head_matches_reference_golden_vectors() -> None:
    import torch

    from deciax_amd import clef_head

    say("clef head: reference fixture")
    params, arrays, hidden, embedding, expected = load_fixture()
    p = _dev_params(params)
    lexical = clef_head.lexical_vectors(torch.as_tensor(embedding).cuda(), arrays["lexical_ids"],
                                        arrays["lexical_spans"])
    out = clef_head.forward(p, hidden, lexical, arrays, heads=4, routing_layers=2, layers=2).cpu().numpy()
    for i, e in expected.items():
        np.testing.assert_allclose(out[i, :len(e)], e, atol=3e-6, rtol=3e-5)
        assert (out[i, len(e):] == np.float32(-1e9)).all()
    changed = np.where(arrays["mask"][..., None], hidden, np.float32(10000.0))
    second = clef_head.forward(p, changed, lexical, arrays, heads=4, routing_layers=2, layers=2).cpu().numpy()
    np.testing.assert_allclose(out[:3], second[:3], atol=1e-6)


def _random_case(seed: int, batch: int, seq: int, hidden: int, width: int, ff: int, nq: int, no: int, ntypes: int,
                 routing_layers: int, layers: int):
    r = rng(seed)
    f = lambda *s, scale=0.2: (r.normal(size=s) * scale).astype(np.float32)  # noqa: E731
    p = {"hidden_norm.weight": 1 + f(hidden), "hidden_norm.bias": f(hidden),
         "memory_projection.weight": f(width, hidden), "memory_projection.bias": f(width),
         "option_context_projection.weight": f(width, hidden), "option_lexical_projection.weight": f(width, hidden),
         "option_question_projection.weight": f(width, hidden), "question_projection.weight": f(width, hidden),
         "question_projection.bias": f(width), "option_summary_norm.weight": 1 + f(width),
         "option_summary_norm.bias": f(width), "global_projection.weight": f(width, hidden),
         "type_embedding.weight": f(ntypes, width), "field_norm.weight": 1 + f(width), "field_norm.bias": f(width),
         "option_norm.weight": 1 + f(width), "option_norm.bias": f(width),
         "residual_scorer.0.weight": f(ff, 4 * width), "residual_scorer.0.bias": f(ff),
         "residual_scorer.3.weight": f(1, ff), "residual_scorer.3.bias": f(1),
         "prior_logit_scale": np.float32(2.0), "joint_logit_scale": np.float32(5.0),
         "residual_gate": np.float32(0.3)}

    def attn(n):
        p.update({n + ".in_proj_weight": f(3 * width, width), n + ".in_proj_bias": f(3 * width),
                  n + ".out_proj.weight": f(width, width), n + ".out_proj.bias": f(width)})

    def ln(n):
        p.update({n + ".weight": 1 + f(width), n + ".bias": f(width)})

    for i in range(routing_layers):
        n = f"evidence_layers.{i}"
        attn(n + ".attention")
        for m in ("query_norm", "memory_norm", "feedforward_norm"):
            ln(f"{n}.{m}")
        p.update({n + ".feedforward.0.weight": f(ff, width), n + ".feedforward.0.bias": f(ff),
                  n + ".feedforward.3.weight": f(width, ff), n + ".feedforward.3.bias": f(width)})
    for i in range(layers):
        n = f"layers.{i}"
        attn(n + ".self_attn")
        attn(n + ".multihead_attn")
        for m in ("norm1", "norm2", "norm3"):
            ln(f"{n}.{m}")
        p.update({n + ".linear1.weight": f(ff, width), n + ".linear1.bias": f(ff),
                  n + ".linear2.weight": f(width, ff), n + ".linear2.bias": f(width)})
    lens = r.integers(seq // 2, seq + 1, batch)
    mask = np.arange(seq)[None, :] < lens[:, None]
    a = {"mask": mask, "question_spans": np.zeros((batch, nq, 2), np.int32),
         "option_spans": np.zeros((batch, no, 2), np.int32), "option_field": np.zeros((batch, no), np.int32),
         "option_mask": np.zeros((batch, no), bool), "question_mask": np.zeros((batch, nq), bool),
         "types": r.integers(0, ntypes, (batch, nq)).astype(np.int32)}
    for b in range(batch):
        q_here = int(r.integers(1, nq + 1))
        a["question_mask"][b, :q_here] = True
        for q in range(q_here):
            s0 = int(r.integers(0, lens[b] - 4))
            a["question_spans"][b, q] = (s0, s0 + int(r.integers(1, 4)))
        o_here = int(r.integers(q_here, no + 1))
        a["option_mask"][b, :o_here] = True
        a["option_field"][b, :o_here] = np.sort(r.integers(0, q_here, o_here))
        a["option_field"][b, :q_here] = np.arange(q_here)  # every field owns an option
        for o in range(o_here):
            s0 = int(r.integers(0, lens[b] - 4))
            a["option_spans"][b, o] = (s0, s0 + int(r.integers(0, 4)))  # empty spans included
    hidden_x = f(batch, seq, hidden, scale=1.0)
    lexical = f(batch, no, hidden, scale=1.0)
    return p, a, hidden_x, lexical


@pytest.mark.parametrize("shape", [
    dict(batch=2, seq=300, hidden=64, width=32, ff=48, nq=5, no=17, ntypes=3, routing_layers=2, layers=2),
    dict(batch=3, seq=131, hidden=96, width=48, ff=80, nq=7, no=70, ntypes=4, routing_layers=1, layers=3),
])
def test_head_matches_oracle_random_shapes(shape: dict) -> None:
    from deciax_amd import clef_head
    from oracle import clef_head as oc

    say(f"clef head random {shape}")
    heads = 4
    p, a, hidden, lexical = _random_case(7 + shape["batch"], **shape)
    want = oc.forward(p, hidden, lexical, a, heads=heads, routing_layers=shape["routing_layers"],
                      layers=shape["layers"])
    got = clef_head.forward(_dev_params(p), hidden, lexical, a, heads=heads, routing_layers=shape["routing_layers"],
                            layers=shape["layers"]).cpu().numpy()
    live = a["option_mask"]
    np.testing.assert_allclose(got[live], want[live], atol=2e-5, rtol=2e-4)
    assert (got[~live] == np.float32(-1e9)).all()


def test_encoded_requests_through_head() -> None:
    """Requests encoded by deciax_amd.schema, laid out by `head_inputs` (the reference's collate,
    src/deciax/models/clef/input.py:140-182), with lexical vectors gathered on the GPU: the head's
    logits match the oracle fed the same arrays, and decode to the same answers."""
    import torch

    from deciax_amd import clef_head
    from deciax_amd.schema import ByteTokenizer, decode, encode, head_inputs
    from oracle import clef_head as oc

    say("clef head: encoded requests")
    tok = ByteTokenizer()
    questions = {"mood": {"type": "choice", "criteria": {"pos": "positive", "neg": "negative", "mix": None}},
                 "late": {"type": "noul"}, "stars": {"type": "score", "criteria": ["bad", "ok", "good"]}}
    records = [encode(tok, s, questions, 2048) for s in ("the parcel came late", {"ticket": 7, "text": "great"})]
    a = head_inputs(records, tok.pad_token_id)
    r = rng(11)
    batch, seq = a["input_ids"].shape
    hidden_dim = 64
    p, _, _, _ = _random_case(5, batch=batch, seq=seq, hidden=hidden_dim, width=32, ff=48, nq=3, no=8, ntypes=3,
                              routing_layers=1, layers=2)
    hidden = r.normal(size=(batch, seq, hidden_dim)).astype(np.float32)
    embedding = r.normal(size=(tok.vocab, hidden_dim)).astype(np.float32)
    lexical = clef_head.lexical_vectors(torch.as_tensor(embedding).cuda(), a["lexical_ids"], a["lexical_spans"])
    want_lex = oc.means(embedding[a["lexical_ids"]], a["lexical_spans"])
    np.testing.assert_allclose(lexical.cpu().numpy(), want_lex, atol=1e-5, rtol=1e-5)
    got = clef_head.forward(_dev_params(p), hidden, lexical, a, heads=4, routing_layers=1, layers=2).cpu().numpy()
    want = oc.forward(p, hidden, want_lex, a, heads=4, routing_layers=1, layers=2)
    live = a["option_mask"]
    np.testing.assert_allclose(got[live], want[live], atol=2e-5, rtol=2e-4)
    for i, record in enumerate(records):
        n = int(live[i].sum())
        ours, theirs = decode(record, got[i, :n], questions, "m"), decode(record, want[i, :n], questions, "m")
        assert ours["answers"]["mood"]["choice"] == theirs["answers"]["mood"]["choice"]
        assert ours["answers"]["late"]["noul"] == pytest.approx(theirs["answers"]["late"]["noul"], abs=2e-4)
        assert ours["answers"]["stars"]["score"] == pytest.approx(theirs["answers"]["stars"]["score"], abs=2e-4)
