"""Pins the oracle's layer pieces and decision forward (oracle/model.py, oracle/numerics.py) on the CPU.

Independent implementations checked against, each at fp32 (the oracle's `bf16=False` mode):
  * transformers' Gemma-2 modules on torch CPU — Gemma2RMSNorm, Gemma2MLP, the rotary
    embedding and the whole Gemma2ForCausalLM (random init from a local tiny config,
    eager attention; TF/models/gemma2/modeling_gemma2.py), whose logits at the option
    positions and label ids must equal the oracle's readout before the softmax;
  * closed forms: RMSNorm of a constant row, RoPE invariants of the reference's
    tests/test_nn.py:25-31 (position 0 unchanged, norm preserved), the full-vocabulary
    brute force of the readout, torch's own bf16 cast and tanh-GELU;
  * the reference's decode KATs (tests/clef/test_input.py:42-44, 78-83).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import model as om
from oracle.numerics import bf16, bf16_bits, from_bits, gelu_tanh, silu, softcap, softmax
from tests.conftest import rng

torch = pytest.importorskip("torch")


def test_bf16_rounding_matches_torch_cast() -> None:
    r = rng(0)
    x = np.concatenate([r.normal(size=4096).astype(np.float32) * 10 ** r.uniform(-30, 30, 4096).astype(np.float32),
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.0e38, -3.0e38, 1e-40], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf16_bits(x), want)
    np.testing.assert_array_equal(from_bits(want), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_activations_match_torch() -> None:
    x = np.linspace(-12, 12, 20001, dtype=np.float32)
    t = torch.from_numpy(x)
    np.testing.assert_allclose(gelu_tanh(x), torch.nn.functional.gelu(t, approximate="tanh").numpy(), rtol=1e-6,
                               atol=1e-6)
    np.testing.assert_allclose(silu(x), torch.nn.functional.silu(t).numpy(), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(softcap(x * 10, 30.0), (30 * torch.tanh(t * 10 / 30)).numpy(), rtol=1e-6, atol=1e-5)
    assert np.array_equal(softcap(x, 0.0), x)


def test_rmsnorm_closed_form_and_transformers() -> None:
    from transformers.models.gemma2.modeling_gemma2 import Gemma2RMSNorm

    w = rng(1).normal(size=64).astype(np.float32) * 0.1
    const = np.full((1, 64), 3.0, np.float32)  # rms = 3 -> x / rms = 1 -> output = 1 + w
    np.testing.assert_allclose(om.rmsnorm(const, w, 0.0, bf16=False)[0], 1 + w, rtol=1e-6)
    x = rng(2).normal(size=(17, 64)).astype(np.float32) * 4
    mod = Gemma2RMSNorm(64, eps=1e-6)
    with torch.no_grad():
        mod.weight.copy_(torch.from_numpy(w))
        want = mod(torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(om.rmsnorm(x, w, 1e-6, bf16=False), want, rtol=1e-5, atol=1e-6)


def test_gated_mlp_matches_transformers() -> None:
    from transformers import Gemma2Config
    from transformers.models.gemma2.modeling_gemma2 import Gemma2MLP

    cfg = Gemma2Config(hidden_size=64, intermediate_size=96, hidden_activation="gelu_pytorch_tanh")
    mod = Gemma2MLP(cfg)
    r = rng(3)
    gate, up = (r.normal(size=(96, 64)).astype(np.float32) * 0.2 for _ in range(2))
    down = r.normal(size=(64, 96)).astype(np.float32) * 0.2
    with torch.no_grad():
        mod.gate_proj.weight.copy_(torch.from_numpy(gate))
        mod.up_proj.weight.copy_(torch.from_numpy(up))
        mod.down_proj.weight.copy_(torch.from_numpy(down))
        x = r.normal(size=(9, 64)).astype(np.float32)
        want = mod(torch.from_numpy(x)).numpy()
    got = om.linear(om.gated(x, gate, up, "gelu_tanh", bf16=False), down, bf16=False)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    # with a unit norm weight of zero, mlp() is rms-normalise then the same chain
    xn = om.rmsnorm(x, np.zeros(64, np.float32), 1e-6, bf16=False)
    np.testing.assert_allclose(om.mlp(x, np.zeros(64, np.float32), gate, up, down, eps=1e-6, bf16=False),
                               om.linear(om.gated(xn, gate, up, bf16=False), down, bf16=False), rtol=1e-6, atol=1e-6)


def test_rope_invariants_and_transformers_rotary() -> None:
    from transformers import Gemma2Config
    from transformers.models.gemma2.modeling_gemma2 import Gemma2RotaryEmbedding, apply_rotary_pos_emb

    d, n = 32, 50
    cos, sin = om.rope_tables(n, d, 10000.0, bf16=False)
    x = rng(4).normal(size=(n, 3, d)).astype(np.float32)
    pos = np.arange(n)
    y = om.rope(x, pos, cos, sin, bf16=False)
    np.testing.assert_allclose(y[0], x[0], rtol=1e-6)  # tests/test_nn.py:29
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)  # :30
    cfg = Gemma2Config(head_dim=d, hidden_size=64, num_attention_heads=2, rope_theta=10000.0)
    rot = Gemma2RotaryEmbedding(cfg)
    tx = torch.from_numpy(x).permute(1, 0, 2)[None]
    tc, ts = rot(tx, torch.from_numpy(pos)[None])
    want, _ = apply_rotary_pos_emb(tx, tx, tc, ts)
    np.testing.assert_allclose(y, want[0].permute(1, 0, 2).numpy(), rtol=1e-5, atol=1e-5)
    # relative-position property: <rope(q, i), rope(k, j)> depends only on i - j
    q1, k1 = x[:1, :1], x[1:2, :1]
    a = om.rope(np.repeat(q1, n, 0), pos, cos, sin, bf16=False)
    b = om.rope(np.repeat(k1, n, 0), pos, cos, sin, bf16=False)
    dots = [float(np.dot(a[i + 3, 0], b[i, 0])) for i in range(n - 3)]
    np.testing.assert_allclose(dots, dots[0], rtol=1e-4, atol=1e-4)


TINY = om.Shape(hidden=64, heads=4, kv_heads=2, head_dim=32, intermediate=128, vocab=300, layers=4, window=8,
                query_scale=24.0 ** -0.5)


def tiny_weights(seed: int = 0) -> dict[str, np.ndarray]:
    r = rng(seed)
    s = TINY

    def m(*shape, std=0.08):
        return (r.normal(size=shape) * std).astype(np.float32)

    w = {"embed": m(s.vocab, s.hidden, std=0.5), "final_norm": m(s.hidden, std=0.2)}
    for i in range(s.layers):
        p = f"layers.{i}."
        w.update({p + "input_norm": m(s.hidden, std=0.2), p + "q": m(s.heads * s.head_dim, s.hidden),
                  p + "k": m(s.kv_heads * s.head_dim, s.hidden), p + "v": m(s.kv_heads * s.head_dim, s.hidden),
                  p + "o": m(s.hidden, s.heads * s.head_dim), p + "post_attn_norm": m(s.hidden, std=0.2),
                  p + "pre_ffn_norm": m(s.hidden, std=0.2), p + "gate": m(s.intermediate, s.hidden),
                  p + "up": m(s.intermediate, s.hidden), p + "down": m(s.hidden, s.intermediate),
                  p + "post_ffn_norm": m(s.hidden, std=0.2)})
    return w


def transformers_model(w: dict[str, np.ndarray]):
    from transformers import Gemma2Config, Gemma2ForCausalLM

    s = TINY
    cfg = Gemma2Config(vocab_size=s.vocab, hidden_size=s.hidden, intermediate_size=s.intermediate,
                       num_hidden_layers=s.layers, num_attention_heads=s.heads, num_key_value_heads=s.kv_heads,
                       head_dim=s.head_dim, query_pre_attn_scalar=24, sliding_window=s.window,
                       attn_logit_softcapping=s.attn_softcap, final_logit_softcapping=s.final_softcap,
                       rms_norm_eps=s.eps, rope_theta=s.rope_theta, hidden_activation="gelu_pytorch_tanh",
                       max_position_embeddings=256, attn_implementation="eager", tie_word_embeddings=True,
                       pad_token_id=0)
    model = Gemma2ForCausalLM(cfg).eval()
    names = {"input_norm": "input_layernorm", "post_attn_norm": "post_attention_layernorm",
             "pre_ffn_norm": "pre_feedforward_layernorm", "post_ffn_norm": "post_feedforward_layernorm",
             "q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
             "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
    sd = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["final_norm"]}
    for i in range(s.layers):
        for ours, theirs in names.items():
            sd[f"model.layers.{i}.{theirs}.weight"] = w[f"layers.{i}.{ours}"]
    with torch.no_grad():
        params = dict(model.named_parameters())
        for k, v in sd.items():
            params[k].copy_(torch.from_numpy(v))
    return model


def test_decision_forward_matches_transformers_gemma2() -> None:
    """The whole fp32 oracle path — sqrt(H)-scaled embedding, sandwich layers with sliding (even)
    and global (odd) causal attention and softcap 50, GELU-tanh MLP, final norm, tied head,
    final softcap 30 — against Gemma2ForCausalLM; two packed sequences, so rows of the second
    restart at position 0 and never see the first."""
    w = tiny_weights()
    model = transformers_model(w)
    r = rng(7)
    lengths = [37, 20]
    seqs = [r.integers(0, TINY.vocab, n) for n in lengths]
    ids = np.concatenate(seqs)
    pos = np.concatenate([np.arange(n) for n in lengths])
    x = om.forward(w, TINY, ids, [0, lengths[0]], lengths, pos, bf16=False)
    ours = om.lm_logits(x, w["final_norm"], w["embed"], eps=TINY.eps, cap=TINY.final_softcap)
    start = 0
    for seq in seqs:
        with torch.no_grad():
            want = model(torch.from_numpy(seq)[None]).logits[0].numpy()
        np.testing.assert_allclose(ours[start:start + len(seq)], want, rtol=2e-4, atol=2e-4)
        start += len(seq)

    # the readout is the LM logit of each option's label at its position, softmaxed per question
    opt_pos = [36, 30, 12, 40, 56, 50]
    opt_label = [5, 17, 200, 3, 299, 0]
    q_off = [0, 3, 6]
    z, p = om.readout(x, w["final_norm"], w["embed"], opt_pos, opt_label, q_off, eps=TINY.eps,
                      cap=TINY.final_softcap, bf16=False)
    np.testing.assert_allclose(z, ours[opt_pos, opt_label], rtol=1e-5, atol=1e-5)
    for a, b in zip(q_off[:-1], q_off[1:]):
        e = np.exp(z[a:b].astype(np.float64) - z[a:b].max())
        np.testing.assert_allclose(p[a:b], e / e.sum(), rtol=1e-6)


def test_bf16_forward_tracks_fp32_forward() -> None:
    """The bf16 rounding points perturb the tiny forward by bf16 noise only (a misplaced rounding
    that truncates, or a wrong dtype round trip, shows up as a large deviation)."""
    w = {k: bf16(v) for k, v in tiny_weights(1).items()}
    ids = rng(8).integers(0, TINY.vocab, 45)
    pos = np.arange(45)
    a = om.forward(w, TINY, ids, [0], [45], pos, bf16=False)
    b = om.forward(w, TINY, ids, [0], [45], pos, bf16=True)
    assert np.array_equal(b, bf16(b)), "bf16 mode must return bf16 values"
    rel = np.abs(a - b).max() / np.abs(a).max()
    assert 0 < rel < 0.05, rel


def test_decode_kats() -> None:
    """Zero logits -> uniform per field (noul 0.5; score over 3 levels -> 1.0), as
    tests/clef/test_input.py:42-44; NaN -> FloatingPointError (:78-83)."""
    probs = om.decode_probs(np.zeros(5, np.float32), [2, 3])
    np.testing.assert_allclose(probs[0], [0.5, 0.5])
    assert sum(i * p for i, p in enumerate(probs[1])) == pytest.approx(1.0)
    with pytest.raises(FloatingPointError, match="non-finite"):
        om.decode_probs(np.array([np.nan, 0.0], np.float32), [2])
    np.testing.assert_allclose(softmax(np.array([1000.0, 1000.0], np.float32)), [0.5, 0.5])


@pytest.mark.parametrize("k", [1, 64, 100, 3584])
def test_summation_orders_agree_with_the_exact_product(k: int) -> None:
    """Every summation order of the oracle's matmul is the same product up to fp32 rounding (a dropped
    or repeated K tile would be off by a whole tile's share), and in fp64 the orders coincide."""
    from oracle.numerics import ORDERS, accumulation, matmul

    r = np.random.Generator(np.random.PCG64(k))
    a = r.normal(size=(7, k)).astype(np.float32)
    b = r.normal(size=(k, 5)).astype(np.float32)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    tol = 1e-6 * np.sqrt(k) * np.abs(a).max() * np.abs(b).max() * 8
    got = {}
    for order in ORDERS:
        with accumulation(np.float32, order):
            got[order] = matmul(a, b)
        np.testing.assert_allclose(got[order], exact, rtol=0, atol=tol)
        with accumulation(np.float64, order):  # summed in fp64, returned rounded once to fp32 (one ulp)
            np.testing.assert_allclose(matmul(a, b), exact, rtol=2.0 ** -23, atol=1e-12)
    if k > 64:  # the orders differ at the fp32 level, or they would not measure anything
        assert any(not np.array_equal(got["blas"], got[o]) for o in ORDERS[1:])
    if k > 128:  # with three tiles or more the walk direction changes the rounding too
        assert not np.array_equal(got["k_tiles"], got["k_tiles_reversed"])
