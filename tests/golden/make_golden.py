"""Writes the golden fixtures of tests/golden/ with the oracle (run: python tests/golden/make_golden.py).

Fixtures (each well under 1 MB):
  attention_packed.npz — three packed sequences (45, 7, 70 rows), GQA 4/2, head_dim 64, causal
      window 16, softcap 50, scale 1/8: bf16 inputs (as uint16 bit patterns) and the oracle's output
      at the bf16 rounding points and in fp32.
  forward_micro.npz — a 2-layer Gemma-2-shaped micro model (H 256, 2/1 heads x 128, MLP 512,
      vocab 300, window 32), its weights regenerated from `seed` by `micro_weights`; two requests of
      40 and 25 tokens with 3 questions; the option logits and per-question probabilities of the
      oracle with exactly summed contractions (truth) and with fp32 sums.
The reference ships no fixture for this path, so these are the oracle's own vectors: they guard
regressions of the oracle (tests/test_golden.py) and give the GPU path fixed targets
(tests/test_gpu_golden.py).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import model as om  # noqa: E402
from oracle.attention import attention_packed  # noqa: E402
from oracle.numerics import accumulation, bf16, bf16_bits  # noqa: E402

MICRO = om.Shape(hidden=256, heads=2, kv_heads=1, head_dim=128, intermediate=512, vocab=300, layers=2, window=32,
                 query_scale=128.0 ** -0.5)
MICRO_SEED = 7
ATTN = dict(lengths=[45, 7, 70], hq=4, hkv=2, d=64, window=16, softcap=50.0, scale=0.125, seed=3)


def micro_weights(seed: int = MICRO_SEED) -> dict[str, np.ndarray]:
    """bf16-valued fp32 weights of the micro model: matrices ~ N(0, 0.05), norm weights ~ N(0, 0.3)."""
    r = np.random.Generator(np.random.PCG64(seed))
    s = MICRO

    def m(*shape: int, std: float = 0.05) -> np.ndarray:
        return bf16(r.normal(size=shape).astype(np.float32) * np.float32(std))

    w = {"embed": m(s.vocab, s.hidden, std=0.5), "final_norm": m(s.hidden, std=0.3)}
    for i in range(s.layers):
        p = f"layers.{i}."
        w.update({p + "input_norm": m(s.hidden, std=0.3), p + "q": m(s.heads * s.head_dim, s.hidden),
                  p + "k": m(s.kv_heads * s.head_dim, s.hidden), p + "v": m(s.kv_heads * s.head_dim, s.hidden),
                  p + "o": m(s.hidden, s.heads * s.head_dim), p + "post_attn_norm": m(s.hidden, std=0.3),
                  p + "pre_ffn_norm": m(s.hidden, std=0.3), p + "gate": m(s.intermediate, s.hidden),
                  p + "up": m(s.intermediate, s.hidden), p + "down": m(s.hidden, s.intermediate),
                  p + "post_ffn_norm": m(s.hidden, std=0.3)})
    return w


def micro_batch() -> dict[str, np.ndarray]:
    """Packed ids, positions and the option layout of the forward fixture."""
    r = np.random.Generator(np.random.PCG64(MICRO_SEED + 1))
    lengths = [40, 25]
    ids = np.concatenate([r.integers(0, MICRO.vocab, n) for n in lengths]).astype(np.int32)
    starts = [0, lengths[0]]
    positions = np.concatenate([np.arange(n) for n in lengths]).astype(np.int32)
    # (request, position in request, label) per option; questions own consecutive options
    questions = [[(0, 39, 5), (0, 38, 17), (0, 30, 250)], [(0, 12, 3), (0, 36, 299)],
                 [(1, 24, 0), (1, 20, 77), (1, 5, 140), (1, 0, 8)]]
    opt_pos, opt_label, q_off = [], [], [0]
    for q in questions:
        for req, pos, label in q:
            opt_pos.append(starts[req] + pos)
            opt_label.append(label)
        q_off.append(len(opt_pos))
    return {"ids": ids, "lengths": np.array(lengths, np.int32), "seq_start": np.array(starts, np.int32),
            "positions": positions, "opt_pos": np.array(opt_pos, np.int32),
            "opt_label": np.array(opt_label, np.int32), "q_offsets": np.array(q_off, np.int32)}


def micro_reference(acc: type) -> tuple[np.ndarray, np.ndarray]:
    w = micro_weights()
    b = micro_batch()
    with accumulation(acc):
        x = om.forward(w, MICRO, b["ids"], b["seq_start"].tolist(), b["lengths"].tolist(), b["positions"])
        return om.readout(x, w["final_norm"], w["embed"], b["opt_pos"], b["opt_label"], b["q_offsets"].tolist(),
                          eps=MICRO.eps, cap=MICRO.final_softcap)


def attention_case() -> dict[str, np.ndarray]:
    a = ATTN
    r = np.random.Generator(np.random.PCG64(a["seed"]))
    rows = sum(a["lengths"])
    q = bf16(r.normal(size=(rows, a["hq"], a["d"])).astype(np.float32) * 2)
    k = bf16(r.normal(size=(rows, a["hkv"], a["d"])).astype(np.float32) * 2)
    v = bf16(r.normal(size=(rows, a["hkv"], a["d"])).astype(np.float32))
    starts = np.concatenate([[0], np.cumsum(a["lengths"])[:-1]]).astype(np.int32)
    kw = dict(scale=a["scale"], softcap_value=a["softcap"], window=a["window"], causal=True)
    out_bf16 = attention_packed(q, k, v, starts, a["lengths"], bf16=True, **kw)
    out_f32 = attention_packed(q, k, v, starts, a["lengths"], bf16=False, **kw)
    return {"q_bits": bf16_bits(q), "k_bits": bf16_bits(k), "v_bits": bf16_bits(v), "seq_start": starts,
            "seq_len": np.array(a["lengths"], np.int32), "out_bf16": out_bf16, "out_f32": out_f32}


def main() -> None:
    np.savez_compressed(HERE / "attention_packed.npz", **attention_case())
    truth_z, truth_p = micro_reference(np.float64)
    f32_z, f32_p = micro_reference(np.float32)
    np.savez_compressed(HERE / "forward_micro.npz", seed=np.int64(MICRO_SEED), logits=truth_z, probs=truth_p,
                        logits_f32=f32_z, probs_f32=f32_p, **micro_batch())
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
