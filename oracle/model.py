"""Gemma-2-shaped decision forward and option readout in numpy (test infrastructure only).

Layer skeleton: the reference's layer (src/deciax/models/qwen3_5/text.py:94-102)
with its fp32 RMSNorm (text.py:25-28), fp32-accumulating projections rounded
to bf16 (`dense`, text.py:21-22; `linear`, src/deciax/nn.py:11-19) and the
gated-MLP rounding points of src/deciax/kernels/swiglu.py:100-101; laid out as
the Gemma-2 sandwich layer of TF/models/gemma2/modeling_gemma2.py:291-335
(input norm -> attention -> post-attention norm -> residual; pre-FFN norm ->
MLP -> post-FFN norm -> residual), with the sqrt(H) embedding scale rounded to
bf16 (:338-349) and the tied embedding as the output head.

Driver order: src/deciax/models/clef/model.py:92-102 (embed, layers, final
norm, head). Readout: gather at the option positions as in
src/deciax/models/laya/heads.py:74-78, score each option with the tied
embedding row of its label token (the LM logit of that token), soft-cap 30
(TF/models/gemma2/modeling_gemma2.py:527-530), then a softmax per question
(src/deciax/models/clef/input.py:185-194, src/deciax/protocol/answers.py:44-46).
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from dataclasses import dataclass

import numpy as np

from oracle.attention import attention_seq
from oracle.numerics import ACTIVATIONS, F32, matmul, maybe, softcap, softmax


@dataclass(frozen=True)
class Shape:
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    layers: int
    window: int = 4096
    attn_softcap: float = 50.0
    final_softcap: float = 30.0
    query_scale: float = 256.0 ** -0.5
    eps: float = 1e-6
    rope_theta: float = 10000.0
    activation: str = "gelu_tanh"

    def sliding(self, layer: int) -> bool:
        """Even layers use the sliding window (TF/models/gemma2/configuration_gemma2.py:95-97)."""
        return layer % 2 == 0


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, bf16: bool = True) -> np.ndarray:
    """x * rsqrt(mean(x^2) + eps) * (1 + w) in fp32 — src/deciax/models/qwen3_5/text.py:25-28."""
    x = np.asarray(x, F32)
    inv = (F32(1.0) / np.sqrt(np.mean(x * x, axis=-1, keepdims=True, dtype=F32) + F32(eps))).astype(F32)
    return maybe((x * inv) * (F32(1.0) + np.asarray(w, F32)), bf16)


def linear(x: np.ndarray, w: np.ndarray, bf16: bool = True) -> np.ndarray:
    """x @ w.T, fp32 accumulation, one rounding — src/deciax/nn.py:11-19 + text.py:21-22."""
    return maybe(matmul(x, np.asarray(w, F32).T), bf16)


def gated(x: np.ndarray, gate: np.ndarray, up: np.ndarray, activation: str = "gelu_tanh",
          bf16: bool = True) -> np.ndarray:
    """act(bf16(x gate^T)) -> bf16, times bf16(x up^T) -> bf16: src/deciax/kernels/swiglu.py:99-101."""
    g = linear(x, gate, bf16)
    u = linear(x, up, bf16)
    return maybe(maybe(ACTIVATIONS[activation](g), bf16) * u, bf16)


def mlp(x: np.ndarray, norm_w: np.ndarray, gate: np.ndarray, up: np.ndarray, down: np.ndarray, *, eps: float,
        activation: str = "gelu_tanh", bf16: bool = True, round_out: bool = False) -> np.ndarray:
    """RMSNorm -> gated -> down, fp32 accumulation over all of f
    (`fused_mlp_partial`, src/deciax/kernels/swiglu.py:166-208; fp32 out unless round_out)."""
    a = gated(rmsnorm(x, norm_w, eps, bf16), gate, up, activation, bf16)
    return maybe(matmul(a, np.asarray(down, F32).T), round_out and bf16)


def rope_tables(max_pos: int, head_dim: int, theta: float, bf16: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin [max_pos, D/2] of positions * inv_freq, inv_freq = 1 / theta^(2i/D) in fp32
    (src/deciax/nn.py:31-44; TF Gemma-2 default rotary), rounded to the activation dtype."""
    inv = (F32(1.0) / (F32(theta) ** (np.arange(0, head_dim, 2, dtype=F32) / F32(head_dim)))).astype(F32)
    freqs = (np.arange(max_pos, dtype=F32)[:, None] * inv[None, :]).astype(F32)
    return maybe(np.cos(freqs), bf16), maybe(np.sin(freqs), bf16)


def rope(x: np.ndarray, positions: np.ndarray, cos: np.ndarray, sin: np.ndarray, bf16: bool = True) -> np.ndarray:
    """Rotate-half RoPE on [L, H, D]: x cos + rotate_half(x) sin, each product and the sum rounded
    in bf16 mode (src/deciax/nn.py:39-44)."""
    x = np.asarray(x, F32)
    half = x.shape[-1] // 2
    c = cos[positions][:, None, :]
    s = sin[positions][:, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    o1 = maybe(maybe(x1 * c, bf16) - maybe(x2 * s, bf16), bf16)
    o2 = maybe(maybe(x2 * c, bf16) + maybe(x1 * s, bf16), bf16)
    return np.concatenate([o1, o2], axis=-1)


def embed_scale(hidden: int, bf16: bool = True) -> float:
    """sqrt(H) in the activation dtype (TF/models/gemma2/modeling_gemma2.py:338-349)."""
    return float(maybe(np.array([np.sqrt(F32(hidden))], F32), bf16)[0])


def layer(x: np.ndarray, p: Mapping[str, np.ndarray], shape: Shape, index: int, seq_start: Sequence[int],
          seq_len: Sequence[int], positions: np.ndarray, cos: np.ndarray, sin: np.ndarray,
          bf16: bool = True, rounding: str = "flash") -> np.ndarray:
    """One sandwich layer over packed rows x [R, H]; `rounding` is attention_seq's bf16 rounding
    point of the attention weights."""
    s = shape
    h = rmsnorm(x, p["input_norm"], s.eps, bf16)
    rows = x.shape[0]
    q = linear(h, p["q"], bf16).reshape(rows, s.heads, s.head_dim)
    k = linear(h, p["k"], bf16).reshape(rows, s.kv_heads, s.head_dim)
    v = linear(h, p["v"], bf16).reshape(rows, s.kv_heads, s.head_dim)
    q = rope(q, positions, cos, sin, bf16)
    k = rope(k, positions, cos, sin, bf16)
    att = np.zeros((rows, s.heads, s.head_dim), F32)
    window = s.window if s.sliding(index) else 0
    for start, length in zip(seq_start, seq_len):
        sl = slice(start, start + length)
        att[sl] = attention_seq(q[sl], k[sl], v[sl], scale=s.query_scale, softcap_value=s.attn_softcap,
                                window=window, causal=True, bf16=bf16, rounding=rounding)
    y = linear(att.reshape(rows, -1), p["o"], bf16)
    x = maybe(x + rmsnorm(y, p["post_attn_norm"], s.eps, bf16), bf16)
    h = rmsnorm(x, p["pre_ffn_norm"], s.eps, bf16)
    y = linear(gated(h, p["gate"], p["up"], s.activation, bf16), p["down"], bf16)
    return maybe(x + rmsnorm(y, p["post_ffn_norm"], s.eps, bf16), bf16)


def layer_params(weights: Mapping[str, np.ndarray], i: int) -> dict[str, np.ndarray]:
    prefix = f"layers.{i}."
    return {k[len(prefix):]: v for k, v in weights.items() if k.startswith(prefix)}


def forward(weights: Mapping[str, np.ndarray], shape: Shape, ids: np.ndarray, seq_start: Sequence[int],
            seq_len: Sequence[int], positions: np.ndarray, *, bf16: bool = True,
            layers: int | None = None) -> np.ndarray:
    """Packed token ids [R] -> final hidden states [R, H] before the final norm."""
    s = shape
    cos, sin = rope_tables(int(positions.max()) + 1 if len(positions) else 1, s.head_dim, s.rope_theta, bf16)
    x = maybe(np.asarray(weights["embed"], F32)[ids] * F32(embed_scale(s.hidden, bf16)), bf16)
    for i in range(s.layers if layers is None else layers):
        x = layer(x, layer_params(weights, i), s, i, seq_start, seq_len, positions, cos, sin, bf16)
    return x


def readout(x: np.ndarray, final_norm: np.ndarray, table: np.ndarray, opt_pos: Sequence[int],
            opt_label: Sequence[int], q_offsets: Sequence[int], *, eps: float, cap: float,
            bf16: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """Option logits z_o = softcap(<rms(x[p_o]), E[t_o]>) and per-question softmax probabilities."""
    g = rmsnorm(np.asarray(x, F32)[np.asarray(opt_pos)], final_norm, eps, bf16)
    e = np.asarray(table, F32)[np.asarray(opt_label)]
    z = softcap(np.einsum("od,od->o", g.astype(np.float64), e.astype(np.float64)).astype(F32), cap)
    probs = np.zeros_like(z)
    for a, b in zip(q_offsets[:-1], q_offsets[1:]):
        if b > a:
            probs[a:b] = softmax(z[a:b])
    return z, probs


def lm_logits(x: np.ndarray, final_norm: np.ndarray, table: np.ndarray, *, eps: float, cap: float,
              bf16: bool = False) -> np.ndarray:
    """Full-vocabulary logits softcap(rms(x) E^T): the brute-force form of `readout`."""
    g = rmsnorm(x, final_norm, eps, bf16)
    return softcap(np.asarray(g, F32) @ np.asarray(table, F32).T, cap)


def decode_probs(logits: np.ndarray, counts: Sequence[int]) -> list[np.ndarray]:
    """Per-field softmax of consecutive option logits, as `decode` does
    (src/deciax/models/clef/input.py:185-194), raising on non-finite values (:190-191)."""
    out, offset = [], 0
    for n in counts:
        values = np.asarray(logits[offset:offset + n], F32)
        if not np.isfinite(values).all():
            raise FloatingPointError("non-finite option logits")
        out.append(softmax(values))
        offset += n
    return out
