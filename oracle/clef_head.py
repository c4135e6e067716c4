"""CPU restatement of the Clef joint schema head (test infrastructure only).

Follows src/deciax/models/clef/head.py:1-111 step by step, in fp32 numpy (the reference's
fixture is fp32, tests/fixtures/clef_head.json). Only `tests/` may import this module; the
product path is `deciax_amd.clef_head` on the GPU.

Helpers restate src/deciax/nn.py:11-29 (`linear`, `layer_norm`),
src/deciax/models/qwen3_5/text.py:21-22 (`dense`) and the masked attention of
src/deciax/kernels/attention/blocked.py:9-32 (key mask, MASK_FILL = -1e30, fp32 softmax).

Pinned by the reference's own golden vectors: tests/golden/clef_head.npz is the reference's
tests/fixtures/clef_head.npz (Cloudflare's torch head, seed 131) and
tests/test_oracle_clef_head.py checks this module against it at the reference's tolerance
(tests/clef/test_head.py:11-29).
"""

from __future__ import annotations

import math
from collections.abc import Mapping

import numpy as np
from scipy.special import erf

F32 = np.float32
MASK_FILL = F32(-1e30)
MAX_LOGIT_SCALE = math.log(100.0)  # head.py:17


def layer_norm(x: np.ndarray, w: np.ndarray, b: np.ndarray | None, eps: float) -> np.ndarray:
    """nn.py:22-29: centre, scale by rsqrt(mean(z^2) + eps), then weight and bias."""
    x = x.astype(F32)
    z = x - x.mean(-1, keepdims=True, dtype=F32)
    z = z * (F32(1) / np.sqrt((z * z).mean(-1, keepdims=True, dtype=F32) + F32(eps)))
    z = z * w
    return z if b is None else z + b


def norm(x: np.ndarray, p: Mapping[str, np.ndarray], name: str) -> np.ndarray:
    """head.py:20-21 (eps 1e-5)."""
    return layer_norm(x, p[name + ".weight"], p[name + ".bias"], 1e-5).astype(F32)


def dense(x: np.ndarray, p: Mapping[str, np.ndarray], name: str) -> np.ndarray:
    """text.py:21-22 with nn.py:11-19: x @ W^T (+ b), fp32."""
    y = np.matmul(x.astype(F32), p[name + ".weight"].astype(F32).T)
    b = p.get(name + ".bias")
    return (y if b is None else y + b).astype(F32)


def linear(x: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
    return (np.matmul(x.astype(F32), w.T) + b).astype(F32)


def means(x: np.ndarray, spans: np.ndarray) -> np.ndarray:
    """head.py:24-29: mean of x[b, start:end] per span (fp32 sum; an empty span gives 0)."""
    s = x.shape[1]
    pos = np.arange(s)
    mask = (pos >= spans[..., :1]) & (pos < spans[..., 1:])            # [B, O, S]
    total = np.einsum("bos,bsd->bod", mask.astype(F32), x.astype(F32))
    return (total / np.maximum(mask.sum(-1, keepdims=True), 1)).astype(F32)


def gather(x: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """head.py:32-33: x[b, idx[b, i]]."""
    return np.stack([x[b][idx[b]] for b in range(x.shape[0])])


def normalize(x: np.ndarray, eps: float = 1e-12) -> np.ndarray:
    """head.py:36-38."""
    length = np.sqrt(np.sum(x.astype(F32) ** 2, -1, keepdims=True, dtype=F32)).astype(F32)
    return (x / np.maximum(length, F32(eps))).astype(F32)


def gelu(x: np.ndarray) -> np.ndarray:
    """jax.nn.gelu(approximate=False): 0.5 x (1 + erf(x / sqrt 2))."""
    return (0.5 * x * (1.0 + erf(x.astype(np.float64) / math.sqrt(2.0)))).astype(F32)


def sigmoid(x: np.ndarray) -> np.ndarray:
    return (1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))).astype(F32)


def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    m = x.max(axis, keepdims=True)
    e = np.exp((x - m).astype(F32))
    return (e / e.sum(axis, keepdims=True)).astype(F32)


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, key_mask: np.ndarray) -> np.ndarray:
    """blocked.py:9-32 without causality: [B, Q, H, D] x [B, K, H, D] with key mask [B, K]."""
    d = q.shape[-1]
    scores = np.einsum("bqhd,bkhd->bhqk", q.astype(F32), k.astype(F32)) * F32(d ** -0.5)
    scores = np.where(key_mask[:, None, None, :], scores, MASK_FILL)
    w = softmax(scores, -1)
    return np.einsum("bhqk,bkhd->bqhd", w, v.astype(F32)).astype(F32)


def mha(query: np.ndarray, memory: np.ndarray, mask: np.ndarray, p: Mapping[str, np.ndarray], name: str,
        heads: int) -> np.ndarray:
    """head.py:41-51: packed in_proj split in three, per-head attention, out_proj."""
    wq, wk, wv = np.split(p[name + ".in_proj_weight"], 3)
    bq, bk, bv = np.split(p[name + ".in_proj_bias"], 3)
    hs = (heads, query.shape[-1] // heads)
    q = linear(query, wq, bq).reshape(*query.shape[:2], *hs)
    k = linear(memory, wk, bk).reshape(*memory.shape[:2], *hs)
    v = linear(memory, wv, bv).reshape(*memory.shape[:2], *hs)
    out = attention(q, k, v, mask).reshape(query.shape)
    return dense(out, p, name + ".out_proj")


def forward(p: Mapping[str, np.ndarray], hidden: np.ndarray, lexical: np.ndarray, a: Mapping[str, np.ndarray], *,
            heads: int, routing_layers: int, layers: int) -> np.ndarray:
    """head.py:54-111: option logits [B, O] (fp32, -1e9 at padded options)."""
    h = norm(hidden, p, "hidden_norm")
    memory = dense(h, p, "memory_projection")
    last = np.maximum(a["mask"].sum(-1) - 1, 0)
    global_vector = h[np.arange(h.shape[0]), last]

    questions = means(h, a["question_spans"])
    contexts = means(h, a["option_spans"])
    owners = a["option_field"]

    options = dense(contexts, p, "option_context_projection") + dense(lexical, p, "option_lexical_projection")
    options = options + gather(dense(questions, p, "option_question_projection"), owners)

    for i in range(routing_layers):                                        # head.py:69-74
        n = f"evidence_layers.{i}"
        q, m = norm(options, p, n + ".query_norm"), norm(memory, p, n + ".memory_norm")
        options = options + mha(q, m, a["mask"], p, n + ".attention", heads)
        ff = dense(norm(options, p, n + ".feedforward_norm"), p, n + ".feedforward.0")
        options = options + dense(gelu(ff), p, n + ".feedforward.3")

    base = dense(questions, p, "question_projection")                      # head.py:76-81
    logits = np.einsum("bow,bqw->bqo", options, base).astype(F32) / F32(math.sqrt(base.shape[-1]))
    owns = (owners[:, None, :] == np.arange(base.shape[1])[None, :, None]) & a["option_mask"][:, None, :]
    routing = softmax(np.where(owns, logits, MASK_FILL), -1)

    summary = np.sum(routing[..., None] * options[:, None], axis=2, dtype=F32)  # head.py:83-85
    fields = base + norm(summary, p, "option_summary_norm")
    fields = fields + dense(global_vector, p, "global_projection")[:, None]
    fields = fields + p["type_embedding.weight"][a["types"]]

    for i in range(layers):                                                # head.py:89-95
        n = f"layers.{i}"
        q = norm(fields, p, n + ".norm1")
        fields = fields + mha(q, q, a["question_mask"], p, n + ".self_attn", heads)
        fields = fields + mha(norm(fields, p, n + ".norm2"), memory, a["mask"], p, n + ".multihead_attn", heads)
        ff = dense(norm(fields, p, n + ".norm3"), p, n + ".linear1")
        fields = fields + dense(gelu(ff), p, n + ".linear2")

    fields = gather(norm(fields, p, "field_norm"), owners)                 # head.py:97-100
    anchor = normalize(gather(questions, owners) + global_vector[:, None])
    prior = np.sum(normalize(lexical) * anchor, -1, dtype=F32)
    prior = prior * F32(math.exp(min(float(p["prior_logit_scale"]), MAX_LOGIT_SCALE)))

    options = norm(options, p, "option_norm")                              # head.py:102-109
    cosine = np.sum(normalize(fields, 1e-8) * normalize(options, 1e-8), -1, dtype=F32)
    features = np.concatenate((fields, options, fields * options, np.abs(fields - options)), -1)
    residual = dense(gelu(dense(features, p, "residual_scorer.0")), p, "residual_scorer.3")[..., 0]
    joint = F32(math.exp(min(float(p["joint_logit_scale"]), MAX_LOGIT_SCALE))) * cosine + residual

    return np.where(a["option_mask"], prior + sigmoid(p["residual_gate"]) * joint, F32(-1e9)).astype(F32)
