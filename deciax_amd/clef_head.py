"""Clef joint schema head on the GPU (fp32).

`forward` follows src/deciax/models/clef/head.py:54-111 step by step. Each step is a call into
the head kernels of `libdeciax_hip.so` (deciax_amd/csrc/head.hip, declared in
include/deciax_hip.h); torch only supplies the device buffers. Batched tensors travel as
[batch * n, d] row blocks. `load_params` reads `joint_head.safetensors` as the reference does
(src/deciax/models/clef/weights.py:100).
"""

from __future__ import annotations

import math
from collections.abc import Mapping
from pathlib import Path
from typing import Any

import numpy as np
import torch

from deciax_amd import kernels as K

MAX_LOGIT_SCALE = math.log(100.0)  # head.py:17
EPS = 1e-5                         # head.py:20-21


def load_params(path: str | Path, device: str | torch.device = "cuda") -> dict[str, torch.Tensor]:
    """Head parameters from a safetensors file, fp32 on the device."""
    from deciax_amd.checkpoint import tensors

    return {k: v.to(device=device, dtype=torch.float32).contiguous() for k, v in tensors(path)}


def _dev(x: Any, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        return x.to(device=device, dtype=dtype).contiguous()
    return torch.as_tensor(np.ascontiguousarray(x)).to(device=device, dtype=dtype).contiguous()


def lexical_vectors(embedding: torch.Tensor, lexical_ids: Any, lexical_spans: Any) -> torch.Tensor:
    """Mean embedding of each option's label tokens: embedding[lexical_ids] averaged over
    lexical_spans [B, O, 2] (how the reference builds `lexical`, tests/clef/test_head.py:16,
    with `means` of head.py:24-29). Returns [B, O, H] fp32."""
    ids = _dev(lexical_ids, torch.int32, embedding.device)
    batch, seq = ids.shape
    rows = K.gather_rows_f32(embedding, ids.reshape(1, batch * seq), batch=1)
    spans = _dev(lexical_spans, torch.int32, embedding.device)
    return K.span_means_f32(rows, spans, batch=batch).reshape(batch, spans.shape[1], embedding.shape[1])


def forward(p: Mapping[str, torch.Tensor], hidden: Any, lexical: Any, a: Mapping[str, Any], *, heads: int,
            routing_layers: int, layers: int) -> torch.Tensor:
    """Option logits [B, O] (fp32, -1e9 at padded options).

    hidden [B, S, H] and lexical [B, O, H] (the lexical option vectors) are fp32; `a` holds the
    collate arrays (src/deciax/models/clef/input.py:140-182): mask [B, S], question_spans
    [B, Q, 2], option_spans [B, O, 2], option_field [B, O], option_mask [B, O], question_mask
    [B, Q] and types [B, Q]. Host (numpy) or device inputs are accepted."""
    dev = p["hidden_norm.weight"].device
    hid = _dev(hidden, torch.float32, dev)
    batch, seq, hdim = hid.shape
    mask_np = np.asarray(a["mask"].cpu() if isinstance(a["mask"], torch.Tensor) else a["mask"]).astype(bool)
    mask = _dev(mask_np.astype(np.uint8), torch.uint8, dev)
    q_mask = _dev(np.asarray(a["question_mask"]).astype(np.uint8), torch.uint8, dev)
    opt_mask = _dev(np.asarray(a["option_mask"]).astype(np.uint8), torch.uint8, dev)
    owners = _dev(a["option_field"], torch.int32, dev)
    types = _dev(a["types"], torch.int32, dev)
    q_spans = _dev(a["question_spans"], torch.int32, dev)
    o_spans = _dev(a["option_spans"], torch.int32, dev)
    n_opt = owners.shape[1]
    lex = _dev(lexical, torch.float32, dev).reshape(batch * n_opt, hdim)

    def norm(x: torch.Tensor, name: str) -> torch.Tensor:
        return K.layer_norm_f32(x, p[name + ".weight"], p[name + ".bias"], eps=EPS)

    def dense(x: torch.Tensor, name: str, **kw: Any) -> torch.Tensor:
        return K.linear_f32(x, p[name + ".weight"], p.get(name + ".bias"), **kw)

    def mha(query: torch.Tensor, memory: torch.Tensor, key_mask: torch.Tensor, name: str,
            out: torch.Tensor) -> torch.Tensor:
        """out += mha(query, memory) (head.py:41-51): in_proj split in q | k | v rows."""
        w, b = p[name + ".in_proj_weight"], p[name + ".in_proj_bias"]
        width = query.shape[1]
        q = K.linear_f32(query, w[:width], b[:width])
        kv = K.linear_f32(memory, w[width:], b[width:])
        att = K.mha_f32(q, kv[:, :width], kv[:, width:], key_mask, batch=batch, heads=heads)
        return dense(att, name + ".out_proj", out=out, accumulate=True)

    h = norm(hid.reshape(batch * seq, hdim), "hidden_norm")               # head.py:57-60
    memory = dense(h, "memory_projection")
    last = torch.as_tensor(np.maximum(mask_np.sum(-1) - 1, 0).astype(np.int32)).to(dev).reshape(batch, 1)
    global_vector = K.gather_rows_f32(h, last, batch=batch)

    questions = K.span_means_f32(h, q_spans, batch=batch)                 # head.py:62-67
    contexts = K.span_means_f32(h, o_spans, batch=batch)
    options = dense(contexts, "option_context_projection")
    dense(lex, "option_lexical_projection", out=options, accumulate=True)
    K.gather_rows_f32(dense(questions, "option_question_projection"), owners, batch=batch, out=options,
                      accumulate=True)

    for i in range(routing_layers):                                        # head.py:69-74
        n = f"evidence_layers.{i}"
        mha(norm(options, n + ".query_norm"), norm(memory, n + ".memory_norm"), mask, n + ".attention", options)
        ff = dense(norm(options, n + ".feedforward_norm"), n + ".feedforward.0", gelu=True)
        dense(ff, n + ".feedforward.3", out=options, accumulate=True)

    base = dense(questions, "question_projection")                         # head.py:76-88
    summary = K.head_routing_f32(options, base, owners, opt_mask, batch=batch)
    fields = K.head_fields_init_f32(base, norm(summary, "option_summary_norm"),
                                    dense(global_vector, "global_projection"), p["type_embedding.weight"], types,
                                    batch=batch)

    for i in range(layers):                                                # head.py:89-95
        n = f"layers.{i}"
        q = norm(fields, n + ".norm1")
        mha(q, q, q_mask, n + ".self_attn", fields)
        mha(norm(fields, n + ".norm2"), memory, mask, n + ".multihead_attn", fields)
        ff = dense(norm(fields, n + ".norm3"), n + ".linear1", gelu=True)
        dense(ff, n + ".linear2", out=fields, accumulate=True)

    fields_o = K.gather_rows_f32(norm(fields, "field_norm"), owners, batch=batch)   # head.py:97-109
    prior_scale = math.exp(min(float(p["prior_logit_scale"]), MAX_LOGIT_SCALE))
    features, prior, cosine = K.head_features_f32(fields_o, norm(options, "option_norm"), questions, global_vector,
                                                  lex, owners, batch=batch, prior_scale=prior_scale)
    residual = dense(dense(features, "residual_scorer.0", gelu=True), "residual_scorer.3")
    gate = 1.0 / (1.0 + math.exp(-float(p["residual_gate"])))
    joint_scale = math.exp(min(float(p["joint_logit_scale"]), MAX_LOGIT_SCALE))
    logits = K.head_combine_f32(prior, cosine, residual.reshape(-1), opt_mask.reshape(-1), gate=gate,
                                joint_scale=joint_scale)
    return logits.reshape(batch, n_opt)
