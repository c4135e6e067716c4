"""Request engine: encode -> one packed forward -> decode (the role of `ClefEngine`,
src/deciax/runtime/clef.py:18-40).

The reference runs requests in chunks of two padded to shape buckets
(clef.py:33-38); here every request of a call shares one varlen forward, so the
batch costs exactly its real tokens. A lock serialises device forwards, as the
reference's engine lock does (clef.py:21,36).
"""

from __future__ import annotations

import threading
from collections.abc import Mapping, Sequence
from typing import Any

import numpy as np
import torch

from deciax_amd import gemma
from deciax_amd.schema import MAX_TOKENS, Record, TokenizerLike, decode, encode, readout_layout

# Token budget of one packed forward; larger calls are split at request boundaries.
MAX_BATCH_TOKENS = 1 << 18


class DecisionEngine:
    def __init__(self, weights: gemma.DecisionWeights, tokenizer: TokenizerLike, name: str) -> None:
        self.weights = weights
        self.tokenizer = tokenizer
        self.name = name
        self.max_token_budget = min(MAX_TOKENS, weights.config.max_position)
        self._lock = threading.Lock()
        self._workspace: gemma.Workspace | None = None

    def decide_batch(self, states: Sequence[Any], questions: Mapping[Any, Mapping[str, Any]], *,
                     max_len: int | None = None, head_max_len: int | None = None) -> list[dict[str, Any]]:
        if head_max_len is not None:
            raise ValueError("one joint token budget per request; head_max_len is unsupported")
        budget = self.max_token_budget if max_len is None else max_len
        if isinstance(budget, int) and not isinstance(budget, bool) and budget > self.max_token_budget:
            raise ValueError(f"max_len must be at most {self.max_token_budget}")
        vocab = self.weights.config.vocab
        records = [encode(self.tokenizer, s, questions, budget, vocab=vocab) for s in states]
        results: list[dict[str, Any]] = []
        for part in _chunks(records, MAX_BATCH_TOKENS):
            logits, probs = self.forward_records(part)
            offset = 0
            for r in part:
                n = sum(len(f.option_ids) for f in r.fields)
                results.append(decode(r, logits[offset:offset + n], questions, self.name,
                                      probs=probs[offset:offset + n]))
                offset += n
        return results

    def forward_records(self, records: Sequence[Record]) -> tuple[np.ndarray, np.ndarray]:
        """(logits, probs) on the host for the options of `records`, in request/field order."""
        w = self.weights
        batch = gemma.pack_batch([r.ids for r in records], readout_layout(records), device=w.device)
        with self._lock:
            ws = self._workspace
            if ws is None or not ws.fits(batch.rows, batch.vt_ld):
                ws = self._workspace = gemma.Workspace(w.config, batch.rows, batch.vt_ld, w.device)
            logits, probs = gemma.forward(w, batch, ws)
            torch.cuda.current_stream().synchronize()
        return logits.cpu().numpy(), probs.cpu().numpy()


def _chunks(records: Sequence[Record], budget: int) -> list[list[Record]]:
    out: list[list[Record]] = []
    cur: list[Record] = []
    used = 0
    for r in records:
        if cur and used + len(r.ids) > budget:
            out.append(cur)
            cur, used = [], 0
        cur.append(r)
        used += len(r.ids)
    if cur:
        out.append(cur)
    return out
