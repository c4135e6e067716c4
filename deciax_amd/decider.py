"""Public entry point, mirroring src/deciax/decider.py:22-84.

`load(model, *, revision, dtype, impl)` builds a Gemma-2-shaped decision model
on the MI355X and binds it to an engine; `Decider.decide` / `decide_batch`
keep the reference's signatures. The models here are synthetic (random-init
weights of the named shape, seeded) because no checkpoint is available; the
path they exercise is the one a real checkpoint would take.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from typing import Any, Literal

from deciax_amd import gemma
from deciax_amd.backend import ImplChoice, resolve
from deciax_amd.engine import DecisionEngine
from deciax_amd.schema import ByteTokenizer, TokenizerLike

DtypeChoice = Literal["auto", "bf16", "fp32"]
ModelName = Literal["gemma2-9b", "gemma2-27b", "tiny"]


class Decider:
    """One loaded model bound to its engine (src/deciax/decider.py:22-52)."""

    def __init__(self, engine: DecisionEngine) -> None:
        self.engine = engine
        self.model = engine.weights

    def decide(self, state: Any, questions: Mapping[Any, Mapping[str, Any]], *, max_len: int | None = None,
               head_max_len: int | None = None) -> dict[str, Any]:
        """Answer every question about one state."""
        return self.decide_batch([state], questions, max_len=max_len, head_max_len=head_max_len)[0]

    def decide_batch(self, states: Sequence[Any], questions: Mapping[Any, Mapping[str, Any]], *,
                     max_len: int | None = None, head_max_len: int | None = None) -> list[dict[str, Any]]:
        """Answer the same questions about many states in shared forward passes."""
        return self.engine.decide_batch(states, questions, max_len=max_len, head_max_len=head_max_len)


def load(model: ModelName = "gemma2-9b", *, revision: str | None = None, dtype: DtypeChoice = "auto",
         impl: ImplChoice = "auto", seed: int = 0, tokenizer: TokenizerLike | None = None,
         layers: int | None = None) -> Decider:
    """Build a synthetic decision model of a registered shape on the GPU.

    `impl` resolves as in `deciax_amd.backend.resolve`; the HIP path computes in bf16, so
    `dtype` must be "auto" or "bf16" (the reference likewise rejects Pallas without BF16,
    src/deciax/models/clef/model.py:48-50). `layers` truncates the depth (tests only)."""
    if model not in gemma.CONFIGS:
        raise ValueError(f"unknown model {model!r}; choose one of {sorted(gemma.CONFIGS)}")
    if revision is not None:
        raise ValueError("synthetic models have no revisions")
    if dtype not in ("auto", "bf16", "fp32"):
        raise ValueError(f"dtype must be 'auto', 'bf16' or 'fp32', got {dtype!r}")
    if dtype == "fp32":
        raise ValueError("the HIP decision forward requires bf16 weights")
    resolve(impl)
    config = gemma.CONFIGS[model]
    if layers is not None:
        if not 1 <= layers <= config.layers:
            raise ValueError(f"layers must be in [1, {config.layers}]")
        from dataclasses import replace

        config = replace(config, layers=layers)
    weights = gemma.random_weights(config, seed=seed)
    tok = tokenizer if tokenizer is not None else ByteTokenizer(config.vocab)
    return Decider(DecisionEngine(weights, tok, model))
