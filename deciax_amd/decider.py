"""Public entry point, mirroring src/deciax/decider.py:22-84.

`load(model, *, revision, dtype, impl)` builds a Gemma-2-shaped decision model
on the MI355X and binds it to an engine; `Decider.decide` / `decide_batch`
keep the reference's signatures. `model` is either a registered shape (random-init
weights, seeded) or a local Gemma-2 checkpoint directory (config.json plus
safetensors, read by `deciax_amd.checkpoint`). The reference resolves a Hub name
with `snapshot_download` (src/deciax/decider.py:66-73); there is no network here,
so a checkpoint must already be on disk.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from dataclasses import replace
from pathlib import Path
from typing import Any, Literal

from deciax_amd import gemma
from deciax_amd.backend import ImplChoice, resolve
from deciax_amd.engine import DecisionEngine
from deciax_amd.schema import MAX_TOKENS, ByteTokenizer, TokenizerLike

DtypeChoice = Literal["auto", "bf16", "fp32"]
ModelName = Literal["gemma2-9b", "gemma2-27b", "tiny"]


class GemmaDecisionModel:
    """A loaded Gemma-2-shaped decision model: device weights plus tokenizer. It satisfies the
    reference's `RequestModel` protocol (src/deciax/models/base.py:58-59): `build_engine()` returns
    the request engine that `Decider` drives, as `ClefModel` does for the reference's Clef
    checkpoints (src/deciax/decider.py:25-27)."""

    def __init__(self, weights: gemma.DecisionWeights, tokenizer: TokenizerLike, name: str) -> None:
        self.weights = weights
        self.tokenizer = tokenizer
        self.name = name
        self.config = weights.config
        self.max_token_budget = min(MAX_TOKENS, weights.config.max_position)

    def build_engine(self) -> DecisionEngine:
        return DecisionEngine(self.weights, self.tokenizer, self.name)


class Decider:
    """One loaded model bound to a runtime engine (src/deciax/decider.py:22-52): the engine comes
    from `model.build_engine()`, as in the reference."""

    def __init__(self, model: GemmaDecisionModel) -> None:
        self.model = model
        self.engine = model.build_engine()

    def decide(self, state: Any, questions: Mapping[Any, Mapping[str, Any]], *, max_len: int | None = None,
               head_max_len: int | None = None) -> dict[str, Any]:
        """Answer every question about one state."""
        return self.decide_batch([state], questions, max_len=max_len, head_max_len=head_max_len)[0]

    def decide_batch(self, states: Sequence[Any], questions: Mapping[Any, Mapping[str, Any]], *,
                     max_len: int | None = None, head_max_len: int | None = None) -> list[dict[str, Any]]:
        """Answer the same questions about many states in shared forward passes."""
        return self.engine.decide_batch(states, questions, max_len=max_len, head_max_len=head_max_len)


def load(model: ModelName | str | Path = "gemma2-9b", *, revision: str | None = None, dtype: DtypeChoice = "auto",
         impl: ImplChoice = "auto", seed: int = 0, tokenizer: TokenizerLike | None = None,
         layers: int | None = None) -> Decider:
    """Build a decision model on the GPU: a registered shape with seeded random weights, or a
    Gemma-2 checkpoint directory.

    `impl` resolves as in `deciax_amd.backend.resolve`; the HIP path computes in bf16, so
    `dtype` must be "auto" or "bf16" (the reference likewise rejects Pallas without BF16,
    src/deciax/models/clef/model.py:48-50). `layers` truncates the depth (tests only)."""
    is_dir = isinstance(model, (str, Path)) and Path(model).is_dir()
    if not is_dir and model not in gemma.CONFIGS:
        raise ValueError(f"unknown model {model!r}; choose one of {sorted(gemma.CONFIGS)} or a checkpoint directory")
    if revision is not None:
        raise ValueError("revisions need the Hub; pass a local checkpoint directory instead")
    if dtype not in ("auto", "bf16", "fp32"):
        raise ValueError(f"dtype must be 'auto', 'bf16' or 'fp32', got {dtype!r}")
    if dtype == "fp32":
        raise ValueError("the HIP decision forward requires bf16 weights")
    resolve(impl)
    if is_dir:
        from deciax_amd import checkpoint

        config, host = checkpoint.read_checkpoint(model)
    else:
        config, host = gemma.CONFIGS[model], None
    if layers is not None:
        if not 1 <= layers <= config.layers:
            raise ValueError(f"layers must be in [1, {config.layers}]")
        config = replace(config, layers=layers)
    weights = gemma.weights_from_host(config, host) if host is not None else gemma.random_weights(config, seed=seed)
    tok = tokenizer if tokenizer is not None else ByteTokenizer(config.vocab)
    return Decider(GemmaDecisionModel(weights, tok, config.name if is_dir else str(model)))
