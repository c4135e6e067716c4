"""The `/v1/systemone` wire contract, as data plus the few functions that apply it.

What a client can observe is fixed by the reference's server (src/deciax/protocol/systemone.py:15-194,
src/deciax/serve/app.py:66-80): the request limits, the status code and detail text of every refusal,
which refusal wins when a request breaks several rules, the `x_jev_confidence` value added to choice and
score answers, and the fields the strict projection keeps. Everything here states that contract; the
order of the rules in each table is part of it.
"""

from __future__ import annotations

import json
import math
from collections.abc import Callable, Iterable, Iterator, Mapping, Sequence
from dataclasses import dataclass
from typing import Any

MAX_BODY_BYTES = 2 * 1024 * 1024
MAX_QUESTIONS = 64
MAX_STATE_CHARS = 50000
MAX_BATCH_STATES = 64
MAX_CHOICE_OPTIONS = 100
MAX_SCORE_LEVELS = 32
MAX_TOTAL_OPTIONS = 512

SURROGATE_DETAIL = "request body contains an unpaired surrogate escape; those cannot be encoded as UTF-8"

# Body fields a request may not set: server-side hooks (refused with one message) and controls this
# server does not implement (refused rather than silently ignored).
HOOK_FIELDS = ("hooks", "on_predict_start", "on_predict_end", "hooks_raise", "hooks_timeout")
UNSUPPORTED_FIELDS = ("task", "lang", "lang_guess", "min_confidence", "images", "videos", "media_kwargs")
UNSUPPORTED_BATCH_FIELDS = ("batch_size", "sort_by_length", "diagnostics")
BUDGET_FIELDS = ("max_len", "head_max_len")


class Refusal(Exception):
    """A request the server answers with `status` and a `detail` that is safe to send back."""

    def __init__(self, status: int, detail: str) -> None:
        super().__init__(detail)
        self.status = status
        self.detail = detail


@dataclass(frozen=True)
class Limits:
    """Per-request caps a served model may tighten."""

    state_chars: int = MAX_STATE_CHARS
    choice_options: int = MAX_CHOICE_OPTIONS
    score_levels: int = MAX_SCORE_LEVELS


DEFAULT_LIMITS = Limits()


@dataclass(frozen=True)
class OptionRule:
    """How one question type counts its answer options and which cap applies to them."""

    containers: tuple[type, ...]
    cap: str          # the Limits field
    noun: str         # the words of the 413 detail
    null_levels_refused: bool = False


OPTION_RULES: dict[str, OptionRule] = {
    "choice": OptionRule((dict, list), "choice_options", "choice options"),
    "score": OptionRule((list,), "score_levels", "score levels", null_levels_refused=True),
}


def _state_chars(state: Any) -> int:
    return len(state) if isinstance(state, str) else len(json.dumps(state, ensure_ascii=False))


def _question_refusals(questions: Mapping[Any, Any], limits: Limits) -> Iterator[Refusal]:
    total = 0
    for qid, question in questions.items():
        rule = OPTION_RULES.get(question.get("type")) if isinstance(question, dict) else None
        criteria = question.get("criteria") if rule else None
        if rule is None or not isinstance(criteria, rule.containers):
            continue
        count, cap = len(criteria), getattr(limits, rule.cap)
        total += count
        if count > cap:
            yield Refusal(413, f"too many {rule.noun} for {qid!r} ({count} > {cap})")
        if rule.null_levels_refused and None in criteria:
            yield Refusal(422, f"score question {qid!r} has a null level at index {criteria.index(None)}; "
                               "give every level a description")
    if total > MAX_TOTAL_OPTIONS:
        yield Refusal(413, f"too many answer options across questions ({total} > {MAX_TOTAL_OPTIONS})")


def request_refusals(state: Any, questions: Any, limits: Limits = DEFAULT_LIMITS) -> Iterator[Refusal]:
    """Every rule one (state, questions) pair breaks, lazily, in the contract's order."""
    if state is None:
        yield Refusal(400, "'state' is required")
    if not isinstance(questions, dict):
        yield Refusal(400, "'questions' must be an object")
        return
    if len(questions) > MAX_QUESTIONS:
        yield Refusal(413, f"too many questions ({len(questions)} > {MAX_QUESTIONS})")
    yield from _question_refusals(questions, limits)
    chars = _state_chars(state)
    if chars > limits.state_chars:
        yield Refusal(413, f"state too large ({chars} > {limits.state_chars} chars)")


def batch_refusals(states: Any, questions: Any, limits: Limits = DEFAULT_LIMITS) -> Iterator[Refusal]:
    """As `request_refusals`, for a batch of states sharing one question set."""
    if not isinstance(states, list) or not states:
        yield Refusal(400, "'states' must be a non-empty list")
        return
    if len(states) > MAX_BATCH_STATES:
        yield Refusal(413, f"too many states in batch ({len(states)} > {MAX_BATCH_STATES})")
    for state in states:
        yield from request_refusals(state, questions, limits)


def first(refusals: Iterable[Refusal]) -> None:
    """Raise the first refusal of `refusals`, if there is one: that is the one a client sees."""
    for refusal in refusals:
        raise refusal


def has_lone_surrogate(body: Any) -> bool:
    """True when some string of a parsed JSON body (key or value) cannot be written as UTF-8, which is
    exactly when it holds an unpaired surrogate code point."""
    try:
        json.dumps(body, ensure_ascii=False).encode("utf-8")
    except UnicodeEncodeError:
        return True
    return False


def field_refusals(body: Mapping[str, Any], unsupported: Sequence[str]) -> Iterator[Refusal]:
    """Hook fields are refused when present at all; unsupported controls when set to a value."""
    hooks = [k for k in HOOK_FIELDS if k in body]
    if hooks:
        yield Refusal(422, f"{', '.join(hooks)} cannot be set from a request; hooks belong to the server")
    sent = [k for k in unsupported if body.get(k) is not None]
    if sent:
        yield Refusal(422, f"{', '.join(sent)} is not supported by deciax")


def budgets(body: Mapping[str, Any], cap: int) -> dict[str, int]:
    """The token budgets a request sets, each a positive integer no larger than the server's cap."""
    out: dict[str, int] = {}
    for key in BUDGET_FIELDS:
        value = body.get(key)
        if value is None:
            continue
        if isinstance(value, bool) or not isinstance(value, int):
            raise Refusal(422, f"{key} must be an integer")
        if value <= 0:
            raise Refusal(422, f"{key} must be a positive integer")
        if value > cap:
            raise Refusal(422, f"{key} exceeds the server cap ({value} > {cap})")
        out[key] = value
    return out


# --------------------------------------------------------------------------- answer decorations


def _ordered_probabilities(kind: str, probabilities: Mapping[str, Any]) -> list[float]:
    """The answer's probabilities as floats: score levels by their integer key, choice keys as given."""
    keys = sorted(probabilities, key=int) if kind == "score" else list(probabilities)
    return [float(probabilities[k]) for k in keys]


def _choice_confidence(p: Sequence[float]) -> float:
    """How far the top option is above a uniform pick, 0 (uniform) .. 1 (certain)."""
    floor = 1.0 / len(p)
    return (max(p) - floor) / (1.0 - floor)


def _score_confidence(p: Sequence[float]) -> float:
    """1 minus the expected distance from the most likely level, relative to that distance for a
    uniform distribution around the middle level; clamped at 0."""
    n = len(p)
    mode = max(range(n), key=lambda i: p[i])
    spread = sum(w * abs(i - mode) for i, w in enumerate(p))
    middle = (n - 1) / 2
    uniform = sum(abs(i - middle) for i in range(n)) / n
    return max(0.0, 1.0 - spread / uniform)


CONFIDENCE: dict[str, Callable[[Sequence[float]], float]] = {"choice": _choice_confidence,
                                                             "score": _score_confidence}


def confidence(answer: Mapping[str, Any]) -> float | None:
    """The Jev `confidence` of a choice or score answer from its probabilities; None for other answers
    and for probability maps that are empty, boolean, non-numeric or non-finite."""
    kind, probabilities = answer.get("type"), answer.get("probabilities")
    measure = CONFIDENCE.get(kind)
    if measure is None or not isinstance(probabilities, dict) or not probabilities:
        return None
    if any(isinstance(v, bool) for v in probabilities.values()):
        return None
    try:
        p = _ordered_probabilities(kind, probabilities)
    except (TypeError, ValueError):
        return None
    if not all(map(math.isfinite, p)):
        return None
    if len(p) == 1:
        return 1.0
    total = sum(p)
    p = [w / total for w in p] if total else [1.0 / len(p)] * len(p)
    return measure(p)


# Fields of each answer type under the strict Jev contract.
STRICT_FIELDS: dict[str, tuple[str, ...]] = {
    "choice": ("type", "choice", "confidence", "probabilities"),
    "score": ("type", "score", "confidence", "probabilities", "legend"),
    "noul": ("type", "noul"),
}


def with_confidence(result: Mapping[str, Any]) -> dict[str, Any]:
    """A copy of `result` whose choice and score answers carry `x_jev_confidence` (4 decimals)."""
    def extend(answer: Mapping[str, Any]) -> Mapping[str, Any]:
        value = confidence(answer)
        return answer if value is None else {**answer, "x_jev_confidence": round(value, 4)}

    return {**result, "answers": {qid: extend(a) for qid, a in result["answers"].items()}}


def strict_view(result: Mapping[str, Any]) -> dict[str, Any]:
    """`result` cut down to the strict Jev contract: model, answers with their contract fields only,
    and usage with input / output token counts."""
    def cut(answer: Mapping[str, Any]) -> Mapping[str, Any]:
        keep = STRICT_FIELDS.get(answer.get("type"))
        return answer if keep is None else {k: answer[k] for k in keep}

    usage = result.get("usage") or {}
    return {"model": result["model"],
            "answers": {qid: cut(a) for qid, a in result["answers"].items()},
            "usage": {k: usage.get(k, 0) for k in ("input_tokens", "output_tokens")}}
