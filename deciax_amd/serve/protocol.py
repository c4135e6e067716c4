"""The `/v1/systemone` wire contract: request limits, client errors and the answer decorations.

The limits, status codes and the `x_jev_confidence` / strict-projection formats are the ones the
reference serves (src/deciax/protocol/systemone.py:15-194), so that a client cannot tell the two
servers apart; the code here is this package's own.
"""

from __future__ import annotations

import json
import math
import re
from collections.abc import Mapping
from dataclasses import dataclass
from typing import Any

MAX_BODY_BYTES = 2 * 1024 * 1024        # systemone.py:15
MAX_QUESTIONS = 64                      # :16
MAX_STATE_CHARS = 50000                 # :17
MAX_BATCH_STATES = 64                   # :18
MAX_CHOICE_OPTIONS = 100                # :19
MAX_SCORE_LEVELS = 32                   # :20
MAX_TOTAL_OPTIONS = 512                 # :21

SURROGATE_DETAIL = "request body contains an unpaired surrogate escape; those cannot be encoded as UTF-8"
_SURROGATE = re.compile("[\ud800-\udfff]")


class RequestError(Exception):
    """A client error with its HTTP status and a detail safe to send back."""

    def __init__(self, status: int, detail: str) -> None:
        super().__init__(detail)
        self.status = status
        self.detail = detail


@dataclass(frozen=True)
class Limits:
    state_chars: int = MAX_STATE_CHARS
    choice_options: int = MAX_CHOICE_OPTIONS
    score_levels: int = MAX_SCORE_LEVELS


DEFAULT_LIMITS = Limits()


def _options_of(qid: str, q: Mapping[str, Any], limits: Limits) -> int:
    """Option count of one question for the total, refusing oversized choice / score lists."""
    criteria, kind = q.get("criteria"), q.get("type")
    if kind == "choice" and isinstance(criteria, (dict, list)):
        if len(criteria) > limits.choice_options:
            raise RequestError(413, f"too many choice options for {qid!r} ({len(criteria)} > {limits.choice_options})")
        return len(criteria)
    if kind == "score" and isinstance(criteria, list):
        if len(criteria) > limits.score_levels:
            raise RequestError(413, f"too many score levels for {qid!r} ({len(criteria)} > {limits.score_levels})")
        if any(level is None for level in criteria):
            raise RequestError(422, f"score question {qid!r} has a null level at index {criteria.index(None)}; "
                                    "give every level a description")
        return len(criteria)
    return 0


def check_request(state: Any, questions: Any, limits: Limits = DEFAULT_LIMITS) -> None:
    """400 for a missing state or malformed questions, 413 for oversized ones, 422 for null score
    levels; all before any tokenization."""
    if state is None:
        raise RequestError(400, "'state' is required")
    if not isinstance(questions, dict):
        raise RequestError(400, "'questions' must be an object")
    if len(questions) > MAX_QUESTIONS:
        raise RequestError(413, f"too many questions ({len(questions)} > {MAX_QUESTIONS})")
    total = sum(_options_of(qid, q, limits) for qid, q in questions.items() if isinstance(q, dict))
    if total > MAX_TOTAL_OPTIONS:
        raise RequestError(413, f"too many answer options across questions ({total} > {MAX_TOTAL_OPTIONS})")
    size = len(state) if isinstance(state, str) else len(json.dumps(state, ensure_ascii=False))
    if size > limits.state_chars:
        raise RequestError(413, f"state too large ({size} > {limits.state_chars} chars)")


def check_batch(states: Any, questions: Any, limits: Limits = DEFAULT_LIMITS) -> None:
    if not isinstance(states, list) or not states:
        raise RequestError(400, "'states' must be a non-empty list")
    if len(states) > MAX_BATCH_STATES:
        raise RequestError(413, f"too many states in batch ({len(states)} > {MAX_BATCH_STATES})")
    for state in states:
        check_request(state, questions, limits)


def has_lone_surrogate(value: Any) -> bool:
    """Whether any key or string anywhere in a parsed body holds an unpaired surrogate."""
    pending = [value]
    while pending:
        item = pending.pop()
        if isinstance(item, str):
            if _SURROGATE.search(item):
                return True
        elif isinstance(item, dict):
            pending.extend(item)
            pending.extend(item.values())
        elif isinstance(item, (list, tuple)):
            pending.extend(item)
    return False


def confidence(answer: Mapping[str, Any]) -> float | None:
    """Jev's confidence of a choice or score answer from its probabilities, None otherwise.
    choice: (max p - 1/n) / (1 - 1/n); score: max(0, 1 - E|i - mode| / E_uniform|i - centre|)."""
    kind, probs = answer.get("type"), answer.get("probabilities")
    if kind not in ("choice", "score") or not isinstance(probs, dict) or not probs:
        return None
    if any(isinstance(v, bool) for v in probs.values()):
        return None
    try:
        keys = sorted(probs, key=int) if kind == "score" else list(probs)
        p = [float(probs[k]) for k in keys]
    except (TypeError, ValueError):
        return None
    if not all(math.isfinite(v) for v in p):
        return None
    n = len(p)
    if n == 1:
        return 1.0
    total = sum(p)
    p = [v / total for v in p] if total else [1.0 / n] * n
    if kind == "choice":
        return (max(p) - 1.0 / n) / (1.0 - 1.0 / n)
    mode = p.index(max(p))
    spread = sum(v * abs(i - mode) for i, v in enumerate(p))
    centre = (n - 1) / 2
    uniform = sum(abs(i - centre) for i in range(n)) / n
    return max(0.0, 1.0 - spread / uniform)


def with_confidence(result: Mapping[str, Any]) -> dict[str, Any]:
    """A copy of `result` whose choice and score answers carry `x_jev_confidence` (4 decimals)."""
    answers = {}
    for qid, answer in result["answers"].items():
        c = confidence(answer)
        answers[qid] = answer if c is None else {**answer, "x_jev_confidence": round(c, 4)}
    return {**result, "answers": answers}


STRICT_FIELDS = {
    "choice": ("type", "choice", "confidence", "probabilities"),
    "score": ("type", "score", "confidence", "probabilities", "legend"),
    "noul": ("type", "noul"),
}


def strict_view(result: Mapping[str, Any]) -> dict[str, Any]:
    """Only the fields of the strict Jev contract."""
    answers = {}
    for qid, answer in result["answers"].items():
        fields = STRICT_FIELDS.get(answer.get("type"))
        answers[qid] = answer if fields is None else {k: answer[k] for k in fields}
    usage = result.get("usage") or {}
    return {"model": result["model"], "answers": answers,
            "usage": {"input_tokens": usage.get("input_tokens", 0), "output_tokens": usage.get("output_tokens", 0)}}
