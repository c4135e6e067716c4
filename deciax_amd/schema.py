"""Host-side request encoding, packing and answer decoding for the decision forward.

Follows the Clef input contract of the reference (src/deciax/models/clef/input.py):
question validation (:61-88), schema serialisation with option spans (:91-137),
right-truncation of the state so the schema stays whole (:127-131), and
`decode` (:185-214): per-field softmax of the option logits, noul -> p["true"],
choice -> argmax in criteria order, score -> expected level, 4-decimal rounding,
FloatingPointError on non-finite values.

Differences, both for the varlen GPU forward:
  * `collate` packs requests back to back (no power-of-two buckets,
    src/deciax/runtime/buckets.py) — `deciax_amd.gemma.pack_batch`;
  * each option is read at one position with one label token (the last token
    of its span and the first token of its id) instead of the Clef joint
    schema head (src/deciax/models/clef/head.py:54-107).

`head_inputs` lays encoded requests out for that joint head (`deciax_amd.clef_head`)
as the reference's collate does (:140-182), padded to the batch maxima.
"""

from __future__ import annotations

import json
from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from typing import Any, Protocol

import numpy as np

QTYPES = {"noul": 0, "choice": 1, "score": 2}  # src/deciax/models/clef/input.py:24
MAX_QUESTIONS = 64          # src/deciax/protocol/systemone.py:17
MAX_TOTAL_OPTIONS = 512     # src/deciax/protocol/systemone.py:22
MAX_TOKENS = 16384          # src/deciax/models/clef/input.py:25-26
SYSTEM_PROMPT = ("Read the complete state and schema. Decide every field jointly. "
                 "Each answer must be exactly one of that field's allowed options.")


class TokenizerLike(Protocol):
    def encode_ids(self, text: str) -> list[int]: ...


class ByteTokenizer:
    """Deterministic UTF-8 byte tokenizer for the synthetic models: id = byte + 4
    (0 pad, 1 bos, 2 eos, 3 unknown)."""

    pad_token_id = 0
    offset = 4

    def __init__(self, vocab: int = 260) -> None:
        if vocab < 260:
            raise ValueError("ByteTokenizer needs a vocabulary of at least 260 ids")
        self.vocab = vocab

    def encode_ids(self, text: str) -> list[int]:
        return [b + self.offset for b in text.encode("utf-8")]


class HFTokenizer:
    """Adapter for a `tokenizers.Tokenizer` (ids without special tokens, as the reference encodes)."""

    def __init__(self, tokenizer: Any, pad_token: str = "<pad>") -> None:
        self.tokenizer = tokenizer
        pad = tokenizer.token_to_id(pad_token)
        self.pad_token_id = 0 if pad is None else pad

    def encode_ids(self, text: str) -> list[int]:
        return list(self.tokenizer.encode(text, add_special_tokens=False).ids)


def render(value: Any) -> str:
    return value if isinstance(value, str) else json.dumps(value, ensure_ascii=False, separators=(",", ":"),
                                                           sort_keys=True)


def options(question: Mapping[str, Any]) -> list[tuple[str, Any]]:
    """(option id, description) in the model's option order (src/deciax/models/clef/input.py:34-43)."""
    if question["type"] == "noul":
        criteria = {"true": "The proposition is true or the answer is yes.",
                    "false": "The proposition is false or the answer is no."}
        criteria.update(question.get("criteria") or {})
        return [(k, criteria[k]) for k in ("true", "false")]
    if question["type"] == "choice":
        return sorted((str(k), v) for k, v in question["criteria"].items())
    return [(str(i), v) for i, v in enumerate(question["criteria"])]


def validate_questions(questions: Mapping[Any, Any]) -> None:
    """Schema checks of src/deciax/models/clef/input.py:61-88 (ValueError on any violation)."""
    if not isinstance(questions, Mapping) or not questions:
        raise ValueError("at least one question is required")
    if len(questions) > MAX_QUESTIONS:
        raise ValueError(f"at most {MAX_QUESTIONS} questions per request")
    total = 0
    for qid, q in questions.items():
        if not isinstance(qid, str) or not qid:
            raise ValueError("question ids must be nonempty strings")
        if not isinstance(q, Mapping) or not isinstance(q.get("type"), str) or q["type"] not in QTYPES:
            raise ValueError(f"{qid}: type must be noul, choice, or score")
        if any(k in q for k in ("labels", "option_order")):
            raise ValueError(f"{qid}: labels and option_order are not supported")
        criteria = q.get("criteria")
        if q["type"] == "choice" and (not isinstance(criteria, dict) or not criteria):
            raise ValueError(f"{qid}: choice criteria must be a nonempty object")
        if q["type"] == "score" and (not isinstance(criteria, list) or not criteria):
            raise ValueError(f"{qid}: score criteria must be a nonempty list")
        if q["type"] == "noul" and criteria is not None and (
                not isinstance(criteria, dict) or not set(criteria) <= {"true", "false"}):
            raise ValueError(f"{qid}: noul criteria must use true/false keys")
        total += len(options(q))
    if total > MAX_TOTAL_OPTIONS:
        raise ValueError(f"at most {MAX_TOTAL_OPTIONS} total options per request")


@dataclass(frozen=True)
class Field:
    id: str
    kind: int
    span: tuple[int, int]
    option_spans: tuple[tuple[int, int], ...]
    option_ids: tuple[str, ...]
    option_labels: tuple[int, ...]   # label token id of each option

    def readout(self) -> list[tuple[int, int]]:
        """(position, label token) per option: the last token of the option's span."""
        return [(end - 1, label) for (_, end), label in zip(self.option_spans, self.option_labels)]


@dataclass(frozen=True)
class Record:
    ids: tuple[int, ...]
    fields: tuple[Field, ...]


def encode(tokenizer: TokenizerLike, state: Any, questions: Mapping[str, Any], max_length: int = MAX_TOKENS,
           vocab: int | None = None) -> Record:
    """Serialise system prompt, state and schema; record question and option spans
    (src/deciax/models/clef/input.py:91-137)."""
    validate_questions(questions)
    if isinstance(max_length, bool) or not isinstance(max_length, int) or not 1 <= max_length <= MAX_TOKENS:
        raise ValueError(f"max_len must be between 1 and {MAX_TOKENS}")
    tok = tokenizer.encode_ids

    schema = tok("\n\nSCHEMA FIELDS:\n")
    fields = []
    for i, (qid, q) in enumerate(questions.items()):
        schema += tok(f"\nFIELD {i + 1}\nID: {qid}\nTYPE: {q['type']}\nINSTRUCTION: ")
        start = len(schema)
        instruction = q.get("instructions")
        schema += tok(qid if instruction in (None, "") else render(instruction))
        span = (start, len(schema))
        schema += tok("\nALLOWED OPTIONS:\n")
        spans, ids, labels = [], [], []
        for j, (oid, description) in enumerate(options(q)):
            schema += tok(f"OPTION {j + 1}: ")
            begin = len(schema)
            semantics = {"option_id": oid} if description is None else {"option_id": oid, "description": description}
            schema += tok(render(semantics))
            spans.append((begin, len(schema)))
            ids.append(oid)
            label_ids = tok(oid) or [0]
            labels.append(label_ids[0])
            schema += tok("\n")
        schema += tok("END FIELD\n")
        fields.append(Field(qid, QTYPES[q["type"]], span, tuple(spans), tuple(ids), tuple(labels)))

    prefix = tok(f"<|im_start|>system\n{SYSTEM_PROMPT}<|im_end|>\n<|im_start|>user\nSTATE:\n")
    suffix = tok("\n<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\nJOINT SCHEMA DECISIONS:")
    fixed = len(prefix) + len(schema) + len(suffix)
    if fixed > max_length:
        raise ValueError(f"schema requires {fixed} tokens before state; maximum is {max_length}")
    state_ids = tok(render(state))[: max_length - fixed]
    offset = len(prefix) + len(state_ids)
    shifted = tuple(
        Field(f.id, f.kind, (f.span[0] + offset, f.span[1] + offset),
              tuple((s + offset, e + offset) for s, e in f.option_spans), f.option_ids, f.option_labels)
        for f in fields)
    ids_all = tuple(prefix + state_ids + schema + suffix)
    if vocab is not None and any(not 0 <= t < vocab for t in ids_all):
        raise ValueError("token id outside the model vocabulary")
    return Record(ids_all, shifted)


def head_inputs(records: Sequence[Record], pad_id: int) -> dict[str, np.ndarray]:
    """The Clef joint head's inputs for encoded requests, in the layout and under the names of
    src/deciax/models/clef/input.py:140-182: options flat per request with the index of the field
    that owns them, and `lexical_ids` holding every option's span tokens back to back (the
    option's `lexical_spans` range in it). Shapes are the batch maxima: the reference rounds them
    up to power-of-two buckets so jit compiles once per bucket, and its padding is masked, so that
    rounding changes no output (src/deciax/runtime/buckets.py:1-3)."""
    if not records:
        raise ValueError("no records")
    b = len(records)
    s = max(len(r.ids) for r in records)
    q = max(len(r.fields) for r in records)
    o = max(sum(len(f.option_ids) for f in r.fields) for r in records)
    lex = [[t for f in r.fields for lo, hi in f.option_spans for t in r.ids[lo:hi]] for r in records]
    out = {
        "lexical_ids": np.full((b, max(1, max(map(len, lex)))), pad_id, np.int32),
        "lexical_spans": np.zeros((b, o, 2), np.int32),
        "input_ids": np.full((b, s), pad_id, np.int32),
        "mask": np.zeros((b, s), bool),
        "question_spans": np.zeros((b, q, 2), np.int32),
        "question_mask": np.zeros((b, q), bool),
        "types": np.zeros((b, q), np.int32),
        "option_spans": np.zeros((b, o, 2), np.int32),
        "option_mask": np.zeros((b, o), bool),
        "option_field": np.zeros((b, o), np.int32),
    }
    for i, r in enumerate(records):
        out["input_ids"][i, :len(r.ids)] = r.ids
        out["mask"][i, :len(r.ids)] = True
        out["lexical_ids"][i, :len(lex[i])] = lex[i]
        opt = 0      # flat option index in this request
        cursor = 0   # next free position in lexical_ids[i]
        for k, f in enumerate(r.fields):
            out["question_spans"][i, k] = f.span
            out["question_mask"][i, k] = True
            out["types"][i, k] = f.kind
            for lo, hi in f.option_spans:
                out["option_spans"][i, opt] = (lo, hi)
                out["option_mask"][i, opt] = True
                out["option_field"][i, opt] = k
                out["lexical_spans"][i, opt] = (cursor, cursor + hi - lo)
                cursor += hi - lo
                opt += 1
    return out


def readout_layout(records: Sequence[Record]) -> list[list[list[tuple[int, int]]]]:
    """options[b][q] = [(position, label), ...] for `deciax_amd.gemma.pack_batch`."""
    return [[f.readout() for f in r.fields] for r in records]


def softmax(z: np.ndarray) -> np.ndarray:
    """Max-subtracted fp32 softmax (src/deciax/protocol/answers.py:44-46)."""
    e = np.exp(z - z.max())
    return e / e.sum()


def decode(record: Record, logits: np.ndarray, questions: Mapping[str, Any], model_name: str,
           probs: np.ndarray | None = None) -> dict[str, Any]:
    """Answers for one request (src/deciax/models/clef/input.py:185-214). `logits` (and the
    per-question `probs` the readout kernel computed, when given) hold this request's options in
    field order; without `probs` the per-field softmax is taken here, as the reference does."""
    answers: dict[str, Any] = {}
    offset = 0
    for f in record.fields:
        n = len(f.option_ids)
        values = np.asarray(logits[offset:offset + n], np.float32)
        if not np.isfinite(values).all():
            raise FloatingPointError("non-finite option logits")
        field_probs = softmax(values) if probs is None else np.asarray(probs[offset:offset + n], np.float32)
        p = dict(zip(f.option_ids, field_probs.astype(np.float64).tolist(), strict=True))
        q = questions[f.id]
        if q["type"] == "noul":
            answer: dict[str, Any] = {"type": "noul", "noul": round(p["true"], 4)}
        elif q["type"] == "choice":
            keys = [str(k) for k in q["criteria"]]
            chosen = max(keys, key=p.__getitem__)
            answer = {"type": "choice", "choice": chosen, "confidence": round(p[chosen], 4),
                      "probabilities": {k: round(p[k], 4) for k in keys}}
        else:
            keys = list(f.option_ids)
            answer = {"type": "score", "score": round(sum(i * p[k] for i, k in enumerate(keys)), 4),
                      "confidence": round(max(p.values()), 4), "legend": dict(zip(keys, q["criteria"], strict=True)),
                      "probabilities": {k: round(p[k], 4) for k in keys}}
        answers[f.id] = answer
        offset += n
    return {"model": model_name, "answers": answers, "usage": {"input_tokens": len(record.ids), "output_tokens": 0}}
