"""Host logic on the CPU: the C-ABI library's exports, impl resolution and error mapping, schema
encode/decode (the reference's tests/clef/test_input.py cases restated for this readout), and
varlen batch packing. Nothing here launches a kernel."""

from __future__ import annotations

import ctypes
from typing import Any

import numpy as np
import pytest

from tests.conftest import rng


# ----------------------------------------------------------------------------- C ABI


def test_library_exports_every_header_symbol() -> None:
    from deciax_amd import _lib

    names = _lib.header_symbols()
    assert len(names) >= 18, names
    handle = _lib.lib()
    missing = [n for n in names if not hasattr(handle, n)]
    assert not missing, missing
    assert set(names) == set(_lib.SIGNATURES), "every declared entry point has a ctypes signature"
    assert handle.dx_version().decode().startswith("deciax-mi355x")


def test_workspace_queries_are_host_arithmetic() -> None:
    from deciax_amd import _lib

    lib = _lib.lib()
    # one 64-aligned V^T column block per sequence and kv head
    assert lib.dx_attn_prefill_workspace(3, 100, 2, 128, _lib.DX_BF16) == 128 * 3 * 2 * 128 * 2
    assert lib.dx_attn_prefill_workspace(3, 100, 2, 128, _lib.DX_F32) == 0
    assert lib.dx_norm_project_workspace(10, 512) == 10 * 512 * 2 + (-(10 * 512 * 2)) % 256
    assert lib.dx_mlp_workspace(8, 256, 512) >= 8 * 256 * 2 + 8 * 512 * 2


def test_status_codes_map_to_reference_exceptions(monkeypatch: pytest.MonkeyPatch) -> None:
    from deciax_amd import _lib

    class FakeLib:
        @staticmethod
        def dx_last_error() -> bytes:
            return b"boom"

    monkeypatch.setattr(_lib, "lib", lambda: FakeLib)
    _lib.check(_lib.DX_OK, "x")
    for code in (_lib.DX_ERR_INVALID, _lib.DX_ERR_UNSUPPORTED):
        with pytest.raises(ValueError, match="x: boom"):
            _lib.check(code, "x")
    with pytest.raises(RuntimeError, match="x: boom"):
        _lib.check(_lib.DX_ERR_RUNTIME, "x")


def test_header_constants_match_binding() -> None:
    from deciax_amd import _lib

    text = _lib.HEADER.read_text()
    for name in ("DX_OK", "DX_ERR_INVALID", "DX_ERR_UNSUPPORTED", "DX_ERR_RUNTIME", "DX_BF16", "DX_F32",
                 "DX_ACT_GELU_TANH", "DX_ACT_SILU"):
        assert f"{name} = {getattr(_lib, name)}" in text, name


def test_product_package_never_touches_the_oracle() -> None:
    """The product path has no CPU fallback: no module of deciax_amd imports the oracle."""
    import ast
    from pathlib import Path

    import deciax_amd

    for path in Path(deciax_amd.__file__).parent.rglob("*.py"):
        tree = ast.parse(path.read_text())
        for node in ast.walk(tree):
            names = []
            if isinstance(node, ast.Import):
                names = [a.name for a in node.names]
            elif isinstance(node, ast.ImportFrom):
                names = [node.module or ""]
            assert not any(n.split(".")[0] == "oracle" for n in names), f"{path} imports the oracle"


def test_missing_library_fails_loudly(monkeypatch: pytest.MonkeyPatch, tmp_path: Any) -> None:
    from deciax_amd import _lib

    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(RuntimeError, match="missing"):
        _lib.lib()
    assert isinstance(ctypes.CDLL, type)


# ----------------------------------------------------------------------------- impl seam


def test_resolve_rejects_like_the_reference() -> None:
    """Unknown impls raise ValueError (src/deciax/ops/backend.py:18); the reference's own backends are
    not served here; without a gfx950 device `hip` is refused (src/deciax/models/clef/model.py:46-50)."""
    import torch

    from deciax_amd.backend import resolve

    with pytest.raises(ValueError, match="must be"):
        resolve("cuda")  # type: ignore[arg-type]
    for impl in ("jax", "pallas"):
        with pytest.raises(ValueError, match="reference"):
            resolve(impl)  # type: ignore[arg-type]
    if not torch.cuda.is_available():
        with pytest.raises(ValueError, match="gfx950"):
            resolve("hip")


def test_load_validates_arguments() -> None:
    import deciax_amd

    with pytest.raises(ValueError, match="unknown model"):
        deciax_amd.load("clef-27b")  # type: ignore[arg-type]
    with pytest.raises(ValueError, match="revisions"):
        deciax_amd.load("tiny", revision="main")
    with pytest.raises(ValueError, match="bf16"):
        deciax_amd.load("tiny", dtype="fp32")
    with pytest.raises(ValueError):
        deciax_amd.load("tiny", impl="nope")  # type: ignore[arg-type]


def test_decider_builds_its_engine_from_the_model() -> None:
    """Decider(model) takes a RequestModel and calls model.build_engine() (src/deciax/decider.py:25-27,
    src/deciax/models/base.py:58-59); decide/decide_batch go to that engine with the budgets."""
    from deciax_amd.decider import Decider

    calls: list[tuple[Any, ...]] = []

    class Engine:
        def decide_batch(self, states, questions, *, max_len=None, head_max_len=None):
            calls.append((tuple(states), max_len, head_max_len))
            return [{"state": s} for s in states]

    class Model:
        built = 0

        def build_engine(self):
            Model.built += 1
            return Engine()

    model = Model()
    d = Decider(model)  # type: ignore[arg-type]
    assert d.model is model and Model.built == 1
    assert d.decide("s", {"q": {"type": "noul"}}, max_len=64) == {"state": "s"}
    assert d.decide_batch(["a", "b"], {"q": {"type": "noul"}}) == [{"state": "a"}, {"state": "b"}]
    assert calls == [(("s",), 64, None), (("a", "b"), None, None)]


# ----------------------------------------------------------------------------- schema


@pytest.fixture
def tokenizer() -> Any:
    from tokenizers import Tokenizer, models, pre_tokenizers

    from deciax_amd.schema import HFTokenizer

    tok = Tokenizer(models.WordLevel({"[UNK]": 0, "hello": 1, "world": 2}, unk_token="[UNK]"))
    tok.pre_tokenizer = pre_tokenizers.Whitespace()
    return HFTokenizer(tok)


QUESTIONS = {
    "sentiment": {"type": "choice", "criteria": {"z": "world", "a": "hello"}},
    "yes": {"type": "noul"},
    "score": {"type": "score", "criteria": ["hello", "world", "hello world"]},
}


def test_encode_spans_and_option_order(tokenizer: Any) -> None:
    """tests/clef/test_input.py:17-45: options sorted for choice, (true, false) for noul; spans
    inside the record; the readout position is the last token of each option span."""
    from deciax_amd.schema import encode, readout_layout

    records = [encode(tokenizer, s, QUESTIONS, 512) for s in ("hello", "hello world " * 20)]
    assert records[0].fields[0].option_ids == ("a", "z")
    assert records[0].fields[1].option_ids == ("true", "false")
    for record in records:
        for field in record.fields:
            assert field.span[0] < field.span[1] < len(record.ids)
            for (start, end), (pos, _label) in zip(field.option_spans, field.readout()):
                assert start < end <= len(record.ids) and pos == end - 1
        assert sum(len(f.option_ids) for f in record.fields) == 7
    layout = readout_layout(records)
    assert [len(q) for q in layout[0]] == [2, 2, 3]


def test_decode_kats(tokenizer: Any) -> None:
    """Zero logits -> noul 0.5 and score 1.0 (tests/clef/test_input.py:42-44); NaN ->
    FloatingPointError (:78-83); usage counts the input tokens (:44)."""
    from deciax_amd.schema import decode, encode

    record = encode(tokenizer, "hello", QUESTIONS, 512)
    result = decode(record, np.zeros(7), QUESTIONS, "tiny")
    assert result["answers"]["yes"]["noul"] == 0.5
    assert result["answers"]["score"]["score"] == 1.0
    assert result["answers"]["sentiment"]["choice"] in ("z", "a")
    assert result["usage"]["input_tokens"] == len(record.ids)
    logits = np.array([0.0, 3.0, 2.0, -2.0, 0.0, 0.0, 5.0], np.float32)
    result = decode(record, logits, QUESTIONS, "tiny")
    assert result["answers"]["sentiment"]["choice"] == "z"
    assert result["answers"]["yes"]["noul"] == pytest.approx(1 / (1 + np.exp(-4.0)), abs=1e-4)
    with pytest.raises(FloatingPointError, match="non-finite"):
        decode(encode(tokenizer, "hello", {"yes": {"type": "noul"}}, 512), np.array([np.nan, 0.0]),
               {"yes": {"type": "noul"}}, "tiny")


def test_truncation_keeps_schema_complete(tokenizer: Any) -> None:
    """tests/clef/test_input.py:48-60."""
    from deciax_amd.schema import encode

    q = {"x": {"type": "choice", "criteria": {"a": "hello", "b": "world"}}}
    fixed = encode(tokenizer, "", q, 512)
    limit = len(fixed.ids) + 5
    actual = encode(tokenizer, "hello world " * 500, q, limit)
    assert len(actual.ids) == limit
    for a, b in zip(actual.fields, fixed.fields, strict=True):
        assert a.span == (b.span[0] + 5, b.span[1] + 5)
    with pytest.raises(ValueError, match="schema requires"):
        encode(tokenizer, "", q, len(fixed.ids) - 1)


def test_prompt_text_kat() -> None:
    """The serialised prompt is part of the trained model's input contract
    (src/deciax/models/clef/input.py:98-125). With the byte tokenizer the ids decode back to the
    text, which must equal this worked example character for character; the question span
    covers the instruction and each option span its JSON semantics."""
    from deciax_amd.schema import SYSTEM_PROMPT, ByteTokenizer, encode

    tok = ByteTokenizer()
    record = encode(tok, {"b": 2, "a": "x"}, {"q": {"type": "noul"}}, 4096)
    text = bytes(t - tok.offset for t in record.ids).decode("utf-8")
    yes = '{"description":"The proposition is true or the answer is yes.","option_id":"true"}'
    no = '{"description":"The proposition is false or the answer is no.","option_id":"false"}'
    want = ("<|im_start|>system\n" + SYSTEM_PROMPT + "<|im_end|>\n<|im_start|>user\nSTATE:\n"
            '{"a":"x","b":2}'
            "\n\nSCHEMA FIELDS:\n"
            "\nFIELD 1\nID: q\nTYPE: noul\nINSTRUCTION: q\nALLOWED OPTIONS:\n"
            "OPTION 1: " + yes + "\nOPTION 2: " + no + "\nEND FIELD\n"
            "\n<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\nJOINT SCHEMA DECISIONS:")
    assert text == want
    assert SYSTEM_PROMPT == ("Read the complete state and schema. Decide every field jointly. Each answer must be "
                             "exactly one of that field's allowed options.")

    def piece(span: tuple[int, int]) -> str:
        return bytes(t - tok.offset for t in record.ids[span[0]:span[1]]).decode("utf-8")

    (field,) = record.fields
    assert piece(field.span) == "q"
    assert [piece(s) for s in field.option_spans] == [yes, no]


def test_head_inputs_layout(tokenizer: Any) -> None:
    """Joint-head inputs in the layout of src/deciax/models/clef/input.py:140-182: options flat
    with their owning field, lexical_ids holding each option's span tokens back to back."""
    from deciax_amd.schema import encode, head_inputs

    questions2 = {"only": {"type": "choice", "criteria": {"b": "world", "a": "hello"}}}
    records = [encode(tokenizer, "hello world", QUESTIONS, 512), encode(tokenizer, "hello", questions2, 512)]
    a = head_inputs(records, pad_id=tokenizer.pad_token_id)
    assert a["input_ids"].shape == a["mask"].shape == (2, max(len(r.ids) for r in records))
    assert a["question_spans"].shape == (2, 3, 2) and a["option_spans"].shape == (2, 7, 2)
    assert a["mask"].sum(1).tolist() == [len(r.ids) for r in records]
    assert a["question_mask"].tolist() == [[True] * 3, [True, False, False]]
    assert a["types"][0].tolist() == [1, 0, 2] and a["types"][1, 0] == 1
    assert a["option_mask"].sum(1).tolist() == [7, 2]
    assert a["option_field"][0].tolist() == [0, 0, 1, 1, 2, 2, 2]
    for i, r in enumerate(records):
        assert a["input_ids"][i, :len(r.ids)].tolist() == list(r.ids)
        assert (a["input_ids"][i, len(r.ids):] == tokenizer.pad_token_id).all()
        flat = [(f, s) for f in r.fields for s in f.option_spans]
        cursor = 0
        for o, (f, (lo, hi)) in enumerate(flat):
            assert tuple(a["option_spans"][i, o]) == (lo, hi)
            l0, l1 = a["lexical_spans"][i, o]
            assert (l0, l1) == (cursor, cursor + hi - lo)
            assert a["lexical_ids"][i, l0:l1].tolist() == list(r.ids[lo:hi])
            cursor = l1
        for k, f in enumerate(r.fields):
            assert tuple(a["question_spans"][i, k]) == f.span
    with pytest.raises(ValueError):
        head_inputs([], 0)


@pytest.mark.parametrize("questions", [
    {},
    {"q": {"type": []}},
    {"q": {"type": "score", "criteria": []}},
    {"q": {"type": "noul", "criteria": {"yes": "yes"}}},
    {"q": {"type": "choice", "criteria": {"a": "a"}, "option_order": ["a"]}},
    {f"q{i}": {"type": "noul"} for i in range(65)},
])
def test_invalid_schema(questions: Any) -> None:
    """tests/clef/test_input.py:63-75, plus the 64-question limit (src/deciax/protocol/systemone.py:17)."""
    from deciax_amd.schema import validate_questions

    with pytest.raises(ValueError):
        validate_questions(questions)


# ----------------------------------------------------------------------------- packing


def test_pack_batch_layout() -> None:
    from deciax_amd.gemma import pack_batch

    r = rng(0)
    lengths = [5, 64, 65, 1]
    ids = [r.integers(0, 100, n).tolist() for n in lengths]
    options = [[[(n - 1, 7), (0, 8)]] for n in lengths]
    b = pack_batch(ids, options, device="cpu")
    assert b.rows == sum(lengths) and b.max_len == 65
    np.testing.assert_array_equal(b.seq_start.numpy(), [0, 5, 69, 134])
    np.testing.assert_array_equal(b.vt_start.numpy(), [0, 64, 128, 256])
    assert b.vt_ld == 64 + 64 + 128 + 64
    np.testing.assert_array_equal(b.positions.numpy(), np.concatenate([np.arange(n) for n in lengths]))
    np.testing.assert_array_equal(b.ids.numpy(), np.concatenate(ids))
    np.testing.assert_array_equal(b.opt_pos.numpy(), [4, 0, 68, 5, 133, 69, 134, 134])
    np.testing.assert_array_equal(b.q_offsets.numpy(), [0, 2, 4, 6, 8])
    with pytest.raises(ValueError, match="outside request"):
        pack_batch([[1, 2]], [[[(2, 0)]]], device="cpu")
    with pytest.raises(ValueError, match="at least one token"):
        pack_batch([[]], [[]], device="cpu")


def test_config_flop_counts() -> None:
    """Linear FLOPs per token of the 9B shape (about 16.6 GFLOP) and the attention pair of the
    layer-pair workload (2.750e11 FLOP per layer at B8 S2048 16x256)."""
    from dataclasses import replace

    from deciax_amd.gemma import CONFIGS

    c = CONFIGS["gemma2-9b"]
    assert c.linear_flops_per_token() == pytest.approx(16.65e9, rel=1e-2)
    one = replace(c, layers=1, window=0)
    assert one.attention_flops([2048] * 8) == pytest.approx(2.750e11, rel=1e-3)
    assert c.query_scale == 1 / 16 and CONFIGS["gemma2-27b"].query_scale == pytest.approx(1 / 12)


def test_bench_refuses_several_gpus() -> None:
    """bench.py measures one MI355X: --gpus above 1 exits with a message before touching a GPU."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    res = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120, cwd=root)
    assert res.returncode == 2
    assert "--gpus 1" in res.stderr and res.stdout == ""


def test_bench_causal_pairs() -> None:
    """The visible-pair count behind the single-kernel configurations' FLOPs: brute force on small
    sequences, and the attention-layer figures the benchmark reports at 8 x 2048."""
    import bench

    for s in (1, 2, 7, 64, 65):
        for w in (0, 1, 3, 64, 100):
            want = sum(1 for i in range(s) for j in range(i + 1) if w <= 0 or i - j < w)
            assert bench.causal_pairs(s, w) == want, (s, w)
    assert bench.causal_pairs(2048) == 2_098_176
    assert bench.causal_pairs(2048, 4096) == 2_098_176
    assert bench.causal_pairs(2048, 512) == 917_760
    assert 4 * 256 * 16 * 8 * bench.causal_pairs(2048) == 275_012_124_672  # 2.750e11 FLOP per layer


def test_pack_batch_longest_first_descriptors() -> None:
    """The attention kernel launches sequences in descriptor order; the driver hands it the packed
    batch's (seq_start, seq_len, vt_start) listed longest first (stable among equal lengths), each
    triple unchanged."""
    from deciax_amd.gemma import pack_batch

    b = pack_batch([[1] * 5, [2] * 70, [3] * 70, [4] * 1], [[], [], [], []], device="cpu")
    ss, sl, vs = b.by_length
    order = [1, 2, 0, 3]
    assert sl.tolist() == [70, 70, 5, 1]
    assert ss.tolist() == [b.seq_start.tolist()[i] for i in order]
    assert vs.tolist() == [b.vt_start.tolist()[i] for i in order]


def test_bench_norm_bytes() -> None:
    """add_rmsnorm's algorithmic bytes: 4 bf16 [T, H] tensors per launch, 3 in the last of 2 L."""
    import bench
    from deciax_amd.gemma import CONFIGS

    cfg = CONFIGS["gemma2-9b"]
    t = 70471
    per = bench.algorithmic_bytes(cfg, [t])["add_rmsnorm"]
    assert per * 84 == 83 * 4 * 2 * t * 3584 + 3 * 2 * t * 3584


def test_flash_attention_rejects_bad_shapes() -> None:
    """The packed flash interface checks its shapes before any device work (ValueError where the
    reference TPU kernel asserts, src/deciax/kernels/attention/pallas.py:70,73)."""
    import torch

    from deciax_amd import kernels as K

    qkv = torch.zeros((2, 16, 3 * 2 * 64), dtype=torch.bfloat16)
    mask = torch.ones((2, 16), dtype=torch.int32)
    with pytest.raises(ValueError, match="width"):
        K.flash_attention(qkv, mask, heads=3)
    with pytest.raises(ValueError, match="mask"):
        K.flash_attention(qkv, mask[:, :8], heads=2)
    with pytest.raises(ValueError, match="window"):
        K.flash_attention(qkv, mask, heads=2, window=-1)
    with pytest.raises(ValueError, match="out_dtype"):
        K.flash_attention(qkv, mask, heads=2, out_dtype=torch.float32)
    with pytest.raises(ValueError, match="qkv"):
        K.flash_attention(qkv[0], mask, heads=2)


def test_offsets_registry_pairs_tensors_with_their_host_values() -> None:
    """offsets_tensor remembers the host values a tensor was built from (so the readout validates
    without a device read); other tensors, and tensors that are gone, are not known."""
    import gc

    import torch

    from deciax_amd import kernels as K

    t = K.offsets_tensor([0, 3, 5, 9], "cpu")
    assert t.dtype == torch.int32 and t.tolist() == [0, 3, 5, 9]
    assert K.known_offsets(t) == (0, 3, 5, 9)
    assert K.known_offsets(t.clone()) is None
    assert K.known_offsets(torch.tensor([0, 3, 5, 9], dtype=torch.int32)) is None
    key = id(t)
    del t
    gc.collect()
    assert key not in K._OFFSETS
