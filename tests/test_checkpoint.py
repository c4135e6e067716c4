"""Checkpoint reader (deciax_amd/checkpoint.py) on the CPU.

A tiny Gemma-2 written by transformers' own `save_pretrained`, with sharded safetensors plus an
index, must read back bit-exactly under this package's names. Its config must map field by field,
and a malformed checkpoint must raise ValueError, as the reference's loader does
(src/deciax/models/clef/weights.py:81-98)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from deciax_amd import checkpoint

TINY = dict(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=32, sliding_window=64, query_pre_attn_scalar=32,
            max_position_embeddings=1024)


@pytest.fixture(scope="module")
def hf_dir(tmp_path_factory: pytest.TempPathFactory) -> tuple[Path, dict[str, torch.Tensor]]:
    from transformers import Gemma2Config, Gemma2ForCausalLM

    torch.manual_seed(0)
    model = Gemma2ForCausalLM(Gemma2Config(**TINY)).to(torch.bfloat16)
    with torch.no_grad():  # non-trivial norm weights, so a mix-up between the four norms shows
        for name, p in model.named_parameters():
            if p.ndim == 1:
                p.normal_(0.0, 0.3)
    path = tmp_path_factory.mktemp("gemma2")
    model.save_pretrained(path, max_shard_size="100KB")
    return path, {k: v.clone() for k, v in model.state_dict().items()}


def test_reads_sharded_hf_checkpoint_bit_exact(hf_dir) -> None:
    path, state = hf_dir
    assert (path / "model.safetensors.index.json").exists(), "the fixture must exercise the sharded layout"
    config, host = checkpoint.read_checkpoint(path)
    assert host["embed"].dtype == torch.bfloat16
    assert torch.equal(host["embed"], state["model.embed_tokens.weight"])
    assert torch.equal(host["final_norm"], state["model.norm.weight"])
    for i in range(config.layers):
        for hf, ours in checkpoint.LAYER_NAMES.items():
            assert torch.equal(host[f"layers.{i}.{ours}"], state[f"model.layers.{i}.{hf}"]), (i, hf)
    assert len(host) == 2 + config.layers * len(checkpoint.LAYER_NAMES)


def test_config_mapping(hf_dir) -> None:
    path, _ = hf_dir
    config, _ = checkpoint.read_checkpoint(path)
    assert (config.layers, config.hidden, config.heads, config.kv_heads, config.head_dim) == (2, 128, 4, 2, 32)
    assert (config.intermediate, config.vocab, config.window, config.max_position) == (256, 512, 64, 1024)
    assert (config.attn_softcap, config.final_softcap, config.eps, config.rope_theta) == (50.0, 30.0, 1e-6, 10000.0)
    assert config.activation == "gelu_tanh"
    assert config.query_scale == pytest.approx(32 ** -0.5)


def _write(path: Path, tensors: dict[str, torch.Tensor], config: dict) -> None:
    from safetensors.torch import save_file

    path.mkdir(parents=True, exist_ok=True)
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(path / "model.safetensors"))
    (path / "config.json").write_text(json.dumps(config))


def _hf_config(path: Path) -> dict:
    return json.loads((path / "config.json").read_text())


def test_single_file_and_tied_lm_head(hf_dir, tmp_path: Path) -> None:
    path, state = hf_dir
    tensors = dict(state)
    tensors["lm_head.weight"] = state["model.embed_tokens.weight"].clone()
    _write(tmp_path / "ok", tensors, _hf_config(path))
    config, host = checkpoint.read_checkpoint(tmp_path / "ok")
    assert torch.equal(host["layers.1.down"], state["model.layers.1.mlp.down_proj.weight"])


@pytest.mark.parametrize("case", ["extra", "missing", "untied", "layer_types", "beyond", "model_type"])
def test_rejects_malformed(hf_dir, tmp_path: Path, case: str) -> None:
    path, state = hf_dir
    tensors, cfg = dict(state), _hf_config(path)
    if case == "extra":
        tensors["model.layers.0.self_attn.q_norm.weight"] = torch.ones(32, dtype=torch.bfloat16)
    elif case == "missing":
        del tensors["model.layers.1.pre_feedforward_layernorm.weight"]
    elif case == "untied":
        tensors["lm_head.weight"] = state["model.embed_tokens.weight"] + 1
    elif case == "layer_types":
        cfg["layer_types"] = ["full_attention", "sliding_attention"]
    elif case == "beyond":
        tensors["model.layers.2.input_layernorm.weight"] = torch.ones(128, dtype=torch.bfloat16)
    elif case == "model_type":
        cfg["model_type"] = "gemma3_text"
    _write(tmp_path / case, tensors, cfg)
    with pytest.raises(ValueError):
        checkpoint.read_checkpoint(tmp_path / case)


def test_tensors_reads_f32_and_rejects_truncation(tmp_path: Path) -> None:
    from safetensors.torch import save_file

    a = torch.arange(12, dtype=torch.float32).reshape(3, 4)
    b = torch.tensor([1.5, -2.0], dtype=torch.bfloat16)
    save_file({"a": a, "b": b}, str(tmp_path / "t.safetensors"))
    got = dict(checkpoint.tensors(tmp_path / "t.safetensors"))
    assert torch.equal(got["a"], a) and torch.equal(got["b"], b)
    raw = (tmp_path / "t.safetensors").read_bytes()
    (tmp_path / "cut.safetensors").write_bytes(raw[:-4])
    with pytest.raises(ValueError):
        list(checkpoint.tensors(tmp_path / "cut.safetensors"))
    assert np.frombuffer(raw[:8], "<u8")[0] > 0
