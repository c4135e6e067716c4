"""Gemma-2 checkpoints on disk (Hugging Face safetensors) -> device weights.

The counterpart of the reference's loader, src/deciax/models/clef/weights.py:26-101:

* `tensors` memory-maps one safetensors file from its JSON header. bf16 stays as raw bits
  and becomes a torch bf16 view, so no ml_dtypes is needed (the reference maps BF16 through
  ml_dtypes, weights.py:26-40).
* `read_checkpoint` walks `model.safetensors.index.json` (or the single `model.safetensors`) and
  renames tensors to the layer names of this package. It raises ValueError on an unexpected
  tensor, an incomplete checkpoint or an unsupported shape (weights.py:81-98 does the same).
* `load_weights` packs q|k|v and gate|up once and places everything on the GPU. The reference
  packs at load too (src/deciax/models/clef/model.py:72-76).

`config.json` supplies the decoder shape, `config_from_hf` maps its fields, and the
configuration the forward cannot run is rejected there.
"""

from __future__ import annotations

import json
import struct
import warnings
from collections.abc import Iterator, Mapping
from pathlib import Path
from typing import Any

import numpy as np
import torch

from deciax_amd import gemma

# safetensors dtype -> (numpy storage dtype, torch dtype it is viewed as)
_DTYPES: dict[str, tuple[Any, torch.dtype]] = {
    "BF16": (np.int16, torch.bfloat16),
    "F16": (np.float16, torch.float16),
    "F32": (np.float32, torch.float32),
}

# per-layer tensor name (after "model.layers.{i}.") -> name in DecisionWeights / weights_from_host
LAYER_NAMES = {
    "input_layernorm.weight": "input_norm",
    "self_attn.q_proj.weight": "q",
    "self_attn.k_proj.weight": "k",
    "self_attn.v_proj.weight": "v",
    "self_attn.o_proj.weight": "o",
    "post_attention_layernorm.weight": "post_attn_norm",
    "pre_feedforward_layernorm.weight": "pre_ffn_norm",
    "mlp.gate_proj.weight": "gate",
    "mlp.up_proj.weight": "up",
    "mlp.down_proj.weight": "down",
    "post_feedforward_layernorm.weight": "post_ffn_norm",
}


def tensors(path: str | Path) -> Iterator[tuple[str, torch.Tensor]]:
    """(name, host tensor) for every tensor of one safetensors file, memory-mapped read-only.

    The file is an 8-byte little-endian header length, a JSON header of
    {name: {dtype, shape, data_offsets: [begin, end]}} and the data; offsets count from the end of
    the header."""
    path = Path(path)
    size = path.stat().st_size
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: not a safetensors file")
        n = struct.unpack("<Q", raw)[0]
        if n > size - 8:
            raise ValueError(f"{path}: header length {n} exceeds the file")
        header = json.loads(f.read(n))
    base = 8 + n
    for key, entry in header.items():
        if key == "__metadata__":
            continue
        dtype = entry.get("dtype")
        if dtype not in _DTYPES:
            raise ValueError(f"{path}: tensor {key!r} has unsupported dtype {dtype!r}")
        np_dtype, torch_dtype = _DTYPES[dtype]
        shape = tuple(int(s) for s in entry["shape"])
        begin, end = (int(o) for o in entry["data_offsets"])
        count = int(np.prod(shape)) if shape else 1
        if end - begin != count * np.dtype(np_dtype).itemsize or base + end > size or begin < 0:
            raise ValueError(f"{path}: tensor {key!r} has inconsistent offsets")
        if count == 0:
            yield key, torch.empty(shape, dtype=torch_dtype)
            continue
        arr = np.memmap(path, mode="r", dtype=np_dtype, offset=base + begin, shape=shape)
        with warnings.catch_warnings():  # the map is read-only; it is only ever copied to the device
            warnings.simplefilter("ignore", UserWarning)
            t = torch.from_numpy(arr)
        yield key, t.view(torch_dtype) if torch_dtype == torch.bfloat16 else t


def config_from_hf(cfg: Mapping[str, Any], name: str = "checkpoint") -> gemma.GemmaConfig:
    """GemmaConfig from a Hugging Face Gemma-2 config.json (transformers' Gemma2Config fields)."""
    if cfg.get("model_type") != "gemma2":
        raise ValueError(f"expected a gemma2 checkpoint, got model_type {cfg.get('model_type')!r}")
    layers = int(cfg["num_hidden_layers"])
    types = cfg.get("layer_types")
    if types is not None:
        want = ["sliding_attention" if i % 2 == 0 else "full_attention" for i in range(layers)]
        if list(types) != want:
            raise ValueError("only the Gemma-2 alternation (even layers sliding, odd layers global) is supported")
    rope = cfg.get("rope_parameters") or {}
    if rope.get("rope_type", "default") != "default":
        raise ValueError(f"rope type {rope.get('rope_type')!r} is not supported")
    theta = float(rope.get("rope_theta", cfg.get("rope_theta", 10000.0)))
    act = cfg.get("hidden_activation") or cfg.get("hidden_act") or "gelu_pytorch_tanh"
    if act not in ("gelu_pytorch_tanh", "gelu_tanh", "silu"):
        raise ValueError(f"activation {act!r} is not supported")
    if cfg.get("tie_word_embeddings", True) is False:
        raise ValueError("untied output embeddings are not supported: the readout dots with the embedding table")
    hidden = int(cfg["hidden_size"])
    heads = int(cfg["num_attention_heads"])
    return gemma.GemmaConfig(
        name=name,
        layers=layers,
        hidden=hidden,
        heads=heads,
        kv_heads=int(cfg.get("num_key_value_heads", heads)),
        head_dim=int(cfg.get("head_dim") or hidden // heads),
        intermediate=int(cfg["intermediate_size"]),
        vocab=int(cfg["vocab_size"]),
        window=int(cfg.get("sliding_window") or 0),
        attn_softcap=float(cfg.get("attn_logit_softcapping") or 0.0),
        final_softcap=float(cfg.get("final_logit_softcapping") or 0.0),
        query_pre_attn_scalar=float(cfg.get("query_pre_attn_scalar") or int(cfg.get("head_dim") or hidden // heads)),
        eps=float(cfg.get("rms_norm_eps", 1e-6)),
        rope_theta=theta,
        activation="silu" if act == "silu" else "gelu_tanh",
        max_position=int(cfg.get("max_position_embeddings", 8192)),
    )


def _shard_files(path: Path) -> list[Path]:
    index = path / "model.safetensors.index.json"
    if index.exists():
        weight_map = json.loads(index.read_text())["weight_map"]
        return [path / f for f in sorted(set(weight_map.values()))]
    single = path / "model.safetensors"
    if single.exists():
        return [single]
    raise ValueError(f"{path}: no model.safetensors or model.safetensors.index.json")


def read_checkpoint(path: str | Path) -> tuple[gemma.GemmaConfig, dict[str, torch.Tensor]]:
    """Config and host tensors (memory-mapped) named as `gemma.weights_from_host` expects."""
    path = Path(path)
    if not (path / "config.json").exists():
        raise ValueError(f"{path}: no config.json")
    config = config_from_hf(json.loads((path / "config.json").read_text()), path.name)
    host: dict[str, torch.Tensor] = {}
    lm_head = None
    for file in _shard_files(path):
        for key, t in tensors(file):
            if key == "model.embed_tokens.weight":
                host["embed"] = t
            elif key == "model.norm.weight":
                host["final_norm"] = t
            elif key == "lm_head.weight":
                lm_head = t
            elif key.startswith("model.layers."):
                parts = key.split(".", 3)
                if len(parts) != 4 or not parts[2].isdigit() or parts[3] not in LAYER_NAMES:
                    raise ValueError(f"unexpected tensor {key!r}")
                layer = int(parts[2])
                if layer >= config.layers:
                    raise ValueError(f"tensor {key!r} beyond num_hidden_layers={config.layers}")
                host[f"layers.{layer}.{LAYER_NAMES[parts[3]]}"] = t
            else:
                raise ValueError(f"unexpected tensor {key!r}")
    want = {"embed", "final_norm"} | {f"layers.{i}.{n}" for i in range(config.layers) for n in LAYER_NAMES.values()}
    missing = sorted(want - set(host))
    if missing:
        raise ValueError(f"incomplete Gemma-2 checkpoint: missing {missing[:4]}{' ...' if len(missing) > 4 else ''}")
    if lm_head is not None and not torch.equal(lm_head, host["embed"]):
        raise ValueError("lm_head.weight differs from the embedding table; only tied embeddings are supported")
    return config, host


def load_weights(path: str | Path, *, device: str | torch.device = "cuda",
                 keep_unpacked: bool = False) -> gemma.DecisionWeights:
    """Device weights of a Gemma-2 checkpoint directory (config.json + safetensors)."""
    config, host = read_checkpoint(path)
    return gemma.weights_from_host(config, host, device=device, keep_unpacked=keep_unpacked)
