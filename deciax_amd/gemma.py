"""Gemma-2-shaped decision model on one MI355X: config, device weights, forward driver.

The driver mirrors `ClefModel.forward` (src/deciax/models/clef/model.py:92-102):
embedding gather, L decoder layers, final norm, option head — with each step a
call into the gfx950 kernels:

    embed (+ layer-0 input norm)                      dx_embed
    zero the V^T tail of each sequence (once)         dx_vt_zero_tails
    per layer:
      q|k|v = h @ Wqkv^T (one GEMM), RoPE on q and k   dx_qkv_rope
        in the epilogue, V written transposed (V^T)
      causal GQA flash attention, softcap 50,          dx_attn_prefill_vt
        sliding window 4096 on even layers
      y = att @ Wo^T; x += post_attn_norm(y);          dx_linear_residual_norm
        h = pre_ffn_norm(x)
      a = gelu_tanh(h Wg^T) * (h Wu^T)                 dx_gated_linear
      y = a @ Wd^T; x += post_ffn_norm(y);             dx_linear_residual_norm
        h = next input_norm(x)
    final norm + gather + label dot + softcap 30 +
      per-question softmax                             dx_readout

Layer layout: the Gemma-2 sandwich layer (TF/models/gemma2/modeling_gemma2.py:291-335)
on the reference's fp32-norm / bf16-activation rounding points
(src/deciax/models/qwen3_5/text.py:21-28,94-102). Sequences are packed
back-to-back (varlen) rather than padded to buckets (src/deciax/runtime/buckets.py),
so no compute is spent on padding.
"""

from __future__ import annotations

import math
from collections.abc import Callable, Sequence
from dataclasses import dataclass, field

import numpy as np
import torch

from deciax_amd import kernels as K

BF16 = torch.bfloat16


@dataclass(frozen=True)
class GemmaConfig:
    """Decoder shape. `query_pre_attn_scalar ** -0.5` is the attention scale
    (TF/models/gemma2/modeling_gemma2.py:229)."""

    name: str
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    window: int = 4096
    attn_softcap: float = 50.0
    final_softcap: float = 30.0
    query_pre_attn_scalar: float = 256.0
    eps: float = 1e-6
    rope_theta: float = 10000.0
    activation: str = "gelu_tanh"
    max_position: int = 16384

    @property
    def query_scale(self) -> float:
        return float(self.query_pre_attn_scalar) ** -0.5

    @property
    def qkv_width(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def sliding(self, layer: int) -> bool:
        """Even layers are sliding-window layers (TF/models/gemma2/configuration_gemma2.py:95-97)."""
        return layer % 2 == 0

    def linear_flops_per_token(self) -> int:
        """2 x (qkv + o + gate|up + down) multiply-adds per token per layer, times layers."""
        h, d = self.hidden, self.head_dim
        per_layer = h * self.qkv_width + self.heads * d * h + 3 * h * self.intermediate
        return 2 * per_layer * self.layers

    def attention_flops(self, lengths: Sequence[int]) -> int:
        """4 D Hq x visible (query, key) pairs, summed over layers (masked pairs not counted)."""
        total = 0
        for i in range(self.layers):
            w = self.window if self.sliding(i) else 0
            for n in lengths:
                if w <= 0 or w >= n:
                    pairs = n * (n + 1) // 2
                else:
                    pairs = w * (w + 1) // 2 + (n - w) * w
                total += 4 * self.head_dim * self.heads * pairs
        return total


CONFIGS: dict[str, GemmaConfig] = {
    # 9B shape: 42 layers, H 3584, 16/8 heads x 256, MLP 14336, vocab 256000.
    "gemma2-9b": GemmaConfig("gemma2-9b", 42, 3584, 16, 8, 256, 14336, 256000, query_pre_attn_scalar=256.0),
    # 27B shape: 46 layers, H 4608, 32/16 heads x 128, scale 1/sqrt(144), MLP 36864.
    "gemma2-27b": GemmaConfig("gemma2-27b", 46, 4608, 32, 16, 128, 36864, 256000, query_pre_attn_scalar=144.0),
    # Small shape for tests: every kernel path (GQA 2, windowed and global layers) at seconds of CPU work.
    "tiny": GemmaConfig("tiny", 4, 512, 4, 2, 128, 1024, 1024, window=64, query_pre_attn_scalar=128.0,
                        max_position=4096),
}


def rope_tables(max_pos: int, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """bf16 bit patterns of cos/sin [max_pos, D/2] for positions * inv_freq with
    inv_freq = 1 / theta^(2i/D), all in fp32 before rounding (src/deciax/nn.py:31-44)."""
    inv = (np.float32(1.0) / (np.float32(theta) ** (np.arange(0, head_dim, 2, dtype=np.float32)
                                                    / np.float32(head_dim)))).astype(np.float32)
    freqs = (np.arange(max_pos, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    return _bf16_bits(np.cos(freqs)), _bf16_bits(np.sin(freqs))


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + (((u >> 16) & 1) + np.uint32(0x7FFF))) >> 16).astype(np.uint16)


def _bits_to_tensor(bits: np.ndarray, device: torch.device) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16)).view(BF16).to(device)


@dataclass
class LayerWeights:
    input_norm: torch.Tensor
    qkv: torch.Tensor            # [(Hq + 2 Hkv) D, H], rows q | k | v
    o: torch.Tensor              # [H, Hq D]
    post_attn_norm: torch.Tensor
    pre_ffn_norm: torch.Tensor
    gate_up: torch.Tensor        # [2 I, H], dx_pack_gate_up layout
    down: torch.Tensor           # [H, I]
    post_ffn_norm: torch.Tensor
    gate: torch.Tensor | None = None  # unpacked copies, kept only when requested
    up: torch.Tensor | None = None


@dataclass
class DecisionWeights:
    config: GemmaConfig
    embed: torch.Tensor          # [V, H], tied with the output head
    final_norm: torch.Tensor
    layers: list[LayerWeights]
    cos: torch.Tensor
    sin: torch.Tensor

    @property
    def device(self) -> torch.device:
        return self.embed.device

    def nbytes(self) -> int:
        n = self.embed.numel() + self.final_norm.numel()
        for lw in self.layers:
            n += sum(t.numel() for t in (lw.input_norm, lw.qkv, lw.o, lw.post_attn_norm, lw.pre_ffn_norm,
                                         lw.gate_up, lw.down, lw.post_ffn_norm))
        return 2 * n

    def numpy_weights(self) -> dict[str, np.ndarray]:
        """Host fp32 copies in the oracle's naming (for parity tests; needs unpacked gate/up)."""
        out = {"embed": _to_np(self.embed), "final_norm": _to_np(self.final_norm)}
        for i in range(len(self.layers)):
            out.update({f"layers.{i}.{k}": v for k, v in self.numpy_layer(i).items()})
        return out

    def numpy_layer(self, i: int) -> dict[str, np.ndarray]:
        """Host fp32 copies of layer i's weights under the oracle's per-layer names (one layer at a
        time, so a parity test can stream a deep model through host memory)."""
        c = self.config
        lw = self.layers[i]
        if lw.gate is None or lw.up is None:
            raise ValueError("weights were built without keep_unpacked=True")
        qd, kd = c.heads * c.head_dim, c.kv_heads * c.head_dim
        qkv = _to_np(lw.qkv)
        return {
            "input_norm": _to_np(lw.input_norm), "q": qkv[:qd], "k": qkv[qd:qd + kd], "v": qkv[qd + kd:],
            "o": _to_np(lw.o), "post_attn_norm": _to_np(lw.post_attn_norm), "pre_ffn_norm": _to_np(lw.pre_ffn_norm),
            "gate": _to_np(lw.gate), "up": _to_np(lw.up), "down": _to_np(lw.down),
            "post_ffn_norm": _to_np(lw.post_ffn_norm),
        }


def _to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float32).numpy()


def random_weights(config: GemmaConfig, *, seed: int = 0, device: str | torch.device = "cuda",
                   std: float = 0.02, norm_std: float = 0.1, keep_unpacked: bool = False) -> DecisionWeights:
    """Random-init bf16 weights, generated on the device and packed once (as the reference packs
    at load, src/deciax/models/clef/model.py:72-76). Matrices ~ N(0, std), norm weights ~ N(0, norm_std)."""
    c = config
    dev = torch.device(device)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)

    def normal(shape: tuple[int, ...], s: float) -> torch.Tensor:
        t = torch.empty(shape, dtype=BF16, device=dev)
        # Fill in row chunks so the fp32 temporary stays small.
        rows = shape[0]
        step = max(1, (1 << 26) // max(1, math.prod(shape[1:])))
        for r0 in range(0, rows, step):
            r1 = min(rows, r0 + step)
            t[r0:r1] = (torch.randn((r1 - r0, *shape[1:]), generator=gen, device=dev, dtype=torch.float32) * s).to(BF16)
        return t

    h, d = c.hidden, c.head_dim
    embed = normal((c.vocab, h), std)
    final_norm = normal((h,), norm_std)
    layers = []
    for _ in range(c.layers):
        gate = normal((c.intermediate, h), std)
        up = normal((c.intermediate, h), std)
        lw = LayerWeights(
            input_norm=normal((h,), norm_std),
            qkv=normal((c.qkv_width, h), std),
            o=normal((h, c.heads * d), std),
            post_attn_norm=normal((h,), norm_std),
            pre_ffn_norm=normal((h,), norm_std),
            gate_up=K.pack_gate_up(gate, up),
            down=normal((h, c.intermediate), std),
            post_ffn_norm=normal((h,), norm_std),
        )
        if keep_unpacked:
            lw.gate, lw.up = gate, up
        else:
            del gate, up
        layers.append(lw)
    cos, sin = rope_tables(c.max_position, d, c.rope_theta)
    return DecisionWeights(c, embed, final_norm, layers, _bits_to_tensor(cos, dev), _bits_to_tensor(sin, dev))


def weights_from_host(config: GemmaConfig, tensors: dict[str, np.ndarray | torch.Tensor], *,
                      device: str | torch.device = "cuda", keep_unpacked: bool = False) -> DecisionWeights:
    """Device weights from host arrays named as the oracle names them: `embed` [V, H], `final_norm`,
    and per layer `layers.{i}.` + input_norm, q [Hq D, H], k, v [Hkv D, H], o [H, Hq D],
    post_attn_norm, pre_ffn_norm, gate, up [I, H], down [H, I], post_ffn_norm (PyTorch [out, in]
    layout, values rounded to bf16). q|k|v and gate|up are packed once here, as the reference packs
    at load (src/deciax/models/clef/model.py:72-76, src/deciax/models/qwen3_5/pallas.py:28-59)."""
    c = config
    dev = torch.device(device)

    def dev_bf16(name: str, shape: tuple[int, ...]) -> torch.Tensor:
        if name not in tensors:
            raise ValueError(f"missing weight {name!r}")
        t = torch.as_tensor(np.asarray(tensors[name], np.float32) if not isinstance(tensors[name], torch.Tensor)
                            else tensors[name])
        if tuple(t.shape) != shape:
            raise ValueError(f"weight {name!r} has shape {tuple(t.shape)}, expected {shape}")
        return t.to(device=dev, dtype=BF16).contiguous()

    h, d = c.hidden, c.head_dim
    layers = []
    for i in range(c.layers):
        p = f"layers.{i}."
        gate = dev_bf16(p + "gate", (c.intermediate, h))
        up = dev_bf16(p + "up", (c.intermediate, h))
        lw = LayerWeights(
            input_norm=dev_bf16(p + "input_norm", (h,)),
            qkv=torch.cat([dev_bf16(p + "q", (c.heads * d, h)), dev_bf16(p + "k", (c.kv_heads * d, h)),
                           dev_bf16(p + "v", (c.kv_heads * d, h))]).contiguous(),
            o=dev_bf16(p + "o", (h, c.heads * d)),
            post_attn_norm=dev_bf16(p + "post_attn_norm", (h,)),
            pre_ffn_norm=dev_bf16(p + "pre_ffn_norm", (h,)),
            gate_up=K.pack_gate_up(gate, up),
            down=dev_bf16(p + "down", (h, c.intermediate)),
            post_ffn_norm=dev_bf16(p + "post_ffn_norm", (h,)),
        )
        if keep_unpacked:
            lw.gate, lw.up = gate, up
        layers.append(lw)
    cos, sin = rope_tables(c.max_position, d, c.rope_theta)
    return DecisionWeights(c, dev_bf16("embed", (c.vocab, h)), dev_bf16("final_norm", (h,)), layers,
                           _bits_to_tensor(cos, dev), _bits_to_tensor(sin, dev))


@dataclass
class PackedBatch:
    """A varlen batch on the device.

    Rows of every request are packed back to back: request b owns rows
    [seq_start[b], seq_start[b] + lengths[b]). Options are flat and grouped by
    question: question q owns options [q_offsets[q], q_offsets[q + 1]);
    opt_pos are global row indices, opt_label token ids."""

    lengths: list[int]
    ids: torch.Tensor
    positions: torch.Tensor
    seq_start: torch.Tensor
    seq_len: torch.Tensor
    vt_start: torch.Tensor
    vt_ld: int
    vt_col: torch.Tensor  # per row: vt_start of its sequence + its position (its V^T column)
    opt_pos: torch.Tensor
    opt_label: torch.Tensor
    q_offsets: torch.Tensor
    questions_per_request: list[int] = field(default_factory=list)
    options_per_question: list[int] = field(default_factory=list)
    # (seq_start, seq_len, vt_start) listed longest request first: the attention kernel launches
    # sequences in descriptor order, so the heaviest work starts first (outputs do not depend on it)
    by_length: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None
    q_offsets_host: tuple[int, ...] = ()  # q_offsets on the host, for validation without a device read

    @property
    def rows(self) -> int:
        return int(sum(self.lengths))

    @property
    def max_len(self) -> int:
        return max(self.lengths) if self.lengths else 0


def pack_batch(token_ids: Sequence[Sequence[int]], options: Sequence[Sequence[Sequence[tuple[int, int]]]],
               device: str | torch.device = "cuda") -> PackedBatch:
    """token_ids[b]: the request's ids; options[b][q]: (position within request, label id) per option."""
    lengths = [len(t) for t in token_ids]
    if not lengths or min(lengths) < 1:
        raise ValueError("every request needs at least one token")
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int64)
    padded = [(n + 63) // 64 * 64 for n in lengths]
    vt_start = np.concatenate([[0], np.cumsum(padded)[:-1]]).astype(np.int64)
    ids = np.concatenate([np.asarray(t, np.int64) for t in token_ids]).astype(np.int32)
    positions = np.concatenate([np.arange(n, dtype=np.int32) for n in lengths])
    opt_pos, opt_label, q_off, qpr, opq = [], [], [0], [], []
    for b, qs in enumerate(options):
        qpr.append(len(qs))
        for q in qs:
            for pos, label in q:
                if not 0 <= pos < lengths[b]:
                    raise ValueError(f"option position {pos} outside request {b} of length {lengths[b]}")
                opt_pos.append(int(starts[b]) + int(pos))
                opt_label.append(int(label))
            q_off.append(len(opt_pos))
            opq.append(len(q))
    dev = torch.device(device)

    def i32(a: Sequence[int] | np.ndarray) -> torch.Tensor:
        return torch.as_tensor(np.asarray(a, dtype=np.int64).astype(np.int32)).to(dev)

    vt_col = np.repeat(vt_start, lengths) + positions
    order = np.argsort(-np.asarray(lengths), kind="stable")
    by_length = (i32(starts[order]), i32(np.asarray(lengths)[order]), i32(vt_start[order]))
    return PackedBatch(lengths, i32(ids), i32(positions), i32(starts), i32(lengths), i32(vt_start),
                       int(sum(padded)), i32(vt_col), i32(opt_pos), i32(opt_label), K.offsets_tensor(q_off, dev), qpr, opq,
                       by_length, tuple(q_off))


class Workspace:
    """Activation buffers for one packed batch, reused across layers."""

    def __init__(self, config: GemmaConfig, rows: int, vt_ld: int, device: torch.device) -> None:
        c = config
        self.rows = rows
        self.x = torch.empty((rows, c.hidden), dtype=BF16, device=device)
        self.h = torch.empty_like(self.x)
        self.y = torch.empty_like(self.x)
        self.qkv = torch.empty((rows, c.qkv_width), dtype=BF16, device=device)
        self.att = torch.empty((rows, c.heads * c.head_dim), dtype=BF16, device=device)
        self.act = torch.empty((rows, c.intermediate), dtype=BF16, device=device)
        self.vt = torch.empty((c.kv_heads * c.head_dim, max(vt_ld, 64)), dtype=BF16, device=device)
        self.counters = K.residual_norm_counters(rows, device)  # row blocks of the fused o / down epilogues

    def fits(self, rows: int, vt_ld: int) -> bool:
        return rows <= self.rows and vt_ld <= self.vt.shape[1]


def embed_scale(hidden: int) -> float:
    """sqrt(H) rounded to bf16, the Gemma-2 normaliser (TF/models/gemma2/modeling_gemma2.py:338-349)."""
    return float(torch.tensor(math.sqrt(hidden), dtype=torch.float32).to(BF16).float())


# True folds each post-norm residual update into the o / down GEMM's epilogue
# (dx_linear_residual_norm): bit-identical to the separate GEMM + dx_add_rmsnorm, but slower at
# prefill sizes, since one workgroup per 256-row block normalises its rows after the main loop.
FUSED_NORM = False


def layer_forward(w: DecisionWeights, i: int, batch: PackedBatch, ws: Workspace) -> None:
    """One decoder layer, in place on ws.x (residual) and ws.h (normed input of the next block)."""
    c = w.config
    lw = w.layers[i]
    rows = batch.rows
    x, h, y = ws.x[:rows], ws.h[:rows], ws.y[:rows]
    qkv, att, act = ws.qkv[:rows], ws.att[:rows], ws.act[:rows]
    qd, kd = c.heads * c.head_dim, c.kv_heads * c.head_dim
    vt = ws.vt[:, :batch.vt_ld]
    K.qkv_rope(h, lw.qkv, qkv, vt, batch.positions, batch.vt_col, w.cos, w.sin, num_q_heads=c.heads,
               num_kv_heads=c.kv_heads, head_dim=c.head_dim)
    seq_start, seq_len, vt_start = batch.by_length or (batch.seq_start, batch.seq_len, batch.vt_start)
    K.attention_vt(qkv[:, :qd], qkv[:, qd:qd + kd], vt, seq_start, seq_len, vt_start, batch.max_len,
                   num_q_heads=c.heads, num_kv_heads=c.kv_heads, head_dim=c.head_dim, scale=c.query_scale,
                   softcap=c.attn_softcap, window=c.window if c.sliding(i) else 0, causal=True, out=att)
    nxt = w.layers[i + 1].input_norm if i + 1 < len(w.layers) else None
    if FUSED_NORM:
        K.linear_residual_norm(att, lw.o, y, x, lw.post_attn_norm, eps=c.eps, counters=ws.counters,
                               next_w=lw.pre_ffn_norm, h=h)
        K.gated_linear(h, lw.gate_up, c.activation, out=act)
        K.linear_residual_norm(act, lw.down, y, x, lw.post_ffn_norm, eps=c.eps, counters=ws.counters,
                               next_w=nxt, h=h if nxt is not None else None)
    else:
        K.linear(att, lw.o, out=y)
        K.add_rmsnorm(y, x, eps=c.eps, post_w=lw.post_attn_norm, next_w=lw.pre_ffn_norm, h=h)
        K.gated_linear(h, lw.gate_up, c.activation, out=act)
        K.linear(act, lw.down, out=y)
        K.add_rmsnorm(y, x, eps=c.eps, post_w=lw.post_ffn_norm, next_w=nxt, h=h if nxt is not None else None)


def forward(w: DecisionWeights, batch: PackedBatch, ws: Workspace | None = None, layers: int | None = None,
            on_layer: Callable[[int, torch.Tensor], None] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Decision forward: (option logits [O] fp32, per-question probabilities [O] fp32).

    `on_layer(i, x)`, when given, sees the residual stream x [rows, H] after the embedding (i = 0)
    and after each layer i (i = 1..L), on the current stream (parity tests read it layer by layer)."""
    c = w.config
    if batch.max_len > c.max_position:
        raise ValueError(f"request of {batch.max_len} tokens exceeds max_position {c.max_position}")
    if ws is None or not ws.fits(batch.rows, batch.vt_ld):
        ws = Workspace(c, batch.rows, batch.vt_ld, w.device)
    rows = batch.rows
    x, h = ws.x[:rows], ws.h[:rows]
    K.embed(batch.ids, w.embed, scale=embed_scale(c.hidden), norm_w=w.layers[0].input_norm, eps=c.eps, x=x, h=h)
    K.vt_zero_tails(ws.vt[:, :batch.vt_ld], batch.seq_len, batch.vt_start)
    if on_layer is not None:
        on_layer(0, x)
    n = c.layers if layers is None else layers
    for i in range(n):
        layer_forward(w, i, batch, ws)
        if on_layer is not None:
            on_layer(i + 1, x)
    return K.readout(x, w.final_norm, w.embed, batch.opt_pos, batch.opt_label, batch.q_offsets, eps=c.eps,
                     softcap=c.final_softcap, q_offsets_host=batch.q_offsets_host or None)
