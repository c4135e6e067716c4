"""Decision-forward parity against the oracle, layer by layer and end to end.

Every forward check here does three things, streaming one layer's weights at a time through host
memory so that the 42- and 46-layer shapes fit:

1. Layer by layer. The GPU's residual stream after each layer is compared with the oracle's layer
   applied to the GPU's own input to that layer, with every contraction summed exactly (fp64) at
   the reference's bf16 rounding points. Each layer must agree within the bf16 output tolerance,
   2e-2 of the layer's largest value, and 1e-2 in relative L2. This pins every layer at full depth:
   a wrong but deterministic layer fails here.
2. The readout. The oracle's readout of the GPU's final hidden state must give the GPU's option
   probabilities within 1e-3 absolute, with the same argmax wherever the oracle's top-2 gap exceeds
   1e-3.
3. End to end. The GPU probabilities are compared with the oracle run freely from the embedding
   (exact sums: the truth), and the fp32 oracle's own distance from that truth is measured beside
   them. Through bf16 rounding points the two drift apart layer by layer: each 1-ulp flip of a
   rounded output, caused by a different fp32 summation order, perturbs every output of the next
   contraction in that row. At the 9B and 27B shapes with random-init weights the fp32 oracle
   itself ends 2e-2 from the truth after 42 / 46 layers (it is 4e-3 after 3 layers). So the
   end-to-end distance is recorded rather than held to 1e-3. It must stay below a gross-error
   guard of 5e-2, and the argmax must agree wherever the truth's top-2 gap exceeds twice the fp32
   oracle's drift. The reference itself measured 3.0e-3 between two of its own paths
   (docs/clef-tp.md:48) and accepts 0.02 in bf16 (tests/laya/test_parity.py:21).

Each check appends one line to `RECORDS`; conftest prints them at the end of the pytest run.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle import model as om
from oracle.numerics import F32, accumulation, bf16

LAYER_MAX_REL = 2e-2      # bf16 output tolerance, of the layer's largest |x|
LAYER_REL_L2 = 1e-2
READOUT_ABS = 1e-3        # option probabilities from the GPU's final hidden state
E2E_GUARD = 5e-2          # gross-error guard on the free-running forward (see module docstring)

RECORDS: list[str] = []


@dataclass
class ForwardParity:
    name: str
    layers: int
    worst_layer_rel_l2: float
    worst_layer_max_rel: float
    readout_err: float
    e2e_err: float
    e2e_fp32_floor: float
    argmax_agree: int
    questions: int

    def line(self) -> str:
        return (f"{self.name}: {self.layers} layers; per layer max relL2 {self.worst_layer_rel_l2:.2e}, "
                f"max |dx|/max|x| {self.worst_layer_max_rel:.2e}; readout |dp| {self.readout_err:.2e}; "
                f"end to end |p - truth| {self.e2e_err:.2e} (fp32 oracle {self.e2e_fp32_floor:.2e}); "
                f"argmax {self.argmax_agree}/{self.questions}")


def shape_of(config) -> om.Shape:
    c = config
    return om.Shape(hidden=c.hidden, heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim,
                    intermediate=c.intermediate, vocab=c.vocab, layers=c.layers, window=c.window,
                    attn_softcap=c.attn_softcap, final_softcap=c.final_softcap, query_scale=c.query_scale,
                    eps=c.eps, rope_theta=c.rope_theta, activation=c.activation)


def _top2_gap(p: np.ndarray) -> float:
    if len(p) < 2:
        return np.inf
    top = np.sort(p)[::-1]
    return float(top[0] - top[1])


def check_forward(name: str, weights, batch, rounding: str = "flash") -> ForwardParity:
    """Run the HIP forward on `batch` (weights built with keep_unpacked=True) and check it against
    the oracle as the module docstring describes. Returns the measured numbers.

    `rounding` is where the oracle's attention rounds its weights to bf16: "flash" rounds the
    unnormalised p and divides by the fp32 sum, as the kernel does; "normalized" rounds the
    normalised weights, the reference's point (src/deciax/kernels/attention/blocked.py:27)."""
    import torch

    from deciax_amd import gemma

    cfg = weights.config
    s = shape_of(cfg)
    rows = batch.rows
    xs: list[np.ndarray] = []
    logits, probs = gemma.forward(weights, batch,
                                  on_layer=lambda i, x: xs.append(x[:rows].float().cpu().numpy()))
    torch.cuda.synchronize()
    z_gpu, p_gpu = logits.cpu().numpy(), probs.cpu().numpy()
    assert np.isfinite(p_gpu).all() and np.isfinite(z_gpu).all()

    ids = batch.ids.cpu().numpy()
    starts = batch.seq_start.cpu().tolist()
    pos = batch.positions.cpu().numpy()
    opt_pos, opt_label = batch.opt_pos.cpu().numpy(), batch.opt_label.cpu().numpy()
    q_off = batch.q_offsets.cpu().tolist()
    # only the embedding rows the batch touches come to the host
    used = np.unique(np.concatenate([ids, opt_label]))
    table = weights.embed[torch.as_tensor(used, device=weights.device)].float().cpu().numpy()
    remap = np.zeros(int(used.max()) + 1, np.int64)
    remap[used] = np.arange(len(used))
    final_norm = weights.final_norm.float().cpu().numpy()
    cos, sin = om.rope_tables(int(pos.max()) + 1, s.head_dim, s.rope_theta)

    x0 = bf16(table[remap[ids]] * F32(om.embed_scale(s.hidden)))
    assert np.array_equal(x0, xs[0]), f"{name}: embedding differs from the oracle"

    def readout(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        return om.readout(x, final_norm, table, opt_pos, remap[opt_label], q_off, eps=s.eps, cap=s.final_softcap)

    truth, free32 = x0.copy(), x0.copy()
    worst_l2 = worst_max = 0.0
    for i in range(cfg.layers):
        p = weights.numpy_layer(i)
        args = (p, s, i, starts, batch.lengths, pos, cos, sin, True, rounding)
        with accumulation(np.float64):
            forced = om.layer(xs[i], *args)
            truth = om.layer(truth, *args)
        with accumulation(np.float32):
            free32 = om.layer(free32, *args)
        d = xs[i + 1] - forced
        rel_l2 = float(np.linalg.norm(d) / max(np.linalg.norm(forced), 1e-30))
        max_rel = float(np.abs(d).max() / max(np.abs(forced).max(), 1e-30))
        worst_l2, worst_max = max(worst_l2, rel_l2), max(worst_max, max_rel)
        assert rel_l2 <= LAYER_REL_L2 and max_rel <= LAYER_MAX_REL, (
            f"{name}: layer {i} differs from the oracle on the same input: relL2 {rel_l2:.2e}, "
            f"max |dx|/max|x| {max_rel:.2e}")

    z_ro, p_ro = readout(xs[-1])
    readout_err = float(np.abs(p_gpu - p_ro).max()) if len(p_gpu) else 0.0
    assert readout_err <= READOUT_ABS, f"{name}: readout differs by {readout_err:.2e}"
    _, p_truth = readout(truth)
    _, p_free32 = readout(free32)
    e2e = float(np.abs(p_gpu - p_truth).max()) if len(p_gpu) else 0.0
    floor = float(np.abs(p_free32 - p_truth).max()) if len(p_gpu) else 0.0
    agree, questions = 0, 0
    for a, b in zip(q_off[:-1], q_off[1:]):
        if b - a < 2:
            continue
        questions += 1
        same = int(np.argmax(p_gpu[a:b]) == np.argmax(p_truth[a:b]))
        agree += same
        if _top2_gap(p_ro[a:b]) > READOUT_ABS:
            assert np.argmax(p_gpu[a:b]) == np.argmax(p_ro[a:b]), f"{name}: readout argmax differs"
        if _top2_gap(p_truth[a:b]) > 2 * floor:
            assert same, f"{name}: argmax differs from the truth with top-2 gap {_top2_gap(p_truth[a:b]):.2e}"
    result = ForwardParity(name, cfg.layers, worst_l2, worst_max, readout_err, e2e, floor, agree, questions)
    RECORDS.append(result.line())
    print(result.line(), flush=True)
    assert e2e <= E2E_GUARD, f"{name}: end-to-end error {e2e:.2e} beyond the gross-error guard"
    return result
