"""Decision-prefill benchmark on one MI355X.

Workload (one "step"): the full 9B-shaped decision forward — 42 layers, H 3584,
16/8 GQA heads x 256, MLP 14336, vocab 256000, sliding 4096 / global
alternation, softcap 50 (final 30), random-init bf16 — over a batch of 16
requests with ragged prompt lengths drawn log-uniform in [256, 16384] and
uniform-random token ids; 8 questions per request with 2-8 options each, read
at distinct positions in the last min(L, 512) tokens. Inputs are resident in
HBM before the timed region.

Prints one JSON line: prefill tokens/s (value), decisions/s, TFLOP/s, the
attention kernel's TFLOP/s and MFMA fraction, the dominant kernel's roofline,
and the CPU oracle baseline timed on a bounded sample on this host.

`--model gemma2-27b` runs the 27B shape instead (46 layers, H 4608, 32/16 heads
x 128, MLP 36864) on 4 requests x 16384 tokens with 64 questions x 8 options
each in the last 512 tokens; the default is the 9B workload above.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from collections import defaultdict
from dataclasses import replace
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16 = 2.5e15      # MI355X dense bf16 MFMA, FLOP/s
PEAK_HBM = 8.0e12       # bytes/s
BATCH, QUESTIONS = 16, 8
LEN_LO, LEN_HI = 256, 16384


def synthetic_batch(vocab: int, seed: int = 0):
    r = np.random.Generator(np.random.PCG64(seed))
    lengths = np.rint(np.exp(r.uniform(math.log(LEN_LO), math.log(LEN_HI), BATCH))).astype(int).tolist()
    ids = [r.integers(0, vocab, n).tolist() for n in lengths]
    options = []
    for n in lengths:
        tail = min(n, 512)
        counts = r.integers(2, 9, QUESTIONS)
        pos = r.choice(np.arange(n - tail, n), size=int(counts.sum()), replace=False)
        req, used = [], 0
        for c in counts:
            req.append([(int(p), int(r.integers(0, vocab))) for p in pos[used:used + c]])
            used += int(c)
        options.append(req)
    return lengths, ids, options


def synthetic_batch_27b(vocab: int, seed: int = 0, requests: int = 4, length: int = 16384, questions: int = 64,
                        per_question: int = 8):
    """Long-context batch: `requests` x `length` tokens, `questions` x `per_question` options per request
    at distinct positions of the last questions * per_question tokens."""
    r = np.random.Generator(np.random.PCG64(seed))
    lengths = [length] * requests
    ids = [r.integers(0, vocab, length).tolist() for _ in range(requests)]
    options = []
    for n in lengths:
        pos = r.permutation(np.arange(n - questions * per_question, n))
        options.append([[(int(p), int(r.integers(0, vocab))) for p in pos[q * per_question:(q + 1) * per_question]]
                        for q in range(questions)])
    return lengths, ids, options


class KernelTimer:
    """HIP events around every kernel launch, on the stream the launch uses (torch's current
    stream): per-category launch counts and average durations over the timed steps."""

    def __init__(self, K, config) -> None:
        import torch

        self.torch = torch
        self.K = K
        self.cfg = config
        self.events: dict[str, list] = defaultdict(list)
        self.enabled = False
        self._orig = {}
        qkv_rows = config.qkv_width

        def wrap(fname, label_fn):
            orig = getattr(K, fname)
            self._orig[fname] = orig

            def inner(*args, **kwargs):
                if not self.enabled:
                    return orig(*args, **kwargs)
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                out = orig(*args, **kwargs)
                b.record()
                self.events[label_fn(args, kwargs)].append((a, b))
                return out

            setattr(K, fname, inner)

        def linear_label(args, kwargs):
            w = args[1]
            if w.shape[0] == qkv_rows:
                return "qkv_proj"
            if w.shape[1] == config.intermediate:
                return "down_proj"
            return "o_proj"

        wrap("linear", linear_label)
        wrap("linear_residual_norm",
             lambda a, k: "down_proj+norm" if a[1].shape[1] == config.intermediate else "o_proj+norm")
        wrap("gated_linear", lambda a, k: "gate_up_proj")
        wrap("attention_vt", lambda a, k: "attention_sliding" if k.get("window", 0) else "attention_global")
        wrap("add_rmsnorm", lambda a, k: "add_rmsnorm")
        wrap("qkv_rope", lambda a, k: "qkv_proj")
        wrap("vt_zero_tails", lambda a, k: "vt_zero_tails")
        wrap("embed", lambda a, k: "embed")
        wrap("readout", lambda a, k: "readout")

    def restore(self) -> None:
        for k, v in self._orig.items():
            setattr(self.K, k, v)

    def summary(self) -> dict[str, dict[str, float]]:
        out = {}
        for name, evs in self.events.items():
            ms = [a.elapsed_time(b) for a, b in evs]
            out[name] = {"launches": len(ms), "avg_ms": float(np.mean(ms)), "total_ms": float(np.sum(ms))}
        return out


def algorithmic_work(cfg, lengths: list[int]) -> dict[str, float]:
    """Algorithmic FLOPs of one launch (one layer) of each GEMM / attention category."""
    t = sum(lengths)
    h, d, hq = cfg.hidden, cfg.head_dim, cfg.heads
    # attention_flops of a one-layer config: layer 0 is a sliding layer; window 0 makes it global
    one = replace(cfg, layers=1)
    return {
        "qkv_proj": 2.0 * t * h * cfg.qkv_width,
        "o_proj": 2.0 * t * hq * d * h,
        "gate_up_proj": 2.0 * t * h * 2 * cfg.intermediate,
        "down_proj": 2.0 * t * cfg.intermediate * h,
        "o_proj+norm": 2.0 * t * hq * d * h,               # the GEMM's FLOPs; the fused residual norm adds bytes
        "down_proj+norm": 2.0 * t * cfg.intermediate * h,
        "attention_sliding": float(one.attention_flops(lengths)),
        "attention_global": float(replace(one, window=0).attention_flops(lengths)),
    }


def readout_bytes(hidden: int, options: int, questions: int) -> float:
    """Algorithmic bytes of one readout: per option its hidden row and its label's embedding row (bf16),
    its position and label (int32) and its logit and probability (fp32); the norm weights once and the
    question offsets."""
    return options * (4.0 * hidden + 16.0) + 2.0 * hidden + 4.0 * (questions + 1)


def algorithmic_bytes(cfg, lengths: list[int], options: int = 0, questions: int = 0) -> dict[str, float]:
    """Algorithmic HBM bytes of one average launch of the memory-bound kernels: add_rmsnorm reads y and
    the residual x and writes x and the next block's normed h, bf16 [T, H] each; the last of the 2 L
    launches has no next norm and writes no h. The readout as `readout_bytes`."""
    th = 2.0 * sum(lengths) * cfg.hidden
    launches = 2 * cfg.layers
    return {"add_rmsnorm": ((launches - 1) * 4 * th + 3 * th) / launches,
            "readout": readout_bytes(cfg.hidden, options, questions)}


TRAFFIC_PROFILES = {("gemma2-9b", "gate_up_proj"): ROOT / "profiles" / "gate_up_gemm_traffic.md"}


def measured_traffic(model: str, kernel: str) -> float | None:
    """HBM bytes per launch of `kernel` from its committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (counters scaled by a plain-copy calibration), or None when no such summary exists."""
    path = TRAFFIC_PROFILES.get((model, kernel))
    if path is None or not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline(cfg, seconds_budget: float = 25.0, n: int = 2048) -> dict:
    """The oracle (numpy fp32 restatement of the path, bf16 rounding points) on a bounded sample:
    one request of n tokens through one sliding and one global layer of the 9B shape plus the
    readout, up to 5 runs within the time budget; the measured FLOP rate is extrapolated to the
    full batch by its FLOP count."""
    from oracle import model as om

    try:
        from threadpoolctl import threadpool_info
        threads = max((i.get("num_threads", 1) for i in threadpool_info()), default=1)
    except Exception:  # pragma: no cover
        threads = len(os.sched_getaffinity(0))
    r = np.random.Generator(np.random.PCG64(1))
    layers = 2
    shape = om.Shape(hidden=cfg.hidden, heads=cfg.heads, kv_heads=cfg.kv_heads, head_dim=cfg.head_dim,
                     intermediate=cfg.intermediate, vocab=cfg.vocab, layers=layers, window=cfg.window,
                     query_scale=cfg.query_scale)
    from oracle.numerics import bf16

    def mat(*s):
        return bf16((r.standard_normal(s, dtype=np.float32) * np.float32(0.02)))

    vocab_rows = 4096  # the sample only gathers from these rows
    w = {"embed": mat(vocab_rows, cfg.hidden), "final_norm": mat(cfg.hidden)}
    for i in range(layers):
        p = f"layers.{i}."
        w.update({p + "input_norm": mat(cfg.hidden), p + "q": mat(cfg.heads * cfg.head_dim, cfg.hidden),
                  p + "k": mat(cfg.kv_heads * cfg.head_dim, cfg.hidden),
                  p + "v": mat(cfg.kv_heads * cfg.head_dim, cfg.hidden), p + "o": mat(cfg.hidden, cfg.heads * cfg.head_dim),
                  p + "post_attn_norm": mat(cfg.hidden), p + "pre_ffn_norm": mat(cfg.hidden),
                  p + "gate": mat(cfg.intermediate, cfg.hidden), p + "up": mat(cfg.intermediate, cfg.hidden),
                  p + "down": mat(cfg.hidden, cfg.intermediate), p + "post_ffn_norm": mat(cfg.hidden)})
    ids = r.integers(0, vocab_rows, n)
    pos = np.arange(n)
    opt_pos = np.arange(n - 40, n)
    opt_lab = r.integers(0, vocab_rows, 40)
    q_off = list(range(0, 41, 5))
    times = []
    t_end = time.perf_counter() + seconds_budget
    while len(times) < 5 and (not times or time.perf_counter() + times[-1] < t_end):
        t0 = time.perf_counter()
        x = om.forward(w, shape, ids, [0], [n], pos)
        om.readout(x, w["final_norm"], w["embed"], opt_pos, opt_lab, q_off, eps=cfg.eps, cap=cfg.final_softcap)
        times.append(time.perf_counter() - t0)
    sample_flops = n * replace(cfg, layers=layers).linear_flops_per_token() + replace(cfg, layers=layers).attention_flops([n])
    t = float(np.median(times))
    return {"flop_rate": sample_flops / t, "seconds": t, "runs": len(times), "threads": threads,
            "sample": f"1 request x {n} tokens, 1 sliding + 1 global {cfg.name}-shaped layer + readout, numpy fp32 "
                      f"oracle, median of {len(times)}; tokens/s extrapolated by FLOP count to the "
                      f"{cfg.layers}-layer batch"}


PEAK_FP32 = 157.3e12    # MI355X fp32 matrix / vector, FLOP/s


def causal_pairs(s: int, window: int = 0) -> int:
    """Visible (query, key) pairs of one causal sequence of s tokens, window 0 = global."""
    if window <= 0 or window >= s:
        return s * (s + 1) // 2
    return window * (window + 1) // 2 + (s - window) * window


def config_kernels(reps: int = 5) -> dict:
    """The single-kernel configurations beside the forward, timed with HIP events over `reps` calls
    after one warm-up call (synthetic N(0, 1) inputs scaled as below, random weights):
    - attention, fp32: batch 1 x 512, 8/4 heads x 128, causal, scale 128^-0.5, no softcap;
    - attention layer pair, bf16: batch 8 x 2048, 16/8 heads x 256, softcap 50, scale 1/16, the
      sliding layer (window 4096, inactive at 2048) plus the global layer; and one window-512 layer;
    - the 9B attention layer pair at 8K-token prompts: batch 8 x 8192, 16/8 heads x 256, scale 1/16,
      softcap 50, sliding window 4096 plus global; and the 27B pair at the same lengths (32/16 heads
      x 128, scale 1/sqrt(144));
    - fused MLP, bf16: 8192 rows, H 3584, I 14336, RMSNorm(1 + w) -> GELU-tanh gate|up -> down;
    - the 9B gate|up and down GEMMs at the benchmark batch's 70471 rows, each beside hipBLASLt
      (torch.matmul) on the same product as a yardstick;
    - the 27B readout: 2048 options (4 requests x 64 questions x 8) over 4 x 16384 rows of H 4608
      and the 256000-row embedding table.
    bf16 attention times the kernel on V already transposed (the forward's form, dx_attn_prefill_vt).
    Each entry's FLOPs are algorithmic (4 D Hq per visible pair; 6 T H I), the bytes as
    `readout_bytes`, the inputs already in HBM."""
    import torch

    from deciax_amd import kernels as K

    def timed(fn) -> float:
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        # a short GPU spin first, so the host has queued every call before the first one starts: the
        # events then bracket back-to-back kernels, not host launch gaps (which exceed the shortest
        # kernels here)
        torch.cuda._sleep(2_000_000)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    g = torch.Generator(device="cuda").manual_seed(0)
    out = {}

    def attn_case(b, s, hq, hkv, d, dtype, scale, softcap, windows):
        q = torch.randn((b * s, hq * d), generator=g, device="cuda").to(dtype) * 0.5
        k = torch.randn((b * s, hkv * d), generator=g, device="cuda").to(dtype) * 0.5
        v = torch.randn((b * s, hkv * d), generator=g, device="cuda").to(dtype) * 0.5
        starts = torch.arange(b, dtype=torch.int32, device="cuda") * s
        lens = torch.full((b,), s, dtype=torch.int32, device="cuda")
        o = torch.empty_like(q)
        kw = dict(num_q_heads=hq, num_kv_heads=hkv, head_dim=d, scale=scale, softcap=softcap, out=o)
        if dtype == torch.bfloat16:
            padded = (s + 63) // 64 * 64
            vt = torch.zeros((hkv * d, b * padded), dtype=dtype, device="cuda")
            vt_start = torch.arange(b, dtype=torch.int32, device="cuda") * padded
            K.transpose_v(v, vt, starts, lens, vt_start, s, num_kv_heads=hkv, head_dim=d)
            run = lambda w: K.attention_vt(q, k, vt, starts, lens, vt_start, s, window=w, **kw)  # noqa: E731
        else:
            run = lambda w: K.attention_varlen(q, k, v, starts, lens, s, window=w, **kw)  # noqa: E731
        ms = sum(timed(lambda w=w: run(w)) for w in windows)
        flops = sum(4.0 * d * hq * b * causal_pairs(s, w) for w in windows)
        del q, k, v, o
        return ms, flops

    ms, fl = attn_case(1, 512, 8, 4, 128, torch.float32, 128 ** -0.5, 0.0, [0])
    out["attention_fp32_1x512_8/4x128"] = {"ms": round(ms, 4), "tflops": round(fl / ms / 1e9, 2),
                                           "frac_fp32_peak": round(fl / ms * 1e3 / PEAK_FP32, 4)}
    ms, fl = attn_case(8, 2048, 16, 8, 256, torch.bfloat16, 1 / 16, 50.0, [4096, 0])
    out["attention_layer_pair_bf16_8x2048_16/8x256"] = {"ms": round(ms, 3), "tflops": round(fl / ms / 1e9, 2),
                                                        "frac_bf16_peak": round(fl / ms * 1e3 / PEAK_BF16, 4)}
    ms, fl = attn_case(8, 2048, 16, 8, 256, torch.bfloat16, 1 / 16, 50.0, [512])
    out["attention_window512_bf16_8x2048_16/8x256"] = {"ms": round(ms, 3), "tflops": round(fl / ms / 1e9, 2),
                                                       "frac_bf16_peak": round(fl / ms * 1e3 / PEAK_BF16, 4)}
    for name, hq, hkv, d, scale in (("attention_layer_pair_bf16_8x8192_16/8x256", 16, 8, 256, 1 / 16),
                                    ("attention_layer_pair_bf16_8x8192_32/16x128", 32, 16, 128, 144 ** -0.5)):
        ms, fl = attn_case(8, 8192, hq, hkv, d, torch.bfloat16, scale, 50.0, [4096, 0])
        out[name] = {"ms": round(ms, 3), "tflops": round(fl / ms / 1e9, 2),
                     "frac_bf16_peak": round(fl / ms * 1e3 / PEAK_BF16, 4)}
    t, h, f = 8192, 3584, 14336
    x = torch.randn((t, h), generator=g, device="cuda").to(torch.bfloat16)
    norm = (torch.randn((h,), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    gate_up = (torch.randn((2 * f, h), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    down = (torch.randn((h, f), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    ms = timed(lambda: K.mlp(x, norm, gate_up, down, eps=1e-6))
    fl = 6.0 * t * h * f
    out["mlp_bf16_8192x3584x14336"] = {"ms": round(ms, 3), "tflops": round(fl / ms / 1e9, 2),
                                       "frac_bf16_peak": round(fl / ms * 1e3 / PEAK_BF16, 4)}
    # the 9B forward's gate|up GEMM (70471 rows, the benchmark batch) and, as a yardstick, hipBLASLt on the
    # same product as a plain GEMM (torch.matmul, no epilogue: it writes twice the output bytes)
    t = 70471
    x = torch.randn((t, h), generator=g, device="cuda").to(torch.bfloat16)
    act = torch.empty((t, f), dtype=torch.bfloat16, device="cuda")
    fl = 2.0 * t * h * 2 * f
    ms = timed(lambda: K.gated_linear(x, gate_up, out=act))
    out["gemm_gate_up_bf16_70471x28672x3584"] = {"ms": round(ms, 3), "tflops": round(fl / ms / 1e9, 2),
                                                 "frac_bf16_peak": round(fl / ms * 1e3 / PEAK_BF16, 4)}
    del act
    plain = torch.empty((t, 2 * f), dtype=torch.bfloat16, device="cuda")
    ms = timed(lambda: torch.matmul(x, gate_up.t(), out=plain))
    out["yardstick_hipblaslt_gemm_bf16_70471x28672x3584"] = {
        "ms": round(ms, 3), "tflops": round(fl / ms / 1e9, 2), "frac_bf16_peak": round(fl / ms * 1e3 / PEAK_BF16, 4),
        "note": "torch.matmul (hipBLASLt) plain GEMM of the same shape, a yardstick only"}
    del x, gate_up, plain
    # the 9B down projection (K 14336) and hipBLASLt on the same product: both write the same bf16 output
    act = torch.randn((t, f), generator=g, device="cuda").to(torch.bfloat16)
    y = torch.empty((t, h), dtype=torch.bfloat16, device="cuda")
    fl = 2.0 * t * h * f
    ms = timed(lambda: K.linear(act, down, out=y))
    out["gemm_down_bf16_70471x3584x14336"] = {"ms": round(ms, 3), "tflops": round(fl / ms / 1e9, 2),
                                              "frac_bf16_peak": round(fl / ms * 1e3 / PEAK_BF16, 4)}
    ms = timed(lambda: torch.matmul(act, down.t(), out=y))
    out["yardstick_hipblaslt_gemm_bf16_70471x3584x14336"] = {
        "ms": round(ms, 3), "tflops": round(fl / ms / 1e9, 2), "frac_bf16_peak": round(fl / ms * 1e3 / PEAK_BF16, 4),
        "note": "torch.matmul (hipBLASLt) of the same product, a yardstick only"}
    del act, y, down
    # 27B readout: 4 requests x 16384 rows, 64 questions x 8 options in each request's last 512 rows
    h, rows, vocab, nreq, nq, per = 4608, 4 * 16384, 256000, 4, 64, 8
    hidden = torch.randn((rows, h), generator=g, device="cuda").to(torch.bfloat16)
    table = (torch.randn((vocab, h), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    fnorm = (torch.randn((h,), generator=g, device="cuda") * 0.1).to(torch.bfloat16)
    r = np.random.Generator(np.random.PCG64(0))
    pos = np.concatenate([b * 16384 + r.permutation(np.arange(16384 - nq * per, 16384)) for b in range(nreq)])
    opt_pos = torch.as_tensor(pos.astype(np.int32), device="cuda")
    opt_label = torch.as_tensor(r.integers(0, vocab, len(pos)).astype(np.int32), device="cuda")
    q_off = K.offsets_tensor(range(0, len(pos) + 1, per), "cuda")
    ms = timed(lambda: K.readout(hidden, fnorm, table, opt_pos, opt_label, q_off, eps=1e-6, softcap=30.0))
    nb = readout_bytes(h, len(pos), nreq * nq)
    out["readout_27b_2048_options"] = {"ms": round(ms, 4), "gbps": round(nb / ms / 1e6, 1),
                                       "frac_hbm_peak": round(nb / ms * 1e3 / PEAK_HBM, 4)}
    return out


def decide_batch_throughput(weights, lengths: list[int], questions_per_request: int = QUESTIONS,
                            reps: int = 3) -> dict:
    """End-to-end `decide_batch` on text requests sized like the forward's batch: the byte tokenizer's
    encoding of the prompt and schema, packing, the host-to-device copy of ids and descriptors, the
    forward, the device-to-host copy and the decode, timed on the host clock (median of `reps` after
    one warm-up call). Every request asks the same `questions_per_request` choice questions of 2-8
    options. A request's encoded length is max(L, prompt and schema + 1) for the batch length L: the
    fixed part (3256 tokens at 8 questions) exceeds the shortest lengths, so the call carries more
    tokens than the forward's batch (`tokens` in the result)."""
    from deciax_amd.engine import DecisionEngine
    from deciax_amd.schema import ByteTokenizer, encode

    cfg = weights.config
    tok = ByteTokenizer(cfg.vocab)
    questions = {f"q{i}": {"type": "choice", "criteria": {f"o{j}": f"option {j} of field {i}"
                                                          for j in range(2 + (i * 5) % 7)}}
                 for i in range(questions_per_request)}
    fixed = len(encode(tok, "", questions, vocab=cfg.vocab).ids)
    r = np.random.Generator(np.random.PCG64(7))
    letters = np.frombuffer(b"abcdefghijklmnopqrstuvwxyz ", np.uint8)
    states = [bytes(r.choice(letters, max(1, n - fixed))).decode() for n in lengths]
    engine = DecisionEngine(weights, tok, cfg.name)
    engine.decide_batch(states, questions)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        results = engine.decide_batch(states, questions)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    tokens = sum(r_["usage"]["input_tokens"] for r_ in results)
    return {"ms": round(t * 1e3, 2), "decisions_per_s": round(len(states) / t, 3),
            "tokens_per_s": round(tokens / t, 1), "tokens": tokens, "requests": len(states),
            "questions_per_request": questions_per_request,
            "scope": "encode + pack + host-to-device + forward + device-to-host + decode, host clock, median of "
                     f"{reps}"}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the single-kernel configurations")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end decide_batch timing")
    ap.add_argument("--configs-only", action="store_true",
                    help="run only the single-kernel configurations (for counter profiles) and print them")
    ap.add_argument("--model", choices=("gemma2-9b", "gemma2-27b"), default="gemma2-9b")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the decision path runs on a single GPU (data parallel over requests "
              "needs no exchange); run it with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from deciax_amd import gemma
    from deciax_amd import kernels as K

    if args.configs_only:
        print(json.dumps({"kernel_configs": config_kernels()}))
        return
    cfg = gemma.CONFIGS[args.model]
    t0 = time.time()
    weights = gemma.random_weights(cfg, seed=args.seed)
    torch.cuda.synchronize()
    print(f"# weights {weights.nbytes() / 1e9:.1f} GB in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    make = synthetic_batch if args.model == "gemma2-9b" else synthetic_batch_27b
    lengths, ids, options = make(cfg.vocab, seed=args.seed)
    n_questions = sum(len(q) for q in options)
    batch = gemma.pack_batch(ids, options)
    ws = gemma.Workspace(cfg, batch.rows, batch.vt_ld, weights.device)
    tokens = batch.rows
    print(f"# batch {len(lengths)} requests, {tokens} tokens, lengths {lengths}", file=sys.stderr, flush=True)

    timer = KernelTimer(K, cfg)
    for i in range(args.warmup):
        gemma.forward(weights, batch, ws)
        torch.cuda.synchronize()
        print(f"# warmup {i + 1}/{args.warmup} done", file=sys.stderr, flush=True)

    timer.enabled = True
    torch.cuda.synchronize()
    start = time.perf_counter()
    for i in range(args.steps):
        logits, probs = gemma.forward(weights, batch, ws)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    timer.enabled = False
    timer.restore()
    assert torch.isfinite(probs).all().item(), "non-finite probabilities"
    ms = elapsed / args.steps * 1e3
    print(f"# {args.steps} steps, {ms:.1f} ms/step", file=sys.stderr, flush=True)

    kern = timer.summary()
    work = algorithmic_work(cfg, lengths)
    n_options = sum(len(q) for req in options for q in req)
    nbytes = algorithmic_bytes(cfg, lengths, n_options, n_questions)
    total_flops = tokens * cfg.linear_flops_per_token() + cfg.attention_flops(lengths)
    per_kernel = {}
    for name, s in sorted(kern.items(), key=lambda kv: -kv[1]["total_ms"]):
        entry = dict(s)
        entry["share"] = s["total_ms"] / (ms * args.steps)
        if name in work and s["launches"]:
            entry["tflops"] = work[name] / (s["avg_ms"] * 1e-3) / 1e12
            entry["frac_bf16_peak"] = entry["tflops"] * 1e12 / PEAK_BF16
        if name in nbytes and s["launches"]:
            entry["gbps"] = nbytes[name] / (s["avg_ms"] * 1e-3) / 1e9
            entry["frac_hbm_peak"] = entry["gbps"] * 1e9 / PEAK_HBM
        per_kernel[name] = entry
    dominant = max(kern, key=lambda k: kern[k]["total_ms"])
    dom = per_kernel[dominant]
    roofline = {
        "kernel": dominant,
        "bound": "mfma",
        "achieved": round(dom.get("tflops", 0.0), 2),
        "peak": PEAK_BF16 / 1e12,
        "unit": "TFLOP/s",
        "frac": round(dom.get("frac_bf16_peak", 0.0), 4),
        "traffic": measured_traffic(cfg.name, dominant),
        "algorithmic_flop_per_launch": work.get(dominant, 0.0),
    }
    attn_ms = sum(kern[k]["total_ms"] for k in kern if k.startswith("attention")) / args.steps
    attn_flops = cfg.attention_flops(lengths)

    e2e = None
    if not args.no_e2e:
        print("# end-to-end decide_batch", file=sys.stderr, flush=True)
        e2e = decide_batch_throughput(weights, lengths)

    configs = None
    if not args.no_configs:
        print("# single-kernel configurations", file=sys.stderr, flush=True)
        configs = config_kernels()

    cpu = None
    if not args.no_cpu_baseline:
        print("# cpu baseline (oracle sample)", file=sys.stderr, flush=True)
        cb = cpu_baseline(cfg)
        cpu = {"value": round(cb["flop_rate"] / (total_flops / tokens), 2), "unit": "tokens/s",
               "cores": cb["threads"], "kind": "port", "sample": cb["sample"],
               "sample_seconds": round(cb["seconds"], 3), "extrapolated": True}

    result = {
        "metric": f"prefill tokens/s ({'9B' if args.model == 'gemma2-9b' else '27B'}-shaped decision forward, 1 GPU)",
        "value": round(tokens / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, uniform-random token ids)",
        "config": {"workload": (f"gemma2-9b-shaped decision forward, 42 layers, batch 16, lengths log-uniform "
                                f"[256, 16384] (seed {args.seed}), 8 questions x 2-8 options"
                                if args.model == "gemma2-9b" else
                                f"gemma2-27b-shaped decision forward, 46 layers, batch 4 x 16384 tokens (seed "
                                f"{args.seed}), 64 questions x 8 options per request"),
                   "tokens_per_step": tokens, "requests": len(lengths), "lengths": lengths},
        "decisions_per_s": round(len(lengths) / (ms * 1e-3), 3),
        "questions_per_s": round(n_questions / (ms * 1e-3), 2),
        "tflops": round(total_flops / (ms * 1e-3) / 1e12, 2),
        "frac_bf16_peak": round(total_flops / (ms * 1e-3) / PEAK_BF16, 4),
        "attention": {"tflops": round(attn_flops / (attn_ms * 1e-3) / 1e12, 2),
                      "frac_bf16_peak": round(attn_flops / (attn_ms * 1e-3) / PEAK_BF16, 4),
                      "ms_per_step": round(attn_ms, 2)},
        "kernels": per_kernel,
        "decide_batch": e2e,
        "kernel_configs": configs,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
