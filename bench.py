"""Benchmark of the quantized mat-mul / KV-cache attention path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode decode|gemv]

Prints one JSON line. Default workload (mode "decode"): a random-init Llama-3-8B-shaped decoder
(32 layers, hidden 4096, GQA 32/8 x 128, SwiGLU 14336, vocab 128256, every matmul weight Q4_0,
f16 KV cache) decoding greedily after a 512-token prompt; a step is one decoded token (one launch
of the captured decode graph, inside the on-device generate loop), and `value` is decode tok/s. Mode "gemv": a step is one decoder layer's Q4_0 GEMVs at batch 1
(QKV 4096x6144, O 4096x4096, gate/up 4096x28672, down 14336x4096) over weights rotated past the
256 MB Infinity Cache; `value` is GB/s.

`roofline` is the Q4_0 batch-1 GEMV kernel (algorithmic bytes N*K/32*18 + 4K + 4N per launch)
timed with events on its stream; `cpu_baseline` is the repo's CPU oracle (a restatement of ggml's
CPU semantics, not ggml) on the host cores, on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "ggml-compiler_amd"))

METRIC = "decode tok/s (8B-shape Q4_0, 1 GPU); quant GEMV GB/s and % of HBM peak"
HBM_PEAK_GBS = 8000.0
LAYER_SHAPES = [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)]  # (K, N)
ROTATE_BYTES = 768 << 20  # > 256 MB Infinity Cache


def gemv_bytes(N: int, K: int, B: int = 1) -> int:
    return N * (K // 32) * 18 + B * K * 4 + B * N * 4


def _weights(ops, K: int, N: int, seed: int, copies: int):
    w = ops.QuantWeight.quantize(ops.fill_normal((N, K), seed=seed, std=0.02), "q4_0")
    return [w] + [ops.QuantWeight(w.type, w.N, w.K, w.data.clone()) for _ in range(copies - 1)]


def gemv_roofline(ops, torch, iters: int = 40) -> dict:
    """Average duration of the batch-1 Q4_0 GEMV kernel over the decode layer shapes, each launch
    bracketed by events on the launch stream, weights rotated past the Infinity Cache."""
    total_bytes, total_ms, n = 0, 0.0, 0
    per_shape = {}
    for K, N in LAYER_SHAPES:
        wbytes = N * (K // 32) * 18
        copies = max(2, math.ceil(ROTATE_BYTES / wbytes))
        ws = _weights(ops, K, N, seed=K + N, copies=copies)
        act = ops.quantize_act("q4_0", ops.fill_normal((1, K), seed=1))
        for i in range(copies):
            ops.mul_mat_q(ws[i], act, 1)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
        torch.cuda.synchronize()
        for i in range(iters):
            ev[i][0].record()
            ops.mul_mat_q(ws[i % copies], act, 1)
            ev[i][1].record()
        torch.cuda.synchronize()
        ms = [a.elapsed_time(b) for a, b in ev]
        avg = sum(ms) / len(ms)
        b = gemv_bytes(N, K)
        per_shape[f"{K}x{N}"] = {"us": round(avg * 1e3, 2), "GB/s": round(b / (avg * 1e-3) / 1e9, 1)}
        total_bytes += b * iters
        total_ms += sum(ms)
        n += iters
        del ws
    achieved = total_bytes / (total_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "k_gemv_q0<Q4_0, B=1> (decode layer shapes)", "avg_us": round(total_ms / n * 1e3, 2),
            "shapes": per_shape}


def cpu_gemv_baseline(seconds: float = 10.0) -> dict:
    """The CPU oracle's Q4_0 GEMV (repo restatement of ggml-cpu, OpenMP) on one layer's shapes."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as orc

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    mats = [(orc.quantize(orc.normal((N, K), seed=K + N, std=0.02), "q4_0"), K, N) for K, N in LAYER_SHAPES]
    x = {K: orc.normal((1, K), seed=1) for K, _ in LAYER_SHAPES}
    reps, t0, nbytes = 0, time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        for raw, K, N in mats:
            orc.mul_mat(raw, "q4_0", x[K], K, threads=threads)
            nbytes += gemv_bytes(N, K)
        reps += 1
    dt = time.perf_counter() - t0
    return {"value": round(nbytes / dt / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{reps} passes over one layer's four Q4_0 GEMVs (batch 1), {dt:.1f} s"}


PROMPT = 512
BYTES_PER_TOKEN_NOTE = ("weights 4,221,370,368 B (Q4_0 matmuls incl. lm_head) + embedding row 2,304 B + norm "
                        "weights 1,064,960 B + K/V 131,072 B x (p+1) + logits 513,024 B, p = position")


def decode_bytes(cfg, p: int) -> int:
    """Algorithmic HBM bytes of one decode step at position p (each weight byte read once, the K/V
    rows 0..p once, the logits written once)."""
    w = 0
    for K, N in [(cfg.n_embd, cfg.qkv_dim), (cfg.n_head * cfg.head_dim, cfg.n_embd), (cfg.n_embd, 2 * cfg.n_ff),
                 (cfg.n_ff, cfg.n_embd)]:
        w += N * (K // 32) * 18
    w = w * cfg.n_layer + cfg.n_vocab * (cfg.n_embd // 32) * 18
    norms = (2 * cfg.n_layer + 1) * cfg.n_embd * 4
    kv = cfg.n_layer * 2 * cfg.n_head_kv * cfg.head_dim * 2 * (p + 1)
    return w + (cfg.n_embd // 32) * 18 + norms + kv + cfg.n_vocab * 4


def bench_decode(args, torch) -> tuple[dict, object]:
    import numpy as np

    from ggml_compiler_amd.llm import LlamaConfig, Model

    cfg = LlamaConfig.llama3_8b(max_ctx=PROMPT + max(args.steps, args.warmup) + 64)
    m = Model(cfg, max_prompt=PROMPT)
    m.init_random(seed=0, std=0.02)
    prompt = np.random.default_rng(0).integers(0, cfg.n_vocab, PROMPT).tolist()
    # warmup: one prefill and W decode steps
    first = int(np.argmax(m.prefill(prompt)))
    m.generate(first, args.warmup)
    m.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = m.prefill(prompt)
    t_pp = time.perf_counter() - t0
    first = int(np.argmax(logits))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks = m.generate(first, args.steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    assert len(toks) == args.steps
    gb = sum(decode_bytes(cfg, PROMPT + i) for i in range(args.steps)) / args.steps
    res = {"value": round(args.steps / dt, 2), "unit": "tok/s", "ms_per_step": dt / args.steps * 1e3,
           "dtype": "q4_0 weights x q8_0 activations (int32 dots, fp32 acc), f16 KV",
           "config": {"workload": "Llama-3-8B-shaped decoder, random init N(0,0.02) -> Q4_0: 32 layers, hidden 4096, "
                                  "GQA 32/8 x 128, SwiGLU 14336, RMSNorm 1e-5, RoPE 500000, vocab 128256; "
                                  f"{PROMPT}-token uniform-random prompt, then greedy decode (one step = one token, "
                                  "on-device generate loop of graph launches)",
                      "global_batch": 1, "seq_len": PROMPT, "parallelism": "none"},
           "extra": {"pp512_tok_s": round(PROMPT / t_pp, 1), "decode_bytes_per_token": int(gb),
                     "decode_GB_s": round(gb * args.steps / dt / 1e9, 1),
                     "decode_frac_hbm_peak": round(gb * args.steps / dt / 1e9 / HBM_PEAK_GBS, 4),
                     "decode_bytes_note": BYTES_PER_TOKEN_NOTE}}
    return res, m


def cpu_decode_baseline(m, seconds: float = 15.0) -> dict:
    """The CPU oracle (repo restatement of ggml-cpu, OpenMP) decoding the same 8B-shaped model on the
    host cores: a 4-token prompt, then greedy tokens until `seconds` have passed."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import numpy as np
    from llama_ref import OracleLlama

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    w = {name: m.get_weight(name) for name, *_ in m.weights()}
    o = OracleLlama(m.cfg, w, threads=threads)
    tok = int(np.argmax(o.forward([1, 2, 3, 4])))
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        tok = int(np.argmax(o.forward([tok])))
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} greedy decode steps of the same 8B-shaped Q4_0 model after a 4-token prompt, {dt:.1f} s"}


def bench_gemv(args, ops, torch) -> dict:
    layers = []
    per_layer = sum(N * (K // 32) * 18 for K, N in LAYER_SHAPES)
    copies = max(2, math.ceil(ROTATE_BYTES / per_layer))
    for c in range(copies):
        layers.append([ops.QuantWeight.quantize(ops.fill_normal((N, K), seed=100 * c + K + N, std=0.02), "q4_0")
                       for K, N in LAYER_SHAPES])
    acts = {K: ops.quantize_act("q4_0", ops.fill_normal((1, K), seed=K)) for K, _ in LAYER_SHAPES}

    def step(i):
        for w in layers[i % copies]:
            ops.mul_mat_q(w, acts[w.K], 1)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    step_bytes = sum(gemv_bytes(N, K) for K, N in LAYER_SHAPES)
    return {"value": round(step_bytes * args.steps / dt / 1e9, 1), "unit": "GB/s", "ms_per_step": dt / args.steps * 1e3,
            "dtype": "q4_0 x q8_0 -> int32, fp32 acc",
            "config": {"workload": "Q4_0 GEMV, one Llama-3-8B layer (QKV 4096x6144, O 4096x4096, gate/up "
                                   "4096x28672, down 14336x4096), batch 1, weights rotated past 256 MB",
                       "global_batch": 1, "seq_len": 1, "parallelism": "none"}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--mode", choices=["decode", "gemv"], default="decode")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); multi-GPU sharding is design-only here.",
              file=sys.stderr)
        return 2
    args.steps = args.steps or (128 if args.mode == "decode" else 200)
    args.warmup = args.warmup if args.warmup is not None else 8

    import torch

    from ggml_compiler_amd import ops

    ops.require_device()
    torch.cuda.set_device(0)
    model = None
    if args.mode == "decode":
        res, model = bench_decode(args, torch)
    else:
        res = bench_gemv(args, ops, torch)
    line = {"metric": METRIC, "value": res["value"], "unit": res["unit"], "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(res["ms_per_step"], 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": res["dtype"], "data": "synthetic",
            "config": res["config"]}
    if "extra" in res:
        line["extra"] = res["extra"]
    line["roofline"] = gemv_roofline(ops, torch)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_decode_baseline(model) if model is not None else cpu_gemv_baseline()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
