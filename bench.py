"""Benchmark of the quantized mat-mul / KV-cache attention path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode decode|gemv|roofline|sweep|gemm|ggml]

Prints one JSON line. Default workload (mode "decode"): a random-init Llama-3-8B-shaped decoder
(32 layers, hidden 4096, GQA 32/8 x 128, SwiGLU 14336, vocab 128256, every matmul weight Q4_0,
f16 KV cache) decoding greedily after a 512-token prompt; a step is one decoded token (one launch
of the captured decode graph, inside the on-device generate loop), and `value` is decode tok/s. Mode "gemv": a step is one decoder layer's Q4_0 GEMVs at batch 1
(QKV 4096x6144, O 4096x4096, gate/up 4096x28672, down 14336x4096) over weights rotated past the
256 MB Infinity Cache; `value` is GB/s.

`roofline` is the dominant decode kernel, the row GEMV with the rms_norm + Q8_0 prologue, at the
gate/up projection's shape (algorithmic bytes N*K/32*18 + 8K + 4N per launch), 32 launches over
32 distinct weights replayed from a HIP graph between events on their stream; `traffic` comes
from the committed rocprofv3 --pmc summary. `cpu_baseline` is the repo's CPU oracle (a restatement of ggml's CPU
semantics, not ggml) on the host cores, on a bounded sample of the same workload. Mode "roofline"
runs only the roofline leg plus a 1 GiB copy (the counter calibration) for rocprofv3 --pmc.
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
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
LAYER_SHAPES = [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)]  # (K, N)
ROTATE_BYTES = 768 << 20  # > 256 MB Infinity Cache


def gemv_bytes(N: int, K: int, B: int = 1) -> int:
    return N * (K // 32) * 18 + B * K * 4 + B * N * 4


def _weights(ops, K: int, N: int, seed: int, copies: int):
    w = ops.QuantWeight.quantize(ops.fill_normal((N, K), seed=seed, std=0.02), "q4_0")
    return [w] + [ops.QuantWeight(w.type, w.N, w.K, w.data.clone()) for _ in range(copies - 1)]


# The dominant decode kernel: the row GEMV that takes an f32 row, rms-normalizes and quantizes it in
# its prologue (ggml_rms_norm -> mul -> mul_mat), at the gate/up projection's shape, the step's
# largest (a third of its time); 32 distinct weights, one per layer as in the 8B model.
ROOF_KERNEL = "k_row_gemv<Q4_0, R=2, NBL=2, PRO_NORM, EPI_STORE> (rms_norm + Q8_0 prologue, 1024 threads)"
ROOF_SHAPE = ("ffn_gate_up", 4096, 28672, 32)  # name, K, N, distinct weights
ROOF_EXTRA = [("attn_qkv", 4096, 6144, 32), ("output", 4096, 128256, 1)]
ROOF_BYTES_NOTE = "per launch: N*K/32*18 (Q4_0 weight) + 4K (x) + 4K (norm weight) + 4N (y)"
PMC_SUMMARY = ROOT / "profiles" / "k_row_gemv_norm_q4_0_gate_up_pmc.md"


def _f32_launch_bytes(K: int, N: int) -> int:
    return N * (K // 32) * 18 + 8 * K + 4 * N


def _pmc_traffic():
    """HBM bytes per launch of the roofline kernel from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy's readings), or None."""
    if not PMC_SUMMARY.exists():
        return None
    for line in PMC_SUMMARY.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1].strip())
    return None


def gemv_roofline(ops, torch, passes: int = 10, extra: bool = True) -> dict:
    """The roofline kernel (ROOF_KERNEL) at the gate/up shape: 32 launches over 32 distinct weights
    (2.1 GB, far past the 256 MB Infinity Cache) captured once in a HIP graph, `passes` replays
    bracketed by two events on the stream they run on; avg_us = elapsed / launches. With extra,
    the QKV and lm-head shapes are timed the same way (other instantiations: reported, not the
    roofline)."""
    from ggml_compiler_amd._lib import check, load

    lib = load()
    x = ops.fill_normal((1, 4096), seed=1)
    nw = ops.fill_normal((4096,), seed=2)
    ys = {}

    def weights(K, N, n):
        return [ops.QuantWeight.quantize(ops.fill_normal((N, K), seed=1000 + 7 * i + K + N, std=0.02), "q4_0")
                for i in range(n)]

    def launch(seq):
        s = ops._stream()
        for w in seq:
            if w.N not in ys:
                ys[w.N] = torch.empty(w.N, dtype=torch.float32, device="cuda")
            check(lib.gcq_rms_norm_mul_mat(w.type, ops._p(w.data), w.N, w.K, ops._p(x), ops._p(nw), 1e-5,
                                           ops._p(ys[w.N]), None, None, 0, s))

    def timed(seq):
        launch(seq)  # device queries happen before capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            launch(seq)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(passes):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (passes * len(seq))

    name, K, N, n = ROOF_SHAPE
    ws = weights(K, N, n)
    us = timed(ws)
    f_us, f_cfg = _read_floor_us(torch, [w.data.data_ptr() for w in ws], ws[0].data.numel())
    del ws
    nbytes = _f32_launch_bytes(K, N)
    achieved = nbytes / (us * 1e-6) / 1e9
    traffic = _pmc_traffic()
    out = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": ROOF_KERNEL,
           "shape": f"{name} K={K} N={N}", "avg_us": round(us, 2), "algorithmic_bytes_per_launch": nbytes,
           "bytes_note": ROOF_BYTES_NOTE, "read_floor_us": round(f_us, 2), "read_floor_cfg": f_cfg,
           "read_floor_note": "the fastest one-launch read of the same weight bytes (gcq_stream_read), timed the "
                              "same way"}
    if traffic is not None:
        out["traffic_note"] = f"HBM bytes per launch from {PMC_SUMMARY.relative_to(ROOT)}"
    if extra:
        shapes = {}
        for ename, eK, eN, en in ROOF_EXTRA:
            ews = weights(eK, eN, en)
            e_us = timed(ews)
            ef_us, _ = _read_floor_us(torch, [w.data.data_ptr() for w in ews], ews[0].data.numel())
            del ews
            shapes[f"{ename} {eK}x{eN}"] = {"us": round(e_us, 2),
                                           "GB/s": round(_f32_launch_bytes(eK, eN) / (e_us * 1e-6) / 1e9, 1),
                                           "read_floor_us": round(ef_us, 2)}
        out["other_shapes"] = shapes
    return out


def copy_calibration(torch, nbytes: int = 1 << 30) -> None:
    """A plain device copy of nbytes (reads nbytes, writes nbytes) for scaling the FETCH_SIZE /
    WRITE_SIZE counters of a --pmc run."""
    a = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()


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
    # tg128: 128 tokens from an empty context (the reference's decode protocol, llm.py:671-682)
    m.reset()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    m.generate(first, 128)
    torch.cuda.synchronize()
    tg128 = 128 / (time.perf_counter() - t1)
    gb = sum(decode_bytes(cfg, PROMPT + i) for i in range(args.steps)) / args.steps
    res = {"value": round(args.steps / dt, 2), "unit": "tok/s", "ms_per_step": dt / args.steps * 1e3,
           "dtype": "q4_0 weights x q8_0 activations (int32 dots, fp32 acc), f16 KV",
           "config": {"workload": "Llama-3-8B-shaped decoder, random init N(0,0.02) -> Q4_0: 32 layers, hidden 4096, "
                                  "GQA 32/8 x 128, SwiGLU 14336, RMSNorm 1e-5, RoPE 500000, vocab 128256; "
                                  f"{PROMPT}-token uniform-random prompt, then greedy decode (one step = one token, "
                                  "on-device generate loop of graph launches)",
                      "global_batch": 1, "seq_len": PROMPT, "parallelism": "none"},
           "extra": {"pp512_tok_s": round(PROMPT / t_pp, 1), "tg128_empty_context_tok_s": round(tg128, 2),
                     "decode_bytes_per_token": int(gb),
                     "decode_GB_s": round(gb * args.steps / dt / 1e9, 1),
                     "decode_frac_hbm_peak": round(gb * args.steps / dt / 1e9 / HBM_PEAK_GBS, 4),
                     "decode_bytes_note": BYTES_PER_TOKEN_NOTE}}
    return res, m


def bench_steps(args, torch) -> dict:
    """The decode benchmark's model, its 512-token prefill and --steps greedy decode steps, and
    nothing else: a short run whose every decode-step kernel a profiler pass can count."""
    import numpy as np

    from ggml_compiler_amd.llm import LlamaConfig, Model

    cfg = LlamaConfig.llama3_8b(max_ctx=PROMPT + max(args.steps, args.warmup) + 64)
    m = Model(cfg, max_prompt=PROMPT)
    m.init_random(seed=0, std=0.02)
    prompt = np.random.default_rng(0).integers(0, cfg.n_vocab, PROMPT).tolist()
    first = int(np.argmax(m.prefill(prompt)))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    m.generate(first, args.steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    m.close()
    return {"metric": "decode steps (profiling run)", "steps": args.steps, "ms_per_step": round(dt / args.steps * 1e3, 4)}


def bench_ggml_decode(args) -> dict:
    """The same 8B-shaped model's decode step built node by node with the ggml API
    (ggml_compiler_amd.ggml.DecodeGraph: separate q / k / v and gate / up mul_mats, rope, set_rows,
    flash_attn_ext over cache views with an f16 mask, n_kv = 768 as the reference pads it for
    positions 512..639) and run by ggml_backend_graph_compute, one host round trip per token
    (inputs set, graph replayed, logits read back, greedy argmax on the host) as the reference's
    decode entry runs (llm.py:550-634)."""
    import numpy as np

    from ggml_compiler_amd import ggml as G
    from ggml_compiler_amd.llm import LlamaConfig, Model

    cfg = LlamaConfig.llama3_8b(max_ctx=768)
    m = Model(cfg, max_prompt=16)
    m.init_random(seed=0, std=0.02)
    w = {name: m.get_weight(name) for name, *_ in m.weights()}
    m.close()
    be = G.Backend(0)
    dg = G.DecodeGraph(be, cfg, w, n_kv=768)
    del w
    prompt = np.random.default_rng(0).integers(0, cfg.n_vocab, PROMPT).tolist()
    t0 = time.perf_counter()
    for p, tok in enumerate(prompt):
        lg = dg.step(tok, p)
    t_prompt = time.perf_counter() - t0
    tok = int(np.argmax(lg))
    t0 = time.perf_counter()
    for i in range(args.steps):
        tok = int(np.argmax(dg.step(tok, PROMPT + i)))
    dt = time.perf_counter() - t0
    dg.close()
    be.close()
    return {"metric": "decode tok/s, ggml graph API (host loop)", "value": round(args.steps / dt, 2),
            "unit": "tok/s", "steps": args.steps, "ms_per_step": round(dt / args.steps * 1e3, 4),
            "prompt_tok_s_one_token_graphs": round(PROMPT / t_prompt, 1),
            "config": {"workload": f"Llama-3-8B-shaped Q4_0 decoder (random init), {PROMPT} prompt tokens fed one "
                                   f"per graph, then {args.steps} greedy tokens; n_kv 768"}}


def bench_program_decode(args, w: dict | None = None) -> dict:
    """The same 8B-shaped model as a ggml-compiler program GGUF (ggml_compiler_amd.program: the
    decode stage node for node, symbolic n_kv bound per step like llm.py:527-529), loaded by
    libgcq's loader and run as the reference's runtime runs it: the prompt through the `decode`
    entry one token per call, then the `generate` entry's loop (per step: counter, bound n_kv,
    causal mask set from the host, the decode and argmax stages, the token read back for the
    until test and collected)."""
    import tempfile

    import numpy as np

    from ggml_compiler_amd import runtime
    from ggml_compiler_amd.llm import LlamaConfig, Model
    from ggml_compiler_amd.program import write_llama_program

    import dataclasses

    from ggml_compiler_amd.ops import type_id
    from ggml_compiler_amd.program import q4_k_m_types, synthetic_weights

    cfg = LlamaConfig.llama3_8b(max_ctx=1024)
    wtype = getattr(args, "wtype", "q4_0")
    types = None
    if wtype == "q4_K_M":  # llama.cpp's Q4_K_M mix: Q4_K with Q6_K lm head, and attn_v / ffn_down in some layers
        cfg = dataclasses.replace(cfg, wtype=type_id("q4_K"))
        types = q4_k_m_types(cfg)
        w = synthetic_weights(cfg, seed=0, std=0.02, types=types)
    elif wtype != "q4_0":  # a type the fused decoder does not hold: the same stream, quantized on the GPU
        cfg = dataclasses.replace(cfg, wtype=type_id(wtype))
        w = synthetic_weights(cfg, seed=0, std=0.02)
    if w is None:  # the decode benchmark's weights (random init, seed 0)
        m = Model(cfg, max_prompt=16)
        m.init_random(seed=0, std=0.02)
        w = {name: m.get_weight(name) for name, *_ in m.weights()}
        m.close()
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, f"llama3_8b_{wtype}.gguf")
        t0 = time.perf_counter()
        write_llama_program(path, cfg, w, kv_step=256, n_gen=args.steps, types=types)
        t_write = time.perf_counter() - t0
        t0 = time.perf_counter()
        s = runtime.Session(path)
        t_load = time.perf_counter() - t0
    prompt = np.random.default_rng(0).integers(0, cfg.n_vocab, PROMPT).tolist()
    t0 = time.perf_counter()
    for p, tok in enumerate(prompt):
        n_kv = max(512, (p + 256) // 256 * 256)
        mask = np.where(np.arange(n_kv) <= p, 0.0, -np.inf).astype(np.float32).reshape(1, 1, 1, n_kv)
        lg = s.run(np.array([[tok]], np.int32), np.array([p], np.int32), mask, entry="decode")["logits"]
    t_prompt = time.perf_counter() - t0
    tok = int(np.argmax(lg))
    s.run(np.array([[tok]], np.int32), np.array([PROMPT], np.int32), entry="generate")  # warm: builds n_kv 768
    s.reset()
    for p, t in enumerate(prompt):  # the same cache state again
        n_kv = max(512, (p + 256) // 256 * 256)
        mask = np.where(np.arange(n_kv) <= p, 0.0, -np.inf).astype(np.float32).reshape(1, 1, 1, n_kv)
        s.run(np.array([[t]], np.int32), np.array([p], np.int32), mask, entry="decode")
    t0 = time.perf_counter()
    out = s.run(np.array([[tok]], np.int32), np.array([PROMPT], np.int32), entry="generate")["tokens"]
    dt = time.perf_counter() - t0
    st = s.stats
    s.close()
    return {"metric": "decode tok/s, ggml-compiler program GGUF through libgcq's loader", "value": round(args.steps / dt, 2),
            "unit": "tok/s", "steps": args.steps, "ms_per_step": round(dt / args.steps * 1e3, 4),
            "stage_calls": st["n_calls"], "first_tokens": [int(t) for t in out[:4]],
            "prompt_tok_s_decode_entry": round(PROMPT / t_prompt, 1), "write_s": round(t_write, 1),
            "load_s": round(t_load, 1),
            "config": {"workload": f"Llama-3-8B-shaped {wtype} decoder (random init) as a program GGUF, {PROMPT} prompt "
                                   f"tokens by the decode entry, then the generate entry's {args.steps} greedy steps "
                                   f"(n_kv 768)"}}


def cpu_info() -> dict:
    """The host CPU: model name, logical CPUs, and the CPUs this process may run on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), model)
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "cpus_available": len(os.sched_getaffinity(0))}


def cpu_decode_sample(m, w, threads: int, seconds: float) -> dict:
    """The CPU oracle (repo restatement of ggml-cpu, OpenMP) decoding the same 8B-shaped model at
    positions PROMPT, PROMPT + 1, ...: the prompt's K / V rows are filled with N(0, 1) f16 values
    instead of being computed (5 minutes of CPU prefill), so each step does the work of a decode step
    after a PROMPT-token prompt; greedy tokens until `seconds` have passed."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import numpy as np

    import oracle as orc
    from llama_ref import OracleLlama

    o = OracleLlama(m.cfg, w, threads=threads)
    c = m.cfg
    o.k[:, :, :PROMPT] = orc.fp32_to_fp16(orc.normal((c.n_layer, c.n_head_kv, PROMPT, c.head_dim), seed=9))
    o.v[:, :, :PROMPT] = orc.fp32_to_fp16(orc.normal((c.n_layer, c.n_head_kv, PROMPT, c.head_dim), seed=10))
    o.pos = PROMPT
    tok, n, t0 = 1, 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        tok = int(np.argmax(o.forward([tok])))
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "steps": n, "seconds": round(dt, 1)}


def cpu_config_rates(ops, m, w, threads: int, seconds: float = 0.4) -> dict:
    """The CPU oracle on C1-C4 at their shapes (one call repeated for ~`seconds`): GEMV GB/s of the
    algorithmic bytes (weight + f32 activations in and out), prefill GEMM GOP/s on a 64-row sample
    of its 512 rows, decode attention GB/s of the K/V bytes. Q4_0 weights are the model's layer-0
    matrices; Q8_0 / Q4_K ones are encoded on the GPU (bit-exact to the oracle's encoders)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as orc

    def timed(f):
        f()
        n, t0 = 0, time.perf_counter()
        while True:
            f()
            n += 1
            dt = time.perf_counter() - t0
            if dt >= seconds:
                return dt / n

    out = {}
    layer = {(4096, 6144): "blk.0.attn_qkv", (4096, 4096): "blk.0.attn_output", (4096, 28672): "blk.0.ffn_gate_up",
             (14336, 4096): "blk.0.ffn_down"}

    def gpu_encoded(t, N, K, seed):
        return ops.quantize(ops.fill_normal((N, K), seed=seed, std=0.02), t).cpu().numpy()

    raw = gpu_encoded("q8_0", 4096, 4096, 1)
    x = orc.normal((1, 4096), seed=2)
    out["C1 q8_0 K4096 N4096 B1 GB/s"] = round(gemv_bytes(4096, 4096, 1) * 34 / 18 / timed(
        lambda: orc.mul_mat(raw, "q8_0", x, 4096, threads=threads)) / 1e9, 2)
    for t in ("q4_0", "q4_K"):
        for K, N in LAYER_SHAPES:
            raw = w[layer[(K, N)]] if t == "q4_0" else gpu_encoded(t, N, K, K + N)
            wb = raw.size
            for B in (1, 8):
                x = orc.normal((B, K), seed=3)
                sec = timed(lambda: orc.mul_mat(raw, t, x, K, threads=threads))
                out[f"C2 {t} K{K} N{N} B{B} GB/s"] = round((wb + B * K * 4 + B * N * 4) / sec / 1e9, 2)
    raw = gpu_encoded("q8_0", 14336, 4096, 4)
    x = orc.normal((64, 4096), seed=5)
    sec = timed(lambda: orc.mul_mat(raw, "q8_0", x, 4096, threads=threads))
    out["C3 q8_0 K4096 N14336 (64 of 512 rows) GOP/s"] = round(2 * 64 * 14336 * 4096 / sec / 1e9, 1)
    for ctx in (512, 4096, 32768):
        q = orc.normal((32, 1, 128), seed=6)
        k16 = orc.fp32_to_fp16(orc.normal((8, ctx, 128), seed=7))
        v16 = orc.fp32_to_fp16(orc.normal((8, ctx, 128), seed=8))
        sec = timed(lambda: orc.flash_attn_ext(q, k16, v16, None, 1 / math.sqrt(128), threads=threads))
        out[f"C4 attn ctx{ctx} GB/s"] = round(2 * ctx * 8 * 128 * 2 / sec / 1e9, 2)
    return out


def cpu_baseline(ops, m, w: dict, seconds: float = 10.0) -> dict:
    """The CPU side of the line (the reference measures its CPU backend with 6 threads and with all
    cores): decode tok/s after a PROMPT-token prompt with all available cores (value) and with 6
    threads, the host CPU, and the oracle's C1-C4 rates with all cores."""
    info = cpu_info()
    cores = info["cpus_available"]
    allc = cpu_decode_sample(m, w, cores, seconds)
    six = cpu_decode_sample(m, w, min(6, cores), seconds)
    res = {"value": allc["value"], "unit": "tok/s", "cores": cores, "kind": "port",
           "sample": f"{allc['steps']} greedy decode steps of the same 8B-shaped Q4_0 model at positions "
                     f"{PROMPT}+ (prompt K/V synthetic), {allc['seconds']} s; the repo's C restatement of ggml-cpu",
           "threads_6": six, **info}
    res["configs_all_cores"] = cpu_config_rates(ops, m, w, cores)
    return res


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


def _graph_us(torch, calls, passes: int = 5) -> float:
    """Average µs per call of `calls` (a list of thunks) captured once in a HIP graph and replayed
    `passes` times between two events on the capture's stream."""
    for c in calls[:2]:
        c()  # device queries and allocator warm-up happen before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            c()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(passes):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (passes * len(calls))


FLOOR_CONFIGS = ((16, 4), (32, 4), (16, 2), (32, 1))  # (wavefronts per CU, loads in flight) of the read floor


def _read_floor_us(torch, bufs, nbytes: int, passes: int = 5) -> tuple[float, str]:
    """The fastest one-launch read of nbytes: gcq_stream_read over the rotated buffers `bufs`
    (device pointers, nbytes readable at each), timed like the kernels (a HIP graph of back-to-back
    launches, `_graph_us`), the best of FLOOR_CONFIGS; (µs, "waves/CU x loads")."""
    from ggml_compiler_amd._lib import check, load

    lib = load()
    sink = torch.zeros(64, dtype=torch.int32, device="cuda")
    best = None
    for wpc, unroll in FLOOR_CONFIGS:
        def call(b):
            check(lib.gcq_stream_read(b, nbytes, wpc, unroll, sink.data_ptr(), torch.cuda.current_stream().cuda_stream))

        us = _graph_us(torch, [lambda b=b: call(b) for b in bufs] * max(1, 64 // len(bufs)), passes)
        if best is None or us < best[0]:
            best = (us, f"{wpc}x{unroll}")
    return best


def _rotating_weights(ops, t: str, N: int, K: int, seed: int):
    """Copies of one N x K weight (N(0, 0.02) -> t) covering ROTATE_BYTES, so successive launches
    read HBM, not the 256 MB Infinity Cache."""
    w = ops.QuantWeight.quantize(ops.fill_normal((N, K), seed=seed, std=0.02), t)
    copies = max(2, math.ceil(ROTATE_BYTES / w.data.numel()))
    return [w] + [ops.QuantWeight(w.type, w.N, w.K, w.data.clone()) for _ in range(copies - 1)]


def bench_sweep(ops, torch, only: set[str] | None = None) -> list[dict]:
    """The other measured configurations (ggml_mul_mat GEMV / GEMM, decode flash_attn_ext), each
    op launched back to back from a HIP graph over inputs rotated past the Infinity Cache. only: the
    configuration names to run (C1, C2, K56, C3, C3K, C4), or all."""
    out = []

    def want(cfg):
        return only is None or cfg in only

    floors = {}  # (type, K, N) -> the read floor of the weight's bytes

    def gemv_case(cfg, t, K, N, B):
        ws = _rotating_weights(ops, t, N, K, seed=K + N)
        x = ops.fill_normal((B, K), seed=1)
        us = _graph_us(torch, [lambda w=w: ops.mul_mat(w, x) for w in ws] * max(1, 64 // len(ws)))
        wbytes = ws[0].data.numel()
        if (t, K, N) not in floors:
            floors[(t, K, N)] = _read_floor_us(torch, [w.data.data_ptr() for w in ws], wbytes)
        f_us, f_cfg = floors[(t, K, N)]
        nbytes = wbytes + B * K * 4 + B * N * 4
        out.append({"config": cfg, "op": "mul_mat", "type": t, "K": K, "N": N, "B": B, "us": round(us, 2),
                    "GB/s": round(nbytes / us / 1e3, 1), "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
                    "read_floor_us": round(f_us, 2), "read_floor_cfg": f_cfg, "floor_over_us": round(f_us / us, 3)})
        del ws

    if want("C1"):
        gemv_case("C1", "q8_0", 4096, 4096, 1)
    for t in ("q4_0", "q4_K") if want("C2") else ():
        for K, N in LAYER_SHAPES:
            for B in (1, 2, 4, 8):
                gemv_case("C2", t, K, N, B)
    # the other K-quant storage types at the same layer shapes (Q4_K_M files mix Q4_K with Q6_K)
    for t in ("q5_K", "q6_K") if want("K56") else ():
        for K, N in LAYER_SHAPES:
            for B in (1, 8):
                gemv_case("K56", t, K, N, B)
    def gemm_case(cfg, t, K, N, M):
        ws = _rotating_weights(ops, t, N, K, seed=3)[:4]
        x = ops.fill_normal((M, K), seed=4)
        us = _graph_us(torch, [lambda w=w: ops.mul_mat(w, x) for w in ws] * 4, passes=3)
        flops = 2 * M * N * K
        out.append({"config": cfg, "op": "mul_mat", "type": t, "K": K, "N": N, "M": M,
                    "us": round(us, 1), "TOP/s": round(flops / us / 1e6, 1),
                    "frac_int8_mfma": round(flops / us / 1e6 / INT8_PEAK_TOPS, 4)})
        del ws

    # C3: prefill GEMM, Q8_0 K=4096 N=14336, 512 rows (activation quantization included)
    if want("C3"):
        gemm_case("C3", "q8_0", 4096, 14336, 512)
    # the same prefill with K-quant weights: gate/up in Q4_K, Q5_K; the down projection (K 14336)
    # in Q6_K, as Q4_K_M files store it
    if want("C3K"):
        gemm_case("C3K", "q4_K", 4096, 14336, 512)
        gemm_case("C3K", "q5_K", 4096, 14336, 512)
        gemm_case("C3K", "q6_K", 14336, 4096, 512)
    # C4: decode attention, 32 q heads on 8 KV heads of 128, one query row, every key visible
    for ctx in (512, 4096, 32768) if want("C4") else ():
        kv_bytes = 2 * ctx * 8 * 128 * 2
        copies = max(2, math.ceil(ROTATE_BYTES / kv_bytes))
        k = ops.fill_normal((copies, 8, ctx, 128), seed=5).half()
        v = ops.fill_normal((copies, 8, ctx, 128), seed=6).half()
        q = ops.fill_normal((32, 1, 128), seed=7)
        calls = [lambda i=i: ops.flash_attn_ext(q, k[i], v[i], None, 1 / math.sqrt(128)) for i in range(copies)]
        us = _graph_us(torch, calls * max(1, 64 // copies))
        # the floor reads kv_bytes contiguous: K copy i and the next (the same bytes, one range)
        f_us, f_cfg = _read_floor_us(torch, [k[i].data_ptr() for i in range(copies - 1)], kv_bytes)
        nbytes = kv_bytes + 2 * 32 * 128 * 4
        out.append({"config": "C4", "op": "flash_attn_ext", "ctx": ctx, "us": round(us, 2),
                    "GB/s": round(nbytes / us / 1e3, 1), "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
                    "read_floor_us": round(f_us, 2), "read_floor_cfg": f_cfg, "floor_over_us": round(f_us / us, 3)})
        del k, v
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--mode", choices=["decode", "gemv", "roofline", "sweep", "gemm", "ggml", "program", "steps"],
                    default="decode",
                    help="roofline: only the roofline leg and a 1 GiB copy (for rocprofv3 --pmc runs); "
                         "steps: the decode model's 512-token prefill and --steps decode steps only (for counter "
                         "and kernel-trace runs of the decode kernels); "
                         "sweep: the GEMV / GEMM / attention configurations, one JSON line each; "
                         "gemm: the prefill GEMM configuration alone, --steps launches (for counter runs); "
                         "ggml: the decode step built with the ggml API and run by its graph executor; "
                         "program: the same model as a ggml-compiler program GGUF run by the loader")
    ap.add_argument("--only", default=None,
                    help="sweep: comma-separated configurations to run (C1, C2, K56, C3, C3K, C4); default all")
    ap.add_argument("--wtype", default="q4_0", choices=["q4_0", "q8_0", "q4_K", "q5_K", "q6_K", "q4_K_M"],
                    help="program: the weight type of every projection, the embedding and the lm head (q4_0: "
                         "the decode benchmark's weights; the others: synthetic_weights of that type; q4_K_M: "
                         "llama.cpp's Q4_K_M mix of Q4_K and Q6_K)")
    ap.add_argument("--type", default="q8_0", choices=["q4_0", "q8_0", "q4_K", "q5_K", "q6_K"],
                    help="gemm: the weight type")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-program", action="store_true", help="skip the program-GGUF decode figure")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); multi-GPU sharding is design-only here.",
              file=sys.stderr)
        return 2
    args.steps = args.steps or {"decode": 128, "gemv": 200, "roofline": 10, "sweep": 1, "gemm": 3,
                                "ggml": 128, "program": 128, "steps": 4}[args.mode]
    args.warmup = args.warmup if args.warmup is not None else 8

    import torch

    from ggml_compiler_amd import ops

    ops.require_device()
    torch.cuda.set_device(0)
    model = None
    if args.mode == "gemm":  # K=4096 N=14336 (Q6_K: K=14336 N=4096), 512 rows: the activation quantized once
        N, K = (4096, 14336) if args.type == "q6_K" else (14336, 4096)
        w = ops.QuantWeight.quantize(ops.fill_normal((N, K), seed=3, std=0.02), args.type)
        act = ops.quantize_act(args.type, ops.fill_normal((512, K), seed=4))
        y = torch.empty((512, N), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            ops.mul_mat_q(w, act, 512, out=y)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / args.steps
        print(json.dumps({"metric": "prefill GEMM TOP/s", "value": round(2 * 512 * N * K / us / 1e6, 1),
                          "unit": "TOP/s", "us": round(us, 1), "type": args.type}), flush=True)
        return 0
    if args.mode == "steps":
        print(json.dumps(bench_steps(args, torch)), flush=True)
        return 0
    if args.mode == "ggml":
        print(json.dumps(bench_ggml_decode(args)), flush=True)
        return 0
    if args.mode == "program":
        print(json.dumps(bench_program_decode(args)), flush=True)
        return 0
    if args.mode == "sweep":
        for r in bench_sweep(ops, torch, set(args.only.split(",")) if args.only else None):
            print(json.dumps(r), flush=True)
        return 0
    if args.mode == "roofline":
        roof = gemv_roofline(ops, torch, passes=args.steps, extra=False)
        copy_calibration(torch)
        print(json.dumps({"metric": "roofline kernel GB/s", "value": roof["achieved"], "unit": "GB/s",
                          "roofline": roof}), flush=True)
        return 0
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
    w = None
    if args.mode == "decode" and not (args.no_program and args.no_cpu):
        w = {name: model.get_weight(name) for name, *_ in model.weights()}
    if args.mode == "decode" and not args.no_program:
        # the same model as a ggml-compiler program GGUF run by libgcq's loader (the reference's
        # boundary: ggml_compiler_load + the generate entry), same step count
        prog = bench_program_decode(args, w)
        line["extra"]["program_gguf_decode_tok_s"] = prog["value"]
        line["extra"]["program_gguf_ms_per_step"] = prog["ms_per_step"]
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(ops, model, w) if model is not None else cpu_gemv_baseline()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
