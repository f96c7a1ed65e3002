"""ggml-compiler program GGUFs for a Llama-style decoder, written without the reference compiler.

The reference compiles a model into a GGUF whose "ggml_compiler.program" JSON (format 3,
ggml_compiler/emit/gguf_runtime.py:104-207) the runtime interprets: values with innermost-first
`ne`, stages of ggml-level nodes, entry points with call / loop drivers, state, symbols. This module
writes that format for the decode step of a Llama-style causal LM, node for node the graph
`ggml.DecodeGraph` builds (the reference's decode stage, ggml_compiler/llm.py:361-444), so a
model can be loaded and run by libgcq's loader (`runtime.Session`, include/ggml_compiler_rt.h)
as a reference-produced file would be:

- symbol `n_kv` in [kv_step, max_ctx]: the attended cache length, bound per step from the
  position like the reference's `n_kv = max(512, ceil(end / 256) * 256)` (llm.py:527-529), with
  kv_step in place of 256 and 512;
- stage `decode` (token, pos, mask, the caches) -> (logits, the caches written in place) and stage
  `pick` (argmax of the logits);
- entry `decode`: one call; entry `generate`: a loop of `n_gen` steps over counter `pos` from
  `start` that binds n_kv, fills the causal mask, calls decode and pick, collects each token into
  `tokens` and stops at an end-of-sequence id (llm.py:421-436).
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

from . import gguf

F32, F16, I32 = "f32", "f16", "i32"
TYPE_NAMES = {0: "f32", 1: "f16", 2: "q4_0", 8: "q8_0", 12: "q4_K", 13: "q5_K", 14: "q6_K"}


def _split_weights(cfg, weights: dict[str, np.ndarray]) -> dict[str, np.ndarray]:
    """HIP-model weight names (stacked q/k/v and gate/up rows) -> the separate tensors the
    reference's graph multiplies by."""
    from . import ggml as G

    H, Hkv, D, E, F = cfg.n_head, cfg.n_head_kv, cfg.head_dim, cfg.n_embd, cfg.n_ff
    if "blk.0.attn_q" in weights:  # already the GGUF's separate tensors
        return weights
    row = int(G.lib().ggml_row_size(cfg.wtype, E))
    out = {"token_embd": weights["token_embd"], "output_norm": weights["output_norm"], "output": weights["output"]}
    for l in range(cfg.n_layer):
        b = f"blk.{l}."
        qkv = weights[b + "attn_qkv"].reshape(-1, row)
        out[b + "attn_q"] = qkv[: H * D]
        out[b + "attn_k"] = qkv[H * D: (H + Hkv) * D]
        out[b + "attn_v"] = qkv[(H + Hkv) * D:]
        gu = weights[b + "ffn_gate_up"].reshape(-1, row)
        out[b + "ffn_gate"] = gu[:F]
        out[b + "ffn_up"] = gu[F:]
        for k in ("attn_norm", "attn_output", "ffn_norm", "ffn_down"):
            out[b + k] = weights[b + k]
    return out


class _Stage:
    def __init__(self, name: str) -> None:
        self.name, self.params, self.nodes, self.outputs = name, [], [], []

    def param(self, typ: str, ne: list, shape: list) -> str:
        name = f"a.{len(self.params)}"
        self.params.append({"name": name, "type": typ, "ne": ne, "shape": shape})
        return name

    def node(self, op: str, src: list[str], typ: str, ne: list, **p) -> str:
        nid = f"%{len(self.nodes)}"
        self.nodes.append({"id": nid, "op": op, "src": src, "type": typ, "ne": list(ne) + [1] * (4 - len(ne)),
                           "p": p, "loc": f"decoder.{op}"})
        return nid

    def json(self) -> dict:
        return {"name": self.name, "params": self.params, "outputs": self.outputs, "nodes": self.nodes}


def llama_program(cfg, kv_step: int = 256, n_gen: int = 128, eos: tuple[int, ...] = ()) -> tuple[dict, dict[str, str]]:
    """The program JSON and the GGUF tensor name of each weight (w.N)."""
    H, Hkv, D, E, F, V, C = (cfg.n_head, cfg.n_head_kv, cfg.head_dim, cfg.n_embd, cfg.n_ff, cfg.n_vocab,
                             cfg.max_ctx)
    if not (0 < kv_step <= C):
        raise ValueError("kv_step must be in [1, max_ctx]")
    wtype = TYPE_NAMES[cfg.wtype]
    wname: dict[str, str] = {}

    def w(name: str) -> str:
        if name not in wname:
            wname[name] = f"w.{len(wname)}"
        return wname[name]

    st = _Stage("decode")
    tok = st.param(I32, [1, 1, 1, 1], [1, 1])
    pos = st.param(I32, [1, 1, 1, 1], [1])
    mask = st.param(F32, ["n_kv", 1, 1, 1], [1, 1, 1, "n_kv"])
    caches = []
    for l in range(cfg.n_layer):
        caches.append((st.param(F16, [D, C, Hkv, 1], [Hkv, C, D]), st.param(F16, [D, C, Hkv, 1], [Hkv, C, D])))
    x = st.node("get_rows", [w("token_embd"), tok], F32, [E, 1])
    m16 = st.node("cast", [mask], F16, ["n_kv", 1])
    written = []
    for l in range(cfg.n_layer):
        b = f"blk.{l}."
        n = st.node("mul", [st.node("rms_norm", [x], F32, [E, 1], eps=cfg.rms_eps), w(b + "attn_norm")], F32, [E, 1])
        q = st.node("mul_mat", [w(b + "attn_q"), n], F32, [H * D, 1], acc=1)
        k = st.node("mul_mat", [w(b + "attn_k"), n], F32, [Hkv * D, 1], acc=1)
        v = st.node("mul_mat", [w(b + "attn_v"), n], F32, [Hkv * D, 1], acc=1)
        rope = dict(n_dims=D, mode=2, freq_base=cfg.rope_base, freq_scale=1.0, attn_factor=1.0)
        q = st.node("rope", [st.node("reshape", [q], F32, [D, H, 1]), pos], F32, [D, H, 1], **rope)
        k = st.node("rope", [st.node("reshape", [k], F32, [D, Hkv, 1]), pos], F32, [D, Hkv, 1], **rope)
        v = st.node("reshape", [v], F32, [D, Hkv, 1])
        kc, vc = caches[l]
        kw = st.node("set_rows", [kc, st.node("permute", [k], F32, [D, 1, Hkv], axes=[0, 2, 1, 3]), pos], F16,
                     [D, C, Hkv])
        vw = st.node("set_rows", [vc, st.node("permute", [v], F32, [D, 1, Hkv], axes=[0, 2, 1, 3]), pos], F16,
                     [D, C, Hkv])
        written += [kw, vw]
        kv = st.node("view", [kw], F16, [D, "n_kv", Hkv], dim=1, start=0)
        vv = st.node("view", [vw], F16, [D, "n_kv", Hkv], dim=1, start=0)
        qp = st.node("permute", [q], F32, [D, 1, H], axes=[0, 2, 1, 3])
        att = st.node("flash_attn", [qp, kv, vv, m16], F32, [D, H, 1], scale=1.0 / math.sqrt(D))
        o = st.node("mul_mat", [w(b + "attn_output"), st.node("reshape", [att], F32, [D * H, 1])], F32, [E, 1], acc=1)
        x = st.node("add", [x, o], F32, [E, 1])
        n = st.node("mul", [st.node("rms_norm", [x], F32, [E, 1], eps=cfg.rms_eps), w(b + "ffn_norm")], F32, [E, 1])
        g = st.node("mul_mat", [w(b + "ffn_gate"), n], F32, [F, 1], acc=1)
        u = st.node("mul_mat", [w(b + "ffn_up"), n], F32, [F, 1], acc=1)
        dn = st.node("mul_mat", [w(b + "ffn_down"), st.node("swiglu", [g, u], F32, [F, 1])], F32, [E, 1], acc=1)
        x = st.node("add", [x, dn], F32, [E, 1])
    h = st.node("mul", [st.node("rms_norm", [x], F32, [E, 1], eps=cfg.rms_eps), w("output_norm")], F32, [E, 1])
    logits = st.node("mul_mat", [w("output"), h], F32, [V, 1], acc=1)
    st.outputs = [logits] + written

    pick = _Stage("pick")
    lg = pick.param(F32, [V, 1, 1, 1], [1, 1, V])
    pick.outputs = [pick.node("argmax", [lg], I32, [1])]

    def value(name, typ, ne, shape):
        return {"name": name, "type": typ, "ne": ne, "shape": shape}

    cache_names = [n for l in range(cfg.n_layer) for n in (f"kv.{l}.0", f"kv.{l}.1")]
    values = [value("token", I32, [1, 1, 1, 1], [1, 1]), value("pos", I32, [1, 1, 1, 1], [1]),
              value("mask", F32, ["n_kv", 1, 1, 1], [1, 1, 1, "n_kv"]), value("logits", F32, [V, 1, 1, 1], [1, 1, V]),
              value("start", I32, [1, 1, 1, 1], [1]), value("tokens", I32, [n_gen, 1, 1, 1], [n_gen])]
    values += [value(n, F16, [D, C, Hkv, 1], [Hkv, C, D]) for n in cache_names]
    call_decode = {"op": "call", "stage": "decode", "args": ["token", "pos", "mask"] + cache_names,
                   "out": ["logits"] + cache_names}
    n_kv = ["max", kv_step, ["*", ["//", ["+", "pos", kv_step], kv_step], kv_step]]
    loop = {"op": "loop", "n": n_gen, "carry": [], "scalars": [], "slices": [], "counters": [["pos", "start"]],
            "bind": [["n_kv", n_kv]], "masks": [["mask", "pos"]], "until": [["token", list(eos)]] if eos else [],
            "collect": [["tokens", "token"]],
            "body": [call_decode, {"op": "call", "stage": "pick", "args": ["logits"], "out": ["token"]}]}
    program = {
        "format_version": 3,
        "symbols": [{"name": "n_kv", "min": kv_step, "max": C}],
        "values": values,
        "inputs": ["token", "pos", "mask"],
        "outputs": ["logits"],
        "stages": [st.json(), pick.json()],
        "driver": [call_decode],
        "entries": [{"name": "decode", "inputs": ["token", "pos", "mask"], "outputs": ["logits"],
                     "driver": [call_decode]},
                    {"name": "generate", "inputs": ["token", "start"], "outputs": ["tokens"], "driver": [loop]}],
        "state": cache_names,
    }
    return program, wname


def q4_k_m_types(cfg) -> dict[str, int]:
    """The storage type of each weight in a Q4_K_M file of cfg's shape, as llama.cpp's quantizer
    assigns them (the mix the reference's Q4_K_M rows run, `llm.llama_cpp_policy`): Q6_K for the lm
    head, and for attn_v and ffn_down of the layers i with i < n/8, i >= 7n/8 or (i - n/8) % 3 == 2;
    Q4_K for the rest."""
    n = cfg.n_layer
    more = [i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2 for i in range(n)]
    types = {"token_embd": 12, "output": 14}
    for l in range(n):
        b = f"blk.{l}."
        for k in ("attn_q", "attn_k", "attn_output", "ffn_gate", "ffn_up"):
            types[b + k] = 12
        types[b + "attn_v"] = 14 if more[l] else 12
        types[b + "ffn_down"] = 14 if more[l] else 12
    return types


def synthetic_weights(cfg, seed: int = 0, std: float = 0.02, types: dict[str, int] | None = None) -> dict[str, np.ndarray]:
    """Random-init weights of cfg's decoder under the HIP model's names (q/k/v and gate/up rows
    stacked), as llm.Model.get_weight gives them: ggml block bytes of cfg.wtype (any storage type the
    library encodes: Q4_0, Q8_0, Q4_K, Q5_K, Q6_K; the GPU encoders, bit-exact with ggml's) from the
    library's N(0, std) stream, tensor i from seed + i; norm weights 1. For models the fused decoder
    does not hold (K-quant weights). With types (a type per GGUF tensor name, as q4_k_m_types
    gives): the separate q / k / v and gate / up tensors under their GGUF names, each of its own
    type (the stacked rows' streams, split)."""
    import torch

    from . import ops

    E, F, V = cfg.n_embd, cfg.n_ff, cfg.n_vocab
    H, Hkv, D = cfg.n_head, cfg.n_head_kv, cfg.head_dim
    shapes = [("token_embd", V, E)]
    for l in range(cfg.n_layer):
        b = f"blk.{l}."
        shapes += [(b + "attn_qkv", (H + 2 * Hkv) * D, E), (b + "attn_output", E, H * D),
                   (b + "ffn_gate_up", 2 * F, E), (b + "ffn_down", E, F)]
    shapes.append(("output", V, E))
    out: dict[str, np.ndarray] = {"output_norm": np.ones(E, np.float32)}
    for l in range(cfg.n_layer):
        out[f"blk.{l}.attn_norm"] = np.ones(E, np.float32)
        out[f"blk.{l}.ffn_norm"] = np.ones(E, np.float32)
    for i, (name, rows, cols) in enumerate(shapes):
        x = ops.fill_normal((rows, cols), seed=seed + i, std=std)
        if types is None:
            out[name] = ops.quantize(x, cfg.wtype).cpu().numpy()
        else:
            b = name[: name.rfind(".") + 1]
            if name.endswith("attn_qkv"):
                parts = [("attn_q", 0, H * D), ("attn_k", H * D, (H + Hkv) * D), ("attn_v", (H + Hkv) * D, rows)]
            elif name.endswith("ffn_gate_up"):
                parts = [("ffn_gate", 0, F), ("ffn_up", F, 2 * F)]
            else:
                parts = [(name[len(b):], 0, rows)]
            for part, r0, r1 in parts:
                out[b + part] = ops.quantize(x[r0:r1].contiguous(), types[b + part]).cpu().numpy()
        del x
    torch.cuda.synchronize()
    return out


def write_llama_program(path: str | Path, cfg, weights: dict[str, np.ndarray], kv_step: int = 256, n_gen: int = 128,
                        eos: tuple[int, ...] = (), types: dict[str, int] | None = None) -> None:
    """The GGUF: the program JSON, tensor_names (w.N -> the weight's name), and every weight as
    ggml block bytes. weights: the HIP model's names and bytes (llm.Model.get_weight), or the
    separate tensors of synthetic_weights(..., types) with those types."""
    program, wname = llama_program(cfg, kv_step, n_gen, eos)
    split = _split_weights(cfg, weights)
    E, F, V = cfg.n_embd, cfg.n_ff, cfg.n_vocab
    H, Hkv, D = cfg.n_head, cfg.n_head_kv, cfg.head_dim
    ne = {"token_embd": (E, V), "output_norm": (E,), "output": (E, V)}
    for l in range(cfg.n_layer):
        b = f"blk.{l}."
        ne.update({b + "attn_norm": (E,), b + "attn_q": (E, H * D), b + "attn_k": (E, Hkv * D),
                   b + "attn_v": (E, Hkv * D), b + "attn_output": (H * D, E), b + "ffn_norm": (E,),
                   b + "ffn_gate": (E, F), b + "ffn_up": (E, F), b + "ffn_down": (F, E)})
    wr = gguf.GGUFWriter()
    wr.add("general.architecture", "ggml_compiler")
    wr.add("ggml_compiler.format_version", 3)
    wr.add("ggml_compiler.program", json.dumps(program, separators=(",", ":")))
    wr.add("ggml_compiler.tensor_names", json.dumps({v: k for k, v in wname.items()}, separators=(",", ":")))
    wr.add("ggml_compiler.meta", json.dumps({"eos_token_ids": list(eos), "max_context": cfg.max_ctx},
                                            separators=(",", ":")))
    for name, gname in wname.items():
        typ = 0 if name.endswith("norm") else (types or {}).get(name, cfg.wtype)
        wr.add_tensor(gname, np.ascontiguousarray(split[name]).view(np.uint8), typ, ne[name])
    wr.write(path)
