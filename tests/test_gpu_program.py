"""GGUF programs loaded and run by libgcq's loader (include/ggml_compiler_rt.h, runtime.Session):
a one-call stage against the oracle, the loop driver's carries / scalars / slices / counters /
causal masks / collected rows / until test, and a Llama decoder program (ggml_compiler_amd.program,
the format the reference's compiler writes for llm.py's decode stage) against the oracle's run of
the same model, by its decode entry (symbolic n_kv bound from the mask's shape) and its generate
entry (n_kv bound per step from the position, greedy tokens, stop at an end-of-sequence id)."""

import json
import math

import numpy as np
import pytest
import torch

from ggml_compiler_amd import gguf, runtime

pytestmark = pytest.mark.gpu
TOL = 1e-3
TOL_LM = 1e-2


def _write(path, program, tensors=()):
    w = gguf.GGUFWriter()
    w.add("general.architecture", "ggml_compiler")
    w.add("ggml_compiler.program", json.dumps(program))
    w.add("ggml_compiler.meta", json.dumps({"note": "test"}))
    for name, data, typ, ne in tensors:
        w.add_tensor(name, data, typ, ne)
    w.write(path)
    return str(path)


def _v(name, typ, ne, shape):
    return {"name": name, "type": typ, "ne": list(ne) + [1] * (4 - len(ne)), "shape": shape}


def _n(i, op, src, typ, ne, **p):
    return {"id": f"%{i}", "op": op, "src": src, "type": typ, "ne": list(ne) + [1] * (4 - len(ne)), "p": p, "loc": ""}


def test_one_call_program(tmp_path, orc):
    """y = W x + b: a Q8_0 weight and an f32 bias from the GGUF, one stage, one call."""
    N, K = 300, 512
    raw = orc.quantize(orc.normal((N, K), seed=50, std=0.02), "q8_0")
    bias = orc.normal((N,), seed=51)
    st = {"name": "lin", "params": [_v("a.0", "f32", [K, 1], [1, K])], "outputs": ["%1"],
          "nodes": [_n(0, "mul_mat", ["w.0", "a.0"], "f32", [N, 1]), _n(1, "add", ["%0", "c.0"], "f32", [N, 1])]}
    prog = {"format_version": 3, "symbols": [], "values": [_v("x", "f32", [K, 1], [1, K]), _v("y", "f32", [N, 1], [1, N])],
            "stages": [st], "entries": [{"name": "main", "inputs": ["x"], "outputs": ["y"],
                                         "driver": [{"op": "call", "stage": "lin", "args": ["x"], "out": ["y"]}]}],
            "state": []}
    path = _write(tmp_path / "lin.gguf", prog, [("w.0", raw, 8, (K, N)), ("c.0", bias, 0, (N,))])
    with runtime.Session(path) as s:
        assert s.backend_name and [t.name for t in s.inputs] == ["x"] and s.outputs[0].shape == (1, N)
        assert s.metadata == {"note": "test"}
        for seed in (52, 53):
            x = orc.normal((1, K), seed=seed)
            y = s.run(x)["y"]
            assert orc.parity(y, orc.mul_mat(raw, "q8_0", x, K) + bias) < TOL
        assert s.stats["n_calls"] == 1 and s.stats["stages"]["lin"]["calls"] == 1
        with pytest.raises(ValueError, match="shape"):
            s.run(np.zeros((2, K), np.float32))


def test_profile_env_writes_a_line_per_node(tmp_path, orc, monkeypatch):
    """GGML_COMPILER_PROFILE=<file> (the reference runtime's profile, runtime/src/ggml_compiler_rt.cpp:
    219-240): each run appends one "stage<TAB>node<TAB>op<TAB>ms" line per graph node, in graph
    order, the nodes launched one at a time; the results stay those of the fused run. The variable
    is read when a model loads, so a model loaded without it runs fused as before."""
    N, K = 300, 512
    raw = orc.quantize(orc.normal((N, K), seed=50, std=0.02), "q8_0")
    bias = orc.normal((N,), seed=51)
    st = {"name": "lin", "params": [_v("a.0", "f32", [K, 1], [1, K])], "outputs": ["%1"],
          "nodes": [_n(0, "mul_mat", ["w.0", "a.0"], "f32", [N, 1]), _n(1, "add", ["%0", "c.0"], "f32", [N, 1])]}
    prog = {"format_version": 3, "symbols": [], "values": [_v("x", "f32", [K, 1], [1, K]), _v("y", "f32", [N, 1], [1, N])],
            "stages": [st], "entries": [{"name": "main", "inputs": ["x"], "outputs": ["y"],
                                         "driver": [{"op": "call", "stage": "lin", "args": ["x"], "out": ["y"]}]}],
            "state": []}
    path = _write(tmp_path / "lin.gguf", prog, [("w.0", raw, 8, (K, N)), ("c.0", bias, 0, (N,))])
    x = orc.normal((1, K), seed=52)
    prof = tmp_path / "prof.tsv"
    monkeypatch.setenv("GGML_COMPILER_PROFILE", str(prof))
    with runtime.Session(path) as s:
        for _ in range(2):
            y = s.run(x)["y"]
    monkeypatch.delenv("GGML_COMPILER_PROFILE")
    lines = prof.read_text().splitlines()
    # 2 runs x 3 nodes: the stage's two, then the copy into the output value that the loader
    # appends after them (as the reference's call graphs do, runtime/src/ggml_compiler_rt.cpp:705-713)
    assert len(lines) == 6, lines
    rows = [ln.split("\t") for ln in lines]
    assert all(len(f) == 4 for f in rows), rows
    assert [f[0] for f in rows] == ["lin"] * 6
    assert [f[2] for f in rows] == ["MUL_MAT", "ADD", "CPY"] * 2
    assert [f[1] for f in rows[:2]] == ["%0", "%1"] and [f[1] for f in rows[3:5]] == ["%0", "%1"]
    assert all(float(f[3]) >= 0.0 for f in rows)
    assert orc.parity(y, orc.mul_mat(raw, "q8_0", x, K) + bias) < TOL
    # a model loaded without the variable appends nothing
    with runtime.Session(path) as s:
        y2 = s.run(x)["y"]
    assert len(prof.read_text().splitlines()) == 6
    assert orc.parity(y2, orc.mul_mat(raw, "q8_0", x, K) + bias) < TOL


def test_unfused_glu_and_eager_attention_ops(tmp_path, orc):
    """A program left unfused (silu then mul rather than swiglu; soft_max over scores with an f16
    mask rather than flash_attn), with sub, div and gelu_erf: ops.cpp's binary and unary tables."""
    E, S = 64, 5
    st = {"name": "f", "params": [_v("a.0", "f32", [E, S], [S, E]), _v("a.1", "f32", [E, S], [S, E]),
                                  _v("a.2", "f16", [E, S], [S, E])],
          "outputs": ["%5"],
          "nodes": [_n(0, "silu", ["a.0"], "f32", [E, S]), _n(1, "mul", ["%0", "a.1"], "f32", [E, S]),
                    _n(2, "sub", ["%1", "a.0"], "f32", [E, S]), _n(3, "div", ["%2", "c.0"], "f32", [E, S]),
                    _n(4, "gelu_erf", ["%3"], "f32", [E, S]),
                    _n(5, "soft_max", ["%4", "a.2"], "f32", [E, S], scale=0.5)]}
    c = orc.normal((E,), seed=60) + 3.0
    prog = {"format_version": 3, "symbols": [],
            "values": [_v("g", "f32", [E, S], [S, E]), _v("u", "f32", [E, S], [S, E]), _v("m", "f16", [E, S], [S, E]),
                       _v("y", "f32", [E, S], [S, E])],
            "stages": [st], "entries": [{"name": "main", "inputs": ["g", "u", "m"], "outputs": ["y"],
                                         "driver": [{"op": "call", "stage": "f", "args": ["g", "u", "m"], "out": ["y"]}]}],
            "state": []}
    g, u = orc.normal((S, E), seed=61), orc.normal((S, E), seed=62)
    m = np.triu(np.full((S, E), -np.inf, np.float32), k=E - S + 1)  # causal-style -inf tail per row
    with runtime.Session(_write(tmp_path / "f.gguf", prog, [("c.0", c, 0, (E,))])) as s:
        y = s.run(g, u, m)["y"]  # Session converts values to the input type (f16 here)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    h = (torch.nn.functional.silu(t(g)) * t(u) - t(g)) / t(c)
    want = torch.softmax(torch.nn.functional.gelu(h) * 0.5 + t(m), dim=-1).numpy()
    assert np.allclose(y, want, rtol=1e-5, atol=1e-7)


def test_layer_norm_gelu_mean_program(tmp_path, orc):
    """A GPT-2-style piece: norm, then * weight + bias from the GGUF, gelu (tanh form), clamp, and
    the mean of each row."""
    E, S = 96, 3
    st = {"name": "ln", "params": [_v("a.0", "f32", [E, S], [S, E])], "outputs": ["%5"],
          "nodes": [_n(0, "norm", ["a.0"], "f32", [E, S], eps=1e-5), _n(1, "mul", ["%0", "c.0"], "f32", [E, S]),
                    _n(2, "add", ["%1", "c.1"], "f32", [E, S]), _n(3, "gelu_tanh", ["%2"], "f32", [E, S]),
                    _n(4, "clamp", ["%3"], "f32", [E, S], min=-0.1, max=2.0), _n(5, "mean", ["%4"], "f32", [1, S])]}
    w, b = orc.normal((E,), seed=70) + 1.0, orc.normal((E,), seed=71)
    prog = {"format_version": 3, "symbols": [],
            "values": [_v("x", "f32", [E, S], [S, E]), _v("y", "f32", [1, S], [S, 1])],
            "stages": [st], "entries": [{"name": "main", "inputs": ["x"], "outputs": ["y"],
                                         "driver": [{"op": "call", "stage": "ln", "args": ["x"], "out": ["y"]}]}],
            "state": []}
    x = orc.normal((S, E), seed=72) * 3.0
    with runtime.Session(_write(tmp_path / "ln.gguf", prog, [("c.0", w, 0, (E,)), ("c.1", b, 0, (E,))])) as s:
        y = s.run(x)["y"]
    h = torch.nn.functional.layer_norm(torch.from_numpy(x), (E,), torch.from_numpy(w), torch.from_numpy(b), eps=1e-5)
    want = torch.clamp(torch.nn.functional.gelu(h, approximate="tanh"), -0.1, 2.0).mean(-1, keepdim=True).numpy()
    assert np.allclose(y, want, rtol=1e-5, atol=1e-6)


def test_set_rows_then_get_rows_of_the_same_parameter(tmp_path, orc):
    """A stage that writes a row of its parameter in place (set_rows into an f16 table, as into a KV
    cache) and reads rows of it (get_rows): the read sees the write, as in ggml's expand order (the
    set_rows result is the first output); the loader's move of small get_rows to the front of a
    stage's graph must not reorder them."""
    E, R = 64, 6
    st = {"name": "upd", "params": [_v("a.0", "f16", [E, R], [R, E]), _v("a.1", "f32", [E, 1], [1, E]),
                                    _v("a.2", "i32", [1], [1]), _v("a.3", "i32", [2], [2])],
          "outputs": ["%0", "%1"],
          "nodes": [_n(0, "set_rows", ["a.0", "a.1", "a.2"], "f16", [E, R]),
                    _n(1, "get_rows", ["a.0", "a.3"], "f32", [E, 2])]}
    prog = {"format_version": 3, "symbols": [],
            "values": [_v("tab", "f16", [E, R], [R, E]), _v("row", "f32", [E, 1], [1, E]), _v("i", "i32", [1], [1]),
                       _v("g", "i32", [2], [2]), _v("y", "f32", [E, 2], [2, E])],
            "stages": [st], "entries": [{"name": "main", "inputs": ["tab", "row", "i", "g"], "outputs": ["y", "tab"],
                                         "driver": [{"op": "call", "stage": "upd", "args": ["tab", "row", "i", "g"],
                                                     "out": ["tab", "y"]}]}],
            "state": []}
    tab = orc.normal((R, E), seed=80).astype(np.float16)
    row = orc.normal((1, E), seed=81)
    with runtime.Session(_write(tmp_path / "upd.gguf", prog)) as s:
        out = s.run(tab, row, np.array([3], np.int32), np.array([3, 1], np.int32))
    want = tab.copy()
    want[3] = row[0].astype(np.float16)
    assert np.array_equal(np.asarray(out["tab"]).astype(np.float16), want)
    assert np.array_equal(out["y"], want[[3, 1]].astype(np.float32)), "get_rows ran before the set_rows of its table"


def test_loop_driver(tmp_path):
    """h_{k+1} = h_k * s_k + R[k] (carry from h0, per-iteration scalars, slices of R); the causal
    mask row of position start + k; both collected per iteration; stop once argmax(h) is 7."""
    n, E = 4, 8
    step = {"name": "step", "params": [_v("a.0", "f32", [E], [E]), _v("a.1", "f32", [1], [1]),
                                       _v("a.2", "f32", [E], [E])],
            "outputs": ["%1"], "nodes": [_n(0, "mul", ["a.0", "a.1"], "f32", [E]), _n(1, "add", ["%0", "a.2"], "f32", [E])]}
    cpm = {"name": "cpm", "params": [_v("a.0", "f32", [E], [E])], "outputs": ["%0"],
           "nodes": [_n(0, "cont", ["a.0"], "f32", [E])]}
    am = {"name": "am", "params": [_v("a.0", "f32", [E], [E])], "outputs": ["%0"],
          "nodes": [_n(0, "argmax", ["a.0"], "i32", [1])]}
    values = [_v("h0", "f32", [E], [E]), _v("h", "f32", [E], [E]), _v("s", "f32", [1], [1]), _v("R", "f32", [E, n], [n, E]),
              _v("r", "f32", [E], [E]), _v("i0", "i32", [1], [1]), _v("i", "i32", [1], [1]), _v("m", "f32", [E], [E]),
              _v("mo", "f32", [E], [E]), _v("t", "i32", [1], [1]), _v("hs", "f32", [E, n], [n, E]),
              _v("ms", "f32", [E, n], [n, E])]
    svals = [2.0, 3.0, 0.5, 1.0]
    loop = {"op": "loop", "n": n, "carry": [["h", "h0"]], "scalars": [{"value": "s", "values": svals}],
            "slices": [["r", "R"]], "counters": [["i", "i0"]], "masks": [["m", "i"]],
            "collect": [["hs", "h"], ["ms", "mo"]], "until": [["t", [7]]],
            "body": [{"op": "call", "stage": "step", "args": ["h", "s", "r"], "out": ["h"]},
                     {"op": "call", "stage": "cpm", "args": ["m"], "out": ["mo"]},
                     {"op": "call", "stage": "am", "args": ["h"], "out": ["t"]}]}
    prog = {"format_version": 3, "symbols": [], "values": values, "stages": [step, cpm, am],
            "entries": [{"name": "main", "inputs": ["h0", "R", "i0"], "outputs": ["hs", "ms", "t"], "driver": [loop]}],
            "state": []}
    h0 = np.array([1, 0, 0, 0, 0, 0, 0, 0], np.float32)
    R = np.zeros((n, E), np.float32)
    R[0, 2] = 5.0   # argmax 2 after step 0
    R[1, 4] = 50.0  # 4 after step 1
    R[2, 7] = 90.0  # 7 after step 2: the loop stops there
    R[3, 0] = 1.0
    with runtime.Session(_write(tmp_path / "loop.gguf", prog)) as s:
        out = s.run(h0, R, np.array([3], np.int32))
        h, want = h0.copy(), np.zeros((n, E), np.float32)
        for k in range(3):
            h = h * svals[k] + R[k]
            want[k] = h
        np.testing.assert_array_equal(out["hs"], want)  # row 3 stays zero: stopped
        assert int(out["t"][0]) == 7
        masks = np.zeros((n, E), np.float32)
        for k in range(3):
            masks[k] = np.where(np.arange(E) <= 3 + k, 0.0, -np.inf)
        np.testing.assert_array_equal(out["ms"], masks)
        assert s.stats["n_calls"] == 9
    # without an until test every iteration runs; iterations after the first replay one captured
    # graph, which the second run (other inputs, other start position) replays from its start
    loop.pop("until")
    with runtime.Session(_write(tmp_path / "loop_all.gguf", prog)) as s:
        for start, scale in ((3, 1.0), (1, -2.0)):
            out = s.run(h0 * scale, R * scale, np.array([start], np.int32))
            h, want, masks = h0 * scale, np.zeros((n, E), np.float32), np.zeros((n, E), np.float32)
            for k in range(n):
                h = h * svals[k] + R[k] * scale
                want[k] = h
                masks[k] = np.where(np.arange(E) <= start + k, 0.0, -np.inf)
            np.testing.assert_array_equal(out["hs"], want)
            np.testing.assert_array_equal(out["ms"], masks)
            assert int(out["t"][0]) == int(np.argmax(want[-1]))
            assert s.stats["n_calls"] == 3 * n
            assert {k: v["calls"] for k, v in s.stats["stages"].items()} == {"step": n, "cpm": n, "am": n}


def _llama(orc, wtype):
    from ggml_compiler_amd.llm import LlamaConfig, Model

    cfg = LlamaConfig(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=1000,
                      max_ctx=64, wtype=wtype, rms_eps=1e-5, rope_base=10000.0)
    m = Model(cfg, max_prompt=16)
    m.init_random(seed=12)
    w = {name: m.get_weight(name) for name, *_ in m.weights()}
    m.close()
    return cfg, w


@pytest.mark.parametrize("wtype", [2, 8])
def test_llama_program_decode_and_generate(tmp_path, orc, wtype):
    from ggml_compiler_amd.program import write_llama_program
    from llama_ref import OracleLlama

    cfg, w = _llama(orc, wtype)
    path = str(tmp_path / "llama.gguf")
    write_llama_program(path, cfg, w, kv_step=16, n_gen=24, eos=(999,))
    with runtime.Session(path) as s:
        assert list(s.entries) == ["decode", "generate"] and s.symbols == {"n_kv": (16, 64)}
        o = OracleLlama(cfg, w)
        tok, toks = 17, []
        for p in range(20):  # n_kv 16 then 32: the decode stage is rebuilt for the new binding
            n_kv = max(16, (p + 16) // 16 * 16)
            mask = np.where(np.arange(n_kv) <= p, 0.0, -np.inf).astype(np.float32).reshape(1, 1, 1, n_kv)
            lg = s.run(np.array([[tok]], np.int32), np.array([p], np.int32), mask, entry="decode")["logits"]
            assert s.bound() == {"n_kv": n_kv}
            lo = o.forward([tok])
            assert orc.parity(lg.reshape(-1), lo) < TOL_LM, p
            tok = int(np.argmax(lg))
            toks.append(tok)
        # generate: the same greedy tokens from a fresh cache, n_kv bound per step by the loop
        s.reset()
        gen = s.run(np.array([[17]], np.int32), np.array([0], np.int32), entry="generate")["tokens"]
        assert list(gen[:20]) == toks
        assert s.stats["stages"]["decode"]["calls"] == 24 and s.stats["stages"]["pick"]["calls"] == 24
        # stop at an end-of-sequence id: the first generated token
        path2 = str(tmp_path / "llama_eos.gguf")
        write_llama_program(path2, cfg, w, kv_step=16, n_gen=24, eos=(toks[2],))
    with runtime.Session(path2) as s2:
        gen = s2.run(np.array([[17]], np.int32), np.array([0], np.int32), entry="generate")["tokens"]
        assert list(gen[:3]) == toks[:3] and not gen[3:].any()
        assert s2.stats["n_calls"] == 6


@pytest.mark.parametrize("wtype", [12, 13, 14, "q4_K_M"])
def test_llama_program_kquant_weights(tmp_path, orc, wtype):
    """A Llama decoder program whose weights are all one K-quant type (Q4_K, Q5_K, Q6_K: every
    projection, the embedding table and the lm head), which the fused decoder does not hold, or
    llama.cpp's Q4_K_M mix (Q6_K lm head, and v / down of some layers Q6_K, the rest Q4_K: q / k
    and v of such a layer of two types): the decode entry against the oracle decoder on the same
    bytes, then the generate entry's tokens."""
    from ggml_compiler_amd.llm import LlamaConfig
    from ggml_compiler_amd.program import q4_k_m_types, synthetic_weights, write_llama_program
    from llama_ref import OracleLlama

    mixed = wtype == "q4_K_M"
    cfg = LlamaConfig(n_layer=4 if mixed else 2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512,
                      n_vocab=1000, max_ctx=64, wtype=12 if mixed else wtype, rms_eps=1e-5, rope_base=10000.0)
    types = q4_k_m_types(cfg) if mixed else None
    if mixed:  # of 4 layers, 2 ((i - 0) % 3 == 2) and 3 (i >= 7n/8) take Q6_K v / down
        assert [types[f"blk.{l}.attn_v"] for l in range(4)] == [12, 12, 14, 14] and types["output"] == 14
    w = synthetic_weights(cfg, seed=31, types=types)
    path = str(tmp_path / "llama_kq.gguf")
    write_llama_program(path, cfg, w, kv_step=16, n_gen=12, eos=(999,), types=types)
    with runtime.Session(path) as s:
        o = OracleLlama(cfg, w, types=types)
        tok, toks = 17, []
        for p in range(12):
            n_kv = max(16, (p + 16) // 16 * 16)
            mask = np.where(np.arange(n_kv) <= p, 0.0, -np.inf).astype(np.float32).reshape(1, 1, 1, n_kv)
            lg = s.run(np.array([[tok]], np.int32), np.array([p], np.int32), mask, entry="decode")["logits"]
            assert orc.parity(lg.reshape(-1), o.forward([tok])) < TOL_LM, p
            tok = int(np.argmax(lg))
            toks.append(tok)
        s.reset()
        gen = s.run(np.array([[17]], np.int32), np.array([0], np.int32), entry="generate")["tokens"]
        assert list(gen[:12]) == toks


def test_compiled_builder_replaces_a_stage(tmp_path, orc):
    """ggml_compiler_load_with: a builder (here a ctypes callback, as generated C++ would be)
    builds stage `lin` from its parameter and the GGUF weight by name; the program's own nodes for
    the stage are not used (they compute something else) and the result is the builder's."""
    import ctypes

    from ggml_compiler_amd import _lib

    lib = _lib.load()
    N, K = 64, 256
    raw = orc.quantize(orc.normal((N, K), seed=60, std=0.02), "q4_0")
    st = {"name": "lin", "params": [_v("a.0", "f32", [K, 1], [1, K])], "outputs": ["%0"],
          "nodes": [_n(0, "mul_mat", ["w.0", "a.0"], "f32", [N, 1])]}
    prog = {"format_version": 3, "symbols": [], "values": [_v("x", "f32", [K, 1], [1, K]), _v("y", "f32", [N, 1], [1, N])],
            "stages": [st], "entries": [{"name": "main", "inputs": ["x"], "outputs": ["y"],
                                         "driver": [{"op": "call", "stage": "lin", "args": ["x"], "out": ["y"]}]}],
            "state": []}
    path = _write(tmp_path / "b.gguf", prog, [("w.0", raw, 2, (K, N))])
    calls = []

    @ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)
    def build(b):
        calls.append(1)
        ctx = lib.ggml_compiler_build_ctx(b)
        x = lib.ggml_compiler_build_param(b, 0)
        w = lib.ggml_compiler_build_weight(b, b"w.0")
        assert lib.ggml_compiler_build_gpu(b) and lib.ggml_compiler_build_weight(b, b"nope") is None
        y = lib.ggml_scale(ctx, lib.ggml_mul_mat(ctx, w, x), ctypes.c_float(2.0))
        lib.ggml_compiler_build_output(b, 0, y)
        return 0

    builders = (_lib.Builder * 1)(_lib.Builder(b"lin", ctypes.cast(build, ctypes.c_void_p)))
    m = lib.ggml_compiler_load_with(path.encode(), None, builders, 1)
    assert not m and "no tensor 'nope'" in lib.ggml_compiler_last_error().decode()  # the builder's error fails the load

    @ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)
    def build_ok(b):
        ctx = lib.ggml_compiler_build_ctx(b)
        y = lib.ggml_scale(ctx, lib.ggml_mul_mat(ctx, lib.ggml_compiler_build_weight(b, b"w.0"),
                                                  lib.ggml_compiler_build_param(b, 0)), ctypes.c_float(2.0))
        lib.ggml_compiler_build_output(b, 0, y)
        return 0

    builders = (_lib.Builder * 1)(_lib.Builder(b"lin", ctypes.cast(build_ok, ctypes.c_void_p)))
    m = lib.ggml_compiler_load_with(path.encode(), None, builders, 1)
    assert m, lib.ggml_compiler_last_error().decode()
    try:
        x = orc.normal((1, K), seed=61)
        assert lib.ggml_compiler_set_input(m, b"x", x.ctypes.data, x.nbytes) == 0
        assert lib.ggml_compiler_run(m) == 0, lib.ggml_compiler_last_error().decode()
        y = np.empty((1, N), np.float32)
        assert lib.ggml_compiler_get_output(m, b"y", y.ctypes.data, y.nbytes) == 0
        assert orc.parity(y, 2 * orc.mul_mat(raw, "q4_0", x, K)) < TOL
        assert lib.ggml_compiler_get_output(m, b"y", y.ctypes.data, 4) == -1
        assert "has 256 bytes" in lib.ggml_compiler_last_error().decode()
    finally:
        lib.ggml_compiler_free(m)
    bad = (_lib.Builder * 1)(_lib.Builder(b"other", ctypes.cast(build_ok, ctypes.c_void_p)))
    assert not lib.ggml_compiler_load_with(path.encode(), None, bad, 1)
    assert "builder for stage 'other'" in lib.ggml_compiler_last_error().decode()
