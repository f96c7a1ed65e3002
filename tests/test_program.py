"""The GGUF program loader's host side (include/ggml_compiler_rt.h model API): GGUF and program
JSON errors are reported by name before any device work, and the model API's NULL / index checks.
The runs themselves are in tests/test_gpu_program.py."""

import json

import pytest

from ggml_compiler_amd import _lib, gguf, runtime


def _gguf(tmp_path, program=None, name="p.gguf"):
    w = gguf.GGUFWriter()
    w.add("general.architecture", "ggml_compiler")
    if program is not None:
        w.add("ggml_compiler.program", program if isinstance(program, str) else json.dumps(program))
    p = tmp_path / name
    w.write(p)
    return str(p)


def _load_error(path):
    lib = _lib.load()
    m = lib.ggml_compiler_load(path.encode(), None)
    assert not m
    return lib.ggml_compiler_last_error().decode()


PROG = {"format_version": 3, "symbols": [{"name": "n", "min": 1, "max": 8}],
        "values": [{"name": "x", "type": "f32", "ne": ["n", 1, 1, 1], "shape": ["n"]}],
        "stages": [], "entries": [{"name": "main", "inputs": ["x"], "outputs": ["x"], "driver": []}], "state": []}


def test_load_errors_name_the_problem(tmp_path):
    assert "cannot read GGUF" in _load_error(str(tmp_path / "missing.gguf"))
    (tmp_path / "junk.gguf").write_bytes(b"not a gguf at all")
    assert "not a GGUF file" in _load_error(str(tmp_path / "junk.gguf"))
    assert "has no ggml_compiler.program" in _load_error(_gguf(tmp_path))
    assert "does not parse" in _load_error(_gguf(tmp_path, "{\"format_version\": 3,", "bad.gguf"))
    assert "format_version 9 is not supported" in _load_error(_gguf(tmp_path, dict(PROG, format_version=9), "v9.gguf"))
    bad = json.loads(json.dumps(PROG))
    bad["values"][0]["ne"][0] = "m"
    assert "unknown symbol 'm'" in _load_error(_gguf(tmp_path, bad, "sym.gguf"))
    bad = json.loads(json.dumps(PROG))
    bad["entries"][0]["driver"] = [{"op": "jump"}]
    assert "driver op 'jump' is not supported" in _load_error(_gguf(tmp_path, bad, "drv.gguf"))
    bad = json.loads(json.dumps(PROG))
    bad["entries"][0]["driver"] = [{"op": "loop", "n": 3, "carry": [], "body": [],
                                    "scalars": [{"value": "x", "values": [1.0, 2.0]}]}]
    assert "2 entries for 3 iterations" in _load_error(_gguf(tmp_path, bad, "sc.gguf"))
    bad = json.loads(json.dumps(PROG))
    bad["values"][0]["ne"][0] = ["//", "n", 0]
    assert "division by zero" in _load_error(_gguf(tmp_path, bad, "div.gguf"))


def test_valid_program_needs_a_hip_device(tmp_path):
    if _lib.load().gcq_device_count() > 0:
        pytest.skip("a HIP device is present")
    assert "no HIP device" in _load_error(_gguf(tmp_path, PROG))
    lib = _lib.load()
    opt = lib.ggml_compiler_default_options()
    opt.allow_cpu_fallback = True
    import ctypes
    assert not lib.ggml_compiler_load(_gguf(tmp_path, PROG, "fb.gguf").encode(), ctypes.byref(opt))
    assert "allow_cpu_fallback" in lib.ggml_compiler_last_error().decode()
    with pytest.raises(runtime.GgmlCompilerRuntimeError, match="no HIP device"):
        runtime.Session(_gguf(tmp_path, PROG, "s.gguf"))


def test_model_api_rejects_null_and_bad_indices():
    lib = _lib.load()
    assert lib.ggml_compiler_n_entries(None) == -1
    assert lib.ggml_compiler_entry_name(None, 0) is None
    assert lib.ggml_compiler_run(None) == -1 and "model is NULL" in lib.ggml_compiler_last_error().decode()
    assert lib.ggml_compiler_run_entry(None, b"main") == -1
    assert lib.ggml_compiler_set_input(None, b"x", None, 0) == -1
    assert lib.ggml_compiler_symbol_info(None, 0, None, None, None, None) == -1
    assert lib.ggml_compiler_metadata(None, b"k") is None
    assert lib.ggml_compiler_build_param(None, 0) is None
    lib.ggml_compiler_free(None)


def test_q4_k_m_types_follow_llama_cpp_rule():
    """llama.cpp's Q4_K_M mix at the 8B shape: the lm head and, in layers 0-3, 28-31 and every
    third from 6, attn_v and ffn_down in Q6_K; every other weight Q4_K."""
    from ggml_compiler_amd.llm import LlamaConfig
    from ggml_compiler_amd.program import q4_k_m_types

    t = q4_k_m_types(LlamaConfig.llama3_8b(max_ctx=64))
    six = [0, 1, 2, 3, 6, 9, 12, 15, 18, 21, 24, 27, 28, 29, 30, 31]
    assert [l for l in range(32) if t[f"blk.{l}.attn_v"] == 14] == six
    assert [l for l in range(32) if t[f"blk.{l}.ffn_down"] == 14] == six
    assert t["output"] == 14 and t["token_embd"] == 12
    assert all(t[f"blk.{l}.{k}"] == 12 for l in range(32)
               for k in ("attn_q", "attn_k", "attn_output", "ffn_gate", "ffn_up"))
