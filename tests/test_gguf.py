"""GGUF reading and writing (ggml_compiler_amd.gguf) on the CPU: the reader against bytes laid out
by hand from the GGUF v3 specification (not by this package's writer), writer round trips, the
errors for damaged files, and a Llama-style model in the layout ggml-compiler writes
(ggml_compiler/emit/gguf_runtime.py:200-271: tensors w.N, module paths in
ggml_compiler.tensor_names, eps / RoPE base in the program's rms_norm / rope nodes) mapped onto the
decoder's weights."""

import json
import struct

import numpy as np
import pytest

from ggml_compiler_amd import gguf


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def test_reader_against_hand_laid_bytes(tmp_path):
    a = np.arange(6, dtype=np.float32).reshape(2, 3)  # ggml ne (3, 2)
    q = bytes(range(18))                               # one Q4_0 block
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, 3)
    head += _s("general.architecture") + struct.pack("<I", 8) + _s("ggml_compiler")
    head += _s("general.alignment") + struct.pack("<II", 4, 64)
    head += _s("x.arr") + struct.pack("<IIQ", 9, 5, 3) + struct.pack("<3i", -1, 0, 7)
    head += _s("a") + struct.pack("<I", 2) + struct.pack("<2Q", 3, 2) + struct.pack("<IQ", 0, 0)
    head += _s("b") + struct.pack("<I", 1) + struct.pack("<Q", 32) + struct.pack("<IQ", 2, 64)
    body = head + b"\0" * ((-len(head)) % 64) + a.tobytes() + b"\0" * (64 - 24) + q
    p = tmp_path / "hand.gguf"
    p.write_bytes(body)
    r = gguf.GGUFReader(p)
    assert r.version == 3
    assert r.kv == {"general.architecture": "ggml_compiler", "general.alignment": 64, "x.arr": [-1, 0, 7]}
    assert r.tensors["a"] == gguf.TensorInfo("a", 0, (3, 2), 0, 24)
    assert r.tensors["b"].shape == (32,) and r.tensors["b"].nbytes == 18
    assert np.array_equal(r.data("a"), a)
    assert r.data("b").tobytes() == q
    r.close()


def test_writer_round_trip(tmp_path):
    w = gguf.GGUFWriter()
    w.add("s", "héllo")
    w.add("u", 7)
    w.add("big", -3)
    w.add("f", 0.5)
    w.add("b", True)
    w.add("names", ["x", "yy"])
    w.add("ints", [1, 2, 3])
    rng = np.random.default_rng(0)
    f16 = rng.standard_normal((4, 64)).astype(np.float16)
    q8 = rng.integers(0, 255, (3, 34 * 2), dtype=np.uint8)
    w.add_tensor("t0", f16, 1, (64, 4))
    w.add_tensor("t1", q8, 8, (64, 3))
    p = tmp_path / "rt.gguf"
    w.write(p)
    r = gguf.GGUFReader(p)
    assert r.kv == {"s": "héllo", "u": 7, "big": -3, "f": 0.5, "b": True, "names": ["x", "yy"], "ints": [1, 2, 3]}
    assert np.array_equal(r.data("t0"), f16)
    assert np.array_equal(r.data("t1"), q8)
    assert r.tensors["t1"].offset % 32 == 0 and r.data_offset % 32 == 0
    with pytest.raises(gguf.GGUFError, match="bytes for type"):
        w.add_tensor("bad", q8[:, :-1], 8, (64, 3))


def test_damaged_files_are_errors(tmp_path):
    p = tmp_path / "x.gguf"
    p.write_bytes(b"GGML" + b"\0" * 40)
    with pytest.raises(gguf.GGUFError, match="not a GGUF"):
        gguf.GGUFReader(p)
    w = gguf.GGUFWriter()
    w.add_tensor("t", np.zeros((2, 8), np.float32), 0, (8, 2))
    w.write(p)
    b = p.read_bytes()
    p.write_bytes(b[:-10])
    with pytest.raises(gguf.GGUFError, match="past the end"):
        gguf.GGUFReader(p)
    p.write_bytes(b[:30])
    with pytest.raises(gguf.GGUFError, match="truncated"):
        gguf.GGUFReader(p)


def tiny_lm(orc, wtype=2, n_layer=2, E=256, H=4, Hkv=2, D=64, F=512, V=1000, seed=0):
    """A tiny Llama-style model: matmul weights and embedding quantized by the reference encoder."""
    T = {}
    i = [seed]

    def q(rows, cols):
        i[0] += 1
        return (wtype, (cols, rows), orc.quantize(orc.normal((rows, cols), seed=i[0], std=0.02), wtype))

    def norm(n):
        i[0] += 1
        return (0, (n,), (1.0 + 0.1 * orc.normal((n,), seed=i[0])).astype(np.float32))

    T["token_embd"] = q(V, E)
    for l in range(n_layer):
        b = f"blk.{l}."
        T[b + "attn_norm"] = norm(E)
        T[b + "attn_q"], T[b + "attn_k"], T[b + "attn_v"] = q(H * D, E), q(Hkv * D, E), q(Hkv * D, E)
        T[b + "attn_output"] = q(E, H * D)
        T[b + "ffn_norm"] = norm(E)
        T[b + "ffn_gate"], T[b + "ffn_up"], T[b + "ffn_down"] = q(F, E), q(F, E), q(E, F)
    T["output_norm"] = norm(E)
    T["output"] = q(V, E)
    return gguf.CausalLM(n_layer=n_layer, n_embd=E, n_head=H, n_head_kv=Hkv, head_dim=D, n_ff=F, n_vocab=V,
                         rms_eps=1e-5, rope_base=10000.0, max_context=256, tensors=T,
                         meta={"kind": "causal_lm", "max_context": 256, "vocab": V})


def test_causal_lm_layout_round_trip(tmp_path, orc):
    lm = tiny_lm(orc)
    p = tmp_path / "lm.gguf"
    gguf.write_causal_lm(p, lm)
    r = gguf.GGUFReader(p)
    names = json.loads(r.kv["ggml_compiler.tensor_names"])
    assert names["w.0"] == "model.embed_tokens.weight" and names["w.2"] == "model.layers.0.self_attn.k_proj.weight"
    assert r.tensors["w.2"].ne == (256, 128) and r.tensors["w.2"].type == 2  # [Hkv*D, E] stored as ne (E, Hkv*D)
    r.close()
    back = gguf.read_causal_lm(p)
    assert (back.n_layer, back.n_embd, back.n_head, back.n_head_kv, back.head_dim, back.n_ff, back.n_vocab) == \
        (2, 256, 4, 2, 64, 512, 1000)
    assert back.rms_eps == pytest.approx(1e-5) and back.rope_base == 10000.0 and back.max_context == 256
    cfg = back.config()
    assert cfg.wtype == 2 and cfg.max_ctx == 256
    st = back.stacked()
    T = lm.tensors
    assert np.array_equal(st["blk.1.attn_qkv"], np.concatenate([T["blk.1.attn_q"][2], T["blk.1.attn_k"][2],
                                                                 T["blk.1.attn_v"][2]]))
    assert np.array_equal(st["blk.0.ffn_gate_up"], np.concatenate([T["blk.0.ffn_gate"][2], T["blk.0.ffn_up"][2]]))
    assert np.array_equal(st["output_norm"], T["output_norm"][2])
    mixed = tiny_lm(orc)
    mixed.tensors["output"] = (8, mixed.tensors["output"][1],
                               orc.quantize(orc.normal((1000, 256), seed=99, std=0.02), 8))
    gguf.write_causal_lm(p, mixed)
    with pytest.raises(gguf.GGUFError, match="one type"):
        gguf.read_causal_lm(p).config()
