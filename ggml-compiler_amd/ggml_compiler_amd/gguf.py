"""GGUF files as ggml-compiler writes them, read (and written) without the gguf package.

The file format is GGUF v3: the magic "GGUF", version, tensor and key-value counts, the key-value
pairs (typed values, arrays), then one info record per tensor (name, ne dims innermost first,
ggml type, data offset), padding to `general.alignment` (32 by default), and the tensor data.
The reference writes it with gguf-py's GGUFWriter (ggml_compiler/emit/gguf_runtime.py:200-271):
tensors named "w.N" (weights) and "c.N" (constants), the program JSON under
"ggml_compiler.program", the weights' module paths under "ggml_compiler.tensor_names" and the
entry-point metadata under "ggml_compiler.meta".

`read_causal_lm` maps such a file of a Llama-style model (Hugging Face module paths
model.embed_tokens, model.layers.L.{self_attn.{q,k,v,o}_proj, mlp.{gate,up,down}_proj,
input_layernorm, post_attention_layernorm}, model.norm, lm_head) onto this package's decoder:
its shape from the tensors, eps and RoPE base from the program's rms_norm and rope nodes
(emit/gguf_runtime.py:76-80). Reading uses a memory map; tensor data is not copied until asked.
"""

from __future__ import annotations

import json
import mmap
import re
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np

MAGIC = b"GGUF"
VERSION = 3
DEFAULT_ALIGNMENT = 32

# GGUF value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
           I64: "<q", F64: "<d"}

# ggml types: (elements per block, bytes per block)
TYPE_SIZES = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36),
              10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292),
              24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8), 30: (1, 2)}
TYPE_NAMES = {0: "f32", 1: "f16", 2: "q4_0", 8: "q8_0", 12: "q4_K", 13: "q5_K", 14: "q6_K", 26: "i32", 30: "bf16"}
F32_T, F16_T, Q4_0_T, Q8_0_T, Q4_K_T = 0, 1, 2, 8, 12


class GGUFError(ValueError):
    pass


def tensor_nbytes(ggml_type: int, ne: tuple[int, ...]) -> int:
    if ggml_type not in TYPE_SIZES:
        raise GGUFError(f"unknown ggml type {ggml_type}")
    blck, size = TYPE_SIZES[ggml_type]
    if ne[0] % blck:
        raise GGUFError(f"row of {ne[0]} is not a multiple of type {ggml_type}'s block of {blck}")
    n = ne[0] // blck * size
    for d in ne[1:]:
        n *= d
    return n


@dataclass(frozen=True)
class TensorInfo:
    name: str
    type: int
    ne: tuple[int, ...]  # innermost first (ggml order)
    offset: int          # from the start of the data section
    nbytes: int

    @property
    def shape(self) -> tuple[int, ...]:
        """numpy / PyTorch order (outermost first)."""
        return tuple(reversed(self.ne))


class GGUFReader:
    """Parses the header, key-values and tensor infos; `data(name)` views a tensor's bytes."""

    def __init__(self, path: str | Path) -> None:
        self.path = Path(path)
        with open(self.path, "rb") as f:
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        self._pos = 0
        if self._take(4) != MAGIC:
            raise GGUFError(f"{self.path}: not a GGUF file")
        self.version = self._scalar(U32)
        if self.version not in (2, 3):
            raise GGUFError(f"{self.path}: GGUF version {self.version} (2 or 3 supported)")
        n_tensors, n_kv = self._scalar(U64), self._scalar(U64)
        self.kv: dict[str, Any] = {}
        for _ in range(n_kv):
            key = self._string()
            self.kv[key] = self._value(self._scalar(U32))
        self.tensors: dict[str, TensorInfo] = {}
        for _ in range(n_tensors):
            name = self._string()
            n_dims = self._scalar(U32)
            ne = tuple(self._scalar(U64) for _ in range(n_dims))
            t = self._scalar(U32)
            off = self._scalar(U64)
            if name in self.tensors:
                raise GGUFError(f"duplicate tensor {name!r}")
            self.tensors[name] = TensorInfo(name, t, ne, off, tensor_nbytes(t, ne))
        align = int(self.kv.get("general.alignment", DEFAULT_ALIGNMENT))
        self.data_offset = (self._pos + align - 1) // align * align
        for ti in self.tensors.values():
            if ti.offset % align or self.data_offset + ti.offset + ti.nbytes > len(self._mm):
                raise GGUFError(f"tensor {ti.name!r}: data at {ti.offset} (+{ti.nbytes}) is misaligned or past the end")

    def _take(self, n: int) -> bytes:
        if self._pos + n > len(self._mm):
            raise GGUFError(f"{self.path}: truncated")
        b = self._mm[self._pos:self._pos + n]
        self._pos += n
        return b

    def _scalar(self, t: int):
        fmt = _SCALAR[t]
        return struct.unpack(fmt, self._take(struct.calcsize(fmt)))[0]

    def _string(self) -> str:
        return self._take(self._scalar(U64)).decode("utf-8")

    def _value(self, t: int):
        if t == STRING:
            return self._string()
        if t == ARRAY:
            et, n = self._scalar(U32), self._scalar(U64)
            return [self._value(et) for _ in range(n)]
        if t not in _SCALAR:
            raise GGUFError(f"unknown value type {t}")
        return self._scalar(t)

    def data(self, name: str) -> np.ndarray:
        """The tensor's bytes: f32 / f16 / i32 as that dtype in numpy order, other types as uint8
        [rows, row bytes]."""
        ti = self.tensors[name]
        start = self.data_offset + ti.offset
        raw = np.frombuffer(self._mm, np.uint8, ti.nbytes, start)
        dt = {F32_T: np.float32, F16_T: np.float16, 26: np.int32}.get(ti.type)
        if dt is not None:
            return raw.view(dt).reshape(ti.shape)
        rows = ti.nbytes // (tensor_nbytes(ti.type, (ti.ne[0],)) or 1)
        return raw.reshape(rows, -1)

    def close(self) -> None:
        self._mm.close()


class GGUFWriter:
    """Writes GGUF v3 (the layout gguf-py's GGUFWriter produces): key-values in insertion order,
    tensors in insertion order at 32-byte aligned offsets."""

    def __init__(self, alignment: int = DEFAULT_ALIGNMENT) -> None:
        self.kv: list[tuple[str, int, Any]] = []
        self.tensors: list[tuple[str, int, tuple[int, ...], bytes]] = []
        self.alignment = alignment

    def add(self, key: str, value: Any, vtype: int | None = None) -> None:
        if vtype is None:
            if isinstance(value, bool):
                vtype = BOOL
            elif isinstance(value, int):
                vtype = U32 if 0 <= value < 2 ** 32 else I64
            elif isinstance(value, float):
                vtype = F32
            elif isinstance(value, str):
                vtype = STRING
            elif isinstance(value, (list, tuple)):
                vtype = ARRAY
            else:
                raise GGUFError(f"no GGUF type for {type(value).__name__}")
        self.kv.append((key, vtype, value))

    def add_tensor(self, name: str, data: np.ndarray, ggml_type: int, ne: tuple[int, ...]) -> None:
        b = np.ascontiguousarray(data).tobytes()
        if len(b) != tensor_nbytes(ggml_type, ne):
            raise GGUFError(f"{name}: {len(b)} bytes for type {ggml_type} ne {ne}")
        self.tensors.append((name, ggml_type, tuple(int(d) for d in ne), b))

    @staticmethod
    def _str(s: str) -> bytes:
        b = s.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    def _val(self, t: int, v: Any) -> bytes:
        if t == STRING:
            return self._str(v)
        if t == ARRAY:
            if not v:
                return struct.pack("<IQ", U32, 0)
            et = STRING if isinstance(v[0], str) else F32 if isinstance(v[0], float) else I32
            return struct.pack("<IQ", et, len(v)) + b"".join(self._val(et, x) for x in v)
        return struct.pack(_SCALAR[t], v)

    def write(self, path: str | Path) -> None:
        out = bytearray(MAGIC + struct.pack("<IQQ", VERSION, len(self.tensors), len(self.kv)))
        for k, t, v in self.kv:
            out += self._str(k) + struct.pack("<I", t) + self._val(t, v)
        off = 0
        offsets = []
        for name, t, ne, b in self.tensors:
            offsets.append(off)
            out += self._str(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne)
            out += struct.pack("<IQ", t, off)
            off = (off + len(b) + self.alignment - 1) // self.alignment * self.alignment
        out += b"\0" * ((-len(out)) % self.alignment)
        with open(path, "wb") as f:
            f.write(out)
            for (name, t, ne, b), o in zip(self.tensors, offsets):
                f.write(b)
                f.write(b"\0" * ((-len(b)) % self.alignment))


# ------------------------------------------------------------------------- causal LM mapping

_LAYER = re.compile(r"^model\.layers\.(\d+)\.(.+)\.weight$")
_ROLES = {"self_attn.q_proj": "attn_q", "self_attn.k_proj": "attn_k", "self_attn.v_proj": "attn_v",
          "self_attn.o_proj": "attn_output", "mlp.gate_proj": "ffn_gate", "mlp.up_proj": "ffn_up",
          "mlp.down_proj": "ffn_down", "input_layernorm": "attn_norm", "post_attention_layernorm": "ffn_norm"}


@dataclass
class CausalLM:
    """A Llama-style model read from a ggml-compiler GGUF: its shape and its tensors by role
    (token_embd, blk.L.{attn_norm, attn_q, attn_k, attn_v, attn_output, ffn_norm, ffn_gate, ffn_up,
    ffn_down}, output_norm, output), each (ggml type, ne, bytes)."""
    n_layer: int
    n_embd: int
    n_head: int
    n_head_kv: int
    head_dim: int
    n_ff: int
    n_vocab: int
    rms_eps: float
    rope_base: float
    max_context: int | None
    tensors: dict[str, tuple[int, tuple[int, ...], np.ndarray]]
    meta: dict[str, Any]

    def config(self, max_ctx: int | None = None):
        """The decoder's LlamaConfig; every matmul weight and the embedding must share one type,
        Q4_0 or Q8_0 (the fused decoder's weight storage)."""
        from .llm import LlamaConfig

        types = {t for name, (t, _, _) in self.tensors.items() if not name.endswith("_norm")}
        if len(types) != 1 or next(iter(types)) not in (Q4_0_T, Q8_0_T):
            raise GGUFError("the fused decoder needs every matmul weight and the embedding in one type, Q4_0 or "
                            f"Q8_0; this file has {sorted(TYPE_NAMES.get(t, str(t)) for t in types)}")
        ctx = max_ctx or self.max_context or 4096
        return LlamaConfig(self.n_layer, self.n_embd, self.n_head, self.n_head_kv, self.head_dim, self.n_ff,
                           self.n_vocab, ctx, next(iter(types)), self.rms_eps, self.rope_base)

    def stacked(self) -> dict[str, np.ndarray]:
        """The decoder's weights: q / k / v and gate / up rows stacked (quantized rows are
        independent, so stacking the byte rows stacks the matrices)."""
        T = self.tensors
        out = {"token_embd": T["token_embd"][2], "output_norm": T["output_norm"][2].astype(np.float32),
               "output": T["output"][2]}
        for l in range(self.n_layer):
            b = f"blk.{l}."
            out[b + "attn_norm"] = T[b + "attn_norm"][2].astype(np.float32)
            out[b + "ffn_norm"] = T[b + "ffn_norm"][2].astype(np.float32)
            out[b + "attn_qkv"] = np.concatenate([T[b + "attn_q"][2], T[b + "attn_k"][2], T[b + "attn_v"][2]])
            out[b + "attn_output"] = T[b + "attn_output"][2]
            out[b + "ffn_gate_up"] = np.concatenate([T[b + "ffn_gate"][2], T[b + "ffn_up"][2]])
            out[b + "ffn_down"] = T[b + "ffn_down"][2]
        return out


def _first_param(program: dict[str, Any], op: str, key: str):
    for st in program.get("stages", []):
        for n in st.get("nodes", []):
            if n.get("op") == op and key in n.get("p", {}):
                return n["p"][key]
    return None


def read_causal_lm(path: str | Path) -> CausalLM:
    r = GGUFReader(path)
    try:
        names = json.loads(r.kv.get("ggml_compiler.tensor_names", "{}"))
        program = json.loads(r.kv.get("ggml_compiler.program", "{}"))
        meta = json.loads(r.kv.get("ggml_compiler.meta", "{}"))
    except json.JSONDecodeError as e:
        raise GGUFError(f"{path}: bad ggml_compiler metadata: {e}") from e
    if not names:
        raise GGUFError(f"{path}: no ggml_compiler.tensor_names (not a ggml-compiler file)")
    by_fqn = {fqn: gname for gname, fqn in names.items()}
    T: dict[str, tuple[int, tuple[int, ...], np.ndarray]] = {}

    def take(fqn: str, role: str) -> None:
        gname = by_fqn.get(fqn)
        if gname is None or gname not in r.tensors:
            raise GGUFError(f"{path}: no tensor for {fqn}")
        ti = r.tensors[gname]
        T[role] = (ti.type, ti.ne, np.array(r.data(gname)))

    take("model.embed_tokens.weight", "token_embd")
    take("model.norm.weight", "output_norm")
    take("lm_head.weight" if "lm_head.weight" in by_fqn else "model.embed_tokens.weight", "output")
    layers = sorted({int(m.group(1)) for f in by_fqn if (m := _LAYER.match(f))})
    if layers != list(range(len(layers))) or not layers:
        raise GGUFError(f"{path}: decoder layers {layers[:4]}... are not 0..L-1")
    for l in layers:
        for mod, role in _ROLES.items():
            take(f"model.layers.{l}.{mod}.weight", f"blk.{l}.{role}")
    E = T["token_embd"][1][0]
    n_vocab = T["token_embd"][1][1]
    n_dims = _first_param(program, "rope", "n_dims")
    eps = _first_param(program, "rms_norm", "eps")
    base = _first_param(program, "rope", "freq_base")
    if n_dims is None or eps is None or base is None:
        raise GGUFError(f"{path}: the program has no rms_norm / rope nodes to take eps and the RoPE base from")
    D = int(n_dims)
    q_rows, k_rows = T["blk.0.attn_q"][1][1], T["blk.0.attn_k"][1][1]
    if q_rows % D or k_rows % D:
        raise GGUFError(f"{path}: q / k rows {q_rows} / {k_rows} are not multiples of the rotary size {D}")
    cfg = CausalLM(n_layer=len(layers), n_embd=E, n_head=q_rows // D, n_head_kv=k_rows // D, head_dim=D,
                   n_ff=T["blk.0.ffn_gate"][1][1], n_vocab=n_vocab, rms_eps=float(eps), rope_base=float(base),
                   max_context=meta.get("max_context"), tensors=T, meta=meta)
    r.close()
    return cfg


def write_causal_lm(path: str | Path, lm: CausalLM, program: dict[str, Any] | None = None) -> None:
    """Writes a model in the reference's layout: tensors "w.N" in module order with their module
    paths in ggml_compiler.tensor_names, the program JSON (by default one decode stage's rms_norm
    and rope nodes, enough for read_causal_lm), and the metadata."""
    w = GGUFWriter()
    order = [("model.embed_tokens.weight", "token_embd")]
    for l in range(lm.n_layer):
        for mod, role in _ROLES.items():
            order.append((f"model.layers.{l}.{mod}.weight", f"blk.{l}.{role}"))
    order += [("model.norm.weight", "output_norm"), ("lm_head.weight", "output")]
    if program is None:
        program = {"format_version": 3, "stages": [{"name": "decode", "params": [], "outputs": [], "nodes": [
            {"id": "%0", "op": "rms_norm", "src": ["a.0"], "type": "f32", "ne": [lm.n_embd, 1], "p": {"eps": lm.rms_eps}},
            {"id": "%1", "op": "rope", "src": ["%0", "a.1"], "type": "f32", "ne": [lm.head_dim, lm.n_head, 1],
             "p": {"n_dims": lm.head_dim, "mode": 2, "freq_base": lm.rope_base, "freq_scale": 1.0,
                   "attn_factor": 1.0}}]}]}
    w.add("general.architecture", "ggml_compiler")
    w.add("ggml_compiler.format_version", 3)
    w.add("ggml_compiler.program", json.dumps(program, separators=(",", ":")))
    w.add("ggml_compiler.tensor_names", json.dumps({f"w.{i}": fqn for i, (fqn, _) in enumerate(order)},
                                                   separators=(",", ":")))
    w.add("ggml_compiler.meta", json.dumps(lm.meta, separators=(",", ":")))
    for i, (fqn, role) in enumerate(order):
        t, ne, data = lm.tensors[role]
        w.add_tensor(f"w.{i}", data, t, ne)
    w.write(path)
