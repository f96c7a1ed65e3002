"""Python view of libgcq's ggml API subset (include/ggml.h, ggml-backend.h, ggml-alloc.h).

`lib()` is the ctypes library with the ggml signatures set; `T(ptr)` reads a tensor's fields
(type, ne, nb, op, data ...). `DecodeGraph` builds, through those calls, the decode-step graph
the reference's causal_lm stage builder makes (ggml_compiler/llm.py:361-444, node order of
runtime/src/ops.cpp's dispatcher) over weights and a KV cache held in HIP buffers, and computes
it with ggml_backend_graph_compute.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np

from . import _lib

F32, F16, Q4_0, Q8_0, Q4_K, I32 = 0, 1, 2, 8, 12, 26
ROPE_NEOX = 2
PREC_F32 = 10
FLAG_INPUT, FLAG_OUTPUT = 1, 2
OP = {name: i for i, name in enumerate(
    ["NONE", "ADD", "MUL", "SCALE", "CPY", "CONT", "RESHAPE", "VIEW", "PERMUTE", "TRANSPOSE", "GET_ROWS",
     "SET_ROWS", "RMS_NORM", "MUL_MAT", "ROPE", "FLASH_ATTN_EXT", "ARGMAX", "GLU", "UNARY", "SOFT_MAX", "IM2COL",
     "CONV_2D_DIRECT"])}


class Tensor(ctypes.Structure):
    """struct ggml_tensor (include/ggml.h)."""
    _fields_ = [("type", ctypes.c_int), ("buffer", ctypes.c_void_p), ("ne", ctypes.c_int64 * 4),
                ("nb", ctypes.c_size_t * 4), ("op", ctypes.c_int), ("op_params", ctypes.c_int32 * 16),
                ("flags", ctypes.c_int32), ("src", ctypes.c_void_p * 10), ("view_src", ctypes.c_void_p),
                ("view_offs", ctypes.c_size_t), ("data", ctypes.c_void_p), ("name", ctypes.c_char * 64),
                ("extra", ctypes.c_void_p)]


def lib() -> ctypes.CDLL:
    return _lib.load()


def T(ptr) -> Tensor:
    if not ptr:
        raise _lib.GcqError(lib().ggml_last_error().decode())
    return ctypes.cast(ptr, ctypes.POINTER(Tensor)).contents


def shape(ptr) -> tuple[int, ...]:
    return tuple(T(ptr).ne)


def strides(ptr) -> tuple[int, ...]:
    return tuple(T(ptr).nb)


def init(no_alloc: bool = True):
    ctx = lib().ggml_init(_lib.InitParams(1 << 20, None, no_alloc))
    if not ctx:
        raise _lib.GcqError("ggml_init failed")
    return ctx


def checked(fn, *args):
    """Call a void ggml function; raise with the library's message if it recorded an error."""
    before = lib().gcq_error_count()
    r = fn(*args)
    if lib().gcq_error_count() != before:
        raise _lib.GcqError(lib().ggml_last_error().decode())
    return r


def nbytes(t) -> int:
    return lib().ggml_nbytes(t)


def set_data(t, a: np.ndarray) -> None:
    a = np.ascontiguousarray(a)
    if a.nbytes != nbytes(t):
        raise ValueError(f"{a.nbytes} bytes for a tensor of {nbytes(t)}")
    checked(lib().ggml_backend_tensor_set, t, a.ctypes.data, 0, a.nbytes)


def get_data(t, dtype, count: int | None = None) -> np.ndarray:
    n = nbytes(t)
    out = np.empty(n // np.dtype(dtype).itemsize, dtype)
    checked(lib().ggml_backend_tensor_get, t, out.ctypes.data, 0, n)
    return out if count is None else out[:count]


def compute(backend, graph) -> None:
    st = lib().ggml_backend_graph_compute(backend, graph)
    if st != 0:
        raise _lib.GcqError(f"graph compute: {lib().ggml_status_to_string(st).decode()}: "
                            f"{lib().ggml_last_error().decode()}")


class Backend:
    """A HIP backend (ggml_backend_hip_init) freed on close."""

    def __init__(self, device: int = 0) -> None:
        self.be = lib().ggml_backend_hip_init(device)
        if not self.be:
            raise _lib.GcqError(lib().ggml_last_error().decode())

    def close(self) -> None:
        if self.be:
            lib().ggml_backend_free(self.be)
            self.be = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


class DecodeGraph:
    """The one-token decode step of a Llama-style causal LM as a ggml graph (the graph the
    reference's decode stage builds, llm.py:361-444): get_rows of the token's embedding; per layer
    rms_norm, mul, mul_mat q / k / v, rope (NEOX) of q and k, set_rows of k and v into an f16 cache
    [kv_heads, max_ctx, head_dim], flash_attn_ext over the first n_kv cache rows with an f16 mask,
    mul_mat o, add; rms_norm, mul, mul_mat gate / up, swiglu, mul_mat down, add; then rms_norm, mul
    and the lm_head mul_mat.

    weights: ggml block bytes by the HIP model's names (token_embd, blk.L.attn_norm,
    blk.L.attn_qkv (q, k, v rows stacked), blk.L.attn_output, blk.L.ffn_norm, blk.L.ffn_gate_up
    (gate, up rows stacked), blk.L.ffn_down, output_norm, output); the stacked weights are split
    into the separate q / k / v and gate / up tensors the reference's graph multiplies by.
    """

    def __init__(self, backend: Backend, cfg, weights: dict[str, np.ndarray], n_kv: int) -> None:
        g = lib()
        self.cfg, self.n_kv, self.be = cfg, n_kv, backend.be
        c = cfg
        H, Hkv, D, E, F = c.n_head, c.n_head_kv, c.head_dim, c.n_embd, c.n_ff
        wt = c.wtype
        row = g.ggml_row_size(wt, E)
        # weights and cache: one context, one buffer
        self.wctx = init()
        W = {}

        def leaf(name, typ, *ne):
            t = [g.ggml_new_tensor_1d, g.ggml_new_tensor_2d, g.ggml_new_tensor_3d][len(ne) - 1](self.wctx, typ, *ne)
            g.ggml_set_name(t, name.encode())
            W[name] = t
            return t

        leaf("token_embd", wt, E, c.n_vocab)
        for l in range(c.n_layer):
            b = f"blk.{l}."
            leaf(b + "attn_norm", F32, E)
            leaf(b + "attn_q", wt, E, H * D)
            leaf(b + "attn_k", wt, E, Hkv * D)
            leaf(b + "attn_v", wt, E, Hkv * D)
            leaf(b + "attn_output", wt, H * D, E)
            leaf(b + "ffn_norm", F32, E)
            leaf(b + "ffn_gate", wt, E, F)
            leaf(b + "ffn_up", wt, E, F)
            leaf(b + "ffn_down", wt, F, E)
            leaf(b + "cache_k", F16, D, c.max_ctx, Hkv)
            leaf(b + "cache_v", F16, D, c.max_ctx, Hkv)
        leaf("output_norm", F32, E)
        leaf("output", wt, E, c.n_vocab)
        self.wbuf = g.ggml_backend_alloc_ctx_tensors(self.wctx, self.be)
        if not self.wbuf:
            raise _lib.GcqError(g.ggml_last_error().decode())
        g.ggml_backend_buffer_clear(self.wbuf, 0)
        for name, t in W.items():
            if name.endswith(("cache_k", "cache_v")):
                continue
            src = name
            part = None
            if name.endswith(("attn_q", "attn_k", "attn_v")):
                src = name.rsplit(".", 1)[0] + ".attn_qkv"
                k = {"attn_q": 0, "attn_k": 1, "attn_v": 2}[name.rsplit(".", 1)[1]]
                lo = [0, H * D, (H + Hkv) * D][k]
                part = (lo, lo + (H * D if k == 0 else Hkv * D))
            elif name.endswith(("ffn_gate", "ffn_up")):
                src = name.rsplit(".", 1)[0] + ".ffn_gate_up"
                part = (0, F) if name.endswith("ffn_gate") else (F, 2 * F)
            a = weights[src]
            if part is not None:
                a = a.reshape(-1, row)[part[0]:part[1]]
            set_data(t, a)
        self.W = W
        self._build()

    def _build(self) -> None:
        g, c, W = lib(), self.cfg, self.W
        H, Hkv, D = c.n_head, c.n_head_kv, c.head_dim
        self.ctx = init()
        ctx = self.ctx
        self.tok = g.ggml_new_tensor_1d(ctx, I32, 1)
        self.pos = g.ggml_new_tensor_1d(ctx, I32, 1)
        self.mask = g.ggml_new_tensor_2d(ctx, F16, self.n_kv, 1)
        for t in (self.tok, self.pos, self.mask):
            g.ggml_set_input(t)
        x = g.ggml_get_rows(ctx, W["token_embd"], self.tok)
        for l in range(c.n_layer):
            b = f"blk.{l}."
            n = g.ggml_mul(ctx, g.ggml_rms_norm(ctx, x, c.rms_eps), W[b + "attn_norm"])
            q = g.ggml_mul_mat(ctx, W[b + "attn_q"], n)
            k = g.ggml_mul_mat(ctx, W[b + "attn_k"], n)
            v = g.ggml_mul_mat(ctx, W[b + "attn_v"], n)
            for t in (q, k, v):
                g.ggml_prec_set_acc(t, PREC_F32)
            q = g.ggml_rope_ext(ctx, g.ggml_reshape_3d(ctx, q, D, H, 1), self.pos, None, D, ROPE_NEOX, 0,
                                c.rope_base, 1.0, 0.0, 1.0, 32.0, 1.0)
            k = g.ggml_rope_ext(ctx, g.ggml_reshape_3d(ctx, k, D, Hkv, 1), self.pos, None, D, ROPE_NEOX, 0,
                                c.rope_base, 1.0, 0.0, 1.0, 32.0, 1.0)
            v = g.ggml_reshape_3d(ctx, v, D, Hkv, 1)
            kw = g.ggml_set_rows(ctx, W[b + "cache_k"], g.ggml_permute(ctx, k, 0, 2, 1, 3), self.pos)
            vw = g.ggml_set_rows(ctx, W[b + "cache_v"], g.ggml_permute(ctx, v, 0, 2, 1, 3), self.pos)
            rs = D * 2
            kv = g.ggml_view_3d(ctx, kw, D, self.n_kv, Hkv, rs, rs * c.max_ctx, 0)
            vv = g.ggml_view_3d(ctx, vw, D, self.n_kv, Hkv, rs, rs * c.max_ctx, 0)
            att = g.ggml_flash_attn_ext(ctx, g.ggml_permute(ctx, q, 0, 2, 1, 3), kv, vv, self.mask,
                                        1.0 / math.sqrt(D), 0.0, 0.0)
            g.ggml_prec_set_acc(att, PREC_F32)
            o = g.ggml_mul_mat(ctx, W[b + "attn_output"], g.ggml_reshape_2d(ctx, att, D * H, 1))
            x = g.ggml_add(ctx, x, o)
            n = g.ggml_mul(ctx, g.ggml_rms_norm(ctx, x, c.rms_eps), W[b + "ffn_norm"])
            gate = g.ggml_mul_mat(ctx, W[b + "ffn_gate"], n)
            up = g.ggml_mul_mat(ctx, W[b + "ffn_up"], n)
            x = g.ggml_add(ctx, x, g.ggml_mul_mat(ctx, W[b + "ffn_down"], g.ggml_swiglu_split(ctx, gate, up)))
        h = g.ggml_mul(ctx, g.ggml_rms_norm(ctx, x, c.rms_eps), W["output_norm"])
        self.logits = g.ggml_mul_mat(ctx, W["output"], h)
        T(self.logits)  # raises with the reason if any node failed
        g.ggml_set_output(self.logits)
        self.graph = g.ggml_new_graph_custom(ctx, 4096, False)
        g.ggml_build_forward_expand(self.graph, self.logits)
        self.galloc = g.ggml_gallocr_new(g.ggml_backend_get_default_buffer_type(self.be))
        if not g.ggml_gallocr_alloc_graph(self.galloc, self.graph):
            raise _lib.GcqError(g.ggml_last_error().decode())

    def reset(self) -> None:
        for l in range(self.cfg.n_layer):
            for k in ("cache_k", "cache_v"):
                checked(lib().ggml_backend_tensor_memset, self.W[f"blk.{l}.{k}"], 0, 0, nbytes(self.W[f"blk.{l}.{k}"]))

    def step(self, token: int, position: int) -> np.ndarray:
        """Feed one token at `position` (< n_kv); the logits."""
        mask = np.where(np.arange(self.n_kv) <= position, 0.0, -np.inf).astype(np.float16)
        set_data(self.tok, np.array([token], np.int32))
        set_data(self.pos, np.array([position], np.int32))
        set_data(self.mask, mask)
        compute(self.be, self.graph)
        return get_data(self.logits, np.float32)

    def close(self) -> None:
        g = lib()
        if getattr(self, "galloc", None):
            g.ggml_gallocr_free(self.galloc)
            self.galloc = None
        if getattr(self, "ctx", None):
            g.ggml_free(self.ctx)
            self.ctx = None
        if getattr(self, "wbuf", None):
            g.ggml_backend_buffer_free(self.wbuf)
            self.wbuf = None
        if getattr(self, "wctx", None):
            g.ggml_free(self.wctx)
            self.wctx = None
