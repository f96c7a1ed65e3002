"""The path's ops on device tensors, each one call into libgcq's C ABI (include/gcq.h).

torch provides device memory and the current stream only; every op's arithmetic runs in libgcq's
HIP kernels. Shapes are given in PyTorch order (outermost first); the ggml op each function
stands for and its reference call site are named per function.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from ._lib import GcqError, check, load

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 2, 8, 12, 13, 14, 15
TYPES = {"f32": F32, "f16": F16, "q4_0": Q4_0, "q8_0": Q8_0, "q4_K": Q4_K, "q4_k": Q4_K, "q5_K": Q5_K, "q5_k": Q5_K,
         "q6_K": Q6_K, "q6_k": Q6_K}
KQUANTS = (Q4_K, Q5_K, Q6_K)


def type_id(t: int | str) -> int:
    if isinstance(t, str):
        if t not in TYPES:
            raise ValueError(f"unknown type {t!r}; known: {sorted(TYPES)}")
        return TYPES[t]
    return int(t)


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def device_count() -> int:
    return int(load().gcq_device_count())


def require_device() -> None:
    if device_count() == 0:
        raise GcqError("no HIP device visible to libgcq")


def _cuda(x: torch.Tensor, dtype: torch.dtype, name: str) -> torch.Tensor:
    if not x.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if x.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {x.dtype}")
    return x


def row_size(t: int | str, n: int) -> int:
    return int(load().gcq_row_size(type_id(t), n))


def workspace(nbytes: int, device=None) -> torch.Tensor:
    """A 256-byte aligned scratch buffer (torch's caching allocator aligns to 512 bytes)."""
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device or "cuda")


# ----------------------------------------------------------------------------- weights


def quantize(x: torch.Tensor, t: int | str) -> torch.Tensor:
    """f32 rows [rows, n] -> ggml block bytes uint8 [rows, row_size], encoded on the GPU exactly as
    ggml's reference encoders (ggml_compiler_quantize, runtime/src/ggml_compiler_rt.cpp:859-876)."""
    t = type_id(t)
    x = _cuda(x, torch.float32, "x").contiguous()
    n = x.shape[-1]
    rows = x.numel() // n
    out = torch.empty(x.shape[:-1] + (row_size(t, n),), dtype=torch.uint8, device=x.device)
    check(load().gcq_quantize(t, _p(x), rows, n, _p(out), _stream()))
    return out


@dataclass
class QuantWeight:
    """A weight of N rows x K values in libgcq's packed device layout (gcq_pack_weights)."""

    type: int
    N: int
    K: int
    data: torch.Tensor  # uint8, gcq_weight_size bytes

    @classmethod
    def from_ggml(cls, raw: torch.Tensor, t: int | str, K: int) -> "QuantWeight":
        """From ggml block rows (uint8 [N, row_size], host or device): the weight upload of
        runtime/src/ggml_compiler_rt.cpp:445-479."""
        t = type_id(t)
        rs = row_size(t, K)
        if rs == 0:
            raise GcqError(load().gcq_last_error().decode())
        raw = raw.reshape(-1)
        if raw.numel() % rs:
            raise ValueError(f"{raw.numel()} bytes is not a whole number of {rs}-byte rows")
        N = raw.numel() // rs
        src = raw.to("cuda", non_blocking=False).contiguous()
        data = torch.empty(int(load().gcq_weight_size(t, N, K)), dtype=torch.uint8, device=src.device)
        check(load().gcq_pack_weights(t, _p(src), N, K, _p(data), _stream()))
        return cls(t, N, K, data)

    @classmethod
    def quantize(cls, w: torch.Tensor, t: int | str) -> "QuantWeight":
        return cls.from_ggml(quantize(w, t), t, w.shape[-1])

    def dequantize(self) -> torch.Tensor:
        out = torch.empty((self.N, self.K), dtype=torch.float32, device=self.data.device)
        check(load().gcq_dequantize(self.type, _p(self.data), self.N, self.K, _p(out), _stream()))
        return out


# ------------------------------------------------------------------------------ mul_mat


def act_size(wtype: int | str, B: int, K: int) -> int:
    return int(load().gcq_act_size(type_id(wtype), B, K))


def quantize_act(wtype: int | str, x: torch.Tensor) -> torch.Tensor:
    """x f32 [B, K] -> the weight type's vec_dot_type, device act layout (gcq_quantize_act)."""
    wtype = type_id(wtype)
    x = _cuda(x, torch.float32, "x").contiguous()
    B, K = x.shape
    act = workspace(act_size(wtype, B, K), x.device)
    check(load().gcq_quantize_act(wtype, _p(x), K, B, K, _p(act), _stream()))
    return act


def act_to_ggml(wtype: int | str, act: torch.Tensor, B: int, K: int) -> torch.Tensor:
    wtype = type_id(wtype)
    xt = Q8_K if wtype in KQUANTS else Q8_0
    out = torch.empty((B, row_size(xt, K)), dtype=torch.uint8, device=act.device)
    check(load().gcq_act_to_ggml(wtype, _p(act), B, K, _p(out), _stream()))
    return out


def mul_mat(w: QuantWeight, x: torch.Tensor) -> torch.Tensor:
    """ggml_mul_mat(w, x) (runtime/src/ops.cpp:107-119): x f32 [M, K] -> [M, N]."""
    x = _cuda(x, torch.float32, "x").contiguous()
    M, K = x.shape
    if K != w.K:
        raise ValueError(f"x has {K} columns, the weight {w.K}")
    y = torch.empty((M, w.N), dtype=torch.float32, device=x.device)
    ws_n = int(load().gcq_mul_mat_workspace(w.type, M, K))
    ws = workspace(ws_n, x.device)
    check(load().gcq_mul_mat(w.type, _p(w.data), w.N, K, _p(x), K, M, _p(y), w.N, _p(ws), ws.numel(), _stream()))
    return y


def mul_mat_q(w: QuantWeight, act: torch.Tensor, M: int, res: torch.Tensor | None = None,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """mul_mat on a pre-quantized activation; with res, y = res + W x (ggml_add fused; out may be res)."""
    y = torch.empty((M, w.N), dtype=torch.float32, device=act.device) if out is None else out
    check(load().gcq_mul_mat_q(w.type, _p(w.data), w.N, w.K, _p(act), M, _p(y), w.N, _p(res), _stream()))
    return y


def rms_norm_q8(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """ggml_rms_norm + mul by w + Q8_0 conversion of the result, fused -> act buffer."""
    x = _cuda(x, torch.float32, "x").contiguous()
    rows, n = x.shape
    act = workspace(act_size(Q4_0, rows, n), x.device)
    check(load().gcq_rms_norm_q8(_p(x), n, _p(w), rows, n, float(eps), _p(act), _stream()))
    return act


def rms_norm_mul_mat(w: QuantWeight, x: torch.Tensor, norm_w: torch.Tensor | None, eps: float,
                     res: torch.Tensor | None = None) -> torch.Tensor:
    """One row: ggml_rms_norm -> mul by norm_w -> ggml_mul_mat(w, .) [+ res], fused (norm_w None:
    the mul_mat alone). x f32 [K] or [1, K] -> [1, N]."""
    x = _cuda(x, torch.float32, "x").contiguous().reshape(1, -1)
    K = x.shape[1]
    if K != w.K:
        raise ValueError(f"x has {K} columns, the weight {w.K}")
    nw = None if norm_w is None else _cuda(norm_w, torch.float32, "norm_w").contiguous()
    y = torch.empty((1, w.N), dtype=torch.float32, device=x.device)
    ws = workspace(int(load().gcq_mul_mat_workspace(w.type, 1, K)), x.device)
    check(load().gcq_rms_norm_mul_mat(w.type, _p(w.data), w.N, K, _p(x), _p(nw), float(eps), _p(y), _p(res), _p(ws),
                                      ws.numel(), _stream()))
    return y


def swiglu_q8(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """silu(g) * u + Q8_0 conversion, fused -> act buffer. g, u [rows, n] sharing a row stride."""
    rows, n = g.shape
    act = workspace(act_size(Q4_0, rows, n), g.device)
    check(load().gcq_swiglu_q8(_p(g), _p(u), g.stride(0), rows, n, _p(act), _stream()))
    return act


def block_isums(w: QuantWeight, act: torch.Tensor, B: int) -> torch.Tensor:
    per = w.K // 32 if w.type in (Q4_0, Q8_0) else (17 if w.type == Q6_K else 10) * (w.K // 256)
    out = torch.empty((B, w.N, per), dtype=torch.int32, device=act.device)
    check(load().gcq_block_isums(w.type, _p(w.data), w.N, w.K, _p(act), B, _p(out), _stream()))
    return out


def gemm_block_isums(w: QuantWeight, act: torch.Tensor, M: int, blk: int) -> torch.Tensor:
    """The GEMM's int32 sums of K-block blk: [M, N] (Q4_0 / Q8_0: a 32-value block; Q6_K: a
    super-block's sum sc * dot) or [M, N, 2] (Q4_K / Q5_K: sum sc * dot, sum m * bsums)."""
    shape = (M, w.N, 2) if w.type in KQUANTS and w.type != Q6_K else (M, w.N)
    out = torch.empty(shape, dtype=torch.int32, device=act.device)
    check(load().gcq_gemm_block_isums(w.type, _p(w.data), w.N, w.K, _p(act), M, blk, _p(out), _stream()))
    return out


# ---------------------------------------------------------------------------- attention


def flash_attn_ext(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: torch.Tensor | None, scale: float,
                   n_kv: int | None = None) -> torch.Tensor:
    """ggml_flash_attn_ext with f32 accumulation (runtime/src/ops.cpp:217-243).
    q f32 [H, Sq, D] (strided allowed, unit inner stride); k, v f16 [Hkv, ctx, D] (a cache; the first
    n_kv rows are read); mask f16 [Sq, >= n_kv] or None. Returns f32 [Sq, H, D]."""
    _cuda(q, torch.float32, "q")
    _cuda(k, torch.float16, "k")
    _cuda(v, torch.float16, "v")
    H, Sq, D = q.shape
    Hkv, ctx, Dk = k.shape
    n_kv = ctx if n_kv is None else n_kv
    if q.stride(2) != 1 or k.stride(2) != 1 or v.stride(2) != 1:
        raise ValueError("q, k, v need a unit stride along the head dim")
    if mask is not None:
        _cuda(mask, torch.float16, "mask")
        if mask.stride(1) != 1:
            raise ValueError("mask rows must be contiguous")
    out = torch.empty((Sq, H, v.shape[2]), dtype=torch.float32, device=q.device)
    ws = workspace(int(load().gcq_flash_attn_workspace(Sq, H, Hkv, v.shape[2], n_kv)), q.device)
    check(load().gcq_flash_attn_ext(_p(q), q.stride(0), q.stride(1), _p(k), k.stride(0), k.stride(1), _p(v),
                                    v.stride(0), v.stride(1), _p(mask), 0 if mask is None else mask.stride(0),
                                    _p(out), Dk, v.shape[2], Sq, H, Hkv, n_kv, float(scale), _p(ws), ws.numel(),
                                    _stream()))
    return out


# ------------------------------------------------------------------------ norms and glue


def rms_norm(x: torch.Tensor, eps: float, w: torch.Tensor | None = None) -> torch.Tensor:
    """ggml_rms_norm (runtime/src/ops.cpp:144-148) over the last dim [, then ggml_mul by w]."""
    x = _cuda(x, torch.float32, "x").contiguous()
    n = x.shape[-1]
    y = torch.empty_like(x)
    check(load().gcq_rms_norm(_p(x), n, _p(y), n, _p(w), x.numel() // n, n, float(eps), _stream()))
    return y


def rope_neox(x: torch.Tensor, pos: torch.Tensor, n_dims: int, base: float, freq_scale: float = 1.0,
              attn_factor: float = 1.0, ff: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """ggml_rope_ext NEOX (runtime/src/ops.cpp:277-291): x f32 [S, H, D], pos int32 [S]."""
    _cuda(x, torch.float32, "x")
    _cuda(pos, torch.int32, "pos")
    S, H, D = x.shape
    out = torch.empty((S, H, D), dtype=torch.float32, device=x.device) if out is None else out
    check(load().gcq_rope_neox(_p(x), x.stride(0), x.stride(1), _p(out), out.stride(0), out.stride(1), _p(pos), D, H,
                               S, n_dims, float(base), float(freq_scale), float(attn_factor), _p(ff), _stream()))
    return out


def set_rows_f16(cache: torch.Tensor, src: torch.Tensor, idx: torch.Tensor) -> None:
    """ggml_set_rows into an f16 cache (runtime/src/ops.cpp:260-275): cache f16 [Hrows, ctx, D],
    src f32 [Hrows, n, D] (strided allowed), idx int32 [n]."""
    _cuda(cache, torch.float16, "cache")
    _cuda(src, torch.float32, "src")
    Hrows, n, D = src.shape
    check(load().gcq_set_rows_f16(_p(cache), cache.stride(0), cache.stride(1), _p(src), src.stride(0), src.stride(1),
                                  _p(idx), n, D, Hrows, cache.shape[1], _stream()))


def get_rows(table: torch.Tensor | QuantWeight, idx: torch.Tensor, t: int | str | None = None) -> torch.Tensor:
    """ggml_get_rows (runtime/src/ops.cpp:302-309) -> f32 [n, D]."""
    if isinstance(table, QuantWeight):
        tid, data, nrows, D = table.type, table.data, table.N, table.K
    else:
        tid = type_id(t) if t is not None else (F16 if table.dtype == torch.float16 else F32)
        data, (nrows, D) = table, table.shape
    n = idx.numel()
    out = torch.empty((n, D), dtype=torch.float32, device=idx.device)
    check(load().gcq_get_rows(tid, _p(data), nrows, D, _p(idx), n, _p(out), _stream()))
    return out


def swiglu(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    y = torch.empty_like(g)
    check(load().gcq_swiglu(_p(g.contiguous()), _p(u.contiguous()), _p(y), g.numel(), _stream()))
    return y


def add(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    y = torch.empty_like(a)
    check(load().gcq_add(_p(a), _p(b), _p(y), a.numel(), b.numel(), _stream()))
    return y


def mul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    y = torch.empty_like(a)
    check(load().gcq_mul(_p(a), _p(b), _p(y), a.numel(), b.numel(), _stream()))
    return y


def argmax(x: torch.Tensor) -> torch.Tensor:
    x = x.reshape(-1, x.shape[-1]).contiguous()
    out = torch.empty(x.shape[0], dtype=torch.int32, device=x.device)
    check(load().gcq_argmax(_p(x), x.shape[1], x.shape[0], x.shape[1], _p(out), _stream()))
    return out


def fill_normal(shape, seed: int, std: float = 1.0, offset: int = 0, device="cuda") -> torch.Tensor:
    out = torch.empty(shape, dtype=torch.float32, device=device)
    check(load().gcq_fill_normal(_p(out), out.numel(), seed, offset, float(std), _stream()))
    return out


def fill_ids(n: int, seed: int, vocab: int, offset: int = 0, device="cuda") -> torch.Tensor:
    out = torch.empty(n, dtype=torch.int32, device=device)
    check(load().gcq_fill_ids(_p(out), n, seed, offset, vocab, _stream()))
    return out
