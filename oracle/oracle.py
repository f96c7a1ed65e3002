"""ctypes binding of the CPU oracle (libgcq_oracle.so, built from gcq_oracle.c by oracle/Makefile).

TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the CPU baseline bench.py reports.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.
Every function mirrors one ggml CPU routine of the quantized mat-mul / KV-cache attention path;
gcq_oracle.c names the routine and the reference call site for each.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "lib" / "libgcq_oracle.so"

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 2, 8, 12, 13, 14, 15
TYPES = {"f32": F32, "f16": F16, "q4_0": Q4_0, "q8_0": Q8_0, "q4_K": Q4_K, "q4_k": Q4_K, "q5_K": Q5_K,
         "q5_k": Q5_K, "q6_K": Q6_K, "q6_k": Q6_K, "q8_K": Q8_K}
KQUANTS = (Q4_K, Q5_K, Q6_K)
ACT_AVX2, ACT_SCALAR = 0, 1

_lib: ctypes.CDLL | None = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB.exists():
        build()
    L = ctypes.CDLL(str(LIB))
    p, i64, i32, f = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
    sigs = {
        "orc_fp32_to_fp16": ([f], ctypes.c_uint16),
        "orc_fp16_to_fp32": ([ctypes.c_uint16], f),
        "orc_fp32_to_fp16_n": ([p, p, i64], None),
        "orc_fp16_to_fp32_n": ([p, p, i64], None),
        "orc_rnd64": ([ctypes.c_uint64, ctypes.c_uint64], ctypes.c_uint64),
        "orc_fill_normal": ([p, i64, ctypes.c_uint64, ctypes.c_uint64, f], None),
        "orc_fill_ids": ([p, i64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int32], None),
        "orc_block_size": ([i32], ctypes.c_size_t),
        "orc_type_size": ([i32], ctypes.c_size_t),
        "orc_row_size": ([i32, i64], ctypes.c_size_t),
        "orc_quantize": ([i32, p, i64, i64, p], ctypes.c_size_t),
        "orc_make_qkx2": ([p, p, p, p, i32, f, i32, p], f),
        "orc_make_qx16": ([p, p], f),
        "orc_quantize_act_q8_0": ([p, p, i64, i32], None),
        "orc_quantize_act_q8_K": ([p, p, i64], None),
        "orc_dequantize": ([i32, p, p, i64, i64], i32),
        "orc_block_isums": ([i32, p, p, i64, p], i64),
        "orc_mul_mat": ([i32, p, i64, i64, p, i64, p, i32], i32),
        "orc_rms_norm": ([p, p, i64, i64, f, i32], None),
        "orc_rope_neox": ([p, i64, i64, p, p, i64, i64, i64, i32, f, f, f, p], None),
        "orc_flash_attn_ext": ([p, i64, i64, p, i64, i64, p, i64, i64, p, i64, p,
                                i32, i32, i32, i32, i32, i32, f, i32], None),
        "orc_swiglu": ([p, p, p, i64], None),
        "orc_argmax": ([p, i64], i32),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def _tid(t: int | str) -> int:
    return TYPES[t] if isinstance(t, str) else int(t)


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def row_size(t: int | str, n: int) -> int:
    return int(lib().orc_row_size(_tid(t), n))


def fp32_to_fp16(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().orc_fp32_to_fp16_n(x.ctypes.data, y.ctypes.data, x.size)
    return y


def fp16_to_fp32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().orc_fp16_to_fp32_n(h.ctypes.data, y.ctypes.data, h.size)
    return y


def normal(shape, seed: int, std: float = 1.0, offset: int = 0) -> np.ndarray:
    out = np.empty(shape, np.float32)
    lib().orc_fill_normal(out.ctypes.data, out.size, seed, offset, std)
    return out


def ids(n: int, seed: int, vocab: int, offset: int = 0) -> np.ndarray:
    out = np.empty(n, np.int32)
    lib().orc_fill_ids(out.ctypes.data, n, seed, offset, vocab)
    return out


def quantize(x: np.ndarray, t: int | str) -> np.ndarray:
    """Weight encoder: f32 [rows, n] -> uint8 [rows, row_size]."""
    x = _c(x, np.float32)
    n = x.shape[-1]
    rows = x.size // n
    rs = row_size(t, n)
    if rs == 0:
        raise ValueError(f"type {t} cannot hold rows of {n}")
    out = np.empty(x.shape[:-1] + (rs,), np.uint8)
    lib().orc_quantize(_tid(t), x.ctypes.data, rows, n, out.ctypes.data)
    return out


def make_qkx2(x: np.ndarray, w: np.ndarray, nmax: int, rmin: float, nstep: int, trace: bool = False):
    """One 32-value sub-block's (scale, min) search of the Q4_K / Q5_K encoder: (codes, scale, min),
    and with trace the search's steps, float32 [nstep + 2, 40]: row 0 the min/max fit, row 1 + s
    candidate s, each [iscale, D > 0, scale, min, weighted error, taken, min used, 0, codes[32]]."""
    x, w = _c(x, np.float32), _c(w, np.float32)
    assert x.size == 32 and w.size == 32
    L = np.zeros(32, np.uint8)
    neg_min = ctypes.c_float(0.0)
    tr = np.zeros((nstep + 2, 40), np.float32) if trace else None
    scale = lib().orc_make_qkx2(x.ctypes.data, w.ctypes.data, L.ctypes.data, ctypes.byref(neg_min), nmax, rmin, nstep,
                                tr.ctypes.data if trace else None)
    out = (L, float(scale), -float(neg_min.value))
    return out + (tr,) if trace else out


def make_qx16(x: np.ndarray):
    """One 16-value sub-block's scale search of the Q6_K encoder: (codes l + 32, scale)."""
    x = _c(x, np.float32)
    assert x.size == 16
    L = np.zeros(16, np.uint8)
    scale = lib().orc_make_qx16(x.ctypes.data, L.ctypes.data)
    return L, float(scale)


def quantize_act_q8_0(x: np.ndarray, variant: int = ACT_AVX2) -> np.ndarray:
    x = _c(x, np.float32)
    n = x.shape[-1]
    rows = x.size // n
    out = np.empty(x.shape[:-1] + (row_size(Q8_0, n),), np.uint8)
    for r in range(rows):
        lib().orc_quantize_act_q8_0(x.reshape(rows, n)[r].ctypes.data, out.reshape(rows, -1)[r].ctypes.data, n,
                                    variant)
    return out


def quantize_act_q8_K(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    n = x.shape[-1]
    rows = x.size // n
    out = np.empty(x.shape[:-1] + (row_size(Q8_K, n),), np.uint8)
    x2, o2 = x.reshape(rows, n), out.reshape(rows, -1)
    for r in range(rows):
        lib().orc_quantize_act_q8_K(x2[r].ctypes.data, o2[r].ctypes.data, n)
    return out


def dequantize(q: np.ndarray, t: int | str, n: int) -> np.ndarray:
    q = _c(q, np.uint8)
    rs = row_size(t, n)
    rows = q.size // rs
    out = np.empty(q.shape[:-1] + (n,), np.float32)
    if lib().orc_dequantize(_tid(t), q.ctypes.data, out.ctypes.data, rows, n) != 0:
        raise ValueError("dequantize failed")
    return out


def block_isums(t: int | str, w_row: np.ndarray, xq_row: np.ndarray, k: int) -> np.ndarray:
    t = _tid(t)
    n = k // 32 if t in (Q4_0, Q8_0) else (17 if t == Q6_K else 10) * (k // 256)
    out = np.empty(n, np.int32)
    w_row, xq_row = _c(w_row, np.uint8), _c(xq_row, np.uint8)
    lib().orc_block_isums(t, w_row.ctypes.data, xq_row.ctypes.data, k, out.ctypes.data)
    return out


def mul_mat(wq: np.ndarray, t: int | str, x: np.ndarray, k: int, threads: int = 0) -> np.ndarray:
    """y [M, N] = x [M, K] (f32) times the quantized weight [N, K] transposed."""
    wq, x = _c(wq, np.uint8), _c(x, np.float32)
    N = wq.size // row_size(t, k)
    M = x.size // k
    y = np.empty((M, N), np.float32)
    if lib().orc_mul_mat(_tid(t), wq.ctypes.data, N, k, x.ctypes.data, M, y.ctypes.data, threads) != 0:
        raise ValueError("mul_mat failed")
    return y


def rms_norm(x: np.ndarray, eps: float, threads: int = 0) -> np.ndarray:
    x = _c(x, np.float32)
    n = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_rms_norm(x.ctypes.data, y.ctypes.data, x.size // n, n, eps, threads)
    return y


def rope_neox(x: np.ndarray, pos: np.ndarray, n_dims: int, base: float, freq_scale: float = 1.0,
              attn_factor: float = 1.0, freq_factors: np.ndarray | None = None) -> np.ndarray:
    """x [S, H, D] f32, pos [S] int32 -> [S, H, D]."""
    x = _c(x, np.float32)
    pos = _c(pos, np.int32)
    S, H, D = x.shape
    out = np.empty_like(x)
    ff = None if freq_factors is None else _c(freq_factors, np.float32)
    lib().orc_rope_neox(x.ctypes.data, H * D, D, out.ctypes.data, pos.ctypes.data, D, H, S, n_dims, base, freq_scale,
                        attn_factor, None if ff is None else ff.ctypes.data)
    return out


def flash_attn_ext(q: np.ndarray, k16: np.ndarray, v16: np.ndarray, mask16: np.ndarray | None, scale: float,
                   threads: int = 0) -> np.ndarray:
    """q [H, Sq, D] f32; k16/v16 [Hkv, n_kv, D] uint16 (f16 bits); mask16 [Sq, n_kv] uint16 or None.
    Returns [Sq, H, Dv] f32 (ggml's [Dv, H, Sq] layout)."""
    q = _c(q, np.float32)
    k16, v16 = _c(k16, np.uint16), _c(v16, np.uint16)
    H, Sq, D = q.shape
    Hkv, n_kv, _ = k16.shape
    Dv = v16.shape[2]
    out = np.empty((Sq, H, Dv), np.float32)
    m = None if mask16 is None else _c(mask16, np.uint16)
    lib().orc_flash_attn_ext(q.ctypes.data, Sq * D, D, k16.ctypes.data, n_kv * D, D, v16.ctypes.data, n_kv * Dv, Dv,
                             None if m is None else m.ctypes.data, n_kv, out.ctypes.data, D, Dv, Sq, H, Hkv, n_kv,
                             scale, threads)
    return out


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g, u = _c(g, np.float32), _c(u, np.float32)
    y = np.empty_like(g)
    lib().orc_swiglu(g.ctypes.data, u.ctypes.data, y.ctypes.data, g.size)
    return y


def argmax(x: np.ndarray) -> int:
    x = _c(x, np.float32)
    return int(lib().orc_argmax(x.ctypes.data, x.size))


def parity(out: np.ndarray, ref: np.ndarray) -> float:
    """max |out - ref| / max(1, max |ref|), inf when out is not finite where ref is
    (ggml_compiler/verify/parity.py:22-36)."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    if out.shape != ref.shape:
        raise ValueError(f"shape {out.shape} vs {ref.shape}")
    if ref.size == 0:
        return 0.0
    if not np.isfinite(out[np.isfinite(ref)]).all():
        return float("inf")
    return float(np.max(np.abs(out - ref))) / max(1.0, float(np.max(np.abs(ref))))


def logit_kl(out: np.ndarray, ref: np.ndarray) -> float:
    """KL(ref || out) of the next-token distributions of one row of logits, as
    ggml_compiler/verify/parity.py:55-71 (token_stats) computes it; inf if out is not finite."""
    r = np.asarray(ref, np.float64)
    o = np.asarray(out, np.float64)
    if not np.isfinite(o).all():
        return float("inf")
    lr = r - r.max()
    lr -= np.log(np.exp(lr).sum())
    lo = o - o.max()
    lo -= np.log(np.exp(lo).sum())
    return float((np.exp(lr) * (lr - lo)).sum())
