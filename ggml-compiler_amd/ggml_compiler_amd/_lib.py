"""ctypes binding of libgcq.so (include/gcq.h and include/ggml_compiler_rt.h).

The library is found through $GCQ_LIB, else in this package's source tree
(ggml-compiler_amd/lib/libgcq.so), as the reference's bindings find libggml_compiler_rt
(ggml_compiler/runtime/session.py:47-63). There is no fallback: every op runs in libgcq's HIP
kernels, and a missing library or device is an error.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIBRARY = _PKG.parent / "lib" / "libgcq.so"
HEADERS = [_PKG.parents[1] / "include" / "gcq.h", _PKG.parents[1] / "include" / "ggml_compiler_rt.h"]


class GcqError(RuntimeError):
    """An error reported by libgcq (its gcq_last_error / ggml_compiler_last_error text)."""


class _Options(ctypes.Structure):
    _fields_ = [("backend", ctypes.c_int), ("device", ctypes.c_int), ("n_threads", ctypes.c_int),
                ("allow_cpu_fallback", ctypes.c_bool)]


def library_path() -> Path:
    env = os.environ.get("GCQ_LIB")
    if env:
        return Path(env)
    if LIBRARY.exists():
        return LIBRARY
    raise GcqError(f"{LIBRARY} not found: build it (make -C ggml-compiler_amd, or __graft_entry__.build())")


_lib: ctypes.CDLL | None = None

p, i32, i64, u64, sz, f32 = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_size_t,
                             ctypes.c_float)

SIGNATURES = {
    "gcq_version": ([], ctypes.c_char_p),
    "gcq_last_error": ([], ctypes.c_char_p),
    "gcq_device_count": ([], i32),
    "gcq_row_size": ([i32, i64], sz),
    "gcq_weight_size": ([i32, i64, i64], sz),
    "gcq_act_size": ([i32, i64, i64], sz),
    "gcq_mul_mat_workspace": ([i32, i64, i64], sz),
    "gcq_flash_attn_workspace": ([i32, i32, i32, i32, i32], sz),
    "gcq_quantize": ([i32, p, i64, i64, p, p], i32),
    "gcq_pack_weights": ([i32, p, i64, i64, p, p], i32),
    "gcq_dequantize": ([i32, p, i64, i64, p, p], i32),
    "gcq_quantize_act": ([i32, p, i64, i64, i64, p, p], i32),
    "gcq_act_to_ggml": ([i32, p, i64, i64, p, p], i32),
    "gcq_mul_mat": ([i32, p, i64, i64, p, i64, i64, p, i64, p, sz, p], i32),
    "gcq_mul_mat_q": ([i32, p, i64, i64, p, i64, p, i64, p, p], i32),
    "gcq_rms_norm_q8": ([p, i64, p, i64, i64, f32, p, p], i32),
    "gcq_rms_norm_mul_mat": ([i32, p, i64, i64, p, p, f32, p, p, p, sz, p], i32),
    "gcq_swiglu_q8": ([p, p, i64, i64, i64, p, p], i32),
    "gcq_block_isums": ([i32, p, i64, i64, p, i64, p, p], i32),
    "gcq_gemm_block_isums": ([i32, p, i64, i64, p, i64, i32, p, p], i32),
    "gcq_flash_attn_ext": ([p, i64, i64, p, i64, i64, p, i64, i64, p, i64, p, i32, i32, i32, i32, i32, i32, f32, p, sz,
                            p], i32),
    "gcq_rms_norm": ([p, i64, p, i64, p, i64, i64, f32, p], i32),
    "gcq_rope_neox": ([p, i64, i64, p, i64, i64, p, i64, i64, i64, i32, f32, f32, f32, p, p], i32),
    "gcq_set_rows_f16": ([p, i64, i64, p, i64, i64, p, i64, i64, i64, i64, p], i32),
    "gcq_get_rows": ([i32, p, i64, i64, p, i64, p, p], i32),
    "gcq_swiglu": ([p, p, p, i64, p], i32),
    "gcq_add": ([p, p, p, i64, i64, p], i32),
    "gcq_mul": ([p, p, p, i64, i64, p], i32),
    "gcq_argmax": ([p, i64, i64, i64, p, p], i32),
    "gcq_fill_normal": ([p, i64, u64, u64, f32, p], i32),
    "gcq_fill_ids": ([p, i64, u64, u64, ctypes.c_int32, p], i32),
    "gcq_llama_create": ([p, i32], p),
    "gcq_llama_free": ([p], None),
    "gcq_llama_init_random": ([p, u64, f32], i32),
    "gcq_llama_n_weights": ([p], i32),
    "gcq_llama_weight_info": ([p, i32, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int),
                               ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)], i32),
    "gcq_llama_set_weight": ([p, ctypes.c_char_p, p, sz], i32),
    "gcq_llama_get_weight": ([p, ctypes.c_char_p, p, sz], i32),
    "gcq_llama_reset": ([p], i32),
    "gcq_llama_position": ([p], i32),
    "gcq_llama_prefill": ([p, p, i32, p], i32),
    "gcq_llama_decode": ([p, ctypes.c_int32, p, p], i32),
    "gcq_llama_generate": ([p, ctypes.c_int32, i32, p], i32),
    "ggml_compiler_version": ([], ctypes.c_char_p),
    "ggml_compiler_last_error": ([], ctypes.c_char_p),
    "ggml_compiler_default_options": ([], _Options),
    "ggml_compiler_has_backend": ([i32], ctypes.c_bool),
    "ggml_compiler_quantize": ([ctypes.c_char_p, p, i64, i64, p, sz], sz),
    "ggml_compiler_row_size": ([ctypes.c_char_p, i64], sz),
}


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    lib = ctypes.CDLL(str(library_path()))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def error() -> GcqError:
    return GcqError(load().gcq_last_error().decode())


def check(rc: int) -> None:
    if rc != 0:
        raise error()
