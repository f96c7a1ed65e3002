"""The reference's ggml_compiler.runtime functions that need no program loader, over libgcq
(ggml_compiler/runtime/session.py:125-149): version, quantize, has_backend."""

from __future__ import annotations

import numpy as np

from ._lib import GcqError, load

_BACKENDS = {"cpu": 0, "cuda": 1, "auto": 2, "hip": 3}

GgmlCompilerRuntimeError = GcqError


def _error() -> GcqError:
    return GcqError(load().ggml_compiler_last_error().decode())


def version() -> str:
    return load().ggml_compiler_version().decode()


def quantize(data: np.ndarray, type_name: str) -> np.ndarray:
    """Encode f32 data (rows along the last axis) in a ggml type; uint8 [rows..., row_bytes]
    (session.py:133-145). The encoding runs in libgcq's GPU encoders."""
    lib = load()
    x = np.ascontiguousarray(data, dtype=np.float32)
    n = x.shape[-1]
    rows = x.size // n
    row_bytes = lib.ggml_compiler_row_size(type_name.encode(), n)
    if row_bytes == 0:
        raise _error()
    out = np.empty(x.shape[:-1] + (row_bytes,), dtype=np.uint8)
    if lib.ggml_compiler_quantize(type_name.encode(), x.ctypes.data, rows, n, out.ctypes.data, out.nbytes) == 0 \
            and out.nbytes:
        raise _error()
    return out


def has_backend(backend: str) -> bool:
    return bool(load().ggml_compiler_has_backend(_BACKENDS[backend]))
