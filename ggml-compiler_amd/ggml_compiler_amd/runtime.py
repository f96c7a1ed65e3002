"""The reference's ggml_compiler.runtime over libgcq (ggml_compiler/runtime/session.py:125-306):
version, quantize, has_backend, and Session, a GGUF program loaded by libgcq's loader
(include/ggml_compiler_rt.h) and run on the HIP backend."""

from __future__ import annotations

import ctypes
import json
import os
from dataclasses import dataclass
from typing import Any

import numpy as np

from ._lib import GcqError, Stats, TensorInfo as _CInfo, load

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


_DTYPES = {0: ("f32", np.float32), 1: ("f16", np.float16), 2: ("i32", np.int32)}


@dataclass(frozen=True)
class TensorInfo:
    name: str
    shape: tuple[int, ...]
    dtype: str
    nbytes: int


class Session:
    """A loaded ggml-compiler GGUF (session.py:160-306): `run` takes inputs positionally or by
    name and returns the entry's outputs by name. Symbolic dims are bound from the input shapes;
    `entries` maps each entry point to its (inputs, outputs); state (a KV cache) persists across
    runs until `reset()`."""

    def __init__(self, path: str | os.PathLike, backend: str = "auto", device: int = 0, n_threads: int = 0,
                 allow_cpu_fallback: bool = False) -> None:
        lib = load()
        if backend not in _BACKENDS:
            raise ValueError(f"backend must be one of {sorted(_BACKENDS)}")
        opt = lib.ggml_compiler_default_options()
        opt.backend, opt.device, opt.n_threads, opt.allow_cpu_fallback = (
            _BACKENDS[backend], device, n_threads, allow_cpu_fallback)
        self._m = lib.ggml_compiler_load(os.fsencode(path), ctypes.byref(opt))
        if not self._m:
            raise _error()
        self.backend_name: str = lib.ggml_compiler_backend_name(self._m).decode()
        self._np: dict[str, np.dtype] = {}
        self.entries: dict[str, tuple[list[TensorInfo], list[TensorInfo]]] = {}
        for e in range(lib.ggml_compiler_n_entries(self._m)):
            ins = [self._info(lib.ggml_compiler_entry_input_info, e, k)
                   for k in range(lib.ggml_compiler_entry_n_inputs(self._m, e))]
            outs = [self._info(lib.ggml_compiler_entry_output_info, e, k)
                    for k in range(lib.ggml_compiler_entry_n_outputs(self._m, e))]
            self.entries[lib.ggml_compiler_entry_name(self._m, e).decode()] = (ins, outs)
        self.inputs, self.outputs = next(iter(self.entries.values()))
        self.symbols: dict[str, tuple[int, int]] = {}
        for k in range(lib.ggml_compiler_n_symbols(self._m)):
            name, lo, hi = ctypes.c_char_p(), ctypes.c_int64(), ctypes.c_int64()
            lib.ggml_compiler_symbol_info(self._m, k, ctypes.byref(name), ctypes.byref(lo), ctypes.byref(hi), None)
            self.symbols[name.value.decode()] = (lo.value, hi.value)

    def _info(self, fn, e: int, k: int) -> TensorInfo:
        info = _CInfo()
        if fn(self._m, e, k, ctypes.byref(info)) != 0:
            raise _error()
        name, (dtype, np_dtype) = info.name.decode(), _DTYPES[info.dtype]
        self._np[name] = np.dtype(np_dtype)
        return TensorInfo(name, tuple(info.shape[: info.ndim]), dtype, int(info.nbytes))

    @property
    def metadata(self) -> dict[str, Any]:
        """The program's own metadata ("ggml_compiler.meta"), or {}."""
        raw = load().ggml_compiler_metadata(self._m, b"ggml_compiler.meta")
        return json.loads(raw.decode()) if raw else {}

    def set_symbol(self, name: str, value: int) -> None:
        if load().ggml_compiler_set_symbol(self._m, name.encode(), int(value)) != 0:
            raise _error()

    def bound(self) -> dict[str, int]:
        lib, out = load(), {}
        for k in range(len(self.symbols)):
            name, v = ctypes.c_char_p(), ctypes.c_int64()
            lib.ggml_compiler_symbol_info(self._m, k, ctypes.byref(name), None, None, ctypes.byref(v))
            out[name.value.decode()] = v.value
        return out

    def reset(self) -> None:
        if load().ggml_compiler_reset(self._m) != 0:
            raise _error()

    def run(self, *args: Any, entry: str | None = None, **kwargs: Any) -> dict[str, np.ndarray]:
        lib = load()
        entry = entry or next(iter(self.entries))
        if entry not in self.entries:
            raise ValueError(f"no entry point {entry!r}; the model has {list(self.entries)}")
        inputs, outputs = self.entries[entry]
        if len(args) > len(inputs):
            raise TypeError(f"{len(args)} positional inputs for an entry with {len(inputs)} inputs")
        given = {t.name: a for t, a in zip(inputs, args)}
        for k, v in kwargs.items():
            if k in given:
                raise TypeError(f"input {k} given twice")
            given[k] = v
        names = [t.name for t in inputs]
        unknown = sorted(set(given) - set(names))
        if unknown:
            raise TypeError(f"unknown inputs {unknown}; the model takes {names}")
        missing = sorted(set(names) - set(given))
        if missing:
            raise TypeError(f"missing inputs {missing}")
        arrays = {t.name: np.ascontiguousarray(np.asarray(given[t.name]), dtype=self._np[t.name]) for t in inputs}
        for t in inputs:
            x = arrays[t.name]
            if not self.symbols:
                if x.shape != t.shape:
                    raise ValueError(f"input {t.name} has shape {x.shape}, the model expects {t.shape}")
                continue
            shape = (ctypes.c_int64 * max(1, x.ndim))(*x.shape)
            if lib.ggml_compiler_set_input_shape(self._m, t.name.encode(), x.ndim, shape) != 0:
                raise _error()
        for t in inputs:
            x = arrays[t.name]
            if lib.ggml_compiler_set_input(self._m, t.name.encode(), x.ctypes.data, x.nbytes) != 0:
                raise _error()
        if lib.ggml_compiler_run_entry(self._m, entry.encode()) != 0:
            raise _error()
        if self.symbols:
            e = list(self.entries).index(entry)
            outputs = [self._info(lib.ggml_compiler_entry_output_info, e, k) for k in range(len(outputs))]
        out = {}
        for t in outputs:
            y = np.empty(t.shape, dtype=self._np[t.name])
            if lib.ggml_compiler_get_output(self._m, t.name.encode(), y.ctypes.data, y.nbytes) != 0:
                raise _error()
            out[t.name] = y
        return out

    @property
    def stats(self) -> dict[str, Any]:
        lib = load()
        st = Stats()
        if lib.ggml_compiler_last_stats(self._m, ctypes.byref(st)) != 0:
            raise _error()
        stages = {}
        for k in range(lib.ggml_compiler_n_stages(self._m)):
            name, ms, calls = ctypes.c_char_p(), ctypes.c_double(), ctypes.c_int()
            lib.ggml_compiler_stage_stats(self._m, k, ctypes.byref(name), ctypes.byref(ms), ctypes.byref(calls))
            stages[name.value.decode()] = {"ms": ms.value, "calls": calls.value}
        return {"ms_total": st.ms_total, "n_calls": st.n_calls, "stages": stages}

    def close(self) -> None:
        if getattr(self, "_m", None):
            load().ggml_compiler_free(self._m)
            self._m = None

    def __enter__(self) -> "Session":
        return self

    def __exit__(self, *exc: Any) -> None:
        self.close()

    def __del__(self) -> None:
        self.close()
