"""ggml-compiler's Python runtime API on libgcq: version, quantize, has_backend and Session, a
program GGUF written by ggml-compiler loaded by libgcq's loader (include/ggml_compiler_rt.h) and
run on the HIP backend.

The public surface is the reference's (ggml_compiler/runtime/session.py: Session(path, backend,
device, n_threads, allow_cpu_fallback), .run(*inputs, entry=None, **inputs) -> {name: array},
.entries / .inputs / .outputs / .symbols / .metadata / .backend_name, .set_symbol, .bound,
.reset, .stats, .close, context manager), so code written against it runs here unchanged. Inside,
a Session keeps one `_Model` (the C handle and its queries) and an `_EntryPoint` per entry, which
binds a call's arguments with an inspect.Signature of the entry's inputs.
"""

from __future__ import annotations

import ctypes
import inspect
import json
import os
from typing import Any, NamedTuple

import numpy as np

from ._lib import GcqError, Stats, TensorInfo as _CTensorInfo, load

GgmlCompilerRuntimeError = GcqError

_BACKEND_IDS = {"cpu": 0, "cuda": 1, "auto": 2, "hip": 3}
_DTYPE_IDS = {0: "f32", 1: "f16", 2: "i32"}
_NUMPY = {"f32": np.dtype(np.float32), "f16": np.dtype(np.float16), "i32": np.dtype(np.int32)}


def _last_error() -> GcqError:
    return GcqError(load().ggml_compiler_last_error().decode())


def _check(rc: int) -> None:
    if rc != 0:
        raise _last_error()


def version() -> str:
    return load().ggml_compiler_version().decode()


def has_backend(backend: str) -> bool:
    return bool(load().ggml_compiler_has_backend(_BACKEND_IDS[backend]))


def quantize(data: np.ndarray, type_name: str) -> np.ndarray:
    """Encode f32 data in a ggml type, rows along the last axis: uint8 [..., row_bytes]. The
    encoding runs in libgcq's GPU encoders (ggml's reference algorithms)."""
    rows_f32 = np.ascontiguousarray(data, dtype=np.float32)
    n_per_row = rows_f32.shape[-1]
    lib = load()
    row_bytes = int(lib.ggml_compiler_row_size(type_name.encode(), n_per_row))
    if not row_bytes:
        raise _last_error()
    encoded = np.empty(rows_f32.shape[:-1] + (row_bytes,), dtype=np.uint8)
    n_rows = rows_f32.size // n_per_row if n_per_row else 0
    written = lib.ggml_compiler_quantize(type_name.encode(), rows_f32.ctypes.data, n_rows, n_per_row,
                                         encoded.ctypes.data, encoded.nbytes)
    if encoded.nbytes and not written:
        raise _last_error()
    return encoded


class TensorInfo(NamedTuple):
    """One input or output of an entry point: its name, PyTorch-order shape (symbols at the
    current binding), dtype name ("f32", "f16", "i32") and bytes."""
    name: str
    shape: tuple[int, ...]
    dtype: str
    nbytes: int


class _Model:
    """The C handle of a loaded program and the queries on it."""

    def __init__(self, path: str | os.PathLike, backend: str, device: int, n_threads: int,
                 allow_cpu_fallback: bool) -> None:
        if backend not in _BACKEND_IDS:
            raise ValueError(f"backend must be one of {sorted(_BACKEND_IDS)}")
        self.lib = load()
        opts = self.lib.ggml_compiler_default_options()
        opts.backend = _BACKEND_IDS[backend]
        opts.device = device
        opts.n_threads = n_threads
        opts.allow_cpu_fallback = allow_cpu_fallback
        self.ptr = self.lib.ggml_compiler_load(os.fsencode(path), ctypes.byref(opts))
        if not self.ptr:
            raise _last_error()

    def info(self, output: bool, entry: int, k: int) -> TensorInfo:
        raw = _CTensorInfo()
        fn = self.lib.ggml_compiler_entry_output_info if output else self.lib.ggml_compiler_entry_input_info
        _check(fn(self.ptr, entry, k, ctypes.byref(raw)))
        return TensorInfo(raw.name.decode(), tuple(int(d) for d in raw.shape[: raw.ndim]), _DTYPE_IDS[raw.dtype],
                          int(raw.nbytes))

    def symbol(self, k: int) -> tuple[str, int, int, int]:
        name, lo, hi, val = ctypes.c_char_p(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        _check(self.lib.ggml_compiler_symbol_info(self.ptr, k, ctypes.byref(name), ctypes.byref(lo), ctypes.byref(hi),
                                                  ctypes.byref(val)))
        return name.value.decode(), lo.value, hi.value, val.value

    def free(self) -> None:
        if self.ptr:
            self.lib.ggml_compiler_free(self.ptr)
            self.ptr = None


class _EntryPoint:
    """One entry of the program: its index, infos, and the signature its inputs form."""

    def __init__(self, model: _Model, index: int) -> None:
        lib = model.lib
        self.index = index
        self.name = lib.ggml_compiler_entry_name(model.ptr, index).decode()
        self.inputs = [model.info(False, index, k) for k in range(lib.ggml_compiler_entry_n_inputs(model.ptr, index))]
        self.outputs = [model.info(True, index, k) for k in range(lib.ggml_compiler_entry_n_outputs(model.ptr, index))]
        self.signature = inspect.Signature(
            [inspect.Parameter(t.name, inspect.Parameter.POSITIONAL_OR_KEYWORD) for t in self.inputs])

    def bind(self, args: tuple, kwargs: dict) -> dict[str, Any]:
        try:
            bound = self.signature.bind(*args, **kwargs)
        except TypeError as e:
            raise TypeError(f"entry {self.name!r} takes inputs {[t.name for t in self.inputs]}: {e}") from None
        return dict(bound.arguments)


def _host_array(x: Any, dtype: np.dtype) -> np.ndarray:
    if hasattr(x, "detach"):  # a torch tensor, without importing torch here
        x = x.detach().cpu().numpy()
    return np.ascontiguousarray(np.asarray(x), dtype=dtype)


class Session:
    """A ggml-compiler GGUF loaded onto the GPU.

    `run(*inputs, entry=None, **named)` executes one entry point (default: the first) and returns a
    dict of its outputs. Inputs may have any shape the program's symbolic dimensions admit; the
    symbols take their values from those shapes. `entries` gives every entry point's input and
    output descriptions, `inputs` / `outputs` the first one's. Persistent tensors (the KV cache)
    keep their contents from one run to the next; `reset()` clears them."""

    def __init__(self, path: str | os.PathLike, backend: str = "auto", device: int = 0, n_threads: int = 0,
                 allow_cpu_fallback: bool = False) -> None:
        self._model = _Model(path, backend, device, n_threads, allow_cpu_fallback)
        ptr, lib = self._model.ptr, self._model.lib
        self.backend_name: str = lib.ggml_compiler_backend_name(ptr).decode()
        self._entries = {ep.name: ep for ep in (_EntryPoint(self._model, e)
                                                for e in range(lib.ggml_compiler_n_entries(ptr)))}
        self.entries: dict[str, tuple[list[TensorInfo], list[TensorInfo]]] = {
            name: (ep.inputs, ep.outputs) for name, ep in self._entries.items()}
        self.inputs, self.outputs = next(iter(self.entries.values()))
        self.symbols: dict[str, tuple[int, int]] = {}
        for k in range(lib.ggml_compiler_n_symbols(ptr)):
            name, lo, hi, _ = self._model.symbol(k)
            self.symbols[name] = (lo, hi)

    @property
    def metadata(self) -> dict[str, Any]:
        """The JSON object stored under the GGUF key "ggml_compiler.meta" (empty when absent)."""
        text = self._model.lib.ggml_compiler_metadata(self._model.ptr, b"ggml_compiler.meta")
        return json.loads(text.decode()) if text else {}

    def set_symbol(self, name: str, value: int) -> None:
        """Set a symbol by hand: for symbols that no input's shape determines, such as how many
        times a driver loop iterates."""
        _check(self._model.lib.ggml_compiler_set_symbol(self._model.ptr, name.encode(), int(value)))

    def bound(self) -> dict[str, int]:
        """Symbol name -> the value it is bound to now."""
        return {name: val for name, _, _, val in (self._model.symbol(k) for k in range(len(self.symbols)))}

    def reset(self) -> None:
        """Clear every persistent state tensor to zeros, e.g. empty the KV cache before a new
        sequence."""
        _check(self._model.lib.ggml_compiler_reset(self._model.ptr))

    def run(self, *args: Any, entry: str | None = None, **kwargs: Any) -> dict[str, np.ndarray]:
        name = next(iter(self._entries)) if entry is None else entry
        ep = self._entries.get(name)
        if ep is None:
            raise ValueError(f"no entry point {name!r}; the model has {list(self._entries)}")
        given = ep.bind(args, kwargs)
        arrays = [(t, _host_array(given[t.name], _NUMPY[t.dtype])) for t in ep.inputs]
        lib, ptr = self._model.lib, self._model.ptr
        for t, a in arrays:  # shapes first: together they fix the symbols
            if not self.symbols:
                if a.shape != t.shape:
                    raise ValueError(f"input {t.name} has shape {a.shape}, the model expects {t.shape}")
                continue
            dims = (ctypes.c_int64 * max(1, a.ndim))(*a.shape)
            _check(lib.ggml_compiler_set_input_shape(ptr, t.name.encode(), a.ndim, dims))
        for t, a in arrays:
            _check(lib.ggml_compiler_set_input(ptr, t.name.encode(), a.ctypes.data, a.nbytes))
        _check(lib.ggml_compiler_run_entry(ptr, name.encode()))
        outputs = ep.outputs if not self.symbols else [self._model.info(True, ep.index, k)
                                                       for k in range(len(ep.outputs))]
        results = {}
        for t in outputs:
            buf = np.empty(t.shape, dtype=_NUMPY[t.dtype])
            _check(lib.ggml_compiler_get_output(ptr, t.name.encode(), buf.ctypes.data, buf.nbytes))
            results[t.name] = buf
        return results

    @property
    def stats(self) -> dict[str, Any]:
        """The last run: total ms and calls, and per stage {ms, calls} (GPU time of its calls)."""
        lib, ptr = self._model.lib, self._model.ptr
        total = Stats()
        _check(lib.ggml_compiler_last_stats(ptr, ctypes.byref(total)))
        stages = {}
        for k in range(lib.ggml_compiler_n_stages(ptr)):
            name, ms, calls = ctypes.c_char_p(), ctypes.c_double(), ctypes.c_int()
            _check(lib.ggml_compiler_stage_stats(ptr, k, ctypes.byref(name), ctypes.byref(ms), ctypes.byref(calls)))
            stages[name.value.decode()] = {"ms": ms.value, "calls": calls.value}
        return {"ms_total": total.ms_total, "n_calls": total.n_calls, "stages": stages}

    def close(self) -> None:
        model = getattr(self, "_model", None)
        if model is not None:
            model.free()

    def __enter__(self) -> "Session":
        return self

    def __exit__(self, *exc: Any) -> None:
        self.close()

    def __del__(self) -> None:
        self.close()
