"""Causal LM decoding over libgcq (include/gcq.h, gcq_llama_*).

The counterpart of ggml_compiler.llm's Generator and bench (ggml_compiler/llm.py:473-683) for a
Llama-style model whose program runs on libgcq's HIP kernels instead of a compiled GGUF:

    m = Model(LlamaConfig.llama3_8b(), max_prompt=512)
    m.init_random(seed=0)                  # or m.set_weight(name, ggml_bytes) per weight
    gen = Generator(m)
    ids = gen.generate(prompt_ids, max_new=128, device=True)

Prefill, decode and generate are the reference program's entry points (llm.py:12-14, :421-436);
the KV cache is state that persists until reset.
"""

from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass, fields
from typing import Sequence

import numpy as np

from ._lib import GcqError, check, load

Q4_0, Q8_0 = 2, 8


class _Config(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_int), ("n_embd", ctypes.c_int), ("n_head", ctypes.c_int),
                ("n_head_kv", ctypes.c_int), ("head_dim", ctypes.c_int), ("n_ff", ctypes.c_int),
                ("n_vocab", ctypes.c_int), ("max_ctx", ctypes.c_int), ("wtype", ctypes.c_int),
                ("rms_eps", ctypes.c_float), ("rope_base", ctypes.c_float)]


@dataclass(frozen=True)
class LlamaConfig:
    n_layer: int
    n_embd: int
    n_head: int
    n_head_kv: int
    head_dim: int
    n_ff: int
    n_vocab: int
    max_ctx: int
    wtype: int = Q4_0
    rms_eps: float = 1e-5
    rope_base: float = 500000.0

    @classmethod
    def llama3_8b(cls, max_ctx: int = 1024, wtype: int = Q4_0) -> "LlamaConfig":
        """Llama-3-8B's shape: 32 layers, hidden 4096, 32/8 heads of 128, SwiGLU 14336, vocab 128256,
        RMSNorm eps 1e-5, RoPE theta 500000."""
        return cls(32, 4096, 32, 8, 128, 14336, 128256, max_ctx, wtype, 1e-5, 500000.0)

    def c(self) -> _Config:
        return _Config(*(getattr(self, f.name) for f in fields(self)))

    @property
    def qkv_dim(self) -> int:
        return (self.n_head + 2 * self.n_head_kv) * self.head_dim


class Model:
    """One gcq_llama: weights, KV cache and the captured decode step on the current HIP device."""

    def __init__(self, cfg: LlamaConfig, max_prompt: int = 512) -> None:
        self.cfg = cfg
        self._lib = load()
        self._m = self._lib.gcq_llama_create(ctypes.byref(cfg.c()), max_prompt)
        if not self._m:
            raise GcqError(self._lib.gcq_last_error().decode())
        self.max_prompt = max_prompt

    @classmethod
    def from_gguf(cls, path, max_ctx: int | None = None, max_prompt: int = 512) -> "Model":
        """A model loaded from a ggml-compiler GGUF of a Llama-style causal LM (gguf.read_causal_lm:
        Q4_0 or Q8_0 weights, shape from the tensors, eps and RoPE base from the program)."""
        from .gguf import read_causal_lm

        lm = read_causal_lm(path)
        m = cls(lm.config(max_ctx), max_prompt=max_prompt)
        for name, data in lm.stacked().items():
            m.set_weight(name, data)
        return m

    def close(self) -> None:
        if getattr(self, "_m", None):
            self._lib.gcq_llama_free(self._m)
            self._m = None

    def __del__(self) -> None:
        self.close()

    def init_random(self, seed: int = 0, std: float = 0.02) -> None:
        check(self._lib.gcq_llama_init_random(self._m, seed, std))

    def weights(self) -> list[tuple[str, int, int, int]]:
        """(name, type, rows, cols) in seed order."""
        out = []
        for i in range(self._lib.gcq_llama_n_weights(self._m)):
            name, t, r, c = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64()
            check(self._lib.gcq_llama_weight_info(self._m, i, ctypes.byref(name), ctypes.byref(t), ctypes.byref(r),
                                                  ctypes.byref(c)))
            out.append((name.value.decode(), t.value, r.value, c.value))
        return out

    def _nbytes(self, t: int, rows: int, cols: int) -> int:
        return cols * 4 if t == 0 else rows * self._lib.gcq_row_size(t, cols)

    def get_weight(self, name: str) -> np.ndarray:
        """ggml block bytes (uint8 [rows, row_size]) or f32 [cols] for a norm weight."""
        _, t, r, c = next(w for w in self.weights() if w[0] == name)
        n = self._nbytes(t, r, c)
        buf = np.empty(n, np.uint8)
        check(self._lib.gcq_llama_get_weight(self._m, name.encode(), buf.ctypes.data, n))
        return buf.view(np.float32) if t == 0 else buf.reshape(r, -1)

    def set_weight(self, name: str, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data)
        check(self._lib.gcq_llama_set_weight(self._m, name.encode(), data.ctypes.data, data.nbytes))

    def reset(self) -> None:
        check(self._lib.gcq_llama_reset(self._m))

    @property
    def position(self) -> int:
        return int(self._lib.gcq_llama_position(self._m))

    def prefill(self, tokens: Sequence[int], logits: bool = True) -> np.ndarray | None:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.cfg.n_vocab, np.float32) if logits else None
        check(self._lib.gcq_llama_prefill(self._m, t.ctypes.data, len(t), None if out is None else out.ctypes.data))
        return out

    def decode(self, token: int, logits: bool = True) -> tuple[np.ndarray | None, int]:
        out = np.empty(self.cfg.n_vocab, np.float32) if logits else None
        nxt = ctypes.c_int32()
        check(self._lib.gcq_llama_decode(self._m, int(token), None if out is None else out.ctypes.data,
                                         ctypes.byref(nxt)))
        return out, nxt.value

    def generate(self, first: int, n_new: int) -> list[int]:
        out = np.empty(max(1, n_new), np.int32)
        check(self._lib.gcq_llama_generate(self._m, int(first), int(n_new), out.ctypes.data))
        return out[:n_new].tolist()

    def forward_layers(self, x: np.ndarray, pos: int, first: int, count: int = 1) -> tuple[np.ndarray, np.ndarray]:
        """Layers [first, first + count) on given residual rows x [n, n_embd] at positions pos .. pos +
        n - 1 (the prompt kernels for n > 1, the decode step's for n == 1), their K / V cached:
        (output rows [n, n_embd], rows after each layer's attention [count, n, n_embd])."""
        x = np.ascontiguousarray(x, np.float32)
        n = x.shape[0]
        out = np.empty_like(x)
        mid = np.empty((count, n, self.cfg.n_embd), np.float32)
        check(self._lib.gcq_llama_forward_layers(self._m, x.ctypes.data, n, int(pos), int(first), int(count),
                                                 out.ctypes.data, mid.ctypes.data))
        return out, mid


class Generator:
    """Greedy decoding on the host or on the device (ggml_compiler/llm.py:473-634, text only)."""

    def __init__(self, model: Model, eos: Sequence[int] = ()) -> None:
        self.m = model
        self.eos = set(eos)

    def reset(self) -> None:
        self.m.reset()

    @property
    def n_past(self) -> int:
        return self.m.position

    def feed(self, ids: Sequence[int]) -> np.ndarray:
        """Append tokens to the context; the logits after the last one ([vocab])."""
        ids = list(ids)
        if len(ids) == 1:
            return self.m.decode(ids[0])[0]
        return self.m.prefill(ids)

    def generate(self, prompt: Sequence[int], max_new: int, stop: Sequence[int] | None = None,
                 device: bool = False) -> list[int]:
        """Greedy continuation of `prompt` from an empty context, stopping after max_new tokens or at a
        stop id (host loop only; the device loop runs max_new steps, as a benchmark would)."""
        self.reset()
        stop = self.eos if stop is None else set(stop)
        logits = self.feed(prompt)
        first = int(np.argmax(logits))
        if device:
            if max_new <= 1:
                return [first][:max_new]
            return [first] + self.m.generate(first, max_new - 1)
        out = [first]
        tok = first
        while len(out) < max_new and tok not in stop:
            _, tok = self.m.decode(tok, logits=False)
            out.append(tok)
        return out


def bench(model: Model, pp: int = 512, tg: int = 128, reps: int = 3, seed: int = 0,
          device: bool = True) -> dict[str, float]:
    """Tokens per second as llama-bench measures them (ggml_compiler/llm.py:637-683): pp = one
    prefill of pp tokens from an empty context; tg = tg single-token decodes after it, mean over
    reps after a warmup."""
    rng = np.random.default_rng(seed)
    out: dict[str, float] = {}
    pp_t, tg_t = [], []
    for r in range(reps + 1):
        ids = rng.integers(0, model.cfg.n_vocab, pp).tolist()
        model.reset()
        t0 = time.perf_counter()
        logits = model.prefill(ids)
        t1 = time.perf_counter()
        first = int(np.argmax(logits))
        if device:
            model.generate(first, tg)
        else:
            tok = first
            for _ in range(tg):
                _, tok = model.decode(tok, logits=False)
        t2 = time.perf_counter()
        if r:
            pp_t.append(t1 - t0)
            tg_t.append(t2 - t1)
    out[f"pp{pp}"] = pp / float(np.mean(pp_t))
    out[f"tg{tg}"] = tg / float(np.mean(tg_t))
    return out
