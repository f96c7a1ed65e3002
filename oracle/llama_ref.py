"""CPU reference of the Llama-style decoder, composed from the oracle's ggml restatements.

TEST INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke(), bench.py's cpu_baseline leg). It runs
the graph ggml-compiler's causal_lm emits per layer at O3 (ggml_compiler/llm.py:361-444;
tests/unit/test_llm.py:130-134): get_rows, then rms_norm, mul, mul_mat q/k/v, rope (NEOX),
set_rows into an f16 KV cache [kv_heads, max_ctx, head_dim] (llm.py:386), flash_attn_ext with the
causal mask of llm.py:355-358, mul_mat o, add, rms_norm, mul, mul_mat gate/up, swiglu, mul_mat
down, add; final rms_norm, mul and the lm_head mul_mat. Weights are ggml block bytes, q/k/v and
gate/up row-stacked as the HIP model stores them.
"""

from __future__ import annotations

import numpy as np

import oracle as orc


class OracleLlama:
    def __init__(self, cfg, weights: dict[str, np.ndarray], threads: int = 0, types: dict[str, int] | None = None) -> None:
        """weights: the stacked q / k / v and gate / up rows of cfg.wtype, or (with types, a type
        per tensor) the separate GGUF tensors."""
        self.cfg = cfg
        self.w = weights
        self.threads = threads
        self.t = cfg.wtype
        self.types = types or {}
        L, Hkv, ctx, D = cfg.n_layer, cfg.n_head_kv, cfg.max_ctx, cfg.head_dim
        self.k = np.zeros((L, Hkv, ctx, D), np.uint16)
        self.v = np.zeros((L, Hkv, ctx, D), np.uint16)
        self.pos = 0

    def reset(self) -> None:
        self.k[:] = 0
        self.v[:] = 0
        self.pos = 0

    def _mm(self, name: str, x: np.ndarray) -> np.ndarray:
        return orc.mul_mat(self.w[name], self.types.get(name, self.t), x, x.shape[1], threads=self.threads)

    def _mm_stacked(self, b: str, stacked: str, parts: tuple[str, ...], x: np.ndarray) -> np.ndarray:
        """The stacked rows' product, or the separate tensors' products side by side."""
        if b + stacked in self.w:
            return self._mm(b + stacked, x)
        return np.concatenate([self._mm(b + p, x) for p in parts], axis=1)

    def _norm(self, name: str, x: np.ndarray) -> np.ndarray:
        return orc.rms_norm(x, self.cfg.rms_eps, threads=self.threads) * self.w[name][None, :]

    def layer(self, l: int, x: np.ndarray, pos: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        """Layer l on residual rows x [S, n_embd] at positions pos (every key up to a row's position
        visible), K / V written into this model's cache: (rows after attention, output rows)."""
        mid = self.attention(l, x, pos)
        return mid, self.ffn(l, mid)

    def ffn(self, l: int, mid: np.ndarray) -> np.ndarray:
        """Layer l's feed-forward half on the rows after attention: mid + down(swiglu(gate, up))."""
        c = self.cfg
        b = f"blk.{l}."
        gu = self._mm_stacked(b, "ffn_gate_up", ("ffn_gate", "ffn_up"), self._norm(b + "ffn_norm", mid))
        return mid + self._mm(b + "ffn_down", orc.swiglu(gu[:, :c.n_ff], gu[:, c.n_ff:]))

    def attention(self, l: int, x: np.ndarray, pos: np.ndarray) -> np.ndarray:
        """Layer l's attention half: x + attn_output(flash_attn(rope(q), cache k, cache v))."""
        c = self.cfg
        S = x.shape[0]
        H, Hkv, D = c.n_head, c.n_head_kv, c.head_dim
        n_kv = int(pos[-1]) + 1
        mask = np.where(np.arange(n_kv)[None, :] <= pos[:, None], 0.0, -np.inf).astype(np.float32)
        b = f"blk.{l}."
        qkv = self._mm_stacked(b, "attn_qkv", ("attn_q", "attn_k", "attn_v"), self._norm(b + "attn_norm", x))
        q = orc.rope_neox(qkv[:, :H * D].reshape(S, H, D), pos, D, c.rope_base)
        k = orc.rope_neox(qkv[:, H * D:(H + Hkv) * D].reshape(S, Hkv, D), pos, D, c.rope_base)
        v = qkv[:, (H + Hkv) * D:].reshape(S, Hkv, D)
        self.k[l][:, pos] = orc.fp32_to_fp16(k.transpose(1, 0, 2))
        self.v[l][:, pos] = orc.fp32_to_fp16(v.transpose(1, 0, 2))
        att = orc.flash_attn_ext(q.transpose(1, 0, 2), self.k[l][:, :n_kv], self.v[l][:, :n_kv],
                                 orc.fp32_to_fp16(mask), 1.0 / np.sqrt(D), threads=self.threads)
        return x + self._mm(b + "attn_output", att.reshape(S, H * D))

    def embed(self, tokens) -> np.ndarray:
        return orc.dequantize(self.w["token_embd"][np.asarray(tokens)], self.types.get("token_embd", self.t),
                              self.cfg.n_embd)

    def forward(self, tokens) -> np.ndarray:
        """Append tokens at the next positions; logits of the last one."""
        c = self.cfg
        S = len(tokens)
        pos = np.arange(self.pos, self.pos + S, dtype=np.int32)
        x = self.embed(tokens)
        for l in range(c.n_layer):
            x = self.layer(l, x, pos)[1]
        self.pos += S
        h = self._norm("output_norm", x[-1:])
        return self._mm("output", h)[0]


def random_weights(model_weights, seed: int, std: float = 0.02, names=None) -> dict[str, np.ndarray]:
    """The weights gcq_llama_init_random draws (tensor i: the normal stream of seed + i, encoded by
    the reference encoder), regenerated on the CPU. model_weights: (name, type, rows, cols) in order."""
    out = {}
    for i, (name, t, rows, cols) in enumerate(model_weights):
        if names is not None and name not in names:
            continue
        if t == orc.F32:
            out[name] = np.ones(cols, np.float32)
        else:
            out[name] = orc.quantize(orc.normal((rows, cols), seed=seed + i, std=std), t)
    return out
