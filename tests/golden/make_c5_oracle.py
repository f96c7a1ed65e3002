"""Writes c5_oracle.npz: the oracle's run of the 8B-shaped decoder at its benchmark configuration,
for tests/test_gpu_llm.py's full-run comparison.

Configuration (the Llama-3-8B-shaped random-init decoder the decode benchmark runs): 32 layers,
hidden 4096, GQA 32 / 8 heads of 128, SwiGLU 14336, RMSNorm eps 1e-5, RoPE NEOX base 500000, vocab
128256, every matmul weight and the embedding ~N(0, 0.02) encoded as Q4_0 (the synthetic stream
gcq_llama_init_random draws: weight i from seed 0 + i), norm weights 1. A 512-token prompt of
uniform ids (oracle.ids(512, seed=PROMPT_SEED)), then 128 greedy tokens: token 0 is the argmax of
the prompt's last logits, token i the argmax after feeding token i - 1.

Stored per logit row (129 rows: the prompt's last, then one per fed token, the last unused for a
token): the greedy token, the margin between the two largest logits, the log-sum-exp, and the 64
largest logits with their ids; the whole first and last rows as float32. The oracle is the repo's
C restatement of ggml-cpu (oracle/), run on this machine's cores.

Run: python tests/golden/make_c5_oracle.py   (about 10 minutes on 8 cores)
"""

from __future__ import annotations

import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))

import oracle as orc  # noqa: E402
from llama_ref import OracleLlama, random_weights  # noqa: E402

PROMPT_SEED = 5
N_PROMPT = 512
N_GEN = 128
TOP = 64


class Cfg:
    n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab = 32, 4096, 32, 8, 128, 14336, 128256
    max_ctx = N_PROMPT + N_GEN
    wtype = orc.Q4_0
    rms_eps, rope_base = 1e-5, 500000.0


def weight_list(c) -> list[tuple[str, int, int, int]]:
    """(name, type, rows, cols) in gcq_llama_weight_info's order (q / k / v and gate / up row-stacked)."""
    qkv = (c.n_head + 2 * c.n_head_kv) * c.head_dim
    out = [("token_embd", c.wtype, c.n_vocab, c.n_embd)]
    for l in range(c.n_layer):
        b = f"blk.{l}."
        out += [(b + "attn_norm", orc.F32, 1, c.n_embd), (b + "attn_qkv", c.wtype, qkv, c.n_embd),
                (b + "attn_output", c.wtype, c.n_embd, c.n_head * c.head_dim), (b + "ffn_norm", orc.F32, 1, c.n_embd),
                (b + "ffn_gate_up", c.wtype, 2 * c.n_ff, c.n_embd), (b + "ffn_down", c.wtype, c.n_embd, c.n_ff)]
    out += [("output_norm", orc.F32, 1, c.n_embd), ("output", c.wtype, c.n_vocab, c.n_embd)]
    return out


def summarize(logits: np.ndarray):
    top = np.argsort(logits)[::-1][:TOP]
    two = np.sort(logits)[-2:]
    m = logits.max()
    lse = m + np.log(np.exp(logits.astype(np.float64) - m).sum())
    return int(top[0]), float(two[1] - two[0]), float(lse), top.astype(np.int32), logits[top].astype(np.float32)


def main() -> None:
    t0 = time.time()
    c = Cfg()
    w = random_weights(weight_list(c), seed=0)
    print(f"weights {time.time() - t0:.0f} s", flush=True)
    o = OracleLlama(c, w)
    prompt = orc.ids(N_PROMPT, seed=PROMPT_SEED, vocab=c.n_vocab)
    rows = [o.forward(prompt.tolist())]
    print(f"prompt {time.time() - t0:.0f} s", flush=True)
    for i in range(N_GEN):
        tok = int(np.argmax(rows[-1]))
        rows.append(o.forward([tok]))
        if i % 16 == 15:
            print(f"step {i + 1} {time.time() - t0:.0f} s", flush=True)
    s = [summarize(r) for r in rows]
    np.savez_compressed(Path(__file__).with_name("c5_oracle.npz"), prompt=prompt,
                        tokens=np.array([x[0] for x in s[:N_GEN]], np.int32),
                        margin=np.array([x[1] for x in s], np.float32), lse=np.array([x[2] for x in s]),
                        top_ids=np.stack([x[3] for x in s]), top_logits=np.stack([x[4] for x in s]),
                        first=rows[0].astype(np.float32), last=rows[-1].astype(np.float32))
    print(f"done {time.time() - t0:.0f} s", flush=True)


if __name__ == "__main__":
    main()
