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

The noise floor: the same oracle run again, teacher-forced with the first run's tokens, with every
element of every embedding row moved one float32 ulp up or down (a seeded coin per element), the
smallest change any difference in rounding can make. How far that run's logits land from the first
run's (floor_top: its logits at the stored top-64 ids; floor_kl: the first and last rows'
next-token KL) is how much 32 layers of this random-weight model amplify rounding-level noise, so
an implementation that rounds differently anywhere cannot be expected to land closer.

Run: python tests/golden/make_c5_oracle.py [--floor-only]   (about 7 minutes per run on 8 cores;
--floor-only adds the noise floor to an existing c5_oracle.npz)
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
FLOOR_SEED = 11
OUT = Path(__file__).with_name("c5_oracle.npz")


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


class UlpPerturbed(OracleLlama):
    """The oracle with every embedding element moved one ulp, up or down by a seeded coin."""

    def embed(self, tokens) -> np.ndarray:
        x = super().embed(tokens)
        up = np.random.default_rng(FLOOR_SEED + self.pos).random(x.shape) < 0.5
        return np.where(up, np.nextafter(x, np.float32(np.inf)), np.nextafter(x, np.float32(-np.inf)))


def run(o: OracleLlama, prompt: np.ndarray, tokens, t0: float) -> list[np.ndarray]:
    """Logit rows of the prompt, then of each fed token; tokens=None feeds the greedy ones."""
    rows = [o.forward(prompt.tolist())]
    print(f"prompt {time.time() - t0:.0f} s", flush=True)
    for i in range(N_GEN):
        tok = int(np.argmax(rows[-1])) if tokens is None else int(tokens[i])
        rows.append(o.forward([tok]))
        if i % 16 == 15:
            print(f"step {i + 1} {time.time() - t0:.0f} s", flush=True)
    return rows


def main() -> None:
    t0 = time.time()
    c = Cfg()
    w = random_weights(weight_list(c), seed=0)
    print(f"weights {time.time() - t0:.0f} s", flush=True)
    prompt = orc.ids(N_PROMPT, seed=PROMPT_SEED, vocab=c.n_vocab)
    if "--floor-only" in sys.argv:
        fx = dict(np.load(OUT))
    else:
        rows = run(OracleLlama(c, w), prompt, None, t0)
        s = [summarize(r) for r in rows]
        fx = dict(prompt=prompt, tokens=np.array([x[0] for x in s[:N_GEN]], np.int32),
                  margin=np.array([x[1] for x in s], np.float32), lse=np.array([x[2] for x in s]),
                  top_ids=np.stack([x[3] for x in s]), top_logits=np.stack([x[4] for x in s]),
                  first=rows[0].astype(np.float32), last=rows[-1].astype(np.float32))
    rows = run(UlpPerturbed(c, w), prompt, fx["tokens"], t0)
    fx["floor_top"] = np.stack([r[ids] for r, ids in zip(rows, fx["top_ids"])]).astype(np.float32)
    fx["floor_kl"] = np.array([orc.logit_kl(rows[0], fx["first"]), orc.logit_kl(rows[-1], fx["last"])])
    np.savez_compressed(OUT, **fx)
    print(f"done {time.time() - t0:.0f} s", flush=True)


if __name__ == "__main__":
    main()
