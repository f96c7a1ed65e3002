"""The decode step in one persistent launch (decode_step.hip, decode path 1) and with each layer's
attention and output projection in one launch (attn_oproj.hip, path 2) against the
five-launches-per-layer decode (decode path 0): the same operations in the same order, so every
logit is equal bit for bit.

Path 0 is the one compared with the oracle op by op and layer by layer (test_gpu_llm.py); equality
with it carries those checks over to paths 1 and 2. A missed barrier or a stale read between workgroups
(the hazards of a persistent kernel) would change values by far less than a tolerance could be
trusted to catch, which is why the comparison is exact.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _cfg(n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, max_ctx, wtype=2):
    from ggml_compiler_amd.llm import LlamaConfig

    return LlamaConfig(n_layer=n_layer, n_embd=n_embd, n_head=n_head, n_head_kv=n_head_kv, head_dim=head_dim,
                       n_ff=n_ff, n_vocab=n_vocab, max_ctx=max_ctx, wtype=wtype, rms_eps=1e-5, rope_base=10000.0)


def _run(m, path, prompt, feed, n_gen):
    m.decode_path = path
    assert m.decode_path == path
    m.reset()
    m.prefill(prompt, logits=False)
    rows, nexts = [], []
    for t in feed:
        lg, nxt = m.decode(int(t))
        rows.append(lg)
        nexts.append(nxt)
    gen = m.generate(int(feed[-1]), n_gen)
    return np.stack(rows), nexts, gen


CASES = {
    # name: (config, prompt tokens, fed tokens, generated)
    "tiny-d64-g2": (_cfg(2, 256, 4, 2, 64, 512, 1000, 256), 13, 6, 12),
    "tiny-q8": (_cfg(2, 256, 4, 2, 64, 512, 1000, 256, wtype=8), 13, 6, 12),
    "d128-g4-splits": (_cfg(3, 1024, 8, 2, 128, 2816, 3000, 2048), 600, 5, 20),
    "d64-g8-long-ff": (_cfg(2, 512, 8, 1, 64, 14336, 2000, 1024), 40, 4, 8),
}


@pytest.mark.parametrize("name", list(CASES))
def test_decode_paths_equal(gops, orc, name):
    from ggml_compiler_amd.llm import Model

    cfg, n_prompt, n_feed, n_gen = CASES[name]
    print(f"decode paths: {name} {cfg}", flush=True)
    m = Model(cfg, max_prompt=min(512, cfg.max_ctx))
    m.init_random(seed=3)
    m.decode_path = 1  # paths 1 and 2 fit every case above
    m.decode_path = 2
    prompt = orc.ids(n_prompt, seed=4, vocab=cfg.n_vocab).tolist()
    feed = orc.ids(n_feed, seed=5, vocab=cfg.n_vocab)
    r0, n0, g0 = _run(m, 0, prompt, feed, n_gen)
    assert np.isfinite(r0).all()
    for path in (1, 2):
        r1, n1, g1 = _run(m, path, prompt, feed, n_gen)
        assert np.array_equal(r0, r1), (name, path, float(np.abs(r0 - r1).max()))
        assert n0 == n1
        assert g0 == g1
    m.close()


def test_decode_step_8b_shape(gops, orc):
    """The 32-layer 8B-shaped Q4_0 decoder of the decode benchmark (max_ctx 640) after a 512-token
    prompt: four fed tokens and 32 generated, every path."""
    from ggml_compiler_amd.llm import LlamaConfig, Model

    cfg = LlamaConfig(n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=14336, n_vocab=128256,
                      max_ctx=640, wtype=2, rms_eps=1e-5, rope_base=500000.0)
    print("decode paths: 8B shape", flush=True)
    m = Model(cfg, max_prompt=512)
    m.init_random(seed=0)
    prompt = orc.ids(512, seed=5, vocab=cfg.n_vocab).tolist()
    feed = orc.ids(4, seed=6, vocab=cfg.n_vocab)
    r0, n0, g0 = _run(m, 0, prompt, feed, 32)
    for path in (1, 2):
        r1, n1, g1 = _run(m, path, prompt, feed, 32)
        assert np.array_equal(r0, r1), (path, float(np.abs(r0 - r1).max()))
        assert n0 == n1 and g0 == g1
    m.close()


def test_decode_path_switch_errors(gops):
    """Paths 1 and 2 are refused where the configuration does not fit them (max_ctx past 2048 keys)."""
    from ggml_compiler_amd._lib import GcqError
    from ggml_compiler_amd.llm import Model

    m = Model(_cfg(1, 256, 4, 2, 64, 512, 1000, 4096), max_prompt=16)
    assert m.decode_path == 0
    with pytest.raises(GcqError, match="does not fit"):
        m.decode_path = 1
    with pytest.raises(GcqError, match="does not fit"):
        m.decode_path = 2
    with pytest.raises(GcqError, match="decode path must be"):
        m.decode_path = 3
    m.close()
