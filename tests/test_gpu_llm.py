"""The Llama-style decoder on libgcq against the oracle's CPU run of the same graph.

Two tolerances, both the reference's own:
- every op of the path (mul_mat, flash_attn_ext, rms_norm, rope) is within 1e-3 of the oracle
  on identical inputs (the op tests; the north star's bar);
- a whole model's logits are within 1e-2 (tests/unit/test_llm.py:130-145 pins an O3 model, with
  flash attention, f16 KV cache and ggml rope, at 1e-2), and the 32-layer 8B-shaped model is
  compared by KL divergence of its next-token distributions (ggml_compiler/verify/parity.py:39-81).
The model-level bar is wider because ggml's own arithmetic has steps: K, V and Q are rounded to
f16 and every matmul input to Q8_0 codes, so a last-bit difference in an f32 value (a different
but equally valid summation order) now and then moves a value by one f16 ulp or one code, and
random-weight layers carry that forward. Kernel bugs show as errors far above these bars.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
TOL_LM = 1e-2


def _tiny(wtype=2, max_ctx=256, n_layer=2):
    from ggml_compiler_amd.llm import LlamaConfig

    return LlamaConfig(n_layer=n_layer, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=1000,
                       max_ctx=max_ctx, wtype=wtype, rms_eps=1e-5, rope_base=10000.0)


def _models(cfg, seed=0, max_prompt=64):
    from ggml_compiler_amd.llm import Model
    from llama_ref import OracleLlama

    m = Model(cfg, max_prompt=max_prompt)
    m.init_random(seed=seed)
    w = {name: m.get_weight(name) for name, *_ in m.weights()}
    return m, OracleLlama(cfg, w), w


def _same_greedy(got, ref):
    """Greedy tokens agree unless the reference's top two are closer than the logits' difference."""
    if int(np.argmax(got)) == int(np.argmax(ref)):
        return True
    top = np.sort(ref)[-2:]
    return top[1] - top[0] <= 2 * np.abs(got - ref).max()


@pytest.mark.parametrize("wtype", [2, 8])
def test_weights_are_the_synthetic_stream(gops, wtype):
    """init_random's weights equal the oracle's regeneration (normal stream + reference encoder)."""
    from llama_ref import random_weights

    cfg = _tiny(wtype)
    m, _, w = _models(cfg, seed=5)
    ref = random_weights(m.weights(), seed=5)
    for name in ref:
        assert np.array_equal(w[name], ref[name]), name
    m.set_weight("blk.1.ffn_down", ref["blk.0.ffn_down"])
    assert np.array_equal(m.get_weight("blk.1.ffn_down"), ref["blk.0.ffn_down"])


@pytest.mark.parametrize("wtype", [2, 8])
@pytest.mark.parametrize("n_prompt", [5, 12])
def test_prefill_and_decode_match_oracle(gops, orc, wtype, n_prompt):
    """5 tokens: the GEMV path; 12: the int8-MFMA GEMM path. Then decode steps through the
    captured graph: each step's logits and greedy token against the oracle."""
    cfg = _tiny(wtype)
    m, o, _ = _models(cfg, seed=1)
    prompt = orc.ids(n_prompt, seed=2, vocab=cfg.n_vocab).tolist()
    lg, lo = m.prefill(prompt), o.forward(prompt)
    assert orc.parity(lg, lo) < TOL_LM
    tok = int(np.argmax(lo))
    for step in range(6):
        lg, nxt = m.decode(tok)
        lo = o.forward([tok])
        assert orc.parity(lg, lo) < TOL_LM, step
        assert nxt == int(np.argmax(lg))
        assert _same_greedy(lg, lo), step
        tok = int(np.argmax(lo))
    assert m.position == n_prompt + 6


def test_device_generate_equals_host_loop(gops):
    """The on-device generate loop makes the tokens the host loop makes (test_llm.py:178-201)."""
    from ggml_compiler_amd.llm import Generator

    cfg = _tiny(2)
    m, _, _ = _models(cfg, seed=3)
    g = Generator(m)
    prompt = list(range(10, 30))
    host = g.generate(prompt, max_new=12)
    dev = g.generate(prompt, max_new=12, device=True)
    assert host == dev and len(dev) == 12


def test_prompt_chunks_and_reset(gops, orc):
    """A prompt longer than max_prompt runs in chunks; reset clears the cache."""
    from ggml_compiler_amd.llm import Model

    cfg = _tiny(2)
    big, o, w = _models(cfg, seed=4, max_prompt=64)
    small = Model(cfg, max_prompt=8)
    for name, arr in w.items():
        small.set_weight(name, arr)
    prompt = orc.ids(30, seed=6, vocab=cfg.n_vocab).tolist()
    a = big.prefill(prompt)
    b = small.prefill(prompt)
    ref = o.forward(prompt)
    assert orc.parity(a, ref) < TOL_LM and orc.parity(b, ref) < TOL_LM
    big.reset()
    assert big.position == 0
    assert np.array_equal(big.prefill(prompt), a)


def test_context_limits(gops):
    from ggml_compiler_amd import GcqError

    cfg = _tiny(2, max_ctx=32)
    m, _, _ = _models(cfg, seed=7, max_prompt=16)
    m.prefill(list(range(30)))
    with pytest.raises(GcqError, match="context full"):
        m.prefill([1, 2, 3])
    with pytest.raises(GcqError, match="out of range"):
        m.decode(cfg.n_vocab)


def _llama3_width(n_layer):
    from ggml_compiler_amd.llm import LlamaConfig

    return LlamaConfig(n_layer=n_layer, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=14336,
                       n_vocab=128256, max_ctx=256, wtype=2, rms_eps=1e-5, rope_base=500000.0)


def _close_lm(lg, lo, orc):
    """Logits of a wide model: finite, next-token KL below 1e-2 (verify/parity.py:39-81), correlation
    above 0.99, and no element off by more than 5% of the largest logit (a gross-error guard)."""
    assert np.isfinite(lg).all()
    assert orc.logit_kl(lg, lo) < 1e-2
    assert np.corrcoef(lg, lo)[0, 1] > 0.99
    assert orc.parity(lg, lo) < 5e-2


@pytest.mark.timeout(300)
def test_llama3_width_one_layer(gops, orc):
    """Every executor kernel at the 8B shapes (hidden 4096, GQA 32/8 x 128, SwiGLU 14336, vocab
    128256, RoPE 500000): a one-layer model, 16-token prompt (GEMM path) and two decode steps."""
    m, o, _ = _models(_llama3_width(1), seed=0, max_prompt=32)
    prompt = orc.ids(16, seed=1, vocab=128256).tolist()
    lg, lo = m.prefill(prompt), o.forward(prompt)
    _close_lm(lg, lo, orc)
    tok = int(np.argmax(lo))
    for _ in range(2):
        lg, _ = m.decode(tok)
        lo = o.forward([tok])
        _close_lm(lg, lo, orc)
        assert _same_greedy(lg, lo)
        tok = int(np.argmax(lo))


@pytest.mark.timeout(600)
def test_llama3_8b_shape_matches_oracle(gops, orc):
    """The 32-layer 8B-shaped Q4_0 decoder: weights pinned to the synthetic stream (two regenerated
    on the CPU), then a 16-token prompt and two decode steps; the next-token distributions within
    KL 1e-2 of the oracle's and the logits correlated above 0.99."""
    from llama_ref import random_weights

    m, o, w = _models(_llama3_width(32), seed=0, max_prompt=32)
    ref = random_weights(m.weights(), seed=0, names={"blk.0.attn_qkv", "blk.31.ffn_down"})
    for n, arr in ref.items():
        assert np.array_equal(w[n], arr), n
    prompt = orc.ids(16, seed=1, vocab=128256).tolist()
    rows = [(m.prefill(prompt), o.forward(prompt))]
    tok = int(np.argmax(rows[0][1]))
    for _ in range(2):
        lg, _ = m.decode(tok)
        lo = o.forward([tok])
        rows.append((lg, lo))
        tok = int(np.argmax(lo))
    for lg, lo in rows:
        assert np.isfinite(lg).all()
        assert orc.logit_kl(lg, lo) < 1e-2
        assert np.corrcoef(lg, lo)[0, 1] > 0.99
        assert orc.parity(lg, lo) < 0.2


@pytest.mark.parametrize("wtype", [2, 8])
def test_model_from_reference_layout_gguf(gops, orc, tmp_path, wtype):
    """A model written in ggml-compiler's GGUF layout (module paths, w.N tensors, eps and RoPE base in
    the program) loads into the decoder and matches the oracle's run of the same tensors."""
    from ggml_compiler_amd import gguf
    from ggml_compiler_amd.llm import Model
    from llama_ref import OracleLlama
    from test_gguf import tiny_lm

    p = tmp_path / "lm.gguf"
    gguf.write_causal_lm(p, tiny_lm(orc, wtype=wtype, seed=40))
    m = Model.from_gguf(p, max_prompt=16)
    assert (m.cfg.n_layer, m.cfg.n_head, m.cfg.n_head_kv, m.cfg.wtype) == (2, 4, 2, wtype)
    o = OracleLlama(m.cfg, gguf.read_causal_lm(p).stacked())
    prompt = orc.ids(9, seed=41, vocab=m.cfg.n_vocab).tolist()
    lg, lo = m.prefill(prompt), o.forward(prompt)
    assert orc.parity(lg, lo) < TOL_LM
    tok = int(np.argmax(lo))
    for step in range(4):
        lg, _ = m.decode(tok)
        lo = o.forward([tok])
        assert orc.parity(lg, lo) < TOL_LM, step
        tok = int(np.argmax(lo))
    m.close()
