"""GPU encoders, repacking, dequantization and activation quantizers against the oracle, byte
for byte (the north star's bit-exactness bar for dequantized weights and quantized codes)."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import to_np

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def test_fill_normal_matches_oracle_stream(gops, orc):
    n = 100_003
    got = to_np(gops.fill_normal((n,), seed=7, std=0.02, offset=12345))
    want = orc.normal((n,), seed=7, std=0.02, offset=12345)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ids = to_np(gops.fill_ids(1000, seed=3, vocab=128256))
    assert np.array_equal(ids, orc.ids(1000, seed=3, vocab=128256))


@pytest.mark.parametrize("t", ["q8_0", "q4_0", "q4_K", "q5_K", "q6_K"])
def test_weight_encoders_bit_exact(gops, orc, t):
    w = orc.normal((64, 1024), seed=11, std=0.02)
    w[3] = 0.0                      # zero row
    w[4] = 0.5                      # constant row
    w[5, :32] = np.linspace(-1, 1, 32, dtype=np.float32)  # exact ties of |x| at the ends
    w[6] *= 1e-4                    # tiny scales (fp16 subnormal d)
    got = to_np(gops.quantize(torch.from_numpy(w).cuda(), t))
    assert np.array_equal(got, orc.quantize(w, t))


@pytest.mark.parametrize("t", ["q4_K", "q5_K", "q6_K"])
def test_weight_encoders_bit_exact_many_superblocks(gops, orc, t):
    """32768 super-blocks (a 2048 x 4096 weight): the K-quant searches are sensitive to the last bit
    of every step (the sub-block weights sqrt(mean x^2) + |x| included, where a sqrt one ulp off
    changed about one super-block in 800), so every byte must still equal the oracle's."""
    w = orc.normal((2048, 4096), seed=31, std=0.02)
    got = to_np(gops.quantize(torch.from_numpy(w).cuda(), t))
    want = orc.quantize(w, t)
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:8].tolist()}"


def test_weight_encoder_kats(gops):
    kats = json.loads((GOLDEN / "quant_kats.json").read_text())
    for name, k in kats.items():
        if k["kind"] != "weight":
            continue
        x = torch.tensor([k["x"]], dtype=torch.float32).cuda()
        assert to_np(gops.quantize(x, k["type"]))[0].tobytes().hex() == k["hex"], name


def test_runtime_quantize_host_api(orc):
    from ggml_compiler_amd import runtime

    w = orc.normal((8, 512), seed=5, std=0.02)
    for t in ("q8_0", "q4_0", "q4_K", "q5_K", "q6_K", "f16"):
        assert np.array_equal(runtime.quantize(w, t), orc.quantize(w, t)), t
    assert runtime.has_backend("hip") and runtime.has_backend("auto") and not runtime.has_backend("cpu")


@pytest.mark.parametrize("t", ["q8_0", "q4_0", "q4_K", "q5_K", "q6_K"])
def test_pack_dequantize_bit_exact(gops, orc, t):
    w = orc.normal((37, 2048), seed=12, std=0.02)
    raw = orc.quantize(w, t)
    qw = gops.QuantWeight.from_ggml(torch.from_numpy(raw), t, 2048)
    got = to_np(qw.dequantize())
    want = orc.dequantize(raw, t, 2048)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("wt", ["q4_0", "q4_K", "q6_K"])
@pytest.mark.parametrize("B", [1, 5, 8])
def test_activation_quantizers_bit_exact(gops, orc, wt, B):
    K = 4096
    x = orc.normal((B, K), seed=13 + B)
    x[0, :32] = np.array([127, 2.5, -2.5, 0.5, -0.5, 1.5] + [0] * 26, np.float32)  # rounding ties
    if B > 1:
        x[1, :256] = 0.0  # all-zero blocks
    act = gops.quantize_act(wt, torch.from_numpy(x).cuda())
    got = to_np(gops.act_to_ggml(wt, act, B, K))
    want = orc.quantize_act_q8_K(x) if wt != "q4_0" else orc.quantize_act_q8_0(x, orc.ACT_AVX2)
    assert np.array_equal(got, want)


def test_activation_kats(gops):
    kats = json.loads((GOLDEN / "quant_kats.json").read_text())
    for name, k in kats.items():
        x = torch.tensor([k["x"]], dtype=torch.float32).cuda()
        if k["kind"] == "act_q8_0" and k["variant"] == "avx2":
            got = gops.act_to_ggml("q4_0", gops.quantize_act("q4_0", x), 1, x.shape[1])
        elif k["kind"] == "act_q8_K":
            got = gops.act_to_ggml("q4_K", gops.quantize_act("q4_K", x), 1, x.shape[1])
        else:
            continue
        assert to_np(got)[0].tobytes().hex() == k["hex"], name

