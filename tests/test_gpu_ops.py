"""rms_norm, rope, set_rows, get_rows and the decode step's glue ops against the oracle."""

import numpy as np
import pytest
import torch

from conftest import to_np

pytestmark = pytest.mark.gpu


def test_rms_norm(gops, orc):
    x = orc.normal((7, 4096), seed=50) * 3
    w = orc.normal((4096,), seed=51)
    tx = torch.from_numpy(x).cuda()
    assert orc.parity(to_np(gops.rms_norm(tx, 1e-5)), orc.rms_norm(x, 1e-5)) < 1e-5
    y = to_np(gops.rms_norm(tx, 1e-6, torch.from_numpy(w).cuda()))
    assert orc.parity(y, orc.rms_norm(x, 1e-6) * w) < 1e-5


@pytest.mark.parametrize("n_dims,base", [(128, 500000.0), (64, 10000.0)])
def test_rope_neox(gops, orc, n_dims, base):
    S, H, D = 9, 32, 128
    x = orc.normal((S, H, D), seed=52)
    pos = np.array([0, 1, 2, 63, 511, 512, 640, 1000, 4095], np.int32)
    y = to_np(gops.rope_neox(torch.from_numpy(x).cuda(), torch.from_numpy(pos).cuda(), n_dims, base))
    assert orc.parity(y, orc.rope_neox(x, pos, n_dims, base)) < 1e-4
    assert np.array_equal(y[0], x[0])  # position 0 is the identity


def test_rope_strided_in_place(gops, orc):
    """q/k heads rotated inside a fused QKV row, in place, as the decode step does."""
    S, D = 2, 128
    qkv = orc.normal((S, 48 * D), seed=53)
    pos = np.array([5, 6], np.int32)
    t = torch.from_numpy(qkv.copy()).cuda()
    qview = t[:, : 32 * D].view(S, 32, D)
    gops.rope_neox(qview, torch.from_numpy(pos).cuda(), D, 500000.0, out=qview)
    got = to_np(t)
    ref = orc.rope_neox(qkv[:, : 32 * D].reshape(S, 32, D), pos, D, 500000.0)
    assert orc.parity(got[:, : 32 * D].reshape(S, 32, D), ref) < 1e-4
    assert np.array_equal(got[:, 32 * D:], qkv[:, 32 * D:])


def test_set_rows_f16(gops, orc):
    Hkv, ctx, D, n = 8, 64, 128, 3
    cache = torch.zeros((Hkv, ctx, D), dtype=torch.float16, device="cuda")
    src = orc.normal((n, Hkv, D), seed=54)  # [s][h][d], written through a transposed view
    idx = np.array([5, 0, 63], np.int32)
    gops.set_rows_f16(cache, torch.from_numpy(src).cuda().permute(1, 0, 2), torch.from_numpy(idx).cuda())
    got = to_np(cache).view(np.uint16)
    want = np.zeros((Hkv, ctx, D), np.uint16)
    want[:, idx] = orc.fp32_to_fp16(src.transpose(1, 0, 2))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("t", ["q4_0", "q8_0", "q4_K", "q5_K", "q6_K"])
def test_get_rows_quantized_table(gops, orc, t):
    raw = orc.quantize(orc.normal((100, 4096), seed=55, std=0.02), t)
    qw = gops.QuantWeight.from_ggml(torch.from_numpy(raw), t, 4096)
    idx = np.array([99, 0, 7, 7], np.int32)
    got = to_np(gops.get_rows(qw, torch.from_numpy(idx).cuda()))
    want = orc.dequantize(raw[idx], t, 4096)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_get_rows_float_tables(gops, orc):
    tab = orc.normal((10, 64), seed=56)
    idx = torch.tensor([3, 9], dtype=torch.int32, device="cuda")
    assert np.array_equal(to_np(gops.get_rows(torch.from_numpy(tab).cuda(), idx)), tab[[3, 9]])
    t16 = torch.from_numpy(tab).cuda().half()
    assert np.array_equal(to_np(gops.get_rows(t16, idx)), to_np(t16.float())[[3, 9]])


def test_swiglu_add_mul(gops, orc):
    g = orc.normal((14336,), seed=57)
    u = orc.normal((14336,), seed=58)
    tg, tu = torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()
    assert orc.parity(to_np(gops.swiglu(tg, tu)), orc.swiglu(g, u)) < 1e-5
    a = orc.normal((4, 4096), seed=59)
    b = orc.normal((4096,), seed=60)
    ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    assert np.array_equal(to_np(gops.add(ta, tb)), a + b)
    assert np.array_equal(to_np(gops.mul(ta, tb)), a * b)


def test_argmax_first_of_ties(gops, orc):
    x = orc.normal((3, 128256), seed=61)
    x[1, 7] = x[1, 100000] = 50.0
    x[2] = -np.inf
    got = to_np(gops.argmax(torch.from_numpy(x).cuda()))
    assert list(got) == [orc.argmax(x[0]), 7, 0]
