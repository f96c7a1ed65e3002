"""Fused decode-step nodes equal their unfused ggml op sequence, byte for byte."""

import numpy as np
import pytest
import torch

from conftest import to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,n", [(1, 256), (3, 4096), (12, 14336)])
def test_rms_norm_q8_equals_norm_then_quantize(gops, orc, rows, n):
    x = torch.from_numpy(orc.normal((rows, n), seed=70) * 2).cuda()
    w = torch.from_numpy(orc.normal((n,), seed=71)).cuda()
    fused = gops.rms_norm_q8(x, w, 1e-5)
    unfused = gops.quantize_act("q4_0", gops.rms_norm(x, 1e-5, w))
    assert torch.equal(gops.act_to_ggml("q4_0", fused, rows, n), gops.act_to_ggml("q4_0", unfused, rows, n))


@pytest.mark.parametrize("rows,n", [(1, 512), (5, 14336)])
def test_swiglu_q8_equals_swiglu_then_quantize(gops, orc, rows, n):
    gu = torch.from_numpy(orc.normal((rows, 2 * n), seed=72)).cuda()
    g, u = gu[:, :n], gu[:, n:]
    fused = gops.swiglu_q8(g, u)
    unfused = gops.quantize_act("q4_0", gops.swiglu(g.contiguous(), u.contiguous()))
    assert torch.equal(gops.act_to_ggml("q4_0", fused, rows, n), gops.act_to_ggml("q4_0", unfused, rows, n))


@pytest.mark.parametrize("t", ["q4_0", "q8_0", "q4_K", "q5_K", "q6_K"])
@pytest.mark.parametrize("B,N,K", [(1, 512, 256), (1, 1000, 256), (2, 300, 512), (1, 40000, 4096), (3, 4096, 4096),
                                   (12, 256, 512)])
def test_mul_mat_q_with_residual(gops, orc, t, B, N, K):
    """y = res + W x in one launch equals W x then ggml_add; also in place (y is res). N=40000 runs
    the persistent GEMV's multi-group loop; 12 rows run the GEMMs (k_gemm for Q4_0 / Q8_0,
    k_gemm_kq for the K-quants)."""
    raw = orc.quantize(orc.normal((N, K), seed=73, std=0.02), t)
    qw = gops.QuantWeight.from_ggml(torch.from_numpy(raw), t, K)
    x = orc.normal((B, K), seed=74)
    act = gops.quantize_act(t, torch.from_numpy(x).cuda())
    r = torch.from_numpy(orc.normal((B, N), seed=75)).cuda()
    plain = gops.mul_mat_q(qw, act, B)
    fused = gops.mul_mat_q(qw, act, B, res=r)
    assert torch.equal(fused, plain + r)
    inplace = r.clone()
    gops.mul_mat_q(qw, act, B, res=inplace, out=inplace)
    assert torch.equal(inplace, plain + r)
    assert orc.parity(to_np(plain), orc.mul_mat(raw, t, x, K)) < 1e-3


@pytest.mark.parametrize("t", ["q4_0", "q8_0"])
@pytest.mark.parametrize("N,K", [(5, 256), (6144, 4096), (40000, 4096), (4096, 14336), (64, 16384 + 512)])
@pytest.mark.parametrize("norm", [True, False])
def test_rms_norm_mul_mat_equals_separate_launches(gops, orc, t, N, K, norm):
    """gcq_rms_norm_mul_mat (one launch for K <= 16384: the GEMV normalizes and quantizes its row)
    equals gcq_rms_norm_q8 (or gcq_quantize_act) + gcq_mul_mat_q bit for bit, with and without a
    residual, and is within 1e-3 of the oracle's rms_norm -> mul -> mul_mat. N=5 leaves most
    wavefronts without rows; N=40000 walks several row groups per wavefront; K=14336 is the down
    projection's shape (one row per wavefront, activation read from LDS); K=16896 takes the
    two-launch path."""
    raw = orc.quantize(orc.normal((N, K), seed=76, std=0.02), t)
    qw = gops.QuantWeight.from_ggml(torch.from_numpy(raw), t, K)
    x = orc.normal((1, K), seed=77) * 3
    nw = orc.normal((K,), seed=78) if norm else None
    xd = torch.from_numpy(x).cuda()
    nwd = None if nw is None else torch.from_numpy(nw).cuda()
    act = gops.rms_norm_q8(xd, nwd, 1e-5) if norm else gops.quantize_act(t, xd)
    plain = gops.mul_mat_q(qw, act, 1)
    fused = gops.rms_norm_mul_mat(qw, xd, nwd, 1e-5)
    assert torch.equal(fused, plain)
    r = torch.from_numpy(orc.normal((1, N), seed=79)).cuda()
    assert torch.equal(gops.rms_norm_mul_mat(qw, xd, nwd, 1e-5, res=r), plain + r)
    xn = orc.rms_norm(x, 1e-5) * nw[None, :] if norm else x
    assert orc.parity(to_np(fused), orc.mul_mat(raw, t, xn, K)) < 1e-3
