"""Decode attention (ggml_flash_attn_ext over an f16 KV cache) against the oracle within 1e-3."""

import numpy as np
import pytest
import torch

from conftest import to_np

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _case(orc, H, Hkv, Sq, n_kv, D, ctx, seed, causal=True):
    q = orc.normal((H, Sq, D), seed=seed)
    kc = orc.fp32_to_fp16(orc.normal((Hkv, ctx, D), seed=seed + 1))
    vc = orc.fp32_to_fp16(orc.normal((Hkv, ctx, D), seed=seed + 2))
    pos = n_kv - Sq + np.arange(Sq)
    mask = np.where((np.arange(n_kv)[None] <= pos[:, None]) | (not causal), 0.0, -np.inf).astype(np.float32)
    return q, kc, vc, orc.fp32_to_fp16(mask)


def _run(gops, q, kc, vc, m16, n_kv, scale):
    tq = torch.from_numpy(q).cuda()
    tk = torch.from_numpy(kc.view(np.float16)).cuda()
    tv = torch.from_numpy(vc.view(np.float16)).cuda()
    tm = None if m16 is None else torch.from_numpy(m16.view(np.float16)).cuda()
    return to_np(gops.flash_attn_ext(tq, tk, tv, tm, scale, n_kv=n_kv))


@pytest.mark.parametrize("n_kv", [1, 17, 512, 4096, 32768])
def test_decode_llama_heads(gops, orc, n_kv):
    """32 query heads on 8 KV heads, d=128, one query at the last position (every key visible)."""
    H, Hkv, D = 32, 8, 128
    q, kc, vc, m16 = _case(orc, H, Hkv, 1, n_kv, D, n_kv, seed=40)
    out = _run(gops, q, kc, vc, m16, n_kv, 1 / np.sqrt(D))
    ref = orc.flash_attn_ext(q, kc, vc, m16, 1 / np.sqrt(D))
    assert orc.parity(out, ref) < TOL


def test_cache_view_and_masked_tail(gops, orc):
    """K/V are the first n_kv rows of a longer cache; keys past the position are -inf."""
    H, Hkv, D, ctx, n_kv, Sq = 32, 8, 128, 2048, 768, 3
    q, kc, vc, m16 = _case(orc, H, Hkv, Sq, n_kv, D, ctx, seed=41)
    m16 = m16.copy()
    m16[:, 700:] = orc.fp32_to_fp16(np.array([-np.inf], np.float32))[0]
    out = _run(gops, q, kc, vc, m16, n_kv, 0.088)
    ref = orc.flash_attn_ext(q, kc[:, :n_kv], vc[:, :n_kv], m16, 0.088)
    assert orc.parity(out, ref) < TOL


@pytest.mark.parametrize("H,Hkv,D", [(4, 4, 64), (8, 2, 128), (16, 2, 256), (6, 3, 128)])
def test_head_layouts(gops, orc, H, Hkv, D):
    q, kc, vc, m16 = _case(orc, H, Hkv, 2, 300, D, 300, seed=42)
    out = _run(gops, q, kc, vc, m16, 300, 0.1)
    assert orc.parity(out, orc.flash_attn_ext(q, kc, vc, m16, 0.1)) < TOL


def test_no_mask_and_fully_masked_row(gops, orc):
    q, kc, vc, _ = _case(orc, 4, 2, 2, 50, 128, 50, seed=43)
    out = _run(gops, q, kc, vc, None, 50, 0.125)
    assert orc.parity(out, orc.flash_attn_ext(q, kc, vc, None, 0.125)) < TOL
    mask = np.zeros((2, 50), np.float32)
    mask[1] = -np.inf
    m16 = orc.fp32_to_fp16(mask)
    out = _run(gops, q, kc, vc, m16, 50, 0.125)
    assert np.isfinite(out).all() and not out[1].any()
    assert orc.parity(out, orc.flash_attn_ext(q, kc, vc, m16, 0.125)) < TOL


def test_prefill_rows(gops, orc):
    H, Hkv, D, Sq = 32, 8, 128, 64
    q, kc, vc, m16 = _case(orc, H, Hkv, Sq, 512, D, 512, seed=44)
    out = _run(gops, q, kc, vc, m16, 512, 1 / np.sqrt(D))
    assert orc.parity(out, orc.flash_attn_ext(q, kc, vc, m16, 1 / np.sqrt(D))) < TOL


@pytest.mark.parametrize("n_kv", [1, 17, 129, 700, 1024, 1500, 2048, 2049, 4096, 32768])
@pytest.mark.parametrize("H,Hkv,D", [(32, 8, 128), (8, 8, 128), (8, 4, 64), (16, 4, 64), (64, 8, 128), (16, 2, 64)])
def test_decode_kernel_no_mask(gops, orc, n_kv, H, Hkv, D):
    """One query row: up to 2048 keys the lane-group kernel (splits of 64 keys at D = 128, 128 at
    D = 64, at most 512 / H of them, 4, 8 or 16 wavefronts each), beyond it the matrix-core kernel
    (16-key blocks per wavefront, Q·Kᵀ and Vᵀ·P on MFMA, online softmax per head, wavefronts merged
    in LDS); splits merged by k_attn_merge. Against the oracle within 1e-3, 1 to 8 query heads per
    KV head. 17 keys leave most wavefronts without a key; 129 gives three splits of 43 keys; 1500
    ends inside a 16-key block; 2048 / 2049 are the last lane-group and first matrix-core
    lengths."""
    q, kc, vc, _ = _case(orc, H, Hkv, 1, n_kv, D, n_kv, seed=45)
    out = _run(gops, q, kc, vc, None, n_kv, 1 / np.sqrt(D))
    ref = orc.flash_attn_ext(q, kc, vc, None, 1 / np.sqrt(D))
    assert orc.parity(out, ref) < TOL


@pytest.mark.parametrize("H,Hkv", [(32, 8), (16, 2)])
def test_decode_row_with_holes_in_the_mask(gops, orc, H, Hkv):
    """One query row with an f16 mask that drops keys inside blocks and whole blocks, and adds
    finite biases to others: the decode kernel's mask path against the oracle."""
    D, n_kv = 128, 1000
    q, kc, vc, _ = _case(orc, H, Hkv, 1, n_kv, D, n_kv, seed=46)
    mask = (orc.normal((1, n_kv), seed=47) * 0.5).astype(np.float32)
    mask[0, 3:9] = -np.inf
    mask[0, 64:160] = -np.inf
    mask[0, 997] = -np.inf
    m16 = orc.fp32_to_fp16(mask)
    out = _run(gops, q, kc, vc, m16, n_kv, 1 / np.sqrt(D))
    assert orc.parity(out, orc.flash_attn_ext(q, kc, vc, m16, 1 / np.sqrt(D))) < TOL
