"""Quantized mul_mat (GEMV for 1..8 rows, int8-MFMA GEMM beyond) against the oracle: integer
block sums bit-exact, float outputs within 1e-3 of ggml's CPU result by the reference's parity
metric (ggml_compiler/verify/parity.py:22-36)."""

import numpy as np
import pytest
import torch

from conftest import to_np

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _weight(gops, orc, t, N, K, seed):
    raw = orc.quantize(orc.normal((N, K), seed=seed, std=0.02), t)
    return raw, gops.QuantWeight.from_ggml(torch.from_numpy(raw), t, K)


@pytest.mark.parametrize("t", ["q4_0", "q8_0", "q4_K", "q5_K", "q6_K"])
@pytest.mark.parametrize("B", [1, 3, 8])
def test_gemv_block_isums_bit_exact(gops, orc, t, B):
    N, K = 37, 1024
    raw, qw = _weight(gops, orc, t, N, K, 21)
    x = orc.normal((B, K), seed=22)
    act = gops.quantize_act(t, torch.from_numpy(x).cuda())
    got = to_np(gops.block_isums(qw, act, B))
    xq = orc.quantize_act_q8_K(x) if t in ("q4_K", "q5_K", "q6_K") else orc.quantize_act_q8_0(x)
    for b in range(B):
        for n in range(N):
            assert np.array_equal(got[b, n], orc.block_isums(t, raw[n], xq[b], K)), (b, n)


@pytest.mark.parametrize("t", ["q4_0", "q8_0", "q4_K", "q5_K", "q6_K"])
@pytest.mark.parametrize("B", list(range(1, 9)))
def test_gemv_matches_oracle(gops, orc, t, B):
    N, K = 1001, 4096
    raw, qw = _weight(gops, orc, t, N, K, 23)
    x = orc.normal((B, K), seed=24 + B)
    y = to_np(gops.mul_mat(qw, torch.from_numpy(x).cuda()))
    assert orc.parity(y, orc.mul_mat(raw, t, x, K)) < TOL


@pytest.mark.parametrize("t", ["q4_0", "q4_K", "q5_K", "q6_K"])
@pytest.mark.parametrize("N,K", [(6144, 4096), (512, 14336), (300, 256), (64, 16384 + 512)])
def test_gemv_llama_shapes(gops, orc, t, N, K):
    """The decode shapes (fused QKV 4096x6144, down 14336x4096 on a row slice) and K past one pass."""
    raw, qw = _weight(gops, orc, t, N, K, 25)
    x = orc.normal((2, K), seed=26)
    y = to_np(gops.mul_mat(qw, torch.from_numpy(x).cuda()))
    assert orc.parity(y, orc.mul_mat(raw, t, x, K)) < TOL


@pytest.mark.parametrize("t", ["q8_0", "q4_0"])
@pytest.mark.parametrize("M,N,K", [(9, 300, 512), (128, 256, 1024), (200, 333, 4096 + 96)])
def test_gemm_matches_oracle(gops, orc, t, M, N, K):
    raw, qw = _weight(gops, orc, t, N, K, 27)
    x = orc.normal((M, K), seed=28)
    y = to_np(gops.mul_mat(qw, torch.from_numpy(x).cuda()))
    assert orc.parity(y, orc.mul_mat(raw, t, x, K)) < TOL


@pytest.mark.parametrize("t", ["q8_0", "q4_0"])
def test_gemm_mfma_block_sums_bit_exact(gops, orc, t):
    M, N, K = 130, 70, 256
    raw, qw = _weight(gops, orc, t, N, K, 29)
    x = orc.normal((M, K), seed=30)
    act = gops.quantize_act(t, torch.from_numpy(x).cuda())
    xq = orc.quantize_act_q8_0(x)
    for blk in (0, 5, 7):
        got = to_np(gops.gemm_block_isums(qw, act, M, blk))
        want = np.array([[orc.block_isums(t, raw[n], xq[m], K)[blk] for n in range(N)] for m in range(M)])
        assert np.array_equal(got, want), blk


def test_gemm_prefill_shape_row_slices(gops, orc):
    """Q8_0 K=4096, N=14336, M=512 at full size; the oracle checks a slice of rows and columns
    (each output depends only on its own activation row and weight row)."""
    t, M, N, K = "q8_0", 512, 14336, 4096
    w = gops.fill_normal((N, K), seed=31, std=0.02)
    qw = gops.QuantWeight.quantize(w, t)
    x = gops.fill_normal((M, K), seed=32)
    y = to_np(gops.mul_mat(qw, x))
    rows = np.r_[0:8, 250:258, 504:512]
    cols = np.r_[0:64, 7000:7064, 14272:14336]
    raw = orc.quantize(orc.normal((N, K), seed=31, std=0.02)[cols], t)
    ref = orc.mul_mat(raw, t, orc.normal((M, K), seed=32)[rows], K)
    assert orc.parity(y[np.ix_(rows, cols)], ref) < TOL


KQ = ["q4_K", "q5_K", "q6_K"]


@pytest.mark.parametrize("t", KQ)
@pytest.mark.parametrize("M,N,K", [(9, 100, 256), (21, 300, 512), (200, 333, 2816), (256, 512, 1024),
                                   (300, 10958, 256)])
def test_gemm_kquant_matches_oracle(gops, orc, t, M, N, K):
    """The K-quant MFMA GEMM (M > 8 rows): one super-block (K 256), a partial row and column tile
    (9 x 100, 200 x 333), eleven super-blocks, a grid of 8 tiles (256 x 512, tiles renumbered per
    XCD), all with 64-column tiles (grids of at most one workgroup per CU); 300 x 10958 takes the
    128-column tiles (258 of them), partial in both dimensions."""
    raw, qw = _weight(gops, orc, t, N, K, 33)
    x = orc.normal((M, K), seed=34)
    y = to_np(gops.mul_mat(qw, torch.from_numpy(x).cuda()))
    assert orc.parity(y, orc.mul_mat(raw, t, x, K)) < TOL


@pytest.mark.parametrize("t", KQ)
def test_gemm_kquant_superblock_sums_bit_exact(gops, orc, t):
    """Per super-block, the GEMM's two integers (sum sc * sub-block dot; sum m * bsums, whose
    bsums the kernel splits as 64 hi + lo) equal the oracle's at every (m, n), over a partial tile
    in both dimensions. The activation has rows of extreme codes: all +127, all -127, and -127 /
    +127 alternating, so the block sums reach +-32 * 127 and the split's hi byte its ends."""
    M, N, K = 133, 70, 768
    raw, qw = _weight(gops, orc, t, N, K, 29)
    x = orc.normal((M, K), seed=30)
    x[3] = 1.0
    x[4] = -1.0
    x[5, 0::2], x[5, 1::2] = -1.0, 1.0
    act = gops.quantize_act(t, torch.from_numpy(x).cuda())
    xq = orc.quantize_act_q8_K(x)
    per = 17 if t == "q6_K" else 10
    want_all = np.array([[orc.block_isums(t, raw[n], xq[m], K) for n in range(N)] for m in range(M)])
    for sb in (0, 2):
        got = to_np(gops.gemm_block_isums(qw, act, M, sb))
        if t == "q6_K":
            want = want_all[:, :, sb * per + 16]
        else:
            want = want_all[:, :, sb * per + 8:sb * per + 10]
        assert got.shape == want.shape
        assert np.array_equal(got, want), sb
    # 128-column tiles: a 300 x 10958 grid (258 tiles), checked on the rows and columns of its
    # first and last tiles
    M, N, K = 300, 10958, 512
    raw, qw = _weight(gops, orc, t, N, K, 31)
    x = orc.normal((M, K), seed=32)
    act = gops.quantize_act(t, torch.from_numpy(x).cuda())
    xq = orc.quantize_act_q8_K(x)
    got = to_np(gops.gemm_block_isums(qw, act, M, 1))
    for m in (*range(0, 6), *range(290, 300)):
        for n in (*range(0, 40), *range(10900, 10958)):
            v = orc.block_isums(t, raw[n], xq[m], K)[per:]
            want = v[16] if t == "q6_K" else v[8:10]
            assert np.array_equal(got[m, n], want), (m, n)


@pytest.mark.parametrize("t", ["q4_K", "q5_K"])
def test_gemm_kquant_residual(gops, orc, t):
    """mul_mat_q on a pre-quantized K-quant activation of 16 rows with a residual (y = res + W x),
    including res aliased to y."""
    M, N, K = 16, 1000, 2048
    raw, qw = _weight(gops, orc, t, N, K, 44)
    x = orc.normal((M, K), seed=45)
    r = orc.normal((M, N), seed=46)
    act = gops.quantize_act(t, torch.from_numpy(x).cuda())
    want = orc.mul_mat(raw, t, x, K) + r
    y = to_np(gops.mul_mat_q(qw, act, M, res=torch.from_numpy(r).cuda()))
    assert orc.parity(y, want) < TOL
    rr = torch.from_numpy(r).cuda()
    gops.mul_mat_q(qw, act, M, res=rr, out=rr)
    assert np.array_equal(to_np(rr), y)


def test_gemv_is_linear_at_full_size(gops):
    """Size-independent property at the fused gate/up shape (4096 x 28672): the quantized
    activation of 2x is exactly twice that of x's codes scale, so y(2x) = 2 y(x) bit-for-bit."""
    qw = gops.QuantWeight.quantize(gops.fill_normal((28672, 4096), seed=35, std=0.02), "q4_0")
    x = gops.fill_normal((1, 4096), seed=36)
    y1 = gops.mul_mat(qw, x)
    y2 = gops.mul_mat(qw, 2 * x)
    assert torch.equal(2 * y1, y2)


_FULL = {}


def _full_weight(gops, t, N, K):
    """The weight once per (type, shape): N(0, 0.02) from the synthetic stream, encoded on the GPU
    (the encoder equals the oracle's byte for byte, test_gpu_quant.py), as ggml block bytes."""
    key = (t, N, K)
    if key not in _FULL:
        _FULL.clear()
        raw = gops.quantize(gops.fill_normal((N, K), seed=41, std=0.02), t)
        _FULL[key] = (raw.cpu().numpy(), gops.QuantWeight.from_ggml(raw, t, K))
    return _FULL[key]


@pytest.mark.parametrize("t", ["q4_0", "q4_K"])
@pytest.mark.parametrize("N,K", [(4096, 4096), (6144, 4096), (28672, 4096), (4096, 14336)])
@pytest.mark.parametrize("B", [1, 2, 4, 8])
def test_gemv_full_decode_shapes(gops, orc, t, N, K, B):
    """The decode shapes at full size for 1, 2, 4 and 8 rows, every output against the oracle:
    attention output 4096 x 4096, fused QKV 4096 x 6144, fused gate/up 4096 x 28672, down
    14336 x 4096 (the row GEMV's dispatch and the batched kernels' plans depend on N)."""
    raw, qw = _full_weight(gops, t, N, K)
    x = orc.normal((B, K), seed=42 + B)
    y = to_np(gops.mul_mat(qw, torch.from_numpy(x).cuda()))
    assert orc.parity(y, orc.mul_mat(raw, t, x, K)) < TOL


def test_gemv_c1_q8_0_4096(gops, orc):
    """C1 at its shape: Q8_0, 4096 x 4096, one row."""
    raw, qw = _full_weight(gops, "q8_0", 4096, 4096)
    x = orc.normal((1, 4096), seed=43)
    y = to_np(gops.mul_mat(qw, torch.from_numpy(x).cuda()))
    assert orc.parity(y, orc.mul_mat(raw, "q8_0", x, 4096)) < TOL


@pytest.mark.parametrize("t", ["q4_0", "q8_0", "q4_K", "q5_K"])
@pytest.mark.parametrize("B", [2, 3, 5, 8, 16])
@pytest.mark.parametrize("K", [2048, 3104, 14336])
def test_gemv_batches_residual(gops, orc, t, B, K):
    """Batches of 2..8 rows (the K-sliced kernel: one wavefront per 64 tasks of 32 values of K,
    the activation in registers, R-row batches) and 16 (the GEMMs): a row count
    that is not a multiple of the row batch, a residual, K of one wavefront (2048), of a partly
    filled second one (3104 = 97 blocks: lanes past the row; Q4_0 / Q8_0 only, K-quant rows are
    whole 256-value super-blocks) and of seven (14336), B padded to a power of two (3, 5)."""
    if t in ("q4_K", "q5_K") and K % 256:
        pytest.skip("K-quant rows are whole 256-value super-blocks")
    N = 1000
    raw, qw = _weight(gops, orc, t, N, K, 44)
    x = orc.normal((B, K), seed=45)
    r = orc.normal((B, N), seed=46)
    act = gops.quantize_act(t, torch.from_numpy(x).cuda())
    y = to_np(gops.mul_mat_q(qw, act, B, res=torch.from_numpy(r).cuda()))
    assert orc.parity(y, orc.mul_mat(raw, t, x, K) + r) < TOL


def _exact_kquant(t, N, K, seed):
    """A Q4_K / Q5_K weight (ggml bytes) and a row for which every float step of the product is
    exact, so that any summation order gives the same bits: d = dmin = 1/16, the 6-bit scales and
    mins 0 or 1, random codes; each 256-value super-block of the row holds +-127/8 once (so
    iscale = -+8 and d_x = -+1/8 exactly) and otherwise values of |x| < 127/8 whose codes need
    rounding; one super-block all zero, and one with a tie of |max| (+127/8 before -127/8: the first
    one sets the scale, so the second maps to +127 by the clamp)."""
    rng = np.random.default_rng(seed)
    nsb = K // 256
    bb = 144 if t == "q4_K" else 176
    raw = np.zeros((N, nsb, bb), np.uint8)
    raw[:, :, 0:2] = np.frombuffer(np.float16(1 / 16).tobytes(), np.uint8)  # d
    raw[:, :, 2:4] = np.frombuffer(np.float16(1 / 16).tobytes(), np.uint8)  # dmin
    sc = rng.integers(0, 2, (N, nsb, 8), dtype=np.uint8)
    mn = rng.integers(0, 2, (N, nsb, 8), dtype=np.uint8)
    raw[:, :, 4:8] = sc[:, :, 0:4]  # get_scale_min_k4's packing for values below 16
    raw[:, :, 8:12] = mn[:, :, 0:4]
    raw[:, :, 12:16] = sc[:, :, 4:8] | (mn[:, :, 4:8] << 4)
    qs = 16 if t == "q4_K" else 48
    raw[:, :, qs:qs + 128] = rng.integers(0, 256, (N, nsb, 128), dtype=np.uint8)
    if t == "q5_K":
        raw[:, :, 16:48] = rng.integers(0, 256, (N, nsb, 32), dtype=np.uint8)
    top = 127 / 8
    x = rng.uniform(-0.999 * top, 0.999 * top, (1, K)).astype(np.float32)
    for sb in range(nsb):
        x[0, sb * 256 + rng.integers(0, 256)] = top if rng.integers(0, 2) else -top
    x[0, 256:512] = 0.0
    x[0, 512:768] = np.clip(x[0, 512:768], -0.9 * top, 0.9 * top)
    x[0, 512 + 40] = top
    x[0, 512 + 200] = -top
    return raw.reshape(N, nsb * bb), x


@pytest.mark.parametrize("t", ["q4_K", "q5_K"])
@pytest.mark.parametrize("K", [4096, 14336])
def test_gemv_row_kquant_fused_quantizer(gops, orc, t, K):
    """One f32 row times a Q4_K / Q5_K weight: the one-launch kernel quantizes the row to Q8_K
    itself. On a product whose float steps are all exact (_exact_kquant) it must give the same
    bits as the separately quantized row (k_act_q8_K, bit-exact with the oracle's
    quantize_row_q8_K) through the batched kernel, so every code, bsum and d is ggml's (a code off
    by one moves an output by 1/128 at least); on a random weight, within 1e-3 of the oracle."""
    N = 1000
    raw, x = _exact_kquant(t, N, K, 47)
    qw = gops.QuantWeight.from_ggml(torch.from_numpy(raw), t, K)
    xt = torch.from_numpy(x).cuda()
    y = to_np(gops.mul_mat(qw, xt))
    act = gops.quantize_act(t, xt)
    y_sep = to_np(gops.mul_mat_q(qw, act, 1))
    assert np.array_equal(y, y_sep), float(np.abs(y - y_sep).max())
    assert np.array_equal(y, orc.mul_mat(raw, t, x, K).astype(np.float32).reshape(y.shape))
    raw2, qw2 = _weight(gops, orc, t, N, K, 48)
    x2 = orc.normal((1, K), seed=49)
    y2 = to_np(gops.mul_mat(qw2, torch.from_numpy(x2).cuda()))
    assert orc.parity(y2, orc.mul_mat(raw2, t, x2, K)) < TOL


@pytest.mark.parametrize("t", ["q4_K", "q5_K", "q6_K"])
@pytest.mark.parametrize("N,K", [(1, 256), (37, 768), (300, 2304), (4097, 4096), (8192, 8192), (3, 8448),
                                 (4096, 14336), (5, 16384)])
def test_gemv_row_kquant_shapes(gops, orc, t, N, K):
    """The one-launch K-quant row kernel at its edges: a row of one super-block (56 of 64 lanes
    idle; Q6_K: an odd super-block count, whose d alternates its half of a word per row), ragged
    row counts (one row, 37, a group split by N), one to eight tasks per lane (the 8B down
    projection, the longest row), its largest row count."""
    raw, qw = _weight(gops, orc, t, N, K, 50)
    x = orc.normal((1, K), seed=51)
    y = to_np(gops.mul_mat(qw, torch.from_numpy(x).cuda()))
    assert orc.parity(y, orc.mul_mat(raw, t, x, K)) < TOL


@pytest.mark.parametrize("t,N,K", [("q4_K", 14336, 4096), ("q6_K", 4096, 14336)])
def test_gemm_kquant_prefill_shape_row_slices(gops, orc, t, N, K):
    """Prefill of 512 rows at the 8B shapes (gate/up 4096 -> 14336 in Q4_K, down 14336 -> 4096 in
    Q6_K), the whole product on the GPU; the oracle checks a slice of rows and columns (each
    output depends only on its own activation row and weight row)."""
    M = 512
    raw, qw = _full_weight(gops, t, N, K)
    x = gops.fill_normal((M, K), seed=32)
    y = to_np(gops.mul_mat(qw, x))
    rows = np.r_[0:8, 250:258, 504:512]
    cols = np.r_[0:64, N // 2:N // 2 + 64, N - 64:N]
    ref = orc.mul_mat(raw[cols], t, orc.normal((M, K), seed=32)[rows], K)
    assert orc.parity(y[np.ix_(rows, cols)], ref) < TOL
