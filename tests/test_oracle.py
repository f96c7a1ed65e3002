"""Pins the CPU oracle (oracle/gcq_oracle.c) before it is trusted as the checker.

ggml (the reference's arithmetic, llama.cpp b11223) is not available, and the reference commits no
numeric golden vectors for this path, so each oracle function is pinned here by what fixes it
independently of its own code: IEEE conversion in numpy, published test vectors, hand-worked
blocks (tests/golden/quant_kats.json), on-grid round trips (the pattern of the reference's
tests/unit/test_modelopt.py:60-72), integer brute force, and float64 closed forms of the ops
(ggml_compiler/ir/ops.py:158-164 rms_norm, :186-214 mul_mat, :260-288 rope, :450-473
flash_attn). Tolerances follow the reference's pins where it has them.
"""

import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


# ------------------------------------------------------------------------------ fp16, PRNG


def test_fp16_round_trip_matches_ieee(orc):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, np.inf, -np.inf, 2.0 ** -24, 2.0 ** -25,
                  1.5 * 2.0 ** -25, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11],
                 np.float32),
    ]).astype(np.float32)
    got = orc.fp32_to_fp16(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    allh = np.arange(65536, dtype=np.uint16)
    back = orc.fp16_to_fp32(allh)
    ref = allh.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(back[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.isnan(back[np.isnan(ref)]).all()


def test_splitmix64_published_vector(orc):
    # Vigna's splitmix64.c seeded with 1234567.
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
            16408922859458223821]
    assert [orc.lib().orc_rnd64(1234567, i) for i in range(5)] == want


def test_normal_stream_moments_and_offsets(orc):
    x = orc.normal((1 << 20,), seed=0)
    assert abs(float(x.mean())) < 5e-3 and abs(float(x.std()) - 1.0) < 5e-3
    tail = orc.normal((100,), seed=0, offset=(1 << 20) - 100)
    assert np.array_equal(tail, x[-100:])  # counter-based: any slice regenerates alone
    s = orc.normal((1000,), seed=0, std=0.02)
    assert np.array_equal(s, (x[:1000] * np.float32(0.02)).astype(np.float32))


# ------------------------------------------------------------------------- hand-worked KATs


def _kats():
    return json.loads((GOLDEN / "quant_kats.json").read_text())


@pytest.mark.parametrize("name", [k for k in json.loads((GOLDEN / "quant_kats.json").read_text())])
def test_encoder_known_answers(orc, name):
    kat = _kats()[name]
    x = np.array(kat["x"], np.float32)[None]
    if kat["kind"] == "weight":
        got = orc.quantize(x, kat["type"])[0]
    elif kat["kind"] == "act_q8_0":
        got = orc.quantize_act_q8_0(x, orc.ACT_AVX2 if kat["variant"] == "avx2" else orc.ACT_SCALAR)[0]
    else:
        got = orc.quantize_act_q8_K(x)[0]
    assert got.tobytes().hex() == kat["hex"], name


# --------------------------------------------------------------------------- on-grid trips


def _fp16_scales(rng, n):
    return rng.uniform(0.01, 0.1, n).astype(np.float16).astype(np.float32)


def test_q8_0_on_grid_round_trip(orc):
    """A block whose largest |code| is 127 on an fp16 scale s encodes as d = s, codes exact."""
    rng = np.random.default_rng(0)
    rows, n = 8, 256
    k = rng.integers(-127, 128, (rows, n))
    k.reshape(-1, 32)[:, 5] = 127 * np.where(rng.random(rows * n // 32) < 0.5, -1, 1)
    s = _fp16_scales(rng, rows * n // 32)
    w = (k.reshape(-1, 32) * s[:, None]).astype(np.float32).reshape(rows, n)
    q = orc.quantize(w, "q8_0").reshape(-1, 34)
    assert np.array_equal(q[:, :2].copy().view(np.float16)[:, 0].astype(np.float32), s)
    assert np.array_equal(q[:, 2:].view(np.int8), k.reshape(-1, 32))
    assert np.array_equal(orc.dequantize(q.reshape(rows, -1), "q8_0", n), w)


def test_q4_0_on_grid_round_trip(orc):
    """Codes in [-8, 7] with a -8 in each block on an fp16 scale: d = s; stored nibble = code + 8,
    byte j = element j | element j+16 << 4 (ggml_compiler/quant/encode.py:42-51)."""
    rng = np.random.default_rng(1)
    rows, n = 8, 256
    k = rng.integers(-7, 8, (rows * n // 32, 32))
    k[:, 9] = -8
    s = _fp16_scales(rng, rows * n // 32)
    w = (k * s[:, None]).astype(np.float32).reshape(rows, n)
    q = orc.quantize(w, "q4_0").reshape(-1, 18)
    assert np.array_equal(q[:, :2].copy().view(np.float16)[:, 0].astype(np.float32), s)
    nib = (k + 8).astype(np.uint8)
    assert np.array_equal(q[:, 2:], nib[:, :16] | (nib[:, 16:] << 4))
    assert np.array_equal(orc.dequantize(q.reshape(rows, -1), "q4_0", n), w)


# ---------------------------------------------------------------------- encoder invariants


@pytest.mark.parametrize("t,bound", [("q8_0", 1e-2), ("q4_0", 0.2), ("q4_K", 0.15), ("q5_K", 0.08), ("q6_K", 0.04)])
def test_encoder_error_bounds(orc, t, bound):
    """Random weights decode within the type's error (tests/unit/test_frontend.py:299-304 bounds
    4-bit at 0.15 of max |w|; :311-318 orders q8_0 < 1e-2 < q4_0 < 0.2)."""
    w = orc.normal((16, 1024), seed=3, std=0.02)
    back = orc.dequantize(orc.quantize(w, t), t, 1024)
    rel = np.abs(back - w).max() / np.abs(w).max()
    assert 0 < rel < bound
    if t == "q4_0":
        assert rel > 1e-2


def test_q8_0_q4_0_per_element_error(orc):
    """|deq - x| <= d/2 (+ fp16 scale rounding) for Q8_0; <= |d| (Q4_0's clamp at 15 aside)."""
    w = orc.normal((4, 512), seed=4)
    for t, bs, half in (("q8_0", 34, 0.5), ("q4_0", 18, 1.0)):
        q = orc.quantize(w, t)
        d = np.abs(q.reshape(-1, bs)[:, :2].copy().view(np.float16)[:, 0].astype(np.float64))
        err = np.abs(orc.dequantize(q, t, 512).astype(np.float64) - w).reshape(-1, 32)
        amax = np.abs(w.reshape(-1, 32)).max(1)
        assert (err.max(1) <= half * d * (1 + 2 ** -10) + amax * 2 ** -10).all(), t


def test_q4_K_layout_closed_form(orc):
    """A hand-built Q4_K block decodes as d*sc_j*q - dmin*m_j with the 6-bit (sc, m) packing of
    ggml's block_q4_K and sub-block 2c / 2c+1 in the low / high nibbles of bytes 32c..32c+31."""
    rng = np.random.default_rng(5)
    sc = rng.integers(0, 64, 8)
    m = rng.integers(0, 64, 8)
    q = rng.integers(0, 16, 256)
    packed = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            packed[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
            packed[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
        else:
            packed[j + 4] = (sc[j] & 15) | ((m[j] & 15) << 4)
    qs = np.zeros(128, np.uint8)
    for c in range(4):
        qs[32 * c:32 * c + 32] = q[64 * c:64 * c + 32] | (q[64 * c + 32:64 * c + 64] << 4)
    d, dmin = np.float16(0.0123), np.float16(0.0456)
    blk = np.concatenate([np.array([d, dmin], np.float16).view(np.uint8), packed, qs])
    got = orc.dequantize(blk[None], "q4_K", 256)[0].astype(np.float64)
    sub = np.repeat(np.arange(8), 32)
    want = np.float32(d) * sc[sub].astype(np.float32) * q - np.float32(dmin) * m[sub].astype(np.float32)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-6)


def test_q4_K_encoder_special_blocks(orc):
    z = np.zeros((1, 256), np.float32)
    assert not orc.quantize(z, "q4_K").any()  # zero super-block: d = dmin = 0, every code 0
    pos = np.abs(orc.normal((1, 256), seed=6)) + 0.5  # all positive: the fit's min starts at 0
    q = orc.quantize(pos, "q4_K")
    assert q[0, 0:2].view(np.float16)[0] > 0 and q[0, 2:4].view(np.float16)[0] >= 0
    back = orc.dequantize(q, "q4_K", 256)
    assert np.abs(back - pos).max() < 0.1 * pos.max()


# ----------------------------------------------------- K-quant encoders: the search, pinned

def _kr():
    import sys

    sys.path.insert(0, str(GOLDEN))
    import kquant_ref

    return kquant_ref


def _kquant_kats():
    return {k: v for k, v in _kats().items() if v["kind"] == "weight" and v["type"] in ("q4_K", "q5_K", "q6_K")}


def test_kquant_restatement_reproduces_kats():
    """tests/golden/kquant_ref.py (a Python restatement of ggml's make_qkx2_quants /
    make_qx_quants encoders, written apart from the C oracle) gives every K-quant fixture's bytes,
    the hand-worked exact-grid block included; test_encoder_known_answers holds the oracle to the
    same bytes."""
    kr = _kr()
    for name, k in _kquant_kats().items():
        assert kr.ENCODERS[k["type"]](k["x"]).hex() == k["hex"], name


def test_kquant_kats_expose_every_wrong_search_parameter():
    """Each wrong parameter of the encoders' searches (make_qkx2_quants' rmin / rdelta / nstep and
    sub-block weighting, make_qx_quants' candidate range and weighting) changes the bytes of at
    least one fixture, so an oracle with that mistake fails test_encoder_known_answers."""
    kr = _kr()
    rec = json.loads((GOLDEN / "kquant_mutations.json").read_text())
    kats = _kquant_kats()
    for t, muts in rec["mutations"].items():
        for mname, kw in muts.items():
            kw = {k: (range(v[0], v[-1] + 1) if isinstance(v, list) and v else range(0) if isinstance(v, list) else v)
                  for k, v in kw.items()}
            caught = [n for n, c in rec["caught_by"].items() if mname in c["catches"] and kats[n]["type"] == t]
            assert caught, (t, mname)
            x = kats[caught[0]]["x"]
            assert kr.ENCODERS[t](x, **kw).hex() != kats[caught[0]]["hex"], (t, mname, caught[0])


def test_kquant_kats_cover_the_search_branches():
    """The fixtures exercise the branches the reference's error bounds leave open: a candidate of the
    search beating the min/max fit (the exact-grid Q4_K block; the last candidate winning in Q4_K and
    Q5_K), the least-squares min clamped to 0, an fp16-subnormal dmin, and Q6_K's search moving the
    scale away from -nmax / max."""
    kr = _kr()
    seen = {t: set() for t in ("q4_K", "q5_K", "q6_K")}
    for name, k in _kquant_kats().items():
        t, tr = k["type"], []
        h = kr.ENCODERS[t](k["x"], trace=tr)
        if t == "q6_K":
            if any(w != 0 for w in tr):
                seen[t].add("search moves the scale")
            continue
        if any(w >= 0 for w, _ in tr):
            seen[t].add("a candidate beats min/max")
        if any(c for _, c in tr):
            seen[t].add("clamped min wins")
        if any(w == (20 if t == "q4_K" else 15) for w, _ in tr):
            seen[t].add("last candidate wins")
        if 0 < int.from_bytes(h[2:4], "little") < 0x400:
            seen[t].add("subnormal dmin")
    full = {"a candidate beats min/max", "clamped min wins", "last candidate wins", "subnormal dmin"}
    assert seen == {"q4_K": full, "q5_K": full, "q6_K": {"search moves the scale"}}


@pytest.mark.parametrize("t", ["q4_K", "q5_K", "q6_K"])
def test_kquant_oracle_equals_restatement_on_random_blocks(orc, t):
    """The C oracle and the Python restatement agree byte for byte beyond the fixtures."""
    kr = _kr()
    rng = np.random.default_rng(11)
    for trial in range(6):
        x = (rng.normal(0, 0.02, 256) if trial % 2 else rng.standard_t(3, 256) * 0.01).astype(np.float32)
        assert orc.quantize(x[None], t).tobytes() == kr.ENCODERS[t](x.tolist()), (t, trial)


def test_kquant_row_sizes(orc):
    """Bytes per 256 values: 144 / 176 / 210 (ggml_compiler/compiler.py:82)."""
    assert [orc.row_size(t, 512) for t in ("q4_K", "q5_K", "q6_K")] == [288, 352, 420]


def test_kquant_error_order(orc):
    """More bits, less error: q6_K < q5_K < q4_K on the same weights (a misplaced high bit in q5_K
    or q6_K would break the order)."""
    w = orc.normal((32, 1024), seed=30, std=0.02)
    err = [np.abs(orc.dequantize(orc.quantize(w, t), t, 1024) - w).mean() for t in ("q4_K", "q5_K", "q6_K")]
    assert err[0] > 1.6 * err[1] > 0 and err[1] > 1.6 * err[2] > 0


def _pack_scale_min(sc, m):
    packed = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            packed[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
            packed[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
        else:
            packed[j + 4] = (sc[j] & 15) | ((m[j] & 15) << 4)
    return packed


def test_q5_K_layout_closed_form(orc):
    """A hand-built Q5_K block ({d, dmin, scales[12], qh[32], qs[128]}) decodes as
    d*sc_j*q - dmin*m_j, q = nibble + 16 * bit: value 64c + l (l < 32) takes the low nibble of
    qs[32c + l] and bit 2c of qh[l]; value 64c + 32 + l the high nibble and bit 2c + 1."""
    rng = np.random.default_rng(31)
    sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    q = rng.integers(0, 32, 256)
    qs = np.zeros(128, np.uint8)
    qh = np.zeros(32, np.uint8)
    for v in range(256):
        c, r = divmod(v, 64)
        hi, l = divmod(r, 32)
        qs[32 * c + l] |= (q[v] & 15) << (4 * hi)
        qh[l] |= (q[v] >> 4) << (2 * c + hi)
    d, dmin = np.float16(0.0123), np.float16(0.0456)
    blk = np.concatenate([np.array([d, dmin], np.float16).view(np.uint8), _pack_scale_min(sc, m), qh, qs])
    assert blk.size == 176
    got = orc.dequantize(blk[None], "q5_K", 256)[0].astype(np.float64)
    sub = np.repeat(np.arange(8), 32)
    want = np.float32(d) * sc[sub].astype(np.float32) * q - np.float32(dmin) * m[sub].astype(np.float32)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-6)


def _q6_K_block(q, sc, d):
    """ggml block_q6_K bytes from 256 codes q in [0, 63] (value = q - 32), 16 int8 scales, fp16 d.
    Value 128h + 32p + l (h < 2, p < 4, l < 32): low 4 bits in ql[64h + 32(p % 2) + l] (low nibble
    for p < 2, high for p >= 2), high 2 bits at bit 2p of qh[32h + l]."""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for v in range(256):
        h, r = divmod(v, 128)
        p, l = divmod(r, 32)
        ql[64 * h + 32 * (p % 2) + l] |= (q[v] & 15) << (4 * (p // 2))
        qh[32 * h + l] |= (q[v] >> 4) << (2 * p)
    return np.concatenate([ql, qh, np.asarray(sc, np.int8).view(np.uint8), np.array([d], np.float16).view(np.uint8)])


def test_q6_K_layout_closed_form(orc):
    rng = np.random.default_rng(32)
    q = rng.integers(0, 64, 256)
    sc = rng.integers(-128, 128, 16)
    d = np.float16(0.00731)
    blk = _q6_K_block(q, sc, d)
    assert blk.size == 210
    got = orc.dequantize(blk[None], "q6_K", 256)[0]
    want = (np.float32(d) * sc[np.arange(256) // 16].astype(np.float32)) * (q - 32).astype(np.float32)
    assert np.array_equal(got, want.astype(np.float32))


def test_q6_K_on_grid_round_trip(orc):
    """Weights d*sc_j*l with d a power of two, one sub-block scale -128 (the largest magnitude),
    l in [-31, 31] and one l = -32 per sub-block (its largest |x|): the encoder recovers d, every
    scale and every code, so the block round-trips exactly and its bytes are the hand-packed ones."""
    rng = np.random.default_rng(33)
    d = 2.0 ** -12
    sc = rng.integers(-127, 128, 16)
    sc[sc == 0] = 5
    sc[rng.integers(0, 16)] = -128
    l = rng.integers(-31, 32, (16, 16))
    l[np.arange(16), rng.integers(0, 16, 16)] = -32
    w = (d * sc[:, None] * l).astype(np.float32).reshape(1, 256)
    qb = orc.quantize(w, "q6_K")
    assert np.array_equal(qb[0], _q6_K_block((l + 32).reshape(-1), sc, np.float16(d)))
    assert np.array_equal(orc.dequantize(qb, "q6_K", 256), w)


@pytest.mark.parametrize("t", ["q5_K", "q6_K"])
def test_kquant_encoder_special_blocks(orc, t):
    z = np.zeros((1, 256), np.float32)
    assert not orc.quantize(z, t).any()  # an all-zero super-block is all zero bytes
    x = orc.normal((1, 256), seed=34)
    x[0, :16] = 0.0  # a zero sub-block inside a live super-block decodes to zeros
    back = orc.dequantize(orc.quantize(x, t), t, 256)
    if t == "q6_K":
        assert not back[0, :16].any()
    assert np.abs(back - x).max() < 0.1 * np.abs(x).max()


def test_act_q8_K_bsums_and_sign(orc):
    x = orc.normal((2, 512), seed=7)
    q = orc.quantize_act_q8_K(x).reshape(-1, 292)
    d = q[:, :4].copy().view(np.float32)[:, 0]
    codes = q[:, 4:260].view(np.int8).astype(np.int64)
    bsums = q[:, 260:].copy().view(np.int16).astype(np.int64)
    assert np.array_equal(bsums, codes.reshape(-1, 16, 16).sum(-1))
    back = (d[:, None] * codes).reshape(2, 512)
    assert np.abs(back - x).max() <= np.abs(d).max() * 0.5 + 1e-6
    assert (np.abs(codes).max(1) == 127).all()


# ------------------------------------------------------------------- integer block sums


def _codes(t, wrow, k):
    """Signed integer codes of a weight row, unpacked from the documented byte layouts."""
    if t == "q8_0":
        return wrow.reshape(-1, 34)[:, 2:].view(np.int8).astype(np.int64).reshape(-1)
    if t == "q4_0":
        b = wrow.reshape(-1, 18)[:, 2:].astype(np.int64)
        return np.concatenate([(b & 15) - 8, (b >> 4) - 8], axis=1).reshape(-1)
    if t == "q4_K":
        b = wrow.reshape(-1, 144)[:, 16:].astype(np.int64).reshape(-1, 4, 32)
        return np.stack([b & 15, b >> 4], axis=2).reshape(-1)  # chunk c: low 32 then high 32
    if t == "q5_K":
        blk = wrow.reshape(-1, 176).astype(np.int64)
        qh, b = blk[:, 16:48], blk[:, 48:].reshape(-1, 4, 32)
        bit = (qh[:, None, None, :] >> (2 * np.arange(4)[None, :, None, None] + np.arange(2)[None, None, :, None])) & 1
        return (np.stack([b & 15, b >> 4], axis=2) + 16 * bit).reshape(-1)
    blk = wrow.reshape(-1, 210).astype(np.int64)  # q6_K: codes minus 32
    ql, qh = blk[:, :128].reshape(-1, 2, 2, 32), blk[:, 128:192].reshape(-1, 2, 32)
    low = np.stack([ql[:, :, 0] & 15, ql[:, :, 1] & 15, ql[:, :, 0] >> 4, ql[:, :, 1] >> 4], axis=2)  # [sb, h, p, l]
    high = (qh[:, :, None, :] >> (2 * np.arange(4))[None, None, :, None]) & 3
    return (low | (high << 4)).reshape(-1) - 32


@pytest.mark.parametrize("t", ["q8_0", "q4_0", "q4_K", "q5_K", "q6_K"])
def test_block_isums_brute_force(orc, t):
    k = 1024
    w = orc.normal((3, k), seed=8, std=0.02)
    x = orc.normal((k,), seed=9)
    wq = orc.quantize(w, t)
    if t in ("q4_K", "q5_K", "q6_K"):
        xq = orc.quantize_act_q8_K(x)
        xc = xq.reshape(-1, 292)[:, 4:260].view(np.int8).astype(np.int64).reshape(-1)
        bs = xq.reshape(-1, 292)[:, 260:].copy().view(np.int16).astype(np.int64)
    else:
        xq = orc.quantize_act_q8_0(x)
        xc = xq.reshape(-1, 34)[:, 2:].view(np.int8).astype(np.int64).reshape(-1)
    for r in range(3):
        got = orc.block_isums(t, wq[r], xq, k)
        prod = _codes(t, wq[r], k) * xc
        if t in ("q8_0", "q4_0"):
            assert np.array_equal(got, prod.reshape(-1, 32).sum(1))
            continue
        if t == "q6_K":
            got = got.reshape(-1, 17)
            subs = prod.reshape(-1, 16, 16).sum(2)
            sc = wq[r].reshape(-1, 210)[:, 192:208].view(np.int8).astype(np.int64)
            assert np.array_equal(got[:, :16], subs)
            assert np.array_equal(got[:, 16], (sc * subs).sum(1))
            continue
        got = got.reshape(-1, 10)
        dots = prod.reshape(-1, 8, 32).sum(2)
        assert np.array_equal(got[:, :8], dots)
        hdr = wq[r].reshape(-1, 144 if t == "q4_K" else 176)[:, 4:16]
        for b in range(k // 256):
            scm = [_scale_min(hdr[b], j) for j in range(8)]
            assert got[b, 8] == sum(s * dots[b, j] for j, (s, _) in enumerate(scm))
            assert got[b, 9] == sum(mm * (bs[b, 2 * j] + bs[b, 2 * j + 1]) for j, (_, mm) in enumerate(scm))


def _scale_min(p, j):
    p = [int(v) for v in p]
    if j < 4:
        return p[j] & 63, p[j + 4] & 63
    return (p[j + 4] & 15) | ((p[j - 4] >> 6) << 4), (p[j + 4] >> 4) | ((p[j] >> 6) << 4)


# ---------------------------------------------------------------------------- float ops


@pytest.mark.parametrize("t", ["q8_0", "q4_0", "q4_K", "q5_K", "q6_K"])
def test_mul_mat_closed_form(orc, t):
    """y = x_q . w_q^T in float64 from both dequantized operands; oracle (f32 accumulation)
    within 1e-5 of it, and within quantization error of the unquantized product."""
    N, K, M = 64, 512, 3
    w = orc.normal((N, K), seed=10, std=0.02)
    x = orc.normal((M, K), seed=11)
    wq = orc.quantize(w, t)
    y = orc.mul_mat(wq, t, x, K)
    wd = orc.dequantize(wq, t, K).astype(np.float64)
    if t in ("q4_K", "q5_K", "q6_K"):
        xq = orc.quantize_act_q8_K(x).reshape(M, -1, 292)
        xd = (xq[:, :, :4].copy().view(np.float32) * xq[:, :, 4:260].view(np.int8)).reshape(M, K)
    else:
        xq = orc.quantize_act_q8_0(x).reshape(M, -1, 34)
        xd = (xq[:, :, :2].copy().view(np.float16).astype(np.float32) * xq[:, :, 2:].view(np.int8)).reshape(M, K)
    ref = xd.astype(np.float64) @ wd.T
    assert orc.parity(y, ref) < 1e-5
    assert orc.parity(y, x.astype(np.float64) @ w.T.astype(np.float64)) < (0.02 if t == "q8_0" else 0.15)


def test_rms_norm_closed_form(orc):
    x = orc.normal((5, 4096), seed=12) * 3
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-5)
    assert orc.parity(orc.rms_norm(x, 1e-5), ref) < 1e-6


def test_rope_closed_form(orc):
    """theta = pos * base^(-2i/n): ggml's repeated multiplication drifts ~1e-4 at pos 1000
    (ggml_compiler/passes/fuse_rope.py:14-15); position 0 is the identity; pairs keep their norm."""
    S, H, D = 6, 4, 128
    x = orc.normal((S, H, D), seed=13)
    pos = np.array([0, 1, 7, 100, 600, 1000], np.int32)
    out = orc.rope_neox(x, pos, D, 500000.0)
    inv = 500000.0 ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    th = pos[:, None].astype(np.float64) * inv[None]
    c, s = np.cos(th)[:, None], np.sin(th)[:, None]
    x1, x2 = x[..., :D // 2].astype(np.float64), x[..., D // 2:].astype(np.float64)
    ref = np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)
    assert orc.parity(out, ref) < 2e-4
    assert np.array_equal(out[0], x[0])
    n_in = x1 ** 2 + x2 ** 2
    n_out = out[..., :D // 2].astype(np.float64) ** 2 + out[..., D // 2:].astype(np.float64) ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5, atol=1e-6)
    part = orc.rope_neox(x, pos, 64, 10000.0)  # n_dims < D: the rest passes through
    assert np.array_equal(part[..., 64:], x[..., 64:])


def _attn_ref(q, k16, v16, m16, scale):
    H, Sq, D = q.shape
    Hkv = k16.shape[0]
    qf = q.astype(np.float16).astype(np.float64)
    kf = k16.view(np.float16).astype(np.float64)
    vf = v16.view(np.float16).astype(np.float64)
    out = np.zeros((Sq, H, vf.shape[2]))
    for h in range(H):
        hk = h // (H // Hkv)
        s = qf[h] @ kf[hk].T * scale
        if m16 is not None:
            s = s + m16.view(np.float16).astype(np.float64)
        for i in range(Sq):
            row = s[i]
            if np.isneginf(row).all():
                continue  # ggml: no visible key -> S = 0 -> output 0
            p = np.exp(row - row.max())
            out[i, h] = p @ vf[hk] / p.sum()
    return out


@pytest.mark.parametrize("H,Hkv,Sq,n_kv", [(4, 4, 3, 37), (8, 2, 1, 300), (32, 8, 2, 512)])
def test_flash_attn_closed_form(orc, H, Hkv, Sq, n_kv):
    D = 128
    q = orc.normal((H, Sq, D), seed=14)
    k16 = orc.fp32_to_fp16(orc.normal((Hkv, n_kv, D), seed=15))
    v16 = orc.fp32_to_fp16(orc.normal((Hkv, n_kv, D), seed=16))
    pos = n_kv - Sq + np.arange(Sq)
    mask = np.where(np.arange(n_kv)[None] <= pos[:, None], 0.0, -np.inf).astype(np.float32)
    m16 = orc.fp32_to_fp16(mask)
    out = orc.flash_attn_ext(q, k16, v16, m16, 1 / np.sqrt(D))
    assert orc.parity(out, _attn_ref(q, k16, v16, m16, 1 / np.sqrt(D))) < 1e-5


def test_flash_attn_fully_masked_row_is_zero(orc):
    """No visible key: ggml's sum S stays 0 and the row is 0, never NaN
    (tests/unit/test_frontend.py:338-358 requires finite output)."""
    q = orc.normal((2, 2, 64), seed=17)
    k16 = orc.fp32_to_fp16(orc.normal((2, 5, 64), seed=18))
    v16 = orc.fp32_to_fp16(orc.normal((2, 5, 64), seed=19))
    mask = np.zeros((2, 5), np.float32)
    mask[1] = -np.inf
    out = orc.flash_attn_ext(q, k16, v16, orc.fp32_to_fp16(mask), 0.125)
    assert np.isfinite(out).all() and not out[1].any() and out[0].any()


def test_swiglu_argmax(orc):
    g = orc.normal((1000,), seed=20)
    u = orc.normal((1000,), seed=21)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert orc.parity(orc.swiglu(g, u), ref) < 1e-6
    x = np.array([1, 5, 2, 5, -1], np.float32)
    assert orc.argmax(x) == 1


def test_parity_metric(orc):
    assert orc.parity(np.array([1.0, np.nan]), np.array([1.0, 2.0])) == float("inf")
    assert orc.parity(np.array([10.5]), np.array([10.0])) == pytest.approx(0.05)
    assert orc.parity(np.array([0.5]), np.array([0.0])) == pytest.approx(0.5)
