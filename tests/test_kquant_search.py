"""The K-quant encoders' scale searches, checked against what the mathematics fixes.

ggml's Q4_K / Q5_K encoder fits each 32-value sub-block with make_qkx2_quants and its Q6_K encoder
each 16-value sub-block with make_qx_quants (runtime/src/ggml_compiler_rt.cpp:859-876 calls
ggml_quantize_chunk, which runs them; ggml is not in this container). Their published definitions
fix the candidates and the selection rule, so the oracle's choices can be checked in float64 against
closed forms rather than against a second restatement of the search:

* make_qkx2_quants (asymmetric, weights w): a min/max fit (iscale = nmax / (max - min), scale =
  1 / iscale, min = min(x, 0)), then for s = 0 .. nstep the codes l = clamp(rne(iscale_s (x - min)),
  0, nmax) with iscale_s = (rmin + rdelta s + nmax) / (max - min), refit by weighted least squares
  (min clamped to <= 0) and taken when their weighted error is lower; ggml's loop moves `min` to
  the taken fit's, so later candidates depend on earlier choices. The oracle exposes each step
  (make_qkx2's trace) and every step is checked: its iscale against the formula with the published
  constants and the current min, its codes, its (scale, min) against the closed-form weighted
  least-squares solution, its error, and whether it was taken. Independently of the path, the
  result's error is the least of every fit the search made and its (scale, min) is the closed-form
  fit of its codes.
* make_qx_quants (symmetric, weights x^2, nmax 32): candidates iscale = -(nmax + 0.1 s) / max for
  s = -9 .. 9, the codes l = clamp(rne(iscale x), -32, 31), scale = sum w x l / sum w l^2; the
  result maximizes (sum w x l)^2 / sum w l^2 (least weighted error) and its scale is that ratio.

For make_qx_quants each check runs in float64 on diverse sub-blocks: (1) the oracle's codes are one
candidate's codes, (2) their fit is the best over the published set, (3) the returned scale is the
closed-form solution. The same checks with a wrong rdelta, nstep, rmin, weighting or candidate
range reject the oracle's outputs on at least one of these sub-blocks, so the outputs pin the
published parameters. The super-block packing (6-bit scale / min pairs against the largest, fp16 d
and dmin, codes recomputed against the rounded scales) is checked in closed form from the bytes.
"""

from __future__ import annotations

import numpy as np
import pytest

Q4K = dict(nmax=15, rmin=-1.0, rdelta=0.1, nstep=20)
Q5K = dict(nmax=31, rmin=-0.5, rdelta=0.1, nstep=15)
REL = 2e-5  # float32 accumulation in the encoder against the float64 error here


def _blocks(n: int, size: int, seed: int) -> list[np.ndarray]:
    """Sub-blocks of several shapes: normal, one-sided, outliers, clustered, tiny, large, coarse."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        kind = i % 9
        if kind == 0:
            x = rng.normal(0, 1, size)
        elif kind == 1:
            x = rng.uniform(0.05, 1.0, size)          # all positive: min clamps to 0
        elif kind == 2:
            x = -rng.uniform(0.05, 1.0, size)         # all negative
        elif kind == 3:
            x = rng.normal(0, 0.02, size)
            x[rng.integers(size)] *= 40.0             # one outlier
        elif kind == 4:
            x = rng.choice([-1.0, 0.3, 0.7], size) + rng.normal(0, 0.05, size)
        elif kind == 5:
            x = rng.normal(0, 1e-3, size)
        elif kind == 6:
            x = rng.normal(5, 300, size)
        elif kind == 7:
            x = np.round(rng.normal(0, 3, size)) * 0.25  # coarse grid
        else:
            x = rng.laplace(0, 1, size)
        out.append(x.astype(np.float32))
    return out


def _weights(x: np.ndarray, how: str = "ggml") -> np.ndarray:
    """Q4_K / Q5_K sub-block weights: sqrt(mean x^2) + |x| (quantize_row_q4_K_ref)."""
    x = x.astype(np.float32)
    if how == "ggml":
        av = np.float32(np.sqrt(np.float32(np.sum(x * x, dtype=np.float32)) / np.float32(32)))
        return (av + np.abs(x)).astype(np.float32)
    if how == "ones":
        return np.ones_like(x)
    if how == "abs":
        return np.abs(x)
    return x * x


def _rne(v: np.ndarray) -> np.ndarray:
    return np.rint(v).astype(np.int64)


def _wls(x, w, l):
    """Weighted least squares (scale, min) for codes l, min clamped to <= 0; None when singular."""
    x, w, l = (np.asarray(a, np.float64) for a in (x, w, l))
    sw, sl, sl2, sx, sxl = w.sum(), (w * l).sum(), (w * l * l).sum(), (w * x).sum(), (w * l * x).sum()
    D = sw * sl2 - sl * sl
    if D <= 0:
        return None
    scale = (sw * sxl - sx * sl) / D
    mn = (sl2 * sx - sl * sxl) / D
    if mn > 0:
        mn = 0.0
        scale = sxl / sl2
    return scale, mn


def _tiny(x, w) -> float:
    """The weighted error float32 arithmetic cannot resolve: 1e-10 of the block's weighted energy."""
    return 1e-10 * float((np.asarray(w, np.float64) * np.asarray(x, np.float64) ** 2).sum()) + 1e-37


def _err(x, w, l, scale, mn):
    x, w, l = (np.asarray(a, np.float64) for a in (x, w, l))
    d = scale * l + mn - x
    return float((w * d * d).sum())


def _qkx2_violation(x, w, L, scale, mn, trace, nmax, rmin, rdelta, nstep) -> str | None:
    """Why the oracle's search of sub-block x (its step trace, codes L and result (scale, min)) is not
    make_qkx2_quants with these parameters and weights w, or None. Step s makes codes
    clamp(rne(iscale_s (x - min))) against the min of the best fit so far (ggml updates min as the
    search goes), fits them by weighted least squares, and takes the fit if its error is lower."""
    x32 = x.astype(np.float32)
    mn0 = min(np.float32(x32.min()), np.float32(0.0))
    mx = np.float32(x32.max())
    if mx == mn0:
        return None if (L == 0).all() else "constant block: codes not zero"

    def codes_ok(want, got, v):
        return bool(((want == got) | _near_half(v)).all())

    t0 = trace[0]
    isc0 = np.float32(np.float32(nmax) / np.float32(mx - mn0))
    if not np.isclose(t0[0], isc0, rtol=1e-6):
        return "min/max fit: iscale is not nmax / (max - min)"
    v0 = (isc0 * (x32 - mn0)).astype(np.float64)
    if not codes_ok(np.clip(_rne(v0), 0, nmax), t0[8:].astype(np.int64), v0):
        return "min/max fit: codes"
    best = _err(x32, w, t0[8:], float(np.float32(1) / isc0), float(mn0))
    if not np.isclose(t0[4], best, rtol=1e-3, atol=1e-30):
        return "min/max fit: weighted error"
    cur_min, cur_scale, cur_L = float(mn0), float(t0[2]), t0[8:].astype(np.int64)
    tiny = _tiny(x32, w)
    for st in range(nstep + 1):
        t = trace[1 + st]
        if t[6] != np.float32(cur_min):
            return f"step {st}: codes not made against the best fit's min"
        isc = np.float32((np.float32(rmin) + np.float32(rdelta) * np.float32(st) + np.float32(nmax)) /
                         np.float32(mx - np.float32(cur_min)))
        if not np.isclose(t[0], isc, rtol=1e-6):
            return f"step {st}: iscale is not (rmin + rdelta s + nmax) / (max - min)"
        codes = t[8:].astype(np.int64)
        v = (isc * (x32 - np.float32(cur_min))).astype(np.float64)
        if not codes_ok(np.clip(_rne(v), 0, nmax), codes, v):
            return f"step {st}: codes"
        fit = _wls(x32, w, codes)
        if fit is None or t[1] == 0:
            if t[5]:
                return f"step {st}: taken without a fit"
            continue
        xmax = float(np.abs(x32).max())
        if abs(t[2] - fit[0]) > 1e-4 * abs(fit[0]) + 1e-6 * xmax / nmax or \
                abs(t[3] - fit[1]) > 1e-4 * abs(fit[1]) + 1e-5 * xmax:
            return f"step {st}: (scale, min) are not the weighted least-squares fit of the codes"
        e = _err(x32, w, codes, *fit)
        if not np.isclose(t[4], e, rtol=2e-3, atol=tiny):
            return f"step {st}: weighted error"
        taken = bool(t[5])
        if taken != (e < best) and abs(e - best) > 1e-5 * best + tiny:
            return f"step {st}: {'took' if taken else 'left'} a fit of error {e:.9g} against the best {best:.9g}"
        if taken:
            best, cur_min, cur_scale, cur_L = e, float(t[3]), float(t[2]), codes
    if not np.array_equal(L, cur_L) or scale != np.float32(cur_scale) or mn != np.float32(cur_min):
        return "result is not the last fit taken"
    return None


def _qkx2_runs(orc, params, seed):
    out = []
    for x in _blocks(360, 32, seed=seed):
        w = _weights(x)
        L, scale, mn, tr = orc.make_qkx2(x, w, params["nmax"], params["rmin"], params["nstep"], trace=True)
        out.append((x, w, L.astype(np.int64), scale, mn, tr))
    return out


@pytest.mark.parametrize("name,params", [("q4_K", Q4K), ("q5_K", Q5K)])
def test_qkx2_search_follows_its_definition(orc, name, params):
    bad = []
    for i, (x, w, L, scale, mn, tr) in enumerate(_qkx2_runs(orc, params, 11 if name == "q4_K" else 12)):
        why = _qkx2_violation(x, w, L, scale, mn, tr, **params)
        if why:
            bad.append((i, why))
    assert not bad, f"{name}: {len(bad)} sub-blocks break make_qkx2_quants: {bad[:5]}"


@pytest.mark.parametrize("name,params", [("q4_K", Q4K), ("q5_K", Q5K)])
def test_qkx2_search_result_is_its_best_fit(orc, name, params):
    """Whatever the path: the result's (scale, min) is the weighted least-squares fit of its codes
    (or the min/max fit), and its error is the least of every fit the search made."""
    for x, w, L, scale, mn, tr in _qkx2_runs(orc, params, 15 if name == "q4_K" else 16):
        if float(x.max()) == min(float(x.min()), 0.0):
            continue
        fits = [_err(x, w, tr[0, 8:], float(tr[0, 2]), float(tr[0, 3]))]
        for st in range(params["nstep"] + 1):
            f = _wls(x, w, tr[1 + st, 8:]) if tr[1 + st, 1] else None
            if f is not None:
                fits.append(_err(x, w, tr[1 + st, 8:], *f))
        mine = _err(x, w, L, scale, mn)
        assert mine <= min(fits) * (1 + REL) + _tiny(x, w)
        f = _wls(x, w, L)
        minmax = np.array_equal(L, tr[0, 8:].astype(np.int64)) and scale == tr[0, 2] and mn == tr[0, 3]
        assert minmax or (f is not None and np.isclose(scale, f[0], rtol=1e-4, atol=1e-7) and
                          abs(mn - f[1]) <= 1e-4 * abs(f[1]) + 1e-5 * float(np.abs(x).max()))


@pytest.mark.parametrize("name,params", [("q4_K", Q4K), ("q5_K", Q5K)])
def test_qkx2_outputs_reject_every_wrong_parameter(orc, name, params):
    """The oracle's searches are consistent with the published (rmin, rdelta, nstep, weights) only."""
    runs = _qkx2_runs(orc, params, 13 if name == "q4_K" else 14)
    wrong = {
        "rdelta 0.05": dict(params, rdelta=0.05), "rdelta 0.2": dict(params, rdelta=0.2),
        "nstep - 1": dict(params, nstep=params["nstep"] - 1),
        "rmin + 0.5": dict(params, rmin=params["rmin"] + 0.5), "rmin - 0.5": dict(params, rmin=params["rmin"] - 0.5),
        "weights 1": (params, "ones"), "weights |x|": (params, "abs"), "weights x^2": (params, "sq"),
    }
    for label, v in wrong.items():
        p, how = (v if isinstance(v, tuple) else (v, None))
        rejected = 0
        for x, w, L, scale, mn, tr in runs:
            wu = _weights(x, how) if how else w
            rejected += _qkx2_violation(x, wu, L, scale, mn, tr[:p["nstep"] + 2], **p) is not None
        assert rejected > 0, f"{name}: nothing tells the published search from '{label}'"


def _qx16_candidates(x, nmax=32, lo=-9, hi=9, step=0.1, how="sq"):
    x32 = x.astype(np.float32)
    ax = np.abs(x32)
    mx = np.float32(x32[int(np.argmax(ax))])  # first largest |x|, its sign kept
    w = _weights(x32, how).astype(np.float64)
    out = []
    for s in [0] + [k for k in range(lo, hi + 1) if k != 0]:
        isc = np.float32(-np.float32(np.float32(nmax) + np.float32(step) * np.float32(s)) / mx)
        l = np.clip(_rne(isc * x32), -nmax, nmax - 1)
        sl2 = float((w * l * l).sum())
        slx = float((w * x32 * l).sum())
        if sl2 <= 0:
            continue
        out.append((l, slx / sl2, slx * slx / sl2, s))
    return out


def _qx16_violation(x, L, scale, **cand) -> str | None:
    if np.abs(x).max() < 1e-15:
        return None if (L == 0).all() and scale == 0 else "zero block: codes / scale not zero"
    l = L.astype(np.int64) - 32
    c = _qx16_candidates(x, **cand)
    match = [k for k in c if np.array_equal(k[0], l)]
    if not match:
        return "codes are no candidate's"
    best = max(k[2] for k in c)
    mine = match[0][2]
    if mine < best * (1 - REL):
        return f"fit {mine:.9g} below the best candidate's {best:.9g}"
    if not any(np.isclose(scale, k[1], rtol=1e-4) for k in match):
        return "scale is not sum w x l / sum w l^2 of the codes"
    return None


def test_qx16_choice_is_the_best_published_candidate(orc):
    bad = []
    for i, x in enumerate(_blocks(540, 16, seed=21)):
        L, scale = orc.make_qx16(x)
        why = _qx16_violation(x, L, scale)
        if why:
            bad.append((i, why))
    assert not bad, f"q6_K: {len(bad)} sub-blocks break the published search: {bad[:5]}"


def test_qx16_outputs_reject_every_wrong_parameter(orc):
    outs = [(x, *orc.make_qx16(x)) for x in _blocks(540, 16, seed=22)]
    wrong = {"candidates -10..10": dict(lo=-10, hi=10), "candidates -8..8": dict(lo=-8, hi=8),
             "step 0.2": dict(step=0.2), "step 0.05": dict(step=0.05), "weights 1": dict(how="ones"),
             "weights |x|": dict(how="abs")}
    for label, kw in wrong.items():
        rejected = sum(_qx16_violation(x, L, s, **kw) is not None for x, L, s in outs)
        assert rejected > 0, f"q6_K: nothing tells the published search from '{label}'"


def _f16(v: float) -> float:
    return float(np.float32(v).astype(np.float16).astype(np.float32))


def _near_half(v: np.ndarray) -> np.ndarray:
    """Values whose rounding float32 and float64 may decide differently (within 1e-4 of a .5)."""
    return np.abs(np.abs(v - np.floor(v)) - 0.5) < 1e-4


@pytest.mark.parametrize("t", ["q4_K", "q5_K"])
def test_q4_q5_K_packing_from_the_fits(orc, t):
    """quantize_row_q4_K_ref / q5_K_ref after the fits: ls = rne(63 scale / max scale), lm likewise
    (both <= 63), d = fp16(max scale / 63), dmin = fp16(max min / 63), and each code
    rne((x + dmin m) / (d sc)) clamped to [0, nmax], read back from the encoder's bytes."""
    params = Q4K if t == "q4_K" else Q5K
    nmax = params["nmax"]
    rng = np.random.default_rng(31)
    x = rng.normal(0, 1, (24, 256)).astype(np.float32)
    x[3] = np.abs(x[3])
    x[7] *= 1e-3
    q = orc.quantize(x, t)
    deq_codes = _kquant_codes(q, t, nmax)
    for r in range(x.shape[0]):
        fits = [orc.make_qkx2(x[r, 32 * j:32 * j + 32], _weights(x[r, 32 * j:32 * j + 32]), nmax,
                              params["rmin"], params["nstep"]) for j in range(8)]
        scales = np.array([f[1] for f in fits], np.float64)
        mins = np.array([-f[2] for f in fits], np.float64)
        ms, mm = scales.max(), mins.max()
        blk = q[r]
        d, dmin = (np.frombuffer(blk[0:4].tobytes(), np.float16).astype(np.float64))
        assert d == _f16(ms / 63.0) and dmin == _f16(mm / 63.0)
        sc, m = _scale_min(blk[4:16])
        v_ls = scales * (63.0 / ms) if ms > 0 else np.zeros(8)
        v_lm = mins * (63.0 / mm) if mm > 0 else np.zeros(8)
        for want, got, v in ((np.minimum(_rne(v_ls), 63), sc, v_ls), (np.minimum(_rne(v_lm), 63), m, v_lm)):
            ok = (want == got) | _near_half(v)
            assert ok.all(), f"row {r}: 6-bit scales {got} against {want}"
        for j in range(8):
            dj = np.float32(np.float32(d) * np.float32(sc[j]))
            if dj == 0:
                continue
            dm = np.float32(np.float32(dmin) * np.float32(m[j]))
            v = (x[r, 32 * j:32 * j + 32].astype(np.float64) + float(dm)) / float(dj)
            want = np.clip(_rne(v), 0, nmax)
            got = deq_codes[r, 32 * j:32 * j + 32]
            assert ((want == got) | _near_half(v)).all(), f"row {r} sub-block {j}: codes"


def _scale_min(s: np.ndarray):
    """get_scale_min_k4 for j = 0..7 from the 12 packed bytes."""
    s = s.astype(np.int64)
    sc, m = np.zeros(8, np.int64), np.zeros(8, np.int64)
    for j in range(8):
        if j < 4:
            sc[j], m[j] = s[j] & 63, s[j + 4] & 63
        else:
            sc[j] = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4)
            m[j] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
    return sc, m


def _kquant_codes(q: np.ndarray, t: str, nmax: int) -> np.ndarray:
    """Per-value codes of Q4_K / Q5_K rows of one super-block (value 64c + l: low nibble of qs[32c + l],
    64c + 32 + l: its high nibble; Q5_K's fifth bit from qh[l] bit 2c / 2c + 1)."""
    rows = q.shape[0]
    out = np.zeros((rows, 256), np.int64)
    qs = q[:, 16:144] if t == "q4_K" else q[:, 48:176]
    for c in range(4):
        b = qs[:, 32 * c:32 * c + 32].astype(np.int64)
        out[:, 64 * c:64 * c + 32] = b & 0xF
        out[:, 64 * c + 32:64 * c + 64] = b >> 4
        if t == "q5_K":
            qh = q[:, 16:48].astype(np.int64)
            out[:, 64 * c:64 * c + 32] += ((qh >> (2 * c)) & 1) * 16
            out[:, 64 * c + 32:64 * c + 64] += ((qh >> (2 * c + 1)) & 1) * 16
    return out


def test_q6_K_packing_from_the_fits(orc):
    """quantize_row_q6_K_ref after the fits: iscale = -128 / (scale of largest |scale|),
    d = fp16(1 / iscale), int8 scales rne(iscale scale) (<= 127), codes rne(x / (d sc)) in [-32, 31]."""
    rng = np.random.default_rng(41)
    x = rng.normal(0, 1, (24, 256)).astype(np.float32)
    x[5] *= 1e-2
    q = orc.quantize(x, "q6_K")
    for r in range(x.shape[0]):
        sub = [orc.make_qx16(x[r, 16 * j:16 * j + 16])[1] for j in range(16)]
        msc = sub[int(np.argmax(np.abs(sub)))]
        isc = np.float32(np.float32(-128.0) / np.float32(msc))
        blk = q[r]
        d = float(np.frombuffer(blk[208:210].tobytes(), np.float16)[0])
        assert d == _f16(float(np.float32(1) / isc))
        scales = blk[192:208].view(np.int8).astype(np.int64)
        v = np.float32(isc) * np.array(sub, np.float32)
        want = np.minimum(_rne(v), 127)
        assert ((want == scales) | _near_half(v.astype(np.float64))).all()
        ql, qh = blk[0:128].astype(np.int64), blk[128:192].astype(np.int64)
        codes = np.zeros(256, np.int64)
        for h in range(2):
            for l in range(32):
                a, b = ql[64 * h + l], ql[64 * h + l + 32]
                hb = qh[32 * h + l]
                codes[128 * h + l] = (a & 0xF) | (((hb >> 0) & 3) << 4)
                codes[128 * h + l + 32] = (b & 0xF) | (((hb >> 2) & 3) << 4)
                codes[128 * h + l + 64] = (a >> 4) | (((hb >> 4) & 3) << 4)
                codes[128 * h + l + 96] = (b >> 4) | (((hb >> 6) & 3) << 4)
        for j in range(16):
            dj = np.float32(np.float32(d) * np.float32(scales[j]))
            if dj == 0:
                continue
            vv = x[r, 16 * j:16 * j + 16].astype(np.float64) / float(dj)
            want = np.clip(_rne(vv), -32, 31) + 32
            assert ((want == codes[16 * j:16 * j + 16]) | _near_half(vv)).all(), f"row {r} sub-block {j}"
