"""An independent restatement of ggml's K-quant weight encoders, for the known-answer fixtures.

ggml (llama.cpp, the version the reference pins) is not available here, so the Q4_K / Q5_K / Q6_K
encoder bytes cannot be taken from it. This module restates the published algorithms of
ggml-quants.c in Python with float32 arithmetic step by step (one rounding per C operation, no
fused multiply-add, as ggml-base is compiled), separately from the C oracle, so the two check each
other:

  - make_qkx2_quants(n = 32, nmax, x, weights, rmin, rdelta, nstep, use_mad = false): an
    asymmetric (scale, min) fit: start from the min/max fit, then nstep + 1 candidate inverse
    scales (rmin + rdelta * is + nmax) / (max - min), each refit by weighted least squares (the
    offset clamped to <= 0, the scale then refit alone), kept when its weighted squared error is
    strictly smaller;
  - quantize_row_q4_K_ref / quantize_row_q5_K_ref: per 32-value sub-block the fit above with
    weights sqrt(mean x^2) + |x| (Q4_K: nmax 15, rmin -1, rdelta 0.1, nstep 20; Q5_K: 31, -0.5,
    0.1, 15), 6-bit scales and mins relative to the super-block's largest (fp16 d, dmin), codes
    recomputed against the rounded scales (a sub-block whose rounded scale is 0 keeps its codes);
  - make_qx_quants(n = 16, nmax = 32, x, rmse_type = 1, weights x^2): symmetric, start from
    -nmax / max (max = the first value of largest magnitude), least-squares scale, then the
    candidates -(nmax + 0.1 * is) / max for is in -9..9 (0 skipped), kept when
    sumlx^2 > best * suml2;
  - quantize_row_q6_K_ref: the fit above per 16 values, int8 scales against the scale of largest
    magnitude (d = 1 / (-128 / max_scale) as fp16), codes recomputed, 6-bit codes packed low
    nibbles / high bits.

The parameters (rmin, rdelta, nstep, the weighting, the candidate range) are arguments so a test
can show that the fixtures would fail under a wrong value of each.
"""

from __future__ import annotations

import numpy as np

F = np.float32


def _f(v) -> np.float32:
    return np.float32(v)


def nearest_int(v) -> int:
    """ggml's nearest_int: round to nearest, ties to even (lrintf)."""
    return int(np.rint(_f(v)))


def fp16_bits(v) -> int:
    return int(np.array([v], np.float32).astype(np.float16).view(np.uint16)[0])


def fp16_value(bits: int) -> np.float32:
    return _f(np.array([bits], np.uint16).view(np.float16)[0])


# ---------------------------------------------------------------------------------- Q4_K / Q5_K

def make_qkx2(x, w, nmax: int, rmin: float, rdelta: float, nstep: int, trace: list | None = None):
    """-> (scale, the_min, L) for 32 values x with weights w (float32 lists). trace, if given,
    gets (winning candidate step or -1 for the min/max fit, whether its offset was clamped)."""
    n = len(x)
    mn, mx = x[0], x[0]
    sum_w = w[0]
    sum_x = _f(sum_w * x[0])
    for i in range(1, n):
        if x[i] < mn:
            mn = x[i]
        if x[i] > mx:
            mx = x[i]
        sum_w = _f(sum_w + w[i])
        sum_x = _f(sum_x + _f(w[i] * x[i]))
    if mn > 0:
        mn = _f(0)
    if mx == mn:
        if trace is not None:
            trace.append((-1, False))
        return _f(0), _f(-mn), [0] * n
    won, clamped = -1, False
    iscale = _f(_f(nmax) / _f(mx - mn))
    scale = _f(_f(1) / iscale)
    L = []
    best = _f(0)
    for i in range(n):
        l = min(nmax, max(0, nearest_int(_f(iscale * _f(x[i] - mn)))))
        L.append(l)
        diff = _f(_f(_f(scale * _f(l)) + mn) - x[i])
        best = _f(best + _f(w[i] * _f(diff * diff)))
    for step in range(nstep + 1):
        iscale = _f(_f(_f(_f(rmin) + _f(_f(rdelta) * _f(step))) + _f(nmax)) / _f(mx - mn))
        aux = []
        sum_l = sum_l2 = sum_xl = _f(0)
        for i in range(n):
            l = min(nmax, max(0, nearest_int(_f(iscale * _f(x[i] - mn)))))
            aux.append(l)
            wl = _f(w[i] * _f(l))
            sum_l = _f(sum_l + wl)
            sum_l2 = _f(sum_l2 + _f(wl * _f(l)))
            sum_xl = _f(sum_xl + _f(wl * x[i]))
        D = _f(_f(sum_w * sum_l2) - _f(sum_l * sum_l))
        if D > 0:
            this_scale = _f(_f(_f(sum_w * sum_xl) - _f(sum_x * sum_l)) / D)
            this_min = _f(_f(_f(sum_l2 * sum_x) - _f(sum_l * sum_xl)) / D)
            was_clamped = bool(this_min > 0)
            if was_clamped:
                this_min = _f(0)
                this_scale = _f(sum_xl / sum_l2)
            cur = _f(0)
            for i in range(n):
                diff = _f(_f(_f(this_scale * _f(aux[i])) + this_min) - x[i])
                cur = _f(cur + _f(w[i] * _f(diff * diff)))
            if cur < best:
                L, best, scale, mn = aux, cur, this_scale, this_min
                won, clamped = step, was_clamped
    if trace is not None:
        trace.append((won, clamped))
    return scale, _f(-mn), L


def kquant_weights(x, kind: str = "ggml"):
    """Sub-block weights: ggml's sqrt(mean x^2) + |x|, or a variant for mutation tests."""
    if kind == "ggml":
        s2 = _f(0)
        for v in x:
            s2 = _f(s2 + _f(v * v))
        av = _f(np.sqrt(_f(s2 / _f(len(x)))))
        return [_f(av + _f(abs(v))) for v in x]
    if kind == "uniform":
        return [_f(1)] * len(x)
    if kind == "abs":
        return [_f(abs(v)) for v in x]
    if kind == "square":
        return [_f(v * v) for v in x]
    raise ValueError(kind)


def _scale_min_k4(j: int, q: list[int]) -> tuple[int, int]:
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def _kquant_superblock(x, nmax, rmin, rdelta, nstep, weighting, trace=None):
    """Shared part of Q4_K / Q5_K for one 256-value super-block: (d bits, dmin bits, 12 scale
    bytes, 256 codes)."""
    L, scales, mins = [0] * 256, [], []
    for j in range(8):
        sub = x[32 * j:32 * j + 32]
        sc, mn, Lj = make_qkx2(sub, kquant_weights(sub, weighting), nmax, rmin, rdelta, nstep, trace)
        scales.append(sc)
        mins.append(mn)
        L[32 * j:32 * j + 32] = Lj
    max_scale = max_min = _f(0)
    for j in range(8):
        if scales[j] > max_scale:
            max_scale = scales[j]
        if mins[j] > max_min:
            max_min = mins[j]
    inv_scale = _f(_f(63) / max_scale) if max_scale > 0 else _f(0)
    inv_min = _f(_f(63) / max_min) if max_min > 0 else _f(0)
    sb = [0] * 12
    for j in range(8):
        ls = min(63, nearest_int(_f(inv_scale * scales[j])))
        lm = min(63, nearest_int(_f(inv_min * mins[j])))
        if j < 4:
            sb[j] = ls
            sb[j + 4] = lm
        else:
            sb[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            sb[j - 4] |= (ls >> 4) << 6
            sb[j] |= (lm >> 4) << 6
    d_bits = fp16_bits(_f(max_scale / _f(63)))
    dmin_bits = fp16_bits(_f(max_min / _f(63)))
    for j in range(8):
        sc, m = _scale_min_k4(j, sb)
        d = _f(fp16_value(d_bits) * _f(sc))
        if d == 0:
            continue
        dm = _f(fp16_value(dmin_bits) * _f(m))
        for ii in range(32):
            L[32 * j + ii] = min(nmax, max(0, nearest_int(_f(_f(x[32 * j + ii] + dm) / d))))
    return d_bits, dmin_bits, sb, L


def _u16(v: int) -> bytes:
    return int(v).to_bytes(2, "little")


def quantize_q4_K(x, rmin=-1.0, rdelta=0.1, nstep=20, weighting="ggml", trace=None) -> bytes:
    x = [_f(v) for v in x]
    out = b""
    for b in range(0, len(x), 256):
        d, dmin, sb, L = _kquant_superblock(x[b:b + 256], 15, rmin, rdelta, nstep, weighting, trace)
        qs = []
        for j in range(0, 256, 64):
            qs += [L[j + l] | (L[j + l + 32] << 4) for l in range(32)]
        out += _u16(d) + _u16(dmin) + bytes(sb) + bytes(qs)
    return out


def quantize_q5_K(x, rmin=-0.5, rdelta=0.1, nstep=15, weighting="ggml", trace=None) -> bytes:
    x = [_f(v) for v in x]
    out = b""
    for b in range(0, len(x), 256):
        d, dmin, sb, L = _kquant_superblock(x[b:b + 256], 31, rmin, rdelta, nstep, weighting, trace)
        qh, ql = [0] * 32, []
        m1, m2 = 1, 2
        for nn in range(0, 256, 64):
            chunk = [0] * 32
            for j in range(32):
                l1, l2 = L[nn + j], L[nn + j + 32]
                if l1 > 15:
                    l1 -= 16
                    qh[j] |= m1
                if l2 > 15:
                    l2 -= 16
                    qh[j] |= m2
                chunk[j] = l1 | (l2 << 4)
            ql += chunk
            m1 <<= 2
            m2 <<= 2
        out += _u16(d) + _u16(dmin) + bytes(sb) + bytes(qh) + bytes(ql)
    return out


# ----------------------------------------------------------------------------------------- Q6_K

GROUP_MAX_EPS = np.float32(1e-15)


def make_qx(x, nmax: int = 32, search=range(-9, 10), weighting: str = "square", trace: list | None = None):
    """make_qx_quants(n, nmax, x, L, rmse_type = 1, qw = NULL): -> (scale, L) with L in [0, 2 nmax).
    trace, if given, gets the step of the last candidate that won (0: the first fit)."""
    n = len(x)
    mx = amax = _f(0)
    for v in x:
        ax = _f(abs(v))
        if ax > amax:
            amax, mx = ax, v
    if amax < GROUP_MAX_EPS:
        if trace is not None:
            trace.append(0)
        return _f(0), [0] * n

    def weight(v):
        if weighting == "square":
            return _f(v * v)
        if weighting == "uniform":
            return _f(1)
        if weighting == "abs":
            return _f(abs(v))
        raise ValueError(weighting)

    def sums(iscale):
        slx = sl2 = _f(0)
        ls = []
        for v in x:
            l = min(nmax - 1, max(-nmax, nearest_int(_f(iscale * v))))
            ls.append(l)
            w = weight(v)
            slx = _f(slx + _f(_f(w * v) * _f(l)))
            sl2 = _f(sl2 + _f(_f(w * _f(l)) * _f(l)))
        return slx, sl2, ls

    iscale = _f(_f(-nmax) / mx)
    sumlx, suml2, ls = sums(iscale)
    L = [l + nmax for l in ls]
    scale = _f(sumlx / suml2) if suml2 != 0 else _f(0)
    best = _f(scale * sumlx)
    won = 0
    for step in search:
        if step == 0:
            continue
        iscale = _f(-_f(_f(nmax) + _f(_f(0.1) * _f(step))) / mx)
        sumlx, suml2, ls = sums(iscale)
        if suml2 > 0 and _f(sumlx * sumlx) > _f(best * suml2):
            L = [l + nmax for l in ls]
            scale = _f(sumlx / suml2)
            best = _f(scale * sumlx)
            won = step
    if trace is not None:
        trace.append(won)
    return scale, L


def quantize_q6_K(x, search=range(-9, 10), weighting="square", trace=None) -> bytes:
    x = [_f(v) for v in x]
    out = b""
    for b in range(0, len(x), 256):
        xs = x[b:b + 256]
        L, scales = [0] * 256, []
        max_scale = max_abs = _f(0)
        for ib in range(16):
            sc, Lb = make_qx(xs[16 * ib:16 * ib + 16], 32, search, weighting, trace)
            scales.append(sc)
            L[16 * ib:16 * ib + 16] = Lb
            if _f(abs(sc)) > max_abs:
                max_abs, max_scale = _f(abs(sc)), sc
        if max_abs < GROUP_MAX_EPS:
            out += bytes(210)
            continue
        iscale = _f(_f(-128) / max_scale)
        d_bits = fp16_bits(_f(_f(1) / iscale))
        q_scales = [min(127, nearest_int(_f(iscale * sc))) for sc in scales]
        for j in range(16):
            d = _f(fp16_value(d_bits) * _f(q_scales[j]))
            if d == 0:
                continue
            for ii in range(16):
                L[16 * j + ii] = min(31, max(-32, nearest_int(_f(xs[16 * j + ii] / d)))) + 32
        ql, qh = [0] * 128, [0] * 64
        for half in range(2):
            j = 128 * half
            for l in range(32):
                q1, q2, q3, q4 = (L[j + l] & 0xF, L[j + l + 32] & 0xF, L[j + l + 64] & 0xF, L[j + l + 96] & 0xF)
                ql[64 * half + l] = q1 | (q3 << 4)
                ql[64 * half + l + 32] = q2 | (q4 << 4)
                qh[32 * half + l] = ((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4)
                                     | ((L[j + l + 96] >> 4) << 6))
        out += bytes(ql) + bytes(qh) + np.array(q_scales, np.int8).tobytes() + _u16(d_bits)
    return out


ENCODERS = {"q4_K": quantize_q4_K, "q5_K": quantize_q5_K, "q6_K": quantize_q6_K}
