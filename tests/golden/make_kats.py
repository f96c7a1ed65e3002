"""Writes quant_kats.json (encoder blocks: inputs and the bytes ggml's algorithms give) and
kquant_mutations.json (which wrong search parameter each K-quant block would expose).

ggml is not available to run. The Q8_0 / Q4_0 / Q8_K blocks and the exact-grid K-quant blocks were
worked by hand from the published algorithm of the ggml routine named; the only arithmetic done
here is packing those hand-derived values into bytes. The other K-quant blocks are chosen from
seeded candidates so that together they catch every wrong parameter of the searches
(make_qkx2_quants' rmin / rdelta / nstep and sub-block weighting, make_qx_quants' candidate range
and weighting): their bytes come from kquant_ref.py, an independent restatement of the algorithms
(checked against the hand-worked blocks and against the C oracle by the tests), and
kquant_mutations.json records, for each wrong parameter, a block whose bytes it changes.
Run: python tests/golden/make_kats.py
"""

import json
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parent))
import kquant_ref as kr  # noqa: E402


def h16(v):  # fp16 bytes, little-endian
    return np.array([v], np.float16).tobytes().hex()


def i8(vals, n):
    return np.array(list(vals) + [0] * (n - len(vals)), np.int8).tobytes().hex()


def pad(vals, n):
    return list(map(float, vals)) + [0.0] * (n - len(vals))


kats = {}

# quantize_row_q8_0_ref: amax 127 -> d = 1, id = 1; roundf rounds halves away from zero.
x = [127, 2.5, -2.5, 0.5, -0.5, 1.5]
kats["q8_0_ties_half_away"] = {"kind": "weight", "type": "q8_0", "x": pad(x, 32),
                               "hex": h16(1.0) + i8([127, 3, -3, 1, -1, 2], 32)}
# quantize_row_q8_0 (x86 AVX2): id = 127/amax = 1; _mm256_round_ps nearest rounds halves to even.
kats["act_q8_0_avx2_ties_even"] = {"kind": "act_q8_0", "variant": "avx2", "x": pad(x, 32),
                                   "hex": h16(1.0) + i8([127, 2, -2, 0, 0, 2], 32)}
# The generic quantize_row_q8_0 is the reference encoder.
kats["act_q8_0_scalar_half_away"] = {"kind": "act_q8_0", "variant": "scalar", "x": pad(x, 32),
                                     "hex": h16(1.0) + i8([127, 3, -3, 1, -1, 2], 32)}
# All-zero block: d = 0, id = 0, codes 0.
kats["q8_0_zero"] = {"kind": "weight", "type": "q8_0", "x": pad([], 32), "hex": "00" * 34}
# amax = 1e-3: d = 1e-3/127 = 7.874e-6 = 132.1 units of 2^-24 -> fp16 subnormal 0x0084; codes +-127.
kats["q8_0_subnormal_scale"] = {"kind": "weight", "type": "q8_0", "x": pad([1e-3, -1e-3], 32),
                                "hex": "8400" + i8([127, -127], 32)}
# quantize_row_q4_0_ref: max = +7 -> d = 7/-8 = -0.875 (fp16 0xbb00), id = -8/7;
# element 0: 7*id + 8.5 = 0.5 -> 0; zeros: 8.5 -> 8. byte j = code j | code (j+16) << 4.
kats["q4_0_positive_max"] = {"kind": "weight", "type": "q4_0", "x": pad([7], 32),
                             "hex": "00bb" + "80" + "88" * 15}
# |-1| and |1| tie: the first (-1) sets max -> d = 0.125, id = 8; -1 -> 0.5 -> 0; 1 -> 16.5 -> 16
# clamped to 15; 0.5 -> 12.5 -> 12.
kats["q4_0_first_of_equal_magnitudes"] = {"kind": "weight", "type": "q4_0", "x": pad([-1, 1, 0.5], 32),
                                          "hex": h16(0.125) + "808f8c" + "88" * 13}
# Zero super-block: every field 0.
kats["q4_K_zero"] = {"kind": "weight", "type": "q4_K", "x": pad([], 256), "hex": "00" * 144}
# quantize_row_q8_K_ref: first largest |x| is +2 -> iscale = -127/2 = -63.5; codes 2 -> -127,
# -2 -> 127, 1 -> -63.5 -> -64 (nearest, ties even), 0.5 -> -31.75 -> -32; d = 1/iscale (f32);
# bsums[0] = -127 + 127 - 64 - 32 = -96.
d = np.float32(1) / np.float32(-63.5)
kats["q8_K_positive_max_first"] = {
    "kind": "act_q8_K", "x": pad([2, -2, 1, 0.5], 256),
    "hex": np.array([d], np.float32).tobytes().hex() + i8([-127, 127, -64, -32], 256)
    + np.array([-96] + [0] * 15, np.int16).tobytes().hex()}


# ------------------------------------------------------------------------------- K-quants
#
# Exact grids (quantize_row_q4_K_ref, make_qkx2_quants with nmax 15, rmin -1, rdelta 0.1, nstep 20).
# Every sub-block holds x = mn + s * L with L running over 0..14 (both ends present), s = 63 * 2^-8,
# mn = -t with t = 63 * dmin. The min/max fit takes iscale = 15 / (14 s) and misplaces codes
# (15 L / 14 rounds away from L), so its weighted error is positive; the first candidate,
# (rmin + 0 + 15) / (max - min) = 1 / s, puts every value exactly on its code and its least-squares
# refit recovers (s, mn): it wins. Each sub-block's scale and min are then the super-block's
# largest, so the 6-bit scale and min are both 63 (the 12 packed bytes all 0xff), d = s / 63 = 2^-8
# and dmin = t / 63, and the codes recomputed against them are the L themselves. A wrong rmin
# (the candidate numerators then miss 14) leaves an inexact fit and other bytes.


def exact_grid_q4_K(dmin):
    t = 63.0 * dmin
    s = 63.0 * 2.0 ** -8
    L = []
    for j in range(8):  # a different order of the 15 levels in every sub-block
        L += [(7 * i + 3 * j) % 15 for i in range(32)]
    x = [-t + s * v for v in L]
    assert all(np.float32(v) == v for v in x)  # exact in f32
    qs = []
    for c in range(0, 256, 64):
        qs += [L[c + i] | (L[c + i + 32] << 4) for i in range(32)]
    hexs = h16(2.0 ** -8) + h16(dmin) + "ff" * 12 + bytes(qs).hex()
    return x, hexs


x, hexs = exact_grid_q4_K(2.0 ** -9)
kats["q4_K_exact_grid_search_beats_minmax"] = {"kind": "weight", "type": "q4_K", "x": x, "hex": hexs}
assert kr.quantize_q4_K(x).hex() == hexs  # the restatement agrees with the hand-worked block

# Wrong parameters a fixture set must expose (keyword arguments of kquant_ref's encoders).
MUTATIONS = {
    "q4_K": {"rmin -0.5": {"rmin": -0.5}, "rmin -1.5": {"rmin": -1.5}, "rdelta 0.2": {"rdelta": 0.2},
             "rdelta 0.05": {"rdelta": 0.05}, "nstep 19": {"nstep": 19}, "nstep 10": {"nstep": 10},
             "weights 1": {"weighting": "uniform"}, "weights |x|": {"weighting": "abs"},
             "weights x^2": {"weighting": "square"}},
    "q5_K": {"rmin -1": {"rmin": -1.0}, "rmin 0": {"rmin": 0.0}, "rdelta 0.2": {"rdelta": 0.2},
             "rdelta 0.05": {"rdelta": 0.05}, "nstep 14": {"nstep": 14}, "nstep 20": {"nstep": 20},
             "weights 1": {"weighting": "uniform"}, "weights |x|": {"weighting": "abs"},
             "weights x^2": {"weighting": "square"}},
    "q6_K": {"no search": {"search": range(0)}, "search -8..8": {"search": range(-8, 9)},
             "search -10..10": {"search": range(-10, 11)}, "weights 1": {"weighting": "uniform"},
             "weights |x|": {"weighting": "abs"}},
}


def sub_block(rng, kind, n):
    if kind == "normal":
        return rng.normal(0, 0.02, n)
    if kind == "outlier":  # one large value: late candidates (a wider grid) win
        v = rng.uniform(-1, 1, n) * 0.05
        v[rng.integers(0, n)] = rng.uniform(0.1, 0.3)
        return v
    if kind == "positive":  # offset data: the least-squares min comes out > 0 and is clamped
        return 0.2 + np.abs(rng.normal(0, 0.05, n))
    if kind == "tiny":  # mins far below fp16's normal range: subnormal dmin
        return rng.normal(0, 2e-4, n)
    return rng.standard_t(3, n) * 0.01


def candidates(t, rng, count):
    kinds = ["normal", "outlier", "positive", "tiny", "heavy"]
    for c in range(count):
        # every fifth candidate small throughout (the largest min, and so dmin, below fp16's normals)
        mix = ["tiny"] * 8 if c % 5 == 4 else [kinds[k] for k in rng.integers(0, len(kinds), 8)]
        yield np.concatenate([sub_block(rng, k, 32) for k in mix]).astype(np.float32).tolist()


def traits(t, x):
    tr = []
    h = kr.ENCODERS[t](x, trace=tr)
    out = set()
    if t in ("q4_K", "q5_K"):
        if any(c for _, c in tr):
            out.add("clamped min wins")
        if any(w >= (20 if t == "q4_K" else 15) for w, _ in tr):
            out.add("last candidate wins")
        if 0 < int.from_bytes(h[2:4], "little") < 0x400:
            out.add("subnormal dmin")
    elif any(w != 0 for w in tr):
        out.add("search moves the scale")
    return h, out


mutation_record = {}
rng = np.random.default_rng(20261202)
for t in ("q4_K", "q5_K", "q6_K"):
    want_traits = {"q4_K": {"clamped min wins", "last candidate wins", "subnormal dmin"},
                   "q5_K": {"clamped min wins", "last candidate wins", "subnormal dmin"},
                   "q6_K": {"search moves the scale"}}[t]
    uncaught = set(MUTATIONS[t])
    missing = set(want_traits)
    chosen = 0
    for x in candidates(t, rng, 400):
        h, tr = traits(t, x)
        catches = {m for m in uncaught if kr.ENCODERS[t](x, **MUTATIONS[t][m]) != h}
        if not (catches or (tr & missing)):
            continue
        name = f"{t}_search_{chosen}"
        kats[name] = {"kind": "weight", "type": t, "x": x, "hex": h.hex()}
        mutation_record[name] = {"catches": sorted(catches), "traits": sorted(tr)}
        uncaught -= catches
        missing -= tr
        chosen += 1
        if not uncaught and not missing:
            break
    assert not uncaught and not missing, (t, uncaught, missing)
for name in ("q4_K_exact_grid_search_beats_minmax",):
    x, h = kats[name]["x"], bytes.fromhex(kats[name]["hex"])
    mutation_record[name] = {"catches": sorted(m for m, kw in MUTATIONS["q4_K"].items() if kr.quantize_q4_K(x, **kw) != h),
                             "traits": ["exact grid: the first candidate beats the min/max fit"]}

Path(__file__).with_name("quant_kats.json").write_text(json.dumps(kats, indent=1) + "\n")
Path(__file__).with_name("kquant_mutations.json").write_text(json.dumps(
    {"mutations": {t: {m: {k: (list(v) if isinstance(v, range) else v) for k, v in kw.items()}
                       for m, kw in ms.items()} for t, ms in MUTATIONS.items()},
     "caught_by": mutation_record}, indent=1) + "\n")
