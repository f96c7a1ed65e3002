"""Writes quant_kats.json: hand-worked encoder blocks (inputs and the bytes ggml's algorithms give).

Each expected byte string below was derived by hand from the published algorithm of the ggml
routine named (ggml is not available to run); the only arithmetic done here is packing those
hand-derived values into bytes. Run: python tests/golden/make_kats.py
"""

import json
from pathlib import Path

import numpy as np


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

Path(__file__).with_name("quant_kats.json").write_text(json.dumps(kats, indent=1) + "\n")
