"""Writes tests/golden/quant_known_answers.json and gemm_int_small.json.

Known-answer blocks for the GGML formats, built from the PUBLIC layout
(block_q4_0 / block_q8_0 / block_q4_K) and written down here case by case:
each block is given as explicit bytes and its expected 32 / 256 decoded
values come from the hand-chosen quantities of that case (d, nibbles,
6-bit scales and mins), not from a decoder. The reference (vortx) has no
quantized code, so these vectors are this build's own; the Q4_K scale
bytes of case q4k_highbits are asserted against the hand-packed literal
below to pin the 6-bit packing.

gemm_int_small.json: small integer matrices and their product from numpy
int64 matmul (exact in f32 as well).

Run: python tests/golden/make_quant_golden.py
"""
import json
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def half(x: float) -> bytes:
    return struct.pack("<e", x)


def f16bits(bits: int) -> bytes:
    return struct.pack("<H", bits)


cases = []

# ---- Q4_0: {half d; uint8 qs[16]}, w_j = (lo(qs[j]) - 8) d, w_{j+16} = (hi(qs[j]) - 8) d
# A: d = 1, qs[0] = 0x9F (lo 15 -> +7 at element 0, hi 9 -> +1 at element 16), rest 0x88 -> 0
blk = half(1.0) + bytes([0x9F] + [0x88] * 15)
exp = [0.0] * 32
exp[0], exp[16] = 7.0, 1.0
cases.append({"name": "q4_0_onehot", "qtype": 2, "block": blk.hex(), "expected": exp})
# B: d = -0.5, all nibbles 0 -> (0 - 8) * -0.5 = 4
blk = half(-0.5) + bytes([0x00] * 16)
cases.append({"name": "q4_0_negd", "qtype": 2, "block": blk.hex(), "expected": [4.0] * 32})
# C: d = smallest f16 subnormal 2^-24; qs[15] = 0xF0 -> element 15 = -8 * 2^-24, element 31 = 7 * 2^-24
blk = f16bits(0x0001) + bytes([0x88] * 15 + [0xF0])
exp = [0.0] * 32
exp[15], exp[31] = -8.0 * 2.0 ** -24, 7.0 * 2.0 ** -24
cases.append({"name": "q4_0_subnormal_d", "qtype": 2, "block": blk.hex(), "expected": exp})
# D: every element position j gets nibble value v=(j % 16); lo for j < 16, hi for j >= 16 with d = 0.25
qs = bytes([(j & 0xF) | (((15 - j) & 0xF) << 4) for j in range(16)])
blk = half(0.25) + qs
exp = [((j & 0xF) - 8) * 0.25 for j in range(16)] + [(((15 - j) & 0xF) - 8) * 0.25 for j in range(16)]
cases.append({"name": "q4_0_positions", "qtype": 2, "block": blk.hex(), "expected": exp})

# ---- Q8_0: {half d; int8 qs[32]}, w_i = d qs[i]
qs = np.arange(-16, 16, dtype=np.int8)
cases.append({"name": "q8_0_ramp", "qtype": 8, "block": (half(0.25) + qs.tobytes()).hex(),
              "expected": [float(v) * 0.25 for v in range(-16, 16)]})
qs = np.zeros(32, dtype=np.int8)
qs[0], qs[31] = -127, 127
cases.append({"name": "q8_0_maxhalf", "qtype": 8, "block": (f16bits(0x7BFF) + qs.tobytes()).hex(),
              "expected": [-127.0 * 65504.0] + [0.0] * 30 + [127.0 * 65504.0]})
cases.append({"name": "q8_0_zero_d", "qtype": 8, "block": (half(0.0) + np.full(32, 77, np.int8).tobytes()).hex(),
              "expected": [0.0] * 32})


# ---- Q4_K: {half d; half dmin; uint8 scales[12]; uint8 qs[128]}
def pack_q4k_scales(sc, m):
    """6-bit (scale, min) of the 8 sub-blocks -> 12 bytes (public layout)."""
    b = [0] * 12
    for s in range(4):
        b[s] = (sc[s] & 63) | ((sc[s + 4] >> 4) << 6)
        b[s + 4] = (m[s] & 63) | ((m[s + 4] >> 4) << 6)
        b[s + 8] = (sc[s + 4] & 15) | ((m[s + 4] & 15) << 4)
    return bytes(b)


# F: sc_s = s + 1, m_s = 2 s, all nibbles 3, d = 1, dmin = 0.5 -> sub-block s (elements 32s..32s+31)
#    = 3 (s + 1) - 0.5 * 2 s = 2 s + 3
sc = [s + 1 for s in range(8)]
m = [2 * s for s in range(8)]
blk = half(1.0) + half(0.5) + pack_q4k_scales(sc, m) + bytes([0x33] * 128)
cases.append({"name": "q4k_uniform", "qtype": 12, "block": blk.hex(),
              "expected": [float(2 * (i // 32) + 3) for i in range(256)]})

# G: 6-bit values with high bits set; chunk c byte l has lo = l % 16, hi = 15 - l % 16
sc = [10, 20, 30, 40, 63, 33, 17, 1]
m = [1, 2, 3, 4, 5, 48, 60, 0]
scb = pack_q4k_scales(sc, m)
assert list(scb) == [202, 148, 94, 40, 1, 194, 195, 4, 95, 1, 193, 1], list(scb)  # hand-packed literal
qs = bytes([(l % 16) | ((15 - l % 16) << 4) for c in range(4) for l in range(32)])
d, dmin = 0.125, 0.0625
exp = [0.0] * 256
for c in range(4):
    for l in range(32):
        exp[64 * c + l] = d * sc[2 * c] * (l % 16) - dmin * m[2 * c]
        exp[64 * c + 32 + l] = d * sc[2 * c + 1] * (15 - l % 16) - dmin * m[2 * c + 1]
blk = half(d) + half(dmin) + scb + qs
cases.append({"name": "q4k_highbits", "qtype": 12, "block": blk.hex(), "expected": exp,
              "scales": sc, "mins": m})

with open(os.path.join(HERE, "quant_known_answers.json"), "w") as f:
    json.dump({"cases": cases}, f, indent=1)

rng = np.random.default_rng(1234)
a = rng.integers(-9, 10, size=(5, 7))
b = rng.integers(-9, 10, size=(7, 3))
with open(os.path.join(HERE, "gemm_int_small.json"), "w") as f:
    json.dump({"a": a.tolist(), "b": b.tolist(), "c": (a @ b).tolist()}, f)
print("wrote", len(cases), "quant cases and gemm_int_small.json")
