"""Writes gguf_dequant_kats.json: the hand-computed dequantization known-answer
tests of the reference (tests/test_gguf.cpp:355-444), as data.

Each case holds the raw block bytes exactly as the reference test assembles
them, and the expected floats it states. The expected values are exact dyadic
rationals, so they are stored as float32 bit patterns. Run from the repo root:
    python tests/golden/make_gguf_kats.py
"""
import json
import struct
from pathlib import Path

import numpy as np


def u16(x):
    return struct.pack("<H", x)


def u32(x):
    return struct.pack("<I", x)


def nib_pairs(lo_fn, hi_fn):
    return bytes(((lo_fn(j) & 0x0F) | (hi_fn(j) << 4)) & 0xFF for j in range(16))


def bits(vals):
    return [int(v) for v in np.asarray(vals, dtype=np.float32).view(np.uint32)]


cases = []

# Q4_0 (test_gguf.cpp:355-376): block 0 d=0.5, qs[j] = j | (15-j)<<4;
# block 1 d=0.25, qs[j] = (15-j) | j<<4.
blk = u16(0x3800) + nib_pairs(lambda j: j, lambda j: 15 - j) + u16(0x3400) + nib_pairs(lambda j: 15 - j, lambda j: j)
exp = [0.0] * 64
for j in range(16):
    exp[j] = (j - 8) * 0.5
    exp[16 + j] = (7 - j) * 0.5
    exp[32 + j] = (7 - j) * 0.25
    exp[48 + j] = (j - 8) * 0.25
cases.append({"name": "q4_0", "type": 2, "blocks_hex": blk.hex(), "expect_bits": bits(exp), "src": "tests/test_gguf.cpp:355-376"})

# Q4_1 (:378-391): d=0.25, m=-1, qs[j] = j | (15-j)<<4.
blk = u16(0x3400) + u16(0xBC00) + nib_pairs(lambda j: j, lambda j: 15 - j)
exp = [0.0] * 32
for j in range(16):
    exp[j] = j * 0.25 - 1.0
    exp[16 + j] = (15 - j) * 0.25 - 1.0
cases.append({"name": "q4_1", "type": 3, "blocks_hex": blk.hex(), "expect_bits": bits(exp), "src": "tests/test_gguf.cpp:378-391"})

# Q5_0 (:393-415): d=1, qh=0 then qh=0xFFFFFFFF, qs[j] = j | (15-j)<<4.
q = nib_pairs(lambda j: j, lambda j: 15 - j)
blk = u16(0x3C00) + u32(0) + q + u16(0x3C00) + u32(0xFFFFFFFF) + q
exp = [0.0] * 64
for j in range(16):
    exp[j] = j - 16
    exp[16 + j] = -1 - j
    exp[32 + j] = j
    exp[48 + j] = 15 - j
cases.append({"name": "q5_0", "type": 6, "blocks_hex": blk.hex(), "expect_bits": bits(exp), "src": "tests/test_gguf.cpp:393-415"})

# Q5_1 (:417-431): d=0.5, m=0.125, qh=0, qs[j] = j | (15-j)<<4.
blk = u16(0x3800) + u16(0x3000) + u32(0) + nib_pairs(lambda j: j, lambda j: 15 - j)
exp = [0.0] * 32
for j in range(16):
    exp[j] = j * 0.5 + 0.125
    exp[16 + j] = (15 - j) * 0.5 + 0.125
cases.append({"name": "q5_1", "type": 7, "blocks_hex": blk.hex(), "expect_bits": bits(exp), "src": "tests/test_gguf.cpp:417-431"})

# Q8_0 (:433-444): d=0.125, qs[j] = j - 16.
blk = u16(0x3000) + bytes(((j - 16) & 0xFF) for j in range(32))
exp = [(j - 16) * 0.125 for j in range(32)]
cases.append({"name": "q8_0", "type": 8, "blocks_hex": blk.hex(), "expect_bits": bits(exp), "src": "tests/test_gguf.cpp:433-444"})

out = Path(__file__).resolve().parent / "gguf_dequant_kats.json"
out.write_text(json.dumps({"cases": cases}, indent=1) + "\n")
print(f"wrote {out} ({len(cases)} cases)")
