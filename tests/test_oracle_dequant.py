"""Pins the oracle's dequantizers (oracle/oracle.cpp, restating
src/io/trc_gguf.cpp:320-417) on the CPU.

Checks, each chosen so that a plausible slip fails one of them:
  * the reference's hand-computed KATs (tests/test_gguf.cpp:355-444);
  * an exhaustive sweep of every quant value x every finite fp16 scale (x a set
    of mins incl. signed zeros and subnormals) against the closed form
    fl32(fl32(q*d) + m), evaluated with numpy's own IEEE arithmetic from the
    documented block layout (a wrong nibble order, offset, bias, or an FMA,
    changes bits);
  * one-hot and random qh masks for the 5th-bit mapping of Q5_0/Q5_1;
  * the reference library itself (oracle/_ref: gguf_tensor_to_f32 on a GGUF file),
    bit for bit on random blocks.
"""
import json

import numpy as np
import pytest

import oracle_lib as O
from conftest import GOLDEN

TYPES = {"q4_0": 2, "q4_1": 3, "q5_0": 6, "q5_1": 7, "q8_0": 8}
BYTES = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34}
FINITE_HALF = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
FINITE_HALF = FINITE_HALF[np.isfinite(FINITE_HALF.view(np.float16))]
M_SET = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x8400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF,
                  0xAA8F, 0xA1C6, 0x9E4F, 0x2E66, 0x0C00, 0x8C00], dtype=np.uint16)


def load_kats():
    return json.loads((GOLDEN / "gguf_dequant_kats.json").read_text())["cases"]


@pytest.mark.parametrize("case", load_kats(), ids=lambda c: c["name"])
def test_reference_kats(case):
    blocks = np.frombuffer(bytes.fromhex(case["blocks_hex"]), dtype=np.uint8)
    got = O.dequant(case["type"], blocks)
    want = np.array(case["expect_bits"], dtype=np.uint32).view(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def pack_blocks(type_, d, m, qh, q):
    """Assembles raw blocks from per-block fields and the 32 integer quants in
    output order (before the bias), following the block layouts of
    src/io/trc_gguf.cpp:320-417."""
    n = d.size
    bb = BYTES[type_]
    raw = np.zeros((n, bb), dtype=np.uint8)
    raw[:, 0:2] = d.astype("<u2").view(np.uint8).reshape(n, 2)
    off = 2
    if type_ in (3, 7):
        raw[:, 2:4] = m.astype("<u2").view(np.uint8).reshape(n, 2)
        off = 4
    if type_ in (6, 7):
        raw[:, off:off + 4] = qh.astype("<u4").view(np.uint8).reshape(n, 4)
        off += 4
    if type_ == 8:
        raw[:, off:off + 32] = q.astype(np.int8).view(np.uint8)
    else:
        lo = q[:, :16] & 0x0F
        hi = q[:, 16:] & 0x0F
        raw[:, off:off + 16] = (lo | (hi << 4)).astype(np.uint8)
    return raw.reshape(-1)


def closed_form(type_, d, m, qh, q):
    """y = fl32(q' * d) [+ m, rounded again], with q' the integer quant after the
    5th bit and the bias, in numpy float32 arithmetic."""
    e = np.arange(32)
    qq = q.astype(np.int64)
    if type_ in (6, 7):
        qq = (qq & 0x0F) | (((qh[:, None].astype(np.int64) >> e) & 1) << 4)
    bias = {2: 8, 3: 0, 6: 16, 7: 0, 8: 0}[type_]
    qq = qq - bias
    df = d.view(np.float16).astype(np.float32)[:, None]
    p = qq.astype(np.float32) * df
    if type_ in (3, 7):
        p = p + m.view(np.float16).astype(np.float32)[:, None]
    return p.reshape(-1)


def q_patterns(t):
    """Blocks of raw quants (before bias) that put every possible value in the
    low- and high-nibble halves (Q4), every 5-bit value in both halves (Q5) or
    every int8 (Q8)."""
    e = np.arange(32)
    if t in (2, 3):
        return (e % 16)[None, :]
    if t in (6, 7):
        return np.stack([e, (e + 16) % 32])
    return (np.arange(256) - 128).reshape(8, 32)


@pytest.mark.parametrize("name", list(TYPES))
def test_exhaustive_quant_scale_sweep(name):
    t = TYPES[name]
    pats = q_patterns(t)
    ms = M_SET if t in (3, 7) else np.zeros(1, dtype=np.uint16)
    n_d, n_m, n_p = FINITE_HALF.size, ms.size, pats.shape[0]
    d = np.repeat(FINITE_HALF, n_m * n_p)
    m = np.tile(np.repeat(ms, n_p), n_d)
    q = np.tile(pats, (n_d * n_m, 1))
    if t in (6, 7):  # bit 4 of the 5-bit value lives in qh
        qh = (((q >> 4) & 1).astype(np.uint64) << np.arange(32, dtype=np.uint64)).sum(axis=1).astype(np.uint32)
        q = q & 0x0F
    else:
        qh = np.zeros(d.size, dtype=np.uint32)
    raw = pack_blocks(t, d, m, qh, q)
    got = O.dequant(t, raw, threads=8)
    want = closed_form(t, d, m, qh, q)
    assert got.size == d.size * 32
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", ["q5_0", "q5_1"])
def test_fifth_bit_mapping(name):
    t = TYPES[name]
    rng = np.random.default_rng(11)
    onehot = (np.uint64(1) << np.arange(32, dtype=np.uint64)).astype(np.uint32)
    qh = np.concatenate([onehot, rng.integers(0, 2**32, 256, dtype=np.uint64).astype(np.uint32),
                         np.uint32([0, 0xFFFFFFFF, 0x0000FFFF, 0xFFFF0000])])
    n = qh.size
    q = rng.integers(0, 16, (n, 32))
    d = np.full(n, 0x3C00, dtype=np.uint16)  # d = 1: y is the integer itself
    m = np.zeros(n, dtype=np.uint16)
    got = O.dequant(t, pack_blocks(t, d, m, qh, q)).reshape(n, 32)
    e = np.arange(32)
    want = (q | (((qh[:, None].astype(np.int64) >> e) & 1) << 4)) - (16 if t == 6 else 0)
    assert np.array_equal(got, want.astype(np.float32))
    # the one-hot rows: only element b changes by 16
    base = q - (16 if t == 6 else 0)
    assert np.array_equal(got[:32] - base[:32], 16 * np.eye(32, dtype=np.float32))


@pytest.mark.skipif(not O.have_ref(), reason="oracle/_ref not built (reference checkout absent)")
@pytest.mark.parametrize("name", list(TYPES))
def test_bitwise_vs_reference_library(name, tmp_dir):
    t = TYPES[name]
    rng = np.random.default_rng(100 + t)
    n = 4096
    raw = rng.integers(0, 256, (n, BYTES[t]), dtype=np.uint8)
    raw[:, 1] &= 0x7B  # finite d
    if t in (3, 7):
        raw[:, 3] &= 0x7B  # finite m
    raw = raw.reshape(-1)
    got = O.dequant(t, raw)
    want = O.ref_dequant(t, raw, tmp_dir)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", list(TYPES))
def test_threads_do_not_change_bits(name):
    t = TYPES[name]
    rng = np.random.default_rng(5)
    raw = rng.integers(0, 256, (10007, BYTES[t]), dtype=np.uint8)
    raw[:, 1] &= 0x7B
    raw = raw.reshape(-1)
    a = O.dequant(t, raw, threads=1)
    b = O.dequant(t, raw, threads=7)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
