"""Pins the oracle's binary16 conversions (oracle/oracle.cpp) before anything is
compared against them.

fp16 -> fp32 is what every dequantized value starts from (src/core/trc_float.h:23-40).
"""
import numpy as np
import pytest

import oracle_lib as O

ALL_HALF = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def oracle_decode_all():
    out = np.empty(65536, dtype=np.float32)
    O.oracle().orc_fp16_to_fp32_n(ALL_HALF.ctypes.data, out.ctypes.data, 65536)
    return out


def test_fp16_decode_matches_ieee_on_all_finite_patterns():
    got = oracle_decode_all()
    want = ALL_HALF.view(np.float16).astype(np.float32)  # numpy: exact IEEE half -> single
    finite = np.isfinite(want)
    assert finite.sum() == 63488
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    # +-Inf stay Inf, NaNs stay NaN
    assert np.array_equal(np.isinf(got), np.isinf(want))
    assert np.array_equal(np.isnan(got), np.isnan(want))


def test_fp16_decode_special_values():
    dec = O.oracle().orc_fp16_to_fp32
    assert np.float32(dec(0x0000)).view(np.uint32) == 0x00000000  # +0, the bug of trc_float.h:32
    assert np.float32(dec(0x8000)).view(np.uint32) == 0x80000000  # -0
    assert dec(0x0001) == np.float32(2.0**-24)                    # smallest subnormal
    assert dec(0x03FF) == np.float32(1023 * 2.0**-24)             # largest subnormal
    assert dec(0x0400) == np.float32(2.0**-14)                    # smallest normal
    assert dec(0x7BFF) == np.float32(65504.0)
    assert dec(0x3C00) == 1.0 and dec(0xBC00) == -1.0


@pytest.mark.skipif(not O.have_ref(), reason="oracle/_ref not built (reference checkout absent)")
def test_fp16_decode_bitwise_vs_reference_all_patterns():
    got = oracle_decode_all()
    ref = O.ref()
    want = np.array([ref.ref_fp16_to_fp32(int(h)) for h in range(65536)], dtype=np.float32)
    # every pattern, NaN payloads included
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_fp32_to_fp16_is_round_to_nearest_even():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[np.isfinite(vals)]
    # add every tie / boundary around the half grid
    h = np.arange(0x7C00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    mids = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    vals = np.concatenate([vals, mids, -mids, np.float32([65504, 65519.99, 65520, 2**-25, 2**-24, 0.0, -0.0])])
    got = np.empty(vals.size, dtype=np.uint16)
    O.oracle().orc_fp32_to_fp16_n(vals.ctypes.data, got.ctypes.data, vals.size)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.skipif(not O.have_ref(), reason="oracle/_ref not built (reference checkout absent)")
def test_fp32_to_fp16_vs_reference_on_finite_values():
    rng = np.random.default_rng(8)
    vals = np.concatenate([rng.uniform(2e-4, 1e-3, 2000), rng.uniform(-0.05, 0, 2000),
                           rng.standard_normal(2000) * 1000]).astype(np.float32)
    ref = O.ref()
    orc = O.oracle()
    for v in vals:
        assert orc.orc_fp32_to_fp16(float(v)) == ref.ref_fp32_to_fp16(float(v))
