"""Pins the seeded-input generators: the oracle's splitmix64 draws
(oracle/oracle.cpp, restating src/core/trc_rng.cpp:38-68) against the
reference library's own rng (oracle/_ref) and against the published splitmix64
constants, and the package's vectorised numpy generator
(train.cpp_amd/synth.py) against the oracle."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from traincpp_amd import synth


def splitmix64_reference_values(seed, n):
    """Straight from the published splitmix64 algorithm (Steele, Lea, Flood 2014)
    in Python integers: the independent check of the C restatement."""
    out = []
    s = seed
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & (2**64 - 1)
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
        out.append(z ^ (z >> 31))
    return out


def test_splitmix64_known_values():
    st = C.c_uint64(0)
    got = [O.oracle().orc_rng_next_u64(C.byref(st)) for _ in range(5)]
    # first outputs for seed 0 as published with the algorithm
    assert got[0] == 0xE220A8397B1DCDAF
    assert got == splitmix64_reference_values(0, 5)


@pytest.mark.skipif(not O.have_ref(), reason="oracle/_ref not built (reference checkout absent)")
def test_rng_bitwise_vs_reference_library():
    orc, ref = O.oracle(), O.ref()
    for seed in (0, 1, 0x7261696E, 2**63 + 12345):
        a, b = C.c_uint64(seed), C.c_uint64(seed)
        for _ in range(200):
            assert orc.orc_rng_next_u64(C.byref(a)) == ref.ref_rng_next_u64(C.byref(b))
        for _ in range(200):
            assert np.float32(orc.orc_rng_uniform01(C.byref(a))).view(np.uint32) == \
                np.float32(ref.ref_rng_uniform01(C.byref(b))).view(np.uint32)
        for _ in range(200):  # same libm calls in both: identical bits
            assert np.float32(orc.orc_rng_normal(C.byref(a), 0.0, 1.0)).view(np.uint32) == \
                np.float32(ref.ref_rng_normal(C.byref(b), 0.0, 1.0)).view(np.uint32)


def test_numpy_generator_matches_oracle_streams():
    seed, n = 0x1234, 1000
    st = synth.streams(seed, n)
    u64 = synth.next_u64(st.copy())
    for i in (0, 1, 17, 999):
        s = C.c_uint64(seed + i)
        assert int(u64[i]) == O.oracle().orc_rng_next_u64(C.byref(s))
    u = synth.uniform01(synth.streams(seed, n))
    for i in (0, 5, 500):
        s = C.c_uint64(seed + i)
        assert np.float32(u[i]) == np.float32(O.oracle().orc_rng_uniform01(C.byref(s)))
    # Box-Muller in numpy float32 may differ from glibc's logf/cosf in the last ulp
    x = synth.normal(seed, n)
    for i in (0, 3, 400):
        s = C.c_uint64(seed + i)
        assert abs(float(x[i]) - O.oracle().orc_rng_normal(C.byref(s), 0.0, 1.0)) <= 1e-5


def test_quant_block_distributions():
    b = synth.quant_blocks(2, 20000, 7)
    d = b["d"].view(np.float16).astype(np.float32)
    assert d.min() >= 2e-4 * 0.999 and d.max() <= 1e-3 * 1.001
    nib = np.concatenate([b["qs"] & 15, b["qs"] >> 4]).ravel()
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.9 * counts.mean()  # uniform over 0..15
    q8 = synth.quant_blocks(8, 20000, 9)["qs"].ravel()
    assert q8.min() == -127 and q8.max() == 127  # [-127, 127], -128 never drawn
    m = synth.quant_blocks(3, 5000, 11)["m"].view(np.float16).astype(np.float32)
    assert m.min() >= -0.05 * 1.001 and m.max() <= 0.0
