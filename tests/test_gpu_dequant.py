"""H1 parity: trc_hip_dequant (gfx950) against the oracle, bit for bit.

Reference semantics: gguf_tensor_to_f32 -> dequantize_q* (src/io/trc_gguf.cpp:320-417,
966-1049). Bar: identical float32 bit patterns (memcmp) on every element.
"""
import json

import numpy as np
import pytest

import oracle_lib as O
from conftest import GOLDEN, announce
from gpu_util import Dev, empty
from test_oracle_dequant import BYTES, M_SET, TYPES, pack_blocks, q_patterns
from traincpp_amd import hip as H
from traincpp_amd import synth

pytestmark = pytest.mark.gpu

ALL_HALF = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)


def gpu_dequant(t, raw: np.ndarray) -> np.ndarray:
    raw = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
    n = raw.size // BYTES[t]
    src = Dev(raw)
    dst = empty(n * 32)
    H.dequant(t, src.ptr, n, dst.ptr)
    H.sync()
    out = dst.read()
    src.free()
    dst.free()
    return out


def assert_bits_equal(got, want):
    g, w = got.view(np.uint32), want.view(np.uint32)
    if not np.array_equal(g, w):
        bad = np.nonzero(g != w)[0]
        raise AssertionError(f"{bad.size} elements differ; first at {bad[0]}: gpu {got[bad[0]]!r} "
                             f"(0x{g[bad[0]]:08x}) oracle {want[bad[0]]!r} (0x{w[bad[0]]:08x})")


@pytest.mark.parametrize("case", json.loads((GOLDEN / "gguf_dequant_kats.json").read_text())["cases"],
                         ids=lambda c: c["name"])
def test_reference_kats(hip, case):
    announce(f"dequant KAT {case['name']}")
    raw = np.frombuffer(bytes.fromhex(case["blocks_hex"]), dtype=np.uint8)
    got = gpu_dequant(case["type"], raw)
    want = np.array(case["expect_bits"], dtype=np.uint32).view(np.float32)
    assert_bits_equal(got, want)


@pytest.mark.parametrize("name", list(TYPES))
def test_config1_full_tensor(hip, name):
    """4096 x 11008 tensor (1,409,024 blocks) with the benchmark distributions."""
    t = TYPES[name]
    n = 4096 * 11008 // 32
    announce(f"dequant cfg1 {name} n_blocks={n}")
    raw = synth.block_bytes(synth.quant_blocks(t, n, synth.config_seed(1, t)))
    got = gpu_dequant(t, raw)
    want = O.dequant(t, raw, threads=8)
    assert_bits_equal(got, want)


@pytest.mark.parametrize("name", list(TYPES))
def test_exhaustive_scale_sweep(hip, name):
    """Every quant value x every fp16 scale pattern (NaN and Inf included) x a set
    of mins: the GPU's half decode and arithmetic must match the CPU's bits."""
    t = TYPES[name]
    pats = q_patterns(t)
    ms = M_SET if t in (3, 7) else np.zeros(1, dtype=np.uint16)
    n_d, n_m, n_p = ALL_HALF.size, ms.size, pats.shape[0]
    d = np.repeat(ALL_HALF, n_m * n_p)
    m = np.tile(np.repeat(ms, n_p), n_d)
    q = np.tile(pats, (n_d * n_m, 1))
    if t in (6, 7):
        qh = (((q >> 4) & 1).astype(np.uint64) << np.arange(32, dtype=np.uint64)).sum(axis=1).astype(np.uint32)
        q = q & 0x0F
    else:
        qh = np.zeros(d.size, dtype=np.uint32)
    raw = pack_blocks(t, d, m, qh, q)
    announce(f"dequant sweep {name} n_blocks={d.size}")
    got = gpu_dequant(t, raw)
    want = O.dequant(t, raw, threads=8)
    fin = np.isfinite(want)
    assert_bits_equal(got[fin], want[fin])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))


@pytest.mark.parametrize("name", list(TYPES))
def test_nan_payloads_match(hip, name):
    """Non-finite scales: NaN payloads and signs, not just NaN-ness."""
    t = TYPES[name]
    nonfinite = ALL_HALF[~np.isfinite(ALL_HALF.view(np.float16))]
    pats = q_patterns(t)
    d = np.repeat(nonfinite, pats.shape[0])
    q = np.tile(pats, (nonfinite.size, 1))
    m = np.zeros(d.size, dtype=np.uint16)
    qh = np.zeros(d.size, dtype=np.uint32)
    raw = pack_blocks(t, d, m, qh, q & 0x0F if t != 8 else q)
    announce(f"dequant NaN payloads {name}")
    assert_bits_equal(gpu_dequant(t, raw), O.dequant(t, raw))


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("n", [1, 2, 7, 8, 9, 31, 33, 1023, 1025, 100003])
def test_ragged_block_counts(hip, name, n):
    t = TYPES[name]
    announce(f"dequant ragged {name} n={n}")
    raw = synth.block_bytes(synth.quant_blocks(t, n, 1234 + n))
    assert_bits_equal(gpu_dequant(t, raw), O.dequant(t, raw))


def test_zero_blocks_is_a_no_op(hip):
    dst = empty(8)
    H.dequant(H.TYPE_Q4_0, dst.ptr, 0, dst.ptr)
    H.sync()


def test_misaligned_and_bad_type_are_rejected(hip):
    src = empty(1024, np.uint8)
    dst = empty(256)
    with pytest.raises(H.HipError) as e:
        H.dequant(H.TYPE_Q4_0, src.ptr + 1, 4, dst.ptr)
    assert e.value.code == H.E_ALIGN
    with pytest.raises(H.HipError) as e:
        H.dequant(H.TYPE_Q5_1, src.ptr + 2, 4, dst.ptr)
    assert e.value.code == H.E_ALIGN
    with pytest.raises(H.HipError) as e:
        H.dequant(H.TYPE_Q4_0, src.ptr, 4, dst.ptr + 4)
    assert e.value.code == H.E_ALIGN
    with pytest.raises(H.HipError) as e:
        H.dequant(12, src.ptr, 4, dst.ptr)  # Q4_K: not a legacy format
    assert e.value.code == H.E_INVALID
