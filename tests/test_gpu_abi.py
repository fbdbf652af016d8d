"""The C ABI's memory and utility entry points on the GPU: allocation, copies,
fill (Device::fill_tensors), strided copy (OP_CONT/OP_DUP, compute_dup
src/backends/cpu/trc_cpu_ops.cpp:219-236) and the forced-error hook."""
import os

import numpy as np
import pytest

from conftest import announce
from gpu_util import Dev, empty
from traincpp_amd import hip as H

pytestmark = pytest.mark.gpu


def test_props(hip):
    p = H.init(0)
    assert H.device_count() >= 1
    assert p.arch.decode().startswith("gfx950")
    assert p.compute_units > 0 and p.memory_total > p.memory_free > 0
    assert p.abi_version == 1


def test_roundtrip_and_fill(hip):
    announce("abi roundtrip")
    x = np.arange(100003, dtype=np.float32)
    d = Dev(x)
    assert np.array_equal(d.read(), x)
    H.fill_f32(d.ptr + 4, -2.5, 1000)
    H.sync()
    y = d.read()
    assert y[0] == 0 and np.all(y[1:1001] == -2.5) and y[1001] == 1001
    H.check(H.load().trc_hip_memset(d.ptr, 0, 8, None))
    H.sync()
    assert np.all(d.read()[:2] == 0)


@pytest.mark.parametrize("offset,count", [(0, 1003), (16, 8), (0, 3), (32, 2_000_001), (4, 5)])
def test_fill_aligned_and_tails(hip, offset, count):
    """16-byte aligned fills take whole float4 stores plus a tail of count % 4;
    others go float by float. Neighbours on both sides stay untouched."""
    x = np.arange(count + 64, dtype=np.float32)
    d = Dev(x)
    H.fill_f32(d.ptr + offset, 7.25, count)
    H.sync()
    y = d.read()
    o = offset // 4
    assert np.array_equal(y[:o], x[:o])
    assert np.all(y[o:o + count] == 7.25)
    assert np.array_equal(y[o + count:], x[o + count:])
    d.free()


@pytest.mark.parametrize("dtype", [np.float32, np.uint8, np.int16, np.float64])
def test_cpy_transpose_is_cont(hip, dtype):
    announce(f"abi cpy {dtype}")
    code = {np.float32: 0, np.uint8: 24, np.int16: 25, np.float64: 28}[dtype]
    x = (np.arange(3 * 5 * 7 * 2) % 251).astype(dtype).reshape(2, 7, 5, 3)
    src = Dev(x)
    view = np.swapaxes(src.base, 2, 3)  # ggml transpose
    out = empty(view.shape, dtype)
    H.cpy(src.tensor(view, code), out.tensor(None, code))
    H.sync()
    assert np.array_equal(out.read(), np.ascontiguousarray(np.swapaxes(x, 2, 3)))


@pytest.mark.parametrize("shape", [(2, 3, 70, 130), (1, 1, 4096, 4096), (1, 1, 1, 65), (1, 1, 65, 1)])
def test_cpy_transpose_tiles(hip, shape):
    """4-byte transposes through the LDS tiles: ragged tiles over planes, the
    Linear layer's 64 MiB dW^T, and single rows or columns (plain copy path)."""
    announce(f"abi cpy transpose {shape}")
    x = np.random.default_rng(3).standard_normal(shape).astype(np.float32)
    src = Dev(x)
    view = np.swapaxes(src.base, 2, 3)
    out = empty(view.shape, np.float32)
    H.cpy(src.tensor(view), out.tensor())
    H.sync()
    assert np.array_equal(out.read().view(np.uint32), np.ascontiguousarray(np.swapaxes(x, 2, 3)).view(np.uint32))
    src.free()
    out.free()


def test_forced_error_hook(hip):
    os.environ["TRC_HIP_FORCE_ERROR"] = "trc_hip_dequant"
    try:
        with pytest.raises(H.HipError) as e:
            H.dequant(H.TYPE_Q4_0, 0, 1, 0)
        assert e.value.code == H.E_FORCED
        assert "forced" in H.last_error()
    finally:
        del os.environ["TRC_HIP_FORCE_ERROR"]
