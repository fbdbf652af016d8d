"""trc_hip_qmatvec_noalloc: the fused matvec without any allocation (its x
planes live in a fixed device array), checked through the C ABI against
trc_hip_qmatvec on the same inputs, bit for bit, and against the oracle's
dequantize-then-mul_mat (gguf_tensor_to_f32, src/io/trc_gguf.cpp:966-1049,
then compute_mul_mat, src/backends/cpu/trc_cpu_ops.cpp:182-216) within the
row-L2 bar 1e-4. Two calls in a row, the second with a smaller input, so the
second runs over what the first left in the shared array."""
import numpy as np
import pytest

import oracle_lib as O
from conftest import announce
from gpu_util import Dev, empty
from test_oracle_dequant import TYPES
from traincpp_amd import hip as H
from traincpp_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _run(fn, t, raw, K, M, X):
    N = X.shape[2]
    dw, dx = Dev(raw), Dev(X)
    dy = empty((1, 1, N, M))
    fn(t, dw.ptr, K, M, (K // 32) * H.BLOCK_BYTES[t], dx.ptr, N, K * 4, dy.ptr, M * 4)
    H.sync()
    y = np.ascontiguousarray(dy.read())
    for d in (dw, dx, dy):
        d.free()
    return y


@pytest.mark.parametrize("first,second", [
    # (type, K, M, N): the first call fills the whole array (32 columns, two
    # column tiles), the second is smaller (other format, fewer columns, K split)
    (("q4_0", 4096, 4096, 32), ("q5_1", 1024, 300, 5)),
    (("q8_0", 8192, 1024, 16), ("q4_1", 512, 2048, 3)),
    (("q5_0", 4096, 14336, 16), ("q5_0", 4096, 64, 1)),
])
def test_noalloc_matches_qmatvec(hip, first, second):
    for name, K, M, N in (first, second):
        t = TYPES[name]
        announce(f"qmatvec_noalloc {name} K={K} M={M} N={N}")
        raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 700 + K + N))
        X = synth.normal(800 + M + N, K * N).reshape(1, 1, N, K)
        got = _run(H.qmatvec_noalloc, t, raw, K, M, X)
        ref = _run(H.qmatvec, t, raw, K, M, X)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        want = O.mul_mat(O.dequant(t, raw, threads=8).reshape(1, 1, M, K), X, threads=8)
        assert O.row_l2_error(got, want) <= TOL


def test_noalloc_argument_errors(hip):
    w, x, y = empty(4096, np.uint8), empty(4096), empty(4096)
    with pytest.raises(H.HipError) as e:
        H.qmatvec_noalloc(H.TYPE_Q4_0, w.ptr, 64, 4, 36, x.ptr, H.QMATVEC_MAX_N + 1, 256, y.ptr, 16)
    assert e.value.code == H.E_SHAPE
    with pytest.raises(H.HipError) as e:
        H.qmatvec_noalloc(H.TYPE_Q4_0, w.ptr, 64, 4, 36, x.ptr, 1, 256, w.ptr + 32, 16)  # y inside W
    assert e.value.code == H.E_SHAPE
    for d in (w, x, y):
        d.free()
