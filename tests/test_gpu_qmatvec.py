"""H2 parity: trc_hip_qmatvec (fused dequant-matvec) against the oracle's
dequantize-then-mul_mat (gguf_tensor_to_f32, src/io/trc_gguf.cpp:966-1049,
followed by compute_mul_mat, src/backends/cpu/trc_cpu_ops.cpp:182-216).

Bar (written here): for every dst row (ne0-run over M), max|y - yhat| / ||yhat||_2 <= 1e-4.
"""
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


def oracle_qmatvec(t, raw, K, M, X):
    W = O.dequant(t, raw, threads=8).reshape(1, 1, M, K)
    return O.mul_mat(W, X, threads=8)


def gpu_qmatvec(t, raw, K, M, X, x_pad=0, y_pad=0):
    N = X.shape[2]
    if x_pad:
        Xp = np.zeros((1, 1, N, K + x_pad), np.float32)
        Xp[..., :K] = X
    else:
        Xp = X
    dw, dx = Dev(raw), Dev(Xp)
    dy = empty((1, 1, N, M + y_pad))
    H.qmatvec(t, dw.ptr, K, M, (K // 32) * H.BLOCK_BYTES[t], dx.ptr, N, (K + x_pad) * 4, dy.ptr, (M + y_pad) * 4)
    H.sync()
    y = dy.read()[..., :M]
    for d in (dw, dx, dy):
        d.free()
    return np.ascontiguousarray(y)


@pytest.mark.parametrize("name", ["q4_0", "q5_0"])
@pytest.mark.parametrize("N", [1, 16])
def test_config2_decode_shapes(hip, name, N):
    """W 14336 x 4096 (K=4096) times x with N = 1 and 16 columns, N(0,1)."""
    t = TYPES[name]
    K, M = 4096, 14336
    announce(f"qmatvec cfg2 {name} N={N}")
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, synth.config_seed(2, t)))
    X = synth.normal(synth.config_seed(2, 100 + N), K * N).reshape(1, 1, N, K)
    got = gpu_qmatvec(t, raw, K, M, X)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert O.row_l2_error(got, want) <= TOL


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("N", [1, 2, 3, 5, 8, 13, 16])
def test_all_formats_small(hip, name, N):
    t = TYPES[name]
    K, M = 32 * 37, 301  # odd block count per row, M not a multiple of any row tile
    announce(f"qmatvec {name} K={K} M={M} N={N}")
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 99 + t))
    X = synth.normal(7 + N, K * N).reshape(1, 1, N, K)
    got = gpu_qmatvec(t, raw, K, M, X)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert O.row_l2_error(got, want) <= TOL


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("K,M", [(32, 1), (64, 3), (4096, 64), (11008, 257)])
def test_edge_shapes_and_padded_columns(hip, name, K, M):
    t = TYPES[name]
    N = 4
    announce(f"qmatvec edge {name} K={K} M={M}")
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 5 + K + M))
    X = synth.normal(K + M, K * N).reshape(1, 1, N, K)
    got = gpu_qmatvec(t, raw, K, M, X, x_pad=4, y_pad=3)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert O.row_l2_error(got, want) <= TOL


def test_argument_errors(hip):
    w = empty(4096, np.uint8)
    x = empty(4096)
    y = empty(4096)
    with pytest.raises(H.HipError) as e:
        H.qmatvec(H.TYPE_Q4_0, w.ptr, 64, 4, 36, x.ptr, 17, 256, y.ptr, 16)
    assert e.value.code == H.E_SHAPE
    with pytest.raises(H.HipError) as e:
        H.qmatvec(H.TYPE_Q4_0, w.ptr, 48, 4, 36, x.ptr, 1, 192, y.ptr, 16)  # K % 32
    assert e.value.code == H.E_SHAPE
    with pytest.raises(H.HipError) as e:
        H.qmatvec(H.TYPE_Q4_1, w.ptr + 2, 64, 4, 40, x.ptr, 1, 256, y.ptr, 16)
    assert e.value.code == H.E_ALIGN
