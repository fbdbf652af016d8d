"""trc_hip_qmatvec_noalloc: the fused matvec without any allocation (its x
planes live in a fixed device array), checked through the C ABI against
trc_hip_qmatvec on the same inputs, bit for bit, and against the oracle's
dequantize-then-mul_mat (gguf_tensor_to_f32, src/io/trc_gguf.cpp:966-1049,
then compute_mul_mat, src/backends/cpu/trc_cpu_ops.cpp:182-216) within the
row-L2 bar 1e-4.

That it allocates nothing is shown two ways: the first call of each pair runs on
a stream that has never been used, captured into a graph in global capture mode
(a hipMalloc inside such a capture fails the capture), and the free device memory
is the same before and after an eager call on another fresh stream. Every case
has N >= 9, which always runs the x pre-pass into the shared array, and the
second call of each pair is smaller, so it runs over what the first one left."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from conftest import announce
from gpu_util import Dev, Stream, empty, mem_free, runtime
from test_oracle_dequant import TYPES
from traincpp_amd import hip as H
from traincpp_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-4
CAPTURE_GLOBAL = 0  # hipStreamCaptureModeGlobal


def _inputs(name, K, M, N):
    t = TYPES[name]
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 700 + K + N))
    X = synth.normal(800 + M + N, K * N).reshape(1, 1, N, K)
    return t, raw, X


def _call(fn, t, dw, dx, dy, K, M, N, stream):
    fn(t, dw.ptr, K, M, (K // 32) * H.BLOCK_BYTES[t], dx.ptr, N, K * 4, dy.ptr, M * 4, stream)


def _captured_noalloc(t, dw, dx, dy, K, M, N):
    """The call on a fresh stream, captured in global mode, then replayed twice."""
    rt = runtime()
    s = Stream()
    graph, gexec = C.c_void_p(), C.c_void_p()
    assert rt.hipStreamBeginCapture(C.c_void_p(s.handle), CAPTURE_GLOBAL) == 0
    try:
        _call(H.qmatvec_noalloc, t, dw, dx, dy, K, M, N, s.handle)
    finally:
        rc = rt.hipStreamEndCapture(C.c_void_p(s.handle), C.byref(graph))
    assert rc == 0, f"global-mode capture failed (hipError_t {rc}): the entry did something not capturable"
    assert rt.hipGraphInstantiate(C.byref(gexec), graph, None, None, 0) == 0
    outs = []
    for _ in range(2):
        assert rt.hipGraphLaunch(gexec, C.c_void_p(s.handle)) == 0
        H.sync(s.handle)
        outs.append(np.ascontiguousarray(dy.read()))
    rt.hipGraphExecDestroy(gexec)
    rt.hipGraphDestroy(graph)
    s.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    return outs[0]


@pytest.mark.parametrize("first,second", [
    # (type, K, M, N): the first call fills the most of the array (32 columns, two
    # column tiles), the second is smaller (other format, fewer columns, K split)
    (("q4_0", 4096, 4096, 32), ("q5_1", 1024, 300, 12)),
    (("q8_0", 8192, 1024, 16), ("q4_1", 512, 2048, 10)),
    (("q5_0", 4096, 14336, 16), ("q5_0", 4096, 64, 9)),
])
def test_noalloc_matches_qmatvec(hip, first, second):
    for name, K, M, N in (first, second):
        announce(f"qmatvec_noalloc {name} K={K} M={M} N={N}")
        t, raw, X = _inputs(name, K, M, N)
        dw, dx = Dev(raw), Dev(X)
        dy = empty((1, 1, N, M))
        got = _captured_noalloc(t, dw, dx, dy, K, M, N)
        _call(H.qmatvec, t, dw, dx, dy, K, M, N, None)
        H.sync()
        ref = np.ascontiguousarray(dy.read())
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        want = O.mul_mat(O.dequant(t, raw, threads=8).reshape(1, 1, M, K), X, threads=8)
        assert O.row_l2_error(got, want) <= TOL
        for d in (dw, dx, dy):
            d.free()


def test_noalloc_leaves_free_memory_unchanged(hip):
    """An eager call on a stream that has never been used: the per-stream entry
    would allocate its 8.3 MiB workspace there; this one must not."""
    name, K, M, N = "q4_0", 4096, 2048, 16
    announce(f"qmatvec_noalloc free memory {name} K={K} M={M} N={N}")
    t, raw, X = _inputs(name, K, M, N)
    dw, dx = Dev(raw), Dev(X)
    dy = empty((1, 1, N, M))
    s = Stream()
    before = mem_free()
    _call(H.qmatvec_noalloc, t, dw, dx, dy, K, M, N, s.handle)
    H.sync(s.handle)
    after = mem_free()
    assert after == before
    s.close()
    for d in (dw, dx, dy):
        d.free()


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
