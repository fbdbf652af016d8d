"""Helpers for the GPU parity tests: device copies of numpy arrays and views,
described to the C ABI as ggml tensors."""
from __future__ import annotations

import ctypes as C

import numpy as np

import oracle_lib as O
from traincpp_amd import hip as H


class Dev:
    """A device copy of a contiguous numpy base array; views of the base map to
    ggml tensor descriptors at the matching byte offset."""

    def __init__(self, base: np.ndarray):
        self.base = np.ascontiguousarray(base)
        self.buf = H.DeviceBuffer(max(self.base.nbytes, 16)).upload(self.base)

    def tensor(self, view: np.ndarray | None = None, type_: int = H.TYPE_F32) -> H.Tensor:
        v = self.base if view is None else view
        off = v.__array_interface__["data"][0] - self.base.__array_interface__["data"][0]
        assert 0 <= off < self.base.nbytes
        ne, nb = O.view_meta(v)
        return H.tensor(self.buf.ptr + off, ne, nb, type_)

    @property
    def ptr(self) -> int:
        return self.buf.ptr

    def read(self, like: np.ndarray | None = None) -> np.ndarray:
        out = np.empty_like(self.base if like is None else like)
        return self.buf.download(out)

    def free(self):
        self.buf.free()


def empty(shape, dtype=np.float32) -> Dev:
    return Dev(np.zeros(shape, dtype=dtype))


def gpu_mul_mat(a_dev: Dev, a_view, b_dev: Dev, b_view) -> np.ndarray:
    ane, _ = O.view_meta(a_view)
    bne, _ = O.view_meta(b_view)
    out = empty((bne[3], bne[2], bne[1], ane[1]))
    H.mul_mat_f32(a_dev.tensor(a_view), b_dev.tensor(b_view), out.tensor())
    H.sync()
    res = out.read()
    out.free()
    return res


_RT = None


def runtime() -> C.CDLL:
    """The HIP runtime the library links (for streams, graphs and memory queries)."""
    global _RT
    if _RT is None:
        rt = C.CDLL("libamdhip64.so")
        V, PV = C.c_void_p, C.POINTER(C.c_void_p)
        for name, args in {
            "hipStreamCreate": [PV], "hipStreamDestroy": [V], "hipStreamBeginCapture": [V, C.c_int],
            "hipStreamEndCapture": [V, PV], "hipGraphInstantiate": [PV, V, V, V, C.c_size_t],
            "hipGraphLaunch": [V, V], "hipGraphExecDestroy": [V], "hipGraphDestroy": [V],
            "hipMemGetInfo": [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)], "hipDeviceSynchronize": [],
            "hipGetLastError": [],
        }.items():
            fn = getattr(rt, name)
            fn.argtypes = args
            fn.restype = C.c_int
        _RT = rt
    return _RT


def mem_free() -> int:
    """Free device memory (hipMemGetInfo) after the device has gone idle."""
    rt = runtime()
    assert rt.hipDeviceSynchronize() == 0
    free, total = C.c_size_t(), C.c_size_t()
    assert rt.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


class Stream:
    """A HIP stream of the runtime the library uses (hipStreamCreate/Destroy),
    passed to the C ABI as its opaque handle."""

    def __init__(self):
        h = C.c_void_p()
        assert runtime().hipStreamCreate(C.byref(h)) == 0
        self.handle = h.value

    def close(self):
        """Frees the stream's qmatvec workspace (after its work), then destroys it,
        in the order include/trc_hip_abi.h asks of callers."""
        if self.handle:
            H.qmatvec_release_stream(self.handle)
            H.sync(self.handle)
            assert runtime().hipStreamDestroy(C.c_void_p(self.handle)) == 0
            self.handle = None
