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


class Stream:
    """A HIP stream of the runtime the library uses (hipStreamCreate/Destroy),
    passed to the C ABI as its opaque handle."""

    _rt = None

    def __init__(self):
        if Stream._rt is None:
            rt = C.CDLL("libamdhip64.so")
            rt.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
            rt.hipStreamDestroy.argtypes = [C.c_void_p]
            Stream._rt = rt
        h = C.c_void_p()
        assert Stream._rt.hipStreamCreate(C.byref(h)) == 0
        self.handle = h.value

    def close(self):
        if self.handle:
            H.sync(self.handle)
            assert Stream._rt.hipStreamDestroy(C.c_void_p(self.handle)) == 0
            self.handle = None
