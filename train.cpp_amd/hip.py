"""ctypes binding of libtrc_hip.so, the C ABI declared in include/trc_hip_abi.h.

This is how Python callers (the parity tests and bench.py) reach the HIP
kernels. Loading fails loudly when the library has not been built: there is no
CPU fallback behind these calls.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"
LIB_PATH = LIB_DIR / "libtrc_hip.so"

TYPE_F32, TYPE_Q4_0, TYPE_Q4_1, TYPE_Q5_0, TYPE_Q5_1, TYPE_Q8_0 = 0, 2, 3, 6, 7, 8
QUANT_TYPES = {"q4_0": TYPE_Q4_0, "q4_1": TYPE_Q4_1, "q5_0": TYPE_Q5_0, "q5_1": TYPE_Q5_1, "q8_0": TYPE_Q8_0}
BLOCK_BYTES = {TYPE_Q4_0: 18, TYPE_Q4_1: 20, TYPE_Q5_0: 22, TYPE_Q5_1: 24, TYPE_Q8_0: 34}
QMATVEC_MAX_N = 64

OK, E_INVALID, E_SHAPE, E_ALIGN, E_NO_DEVICE, E_FORCED = 0, -1, -2, -3, -4, -5

EXPORTS = (
    "trc_hip_device_count", "trc_hip_init", "trc_hip_sync", "trc_hip_last_error",
    "trc_hip_malloc", "trc_hip_free", "trc_hip_h2d", "trc_hip_d2h", "trc_hip_memset",
    "trc_hip_fill_f32", "trc_hip_dequant", "trc_hip_mul_mat_f32", "trc_hip_qmatvec", "trc_hip_cpy",
    "trc_hip_add_f32", "trc_hip_acc_f32", "trc_hip_repeat_back_f32", "trc_hip_qmatvec_noalloc",
    "trc_hip_mul_f32", "trc_hip_repeat_f32", "trc_hip_sum_f32", "trc_hip_qmatvec_release_stream",
    "trc_hip_mul_mat_acc_f32", "trc_hip_sqr_f32", "trc_hip_scale_f32",
)


class Props(C.Structure):
    _fields_ = [
        ("name", C.c_char * 256), ("arch", C.c_char * 64), ("ordinal", C.c_int32),
        ("compute_units", C.c_int32), ("memory_free", C.c_size_t), ("memory_total", C.c_size_t),
        ("unified_memory", C.c_int32), ("abi_version", C.c_int32),
    ]


class Tensor(C.Structure):
    _fields_ = [
        ("data", C.c_void_p), ("type", C.c_int32), ("flags", C.c_int32),
        ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4),
    ]


def tensor(ptr: int, ne, nb, type_: int = TYPE_F32) -> Tensor:
    t = Tensor()
    t.data = C.c_void_p(ptr)
    t.type = type_
    t.flags = 0
    for i in range(4):
        t.ne[i] = int(ne[i])
        t.nb[i] = int(nb[i])
    return t


def contiguous_nb(ne, elem: int = 4):
    nb = [elem, 0, 0, 0]
    for i in range(1, 4):
        nb[i] = nb[i - 1] * int(ne[i - 1])
    return nb


class HipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


_lib = None


def load() -> C.CDLL:
    """Loads libtrc_hip.so (once) and declares every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
    lib = C.CDLL(str(LIB_PATH))
    P, I, I64, SZ, F = C.c_void_p, C.c_int, C.c_int64, C.c_size_t, C.c_float
    sig = {
        "trc_hip_device_count": ([C.POINTER(C.c_int)], I),
        "trc_hip_init": ([I, C.POINTER(Props)], I),
        "trc_hip_sync": ([P], I),
        "trc_hip_last_error": ([], C.c_char_p),
        "trc_hip_malloc": ([C.POINTER(C.c_void_p), SZ], I),
        "trc_hip_free": ([P], I),
        "trc_hip_h2d": ([P, P, SZ, P], I),
        "trc_hip_d2h": ([P, P, SZ, P], I),
        "trc_hip_memset": ([P, I, SZ, P], I),
        "trc_hip_fill_f32": ([P, F, I64, P], I),
        "trc_hip_dequant": ([I, P, I64, P, P], I),
        "trc_hip_mul_mat_f32": ([C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), P], I),
        "trc_hip_mul_mat_acc_f32": ([C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), P], I),
        "trc_hip_sqr_f32": ([C.POINTER(Tensor), C.POINTER(Tensor), P], I),
        "trc_hip_scale_f32": ([C.POINTER(Tensor), C.POINTER(Tensor), C.c_float, P], I),
        "trc_hip_qmatvec": ([I, P, I64, I64, SZ, P, I64, SZ, P, SZ, P], I),
        "trc_hip_qmatvec_noalloc": ([I, P, I64, I64, SZ, P, I64, SZ, P, SZ, P], I),
        "trc_hip_qmatvec_release_stream": ([P], I),
        "trc_hip_cpy": ([C.POINTER(Tensor), C.POINTER(Tensor), P], I),
        "trc_hip_add_f32": ([C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), P], I),
        "trc_hip_acc_f32": ([C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), SZ, SZ, SZ, SZ, I, P], I),
        "trc_hip_repeat_back_f32": ([C.POINTER(Tensor), C.POINTER(Tensor), P], I),
        "trc_hip_mul_f32": ([C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), P], I),
        "trc_hip_repeat_f32": ([C.POINTER(Tensor), C.POINTER(Tensor), P], I),
        "trc_hip_sum_f32": ([C.POINTER(Tensor), C.POINTER(Tensor), P], I),
    }
    for name, (args, ret) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ret
    _lib = lib
    return lib


def last_error() -> str:
    return load().trc_hip_last_error().decode(errors="replace")


def check(code: int) -> None:
    if code != OK:
        raise HipError(code, last_error())


# ---------------------------------------------------------------- thin wrappers

def device_count() -> int:
    n = C.c_int(0)
    check(load().trc_hip_device_count(C.byref(n)))
    return n.value


def init(ordinal: int = 0) -> Props:
    p = Props()
    check(load().trc_hip_init(ordinal, C.byref(p)))
    return p


def sync(stream: int | None = None) -> None:
    check(load().trc_hip_sync(stream))


def dequant(type_: int, blocks_ptr: int, n_blocks: int, dst_ptr: int, stream: int | None = None) -> None:
    check(load().trc_hip_dequant(type_, blocks_ptr, n_blocks, dst_ptr, stream))


def mul_mat_f32(a: Tensor, b: Tensor, d: Tensor, stream: int | None = None) -> None:
    check(load().trc_hip_mul_mat_f32(C.byref(a), C.byref(b), C.byref(d), stream))


def sqr_f32(a: Tensor, d: Tensor, stream: int | None = None) -> None:
    """d = a * a (trc_hip_sqr_f32)."""
    check(load().trc_hip_sqr_f32(C.byref(a), C.byref(d), stream))


def scale_f32(a: Tensor, d: Tensor, s: float, stream: int | None = None) -> None:
    """d = a * s (trc_hip_scale_f32)."""
    check(load().trc_hip_scale_f32(C.byref(a), C.byref(d), s, stream))


def mul_mat_acc_f32(a: Tensor, b: Tensor, d: Tensor, stream: int | None = None) -> None:
    """d += mul_mat(a, b) (trc_hip_mul_mat_acc_f32)."""
    check(load().trc_hip_mul_mat_acc_f32(C.byref(a), C.byref(b), C.byref(d), stream))


def qmatvec(type_: int, w_ptr: int, K: int, M: int, nb1_w: int, x_ptr: int, N: int, nb1_x: int,
            y_ptr: int, nb1_y: int, stream: int | None = None) -> None:
    check(load().trc_hip_qmatvec(type_, w_ptr, K, M, nb1_w, x_ptr, N, nb1_x, y_ptr, nb1_y, stream))


def qmatvec_release_stream(stream: int | None = None) -> None:
    check(load().trc_hip_qmatvec_release_stream(stream))


def qmatvec_noalloc(type_: int, w_ptr: int, K: int, M: int, nb1_w: int, x_ptr: int, N: int, nb1_x: int,
                    y_ptr: int, nb1_y: int, stream: int | None = None) -> None:
    check(load().trc_hip_qmatvec_noalloc(type_, w_ptr, K, M, nb1_w, x_ptr, N, nb1_x, y_ptr, nb1_y, stream))


def cpy(src: Tensor, dst: Tensor, stream: int | None = None) -> None:
    check(load().trc_hip_cpy(C.byref(src), C.byref(dst), stream))


def add_f32(a: Tensor, b: Tensor, d: Tensor, stream: int | None = None) -> None:
    check(load().trc_hip_add_f32(C.byref(a), C.byref(b), C.byref(d), stream))


def acc_f32(a: Tensor, b: Tensor, d: Tensor, nb1: int, nb2: int, nb3: int, offset: int, inplace: bool,
            stream: int | None = None) -> None:
    check(load().trc_hip_acc_f32(C.byref(a), C.byref(b), C.byref(d), nb1, nb2, nb3, offset, 1 if inplace else 0,
                                 stream))


def repeat_back_f32(a: Tensor, d: Tensor, stream: int | None = None) -> None:
    check(load().trc_hip_repeat_back_f32(C.byref(a), C.byref(d), stream))


def mul_f32(a: Tensor, b: Tensor, d: Tensor, stream: int | None = None) -> None:
    check(load().trc_hip_mul_f32(C.byref(a), C.byref(b), C.byref(d), stream))


def repeat_f32(a: Tensor, d: Tensor, stream: int | None = None) -> None:
    check(load().trc_hip_repeat_f32(C.byref(a), C.byref(d), stream))


def sum_f32(a: Tensor, d: Tensor, stream: int | None = None) -> None:
    check(load().trc_hip_sum_f32(C.byref(a), C.byref(d), stream))


def fill_f32(ptr: int, value: float, count: int, stream: int | None = None) -> None:
    check(load().trc_hip_fill_f32(ptr, value, count, stream))


class DeviceBuffer:
    """Device memory owned through the ABI's own allocator."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        check(load().trc_hip_malloc(C.byref(p), nbytes))
        self.ptr = p.value or 0
        self.nbytes = nbytes

    def upload(self, arr) -> "DeviceBuffer":
        import numpy as np
        a = np.ascontiguousarray(arr)
        assert a.nbytes <= self.nbytes
        check(load().trc_hip_h2d(self.ptr, a.ctypes.data, a.nbytes, None))
        return self

    def download(self, arr):
        import numpy as np
        assert arr.flags["C_CONTIGUOUS"] and arr.nbytes <= self.nbytes
        check(load().trc_hip_d2h(arr.ctypes.data, self.ptr, arr.nbytes, None))
        return arr

    def free(self) -> None:
        if self.ptr:
            check(load().trc_hip_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
