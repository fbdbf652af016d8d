"""ctypes access to the CPU checker for the tests.

oracle/liboracle.so    the C++ restatement of the reference CPU path (oracle/oracle.cpp)
oracle/_ref/libtrc_ref.so  the reference's own sources compiled with a small shim
                           (oracle/ref_shim.cpp); present only where the reference
                           checkout was available at build time.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_PATH = ROOT / "oracle" / "liboracle.so"
REF_PATH = ROOT / "oracle" / "_ref" / "libtrc_ref.so"

P, I, I64, F = C.c_void_p, C.c_int, C.c_int64, C.c_float
NE = C.c_int64 * 4
NB = C.c_size_t * 4
AX = C.c_int * 4

_orc = None
_ref = None


def oracle() -> C.CDLL:
    global _orc
    if _orc is None:
        lib = C.CDLL(str(ORACLE_PATH))
        lib.orc_fp16_to_fp32.argtypes = [C.c_uint16]
        lib.orc_fp16_to_fp32.restype = F
        lib.orc_fp32_to_fp16.argtypes = [F]
        lib.orc_fp32_to_fp16.restype = C.c_uint16
        lib.orc_fp16_to_fp32_n.argtypes = [P, P, I64]
        lib.orc_fp32_to_fp16_n.argtypes = [P, P, I64]
        lib.orc_block_bytes.argtypes = [I]
        lib.orc_block_bytes.restype = I64
        lib.orc_dequant.argtypes = [I, P, I64, P, I]
        lib.orc_dequant.restype = I
        lib.orc_mul_mat.argtypes = [P, NE, NB, P, NE, NB, P, NE, NB, I]
        lib.orc_mul_mat.restype = I
        lib.orc_mul_mat_cols.argtypes = [P, NE, NB, P, NE, NB, P, NE, NB, I64, I64, I]
        lib.orc_mul_mat_cols.restype = I
        lib.orc_add.argtypes = [P, NE, NB, P, NE, NB, P, NE, NB]
        lib.orc_add.restype = I
        lib.orc_acc.argtypes = [P, NE, P, NE, NB, P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, I]
        lib.orc_acc.restype = I
        lib.orc_repeat_back.argtypes = [P, NE, NB, P, NE]
        lib.orc_repeat_back.restype = I
        lib.orc_mul.argtypes = [P, NE, NB, P, NE, NB, P, NE, NB]
        lib.orc_mul.restype = I
        lib.orc_sum.argtypes = [P, NE, NB, C.POINTER(F)]
        lib.orc_sum.restype = I
        lib.orc_repeat.argtypes = [P, NE, NB, P, NE, NB]
        lib.orc_repeat.restype = I
        lib.orc_sqr.argtypes = [P, NE, NB, P, NB]
        lib.orc_sqr.restype = I
        lib.orc_scale.argtypes = [P, NE, NB, P, NB, C.c_float]
        lib.orc_scale.restype = I
        lib.orc_rng_next_u64.argtypes = [C.POINTER(C.c_uint64)]
        lib.orc_rng_next_u64.restype = C.c_uint64
        lib.orc_rng_uniform01.argtypes = [C.POINTER(C.c_uint64)]
        lib.orc_rng_uniform01.restype = F
        lib.orc_rng_normal.argtypes = [C.POINTER(C.c_uint64), F, F]
        lib.orc_rng_normal.restype = F
        _orc = lib
    return _orc


def have_ref() -> bool:
    return REF_PATH.exists()


def ref() -> C.CDLL:
    global _ref
    if _ref is None:
        lib = C.CDLL(str(REF_PATH))
        lib.ref_fp16_to_fp32.argtypes = [C.c_uint16]
        lib.ref_fp16_to_fp32.restype = F
        lib.ref_fp32_to_fp16.argtypes = [F]
        lib.ref_fp32_to_fp16.restype = C.c_uint16
        lib.ref_dequant.argtypes = [I, P, I64, P, C.c_char_p]
        lib.ref_dequant.restype = I
        lib.ref_mul_mat.argtypes = [P, NE, AX, P, NE, AX, P]
        lib.ref_mul_mat.restype = I
        lib.ref_add.argtypes = [P, NE, AX, P, NE, AX, P]
        lib.ref_add.restype = I
        lib.ref_acc.argtypes = [P, NE, P, NE, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, I, P]
        lib.ref_acc.restype = I
        lib.ref_repeat_back.argtypes = [P, NE, AX, NE, P]
        lib.ref_repeat_back.restype = I
        lib.ref_mul.argtypes = [P, NE, AX, P, NE, AX, P]
        lib.ref_mul.restype = I
        lib.ref_sum.argtypes = [P, NE, AX, C.POINTER(F)]
        lib.ref_sum.restype = I
        lib.ref_repeat.argtypes = [P, NE, AX, NE, P]
        lib.ref_repeat.restype = I
        lib.ref_unary.argtypes = [P, NE, AX, I, F, P]
        lib.ref_unary.restype = I
        for n in ("ref_rng_next_u64", "ref_rng_uniform01"):
            getattr(lib, n).argtypes = [C.POINTER(C.c_uint64)]
        lib.ref_rng_next_u64.restype = C.c_uint64
        lib.ref_rng_uniform01.restype = F
        lib.ref_rng_normal.argtypes = [C.POINTER(C.c_uint64), F, F]
        lib.ref_rng_normal.restype = F
        lib.ref_headline_time.argtypes = [I, P, I64, I64, P, P, C.c_double, C.POINTER(I), C.c_char_p]
        lib.ref_headline_time.restype = C.c_double
        lib.ref_dequant_time.argtypes = [I, P, I64, P, C.c_double, C.POINTER(I), C.c_char_p]
        lib.ref_dequant_time.restype = C.c_double
        lib.ref_mul_mat_time.argtypes = [P, I64, I64, P, I64, P, C.c_double, C.POINTER(I)]
        lib.ref_mul_mat_time.restype = C.c_double
        _ref = lib
    return _ref


# ---------------------------------------------------------------- helpers

def dequant(type_: int, blocks: np.ndarray, threads: int = 1) -> np.ndarray:
    raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
    bb = oracle().orc_block_bytes(type_)
    n = raw.size // bb
    out = np.empty(n * 32, dtype=np.float32)
    rc = oracle().orc_dequant(type_, raw.ctypes.data, n, out.ctypes.data, threads)
    assert rc == 0
    return out


def ref_headline(type_: int, blocks: np.ndarray, x: np.ndarray, K: int, M: int, budget_s: float,
                 tmp_path: str) -> tuple[np.ndarray, float, int]:
    """The reference's own CPU path for y = W x with W quantized (gguf_tensor_to_f32
    into the F32 weight, then mul_mat on its CPU Device), repeated for budget_s
    seconds: returns y, mean seconds per repetition and the repetition count."""
    raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
    xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert xv.size == K
    y = np.empty(M, dtype=np.float32)
    reps = I(0)
    dt = ref().ref_headline_time(type_, raw.ctypes.data, K, M, xv.ctypes.data, y.ctypes.data, budget_s,
                                 C.byref(reps), tmp_path.encode())
    assert dt > 0, f"ref_headline_time failed ({dt})"
    return y, dt, reps.value


def ref_dequant_timed(type_: int, blocks: np.ndarray, budget_s: float, tmp_path: str) -> tuple[np.ndarray, float, int]:
    """The reference's gguf_tensor_to_f32 of the blocks, repeated for budget_s
    seconds after one untimed pass: returns the F32 values, mean seconds per
    pass and the pass count."""
    raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
    n = raw.size // oracle().orc_block_bytes(type_) * 32
    out = np.empty(n, dtype=np.float32)
    reps = I(0)
    dt = ref().ref_dequant_time(type_, raw.ctypes.data, n, out.ctypes.data, budget_s, C.byref(reps),
                                tmp_path.encode())
    assert dt > 0, f"ref_dequant_time failed ({dt})"
    return out, dt, reps.value


def ref_mul_mat_timed(a: np.ndarray, K: int, M: int, b: np.ndarray, N: int,
                      budget_s: float) -> tuple[np.ndarray, float, int]:
    """y = mul_mat(A [K, M], B [K, N]) on the reference CPU Device (contiguous
    F32), repeated for budget_s seconds after one untimed pass: returns y
    ([M, N] as N rows of M), mean seconds per pass and the pass count."""
    av = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    bv = np.ascontiguousarray(b, dtype=np.float32).reshape(-1)
    assert av.size == K * M and bv.size == K * N
    y = np.empty(M * N, dtype=np.float32)
    reps = I(0)
    dt = ref().ref_mul_mat_time(av.ctypes.data, K, M, bv.ctypes.data, N, y.ctypes.data, budget_s, C.byref(reps))
    assert dt > 0, f"ref_mul_mat_time failed ({dt})"
    return y, dt, reps.value


def ref_dequant(type_: int, blocks: np.ndarray, tmp_dir: str) -> np.ndarray:
    raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
    bb = oracle().orc_block_bytes(type_)
    n = raw.size // bb
    out = np.empty(n * 32, dtype=np.float32)
    path = os.path.join(tmp_dir, f"ref_{os.getpid()}_{type_}.gguf").encode()
    rc = ref().ref_dequant(type_, raw.ctypes.data, n, out.ctypes.data, path)
    assert rc == 0, rc
    return out


def view_meta(arr: np.ndarray):
    """(ne, nb) in ggml order for a numpy array viewed as a ggml tensor (numpy
    axes reversed: numpy shape (ne3, ne2, ne1, ne0))."""
    assert arr.ndim <= 4
    shape = list(arr.shape)[::-1] + [1] * (4 - arr.ndim)
    strides = list(arr.strides)[::-1]
    nb = strides + [0] * (4 - arr.ndim)
    # fill strides of the padded unit dims with the extent of the last real one
    for i in range(arr.ndim, 4):
        nb[i] = (nb[i - 1] * shape[i - 1]) if i > 0 else arr.itemsize
    return shape, nb


def base_ptr_and_meta(arr: np.ndarray):
    ne, nb = view_meta(arr)
    return arr.__array_interface__["data"][0], ne, nb


def mul_mat(a: np.ndarray, b: np.ndarray, threads: int = 1) -> np.ndarray:
    """Oracle mul_mat of two (possibly strided) numpy views in ggml layout; returns
    a contiguous numpy array of shape (ne3, ne2, ne1, ne0) of the result."""
    pa, ane, anb = base_ptr_and_meta(a)
    pb, bne, bnb = base_ptr_and_meta(b)
    dne = [ane[1], bne[1], bne[2], bne[3]]
    out = np.zeros((dne[3], dne[2], dne[1], dne[0]), dtype=np.float32)
    _, _, dnb = base_ptr_and_meta(out)
    rc = oracle().orc_mul_mat(pa, NE(*ane), NB(*anb), pb, NE(*bne), NB(*bnb), out.ctypes.data,
                              NE(*dne), NB(*dnb), threads)
    assert rc == 0
    return out


def ref_mul_mat(a_base: np.ndarray, pa, b_base: np.ndarray, pb) -> np.ndarray:
    """Reference library mul_mat(permute(A, pa), permute(B, pb)) on its CPU device."""
    a_base = np.ascontiguousarray(a_base, dtype=np.float32)
    b_base = np.ascontiguousarray(b_base, dtype=np.float32)
    ane = list(a_base.shape)[::-1] + [1] * (4 - a_base.ndim)
    bne = list(b_base.shape)[::-1] + [1] * (4 - b_base.ndim)
    ape = [0] * 4
    bpe = [0] * 4
    for i in range(4):  # the reference's permute(): ne_out[i] = ne_in[axes[i]] (src/core/trc_tensor.cpp:303-306)
        ape[i] = ane[pa[i]]
        bpe[i] = bne[pb[i]]
    dne = [ape[1], bpe[1], bpe[2], bpe[3]]
    out = np.zeros((dne[3], dne[2], dne[1], dne[0]), dtype=np.float32)
    rc = ref().ref_mul_mat(a_base.ctypes.data, NE(*ane), AX(*pa), b_base.ctypes.data, NE(*bne), AX(*pb),
                           out.ctypes.data)
    assert rc == 0, rc
    return out


def ggml_shape(ne) -> tuple:
    """numpy shape (ne3, ne2, ne1, ne0) of a ggml ne."""
    return (ne[3], ne[2], ne[1], ne[0])


def add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Oracle add of two (possibly strided) float32 views; result contiguous with a's shape."""
    pa, ane, anb = base_ptr_and_meta(a)
    pb, bne, bnb = base_ptr_and_meta(b)
    out = np.zeros(ggml_shape(ane), dtype=np.float32)
    _, dne, dnb = base_ptr_and_meta(out)
    rc = oracle().orc_add(pa, NE(*ane), NB(*anb), pb, NE(*bne), NB(*bnb), out.ctypes.data, NE(*dne), NB(*dnb))
    assert rc == 0, rc
    return out


def acc(a: np.ndarray, b: np.ndarray, nb1: int, nb2: int, nb3: int, offset: int, inplace: bool = False):
    """Oracle acc: a contiguous (any rank up to 4), b a (possibly strided) view.
    Returns the result array; when inplace, a itself is updated and returned."""
    assert a.flags.c_contiguous and a.dtype == np.float32
    _, ane, _ = base_ptr_and_meta(a)
    pb, bne, bnb = base_ptr_and_meta(b)
    out = a if inplace else np.empty_like(a)
    rc = oracle().orc_acc(a.ctypes.data, NE(*ane), pb, NE(*bne), NB(*bnb), out.ctypes.data, nb1, nb2, nb3, offset,
                          1 if inplace else 0)
    assert rc == 0, rc
    return out


def mul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Oracle mul of two (possibly strided) float32 views; result contiguous with a's shape."""
    pa, ane, anb = base_ptr_and_meta(a)
    pb, bne, bnb = base_ptr_and_meta(b)
    out = np.zeros(ggml_shape(ane), dtype=np.float32)
    _, dne, dnb = base_ptr_and_meta(out)
    rc = oracle().orc_mul(pa, NE(*ane), NB(*anb), pb, NE(*bne), NB(*bnb), out.ctypes.data, NE(*dne), NB(*dnb))
    assert rc == 0, rc
    return out


def sum_all(a: np.ndarray) -> np.float32:
    """Oracle sum of every element of a (possibly strided) float32 view."""
    pa, ane, anb = base_ptr_and_meta(a)
    out = F(0.0)
    rc = oracle().orc_sum(pa, NE(*ane), NB(*anb), C.byref(out))
    assert rc == 0, rc
    return np.float32(out.value)


def sqr(a: np.ndarray) -> np.ndarray:
    """Oracle sqr of a (possibly strided) float32 view; contiguous result with a's shape."""
    pa, ane, anb = base_ptr_and_meta(a)
    out = np.zeros(ggml_shape(ane), dtype=np.float32)
    _, _, dnb = base_ptr_and_meta(out)
    assert oracle().orc_sqr(pa, NE(*ane), NB(*anb), out.ctypes.data, NB(*dnb)) == 0
    return out


def scale(a: np.ndarray, s: float) -> np.ndarray:
    """Oracle scale (a * s) of a (possibly strided) float32 view; contiguous result."""
    pa, ane, anb = base_ptr_and_meta(a)
    out = np.zeros(ggml_shape(ane), dtype=np.float32)
    _, _, dnb = base_ptr_and_meta(out)
    assert oracle().orc_scale(pa, NE(*ane), NB(*anb), out.ctypes.data, NB(*dnb), s) == 0
    return out


def repeat(a: np.ndarray, d_ne) -> np.ndarray:
    """Oracle repeat of a (possibly strided) view to ggml shape d_ne; contiguous result."""
    pa, ane, anb = base_ptr_and_meta(a)
    d_ne = list(d_ne) + [1] * (4 - len(d_ne))
    out = np.zeros(ggml_shape(d_ne), dtype=np.float32)
    _, _, dnb = base_ptr_and_meta(out)
    rc = oracle().orc_repeat(pa, NE(*ane), NB(*anb), out.ctypes.data, NE(*d_ne), NB(*dnb))
    assert rc == 0, rc
    return out


def repeat_back(a: np.ndarray, d_ne) -> np.ndarray:
    """Oracle repeat_back of a (possibly strided) view onto ggml shape d_ne; contiguous result."""
    pa, ane, anb = base_ptr_and_meta(a)
    d_ne = list(d_ne) + [1] * (4 - len(d_ne))
    out = np.zeros(ggml_shape(d_ne), dtype=np.float32)
    rc = oracle().orc_repeat_back(pa, NE(*ane), NB(*anb), out.ctypes.data, NE(*d_ne))
    assert rc == 0, rc
    return out


def _perm_ne(ne, axes):
    # the reference's permute(): ne_out[i] = ne_in[axes[i]] (src/core/trc_tensor.cpp:303-306)
    return [ne[axes[i]] for i in range(4)]


def ref_add(a_base: np.ndarray, pa, b_base: np.ndarray, pb) -> np.ndarray:
    """Reference library add(permute(A, pa), permute(B, pb)) on its CPU device."""
    a_base = np.ascontiguousarray(a_base, dtype=np.float32)
    b_base = np.ascontiguousarray(b_base, dtype=np.float32)
    ane = list(a_base.shape)[::-1] + [1] * (4 - a_base.ndim)
    bne = list(b_base.shape)[::-1] + [1] * (4 - b_base.ndim)
    out = np.zeros(ggml_shape(_perm_ne(ane, pa)), dtype=np.float32)
    rc = ref().ref_add(a_base.ctypes.data, NE(*ane), AX(*pa), b_base.ctypes.data, NE(*bne), AX(*pb), out.ctypes.data)
    assert rc == 0, rc
    return out


def ref_acc(a: np.ndarray, b: np.ndarray, nb1: int, nb2: int, nb3: int, offset: int, inplace: bool) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    ane = list(a.shape)[::-1] + [1] * (4 - a.ndim)
    bne = list(b.shape)[::-1] + [1] * (4 - b.ndim)
    out = np.zeros_like(a)
    rc = ref().ref_acc(a.ctypes.data, NE(*ane), b.ctypes.data, NE(*bne), nb1, nb2, nb3, offset, 1 if inplace else 0,
                       out.ctypes.data)
    assert rc == 0, rc
    return out


def ref_repeat_back(a_base: np.ndarray, pa, d_ne) -> np.ndarray:
    a_base = np.ascontiguousarray(a_base, dtype=np.float32)
    ane = list(a_base.shape)[::-1] + [1] * (4 - a_base.ndim)
    d_ne = list(d_ne) + [1] * (4 - len(d_ne))
    out = np.zeros(ggml_shape(d_ne), dtype=np.float32)
    rc = ref().ref_repeat_back(a_base.ctypes.data, NE(*ane), AX(*pa), NE(*d_ne), out.ctypes.data)
    assert rc == 0, rc
    return out


def row_l2_error(got: np.ndarray, want: np.ndarray) -> float:
    """max over dst rows (ne0-runs) of max|got - want| / max(||want_row||_2, 1e-30)."""
    g = got.reshape(-1, got.shape[-1]).astype(np.float64)
    w = want.reshape(-1, want.shape[-1]).astype(np.float64)
    norms = np.maximum(np.sqrt((w * w).sum(axis=1)), 1e-30)
    return float((np.abs(g - w).max(axis=1) / norms).max())


def ref_mul(a_base: np.ndarray, pa, b_base: np.ndarray, pb) -> np.ndarray:
    """Reference library mul(permute(A, pa), permute(B, pb)) on its CPU device."""
    a_base = np.ascontiguousarray(a_base, dtype=np.float32)
    b_base = np.ascontiguousarray(b_base, dtype=np.float32)
    ane = list(a_base.shape)[::-1] + [1] * (4 - a_base.ndim)
    bne = list(b_base.shape)[::-1] + [1] * (4 - b_base.ndim)
    out = np.zeros(ggml_shape(_perm_ne(ane, pa)), dtype=np.float32)
    rc = ref().ref_mul(a_base.ctypes.data, NE(*ane), AX(*pa), b_base.ctypes.data, NE(*bne), AX(*pb), out.ctypes.data)
    assert rc == 0, rc
    return out


def ref_sum(a_base: np.ndarray, pa) -> np.float32:
    """Reference library sum(permute(A, pa)) on its CPU device."""
    a_base = np.ascontiguousarray(a_base, dtype=np.float32)
    ane = list(a_base.shape)[::-1] + [1] * (4 - a_base.ndim)
    out = F(0.0)
    rc = ref().ref_sum(a_base.ctypes.data, NE(*ane), AX(*pa), C.byref(out))
    assert rc == 0, rc
    return np.float32(out.value)


def ref_repeat(a_base: np.ndarray, pa, d_ne) -> np.ndarray:
    """Reference library repeat(permute(A, pa), target of shape d_ne) on its CPU device."""
    a_base = np.ascontiguousarray(a_base, dtype=np.float32)
    ane = list(a_base.shape)[::-1] + [1] * (4 - a_base.ndim)
    d_ne = list(d_ne) + [1] * (4 - len(d_ne))
    out = np.zeros(ggml_shape(d_ne), dtype=np.float32)
    rc = ref().ref_repeat(a_base.ctypes.data, NE(*ane), AX(*pa), NE(*d_ne), out.ctypes.data)
    assert rc == 0, rc
    return out


def ref_unary(a_base: np.ndarray, pa, sq: bool, s: float = 0.0) -> np.ndarray:
    """Reference library sqr(permute(A, pa)) or scale(permute(A, pa), s) on its CPU device."""
    a_base = np.ascontiguousarray(a_base, dtype=np.float32)
    ane = list(a_base.shape)[::-1] + [1] * (4 - a_base.ndim)
    out = np.zeros(ggml_shape(_perm_ne(ane, pa)), dtype=np.float32)
    rc = ref().ref_unary(a_base.ctypes.data, NE(*ane), AX(*pa), 1 if sq else 0, s, out.ctypes.data)
    assert rc == 0, rc
    return out
