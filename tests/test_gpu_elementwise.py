"""Parity of the element-wise graph ops the mul_mat autograd needs on the device
(trc_hip_add_f32 / trc_hip_acc_f32 / trc_hip_repeat_back_f32) against the
oracle's restatement of the reference CPU kernels (compute_binary, compute_acc,
compute_repeat_back in src/backends/cpu/trc_cpu_ops.cpp).

Bar (written here): bit-identical. Each output element is one IEEE add of the
same two operands (add, acc) or the same ordered sum (repeat_back).
"""
import numpy as np
import pytest

import oracle_lib as O
from conftest import announce
from gpu_util import Dev, empty
from traincpp_amd import hip as H

pytestmark = pytest.mark.gpu


def bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def gpu_add(a_base, a_view, b_base, b_view):
    da, db = Dev(a_base), Dev(b_base)
    ne, _ = O.view_meta(a_view)
    out = empty(O.ggml_shape(ne))
    H.add_f32(da.tensor(a_view), db.tensor(b_view), out.tensor())
    H.sync()
    r = out.read()
    for d in (da, db, out):
        d.free()
    return r


@pytest.mark.parametrize("bshape", [(3, 5, 7, 33), (1, 5, 7, 33), (3, 1, 7, 1), (1, 1, 1, 33), (3, 5, 1, 1),
                                    (1, 1, 1, 1)])
def test_add_broadcast_bitwise(hip, bshape):
    announce(f"add bcast {bshape}")
    rng = np.random.default_rng(11)
    a = rng.standard_normal((3, 5, 7, 33)).astype(np.float32)
    b = rng.standard_normal(bshape).astype(np.float32)
    got = gpu_add(a, a, b, b)
    assert (bits(got) == bits(O.add(a, b))).all()


@pytest.mark.parametrize("bshape", [(3, 5, 7, 64), (1, 5, 7, 64), (3, 1, 7, 1), (1, 1, 1, 64), (3, 5, 1, 1),
                                    (1, 1, 1, 1)])
@pytest.mark.parametrize("op", ["add", "mul"])
def test_binary_four_floats_per_lane_bitwise(hip, bshape, op):
    """Rows of 64 floats, 16-byte aligned: the kernel that reads and writes four
    floats per lane, with b broadcast along every dim (scalar per row along ne0)."""
    announce(f"{op} vec4 bcast {bshape}")
    rng = np.random.default_rng(14)
    a = rng.standard_normal((3, 5, 7, 64)).astype(np.float32)
    b = rng.standard_normal(bshape).astype(np.float32)
    if op == "add":
        assert (bits(gpu_add(a, a, b, b)) == bits(O.add(a, b))).all()
    else:
        assert (bits(gpu_mul(a, a, b, b)) == bits(O.mul(a, b))).all()


def test_add_strided_views_bitwise(hip):
    rng = np.random.default_rng(12)
    A = rng.standard_normal((4, 6, 300, 9)).astype(np.float32)
    B = rng.standard_normal((4, 6, 1, 9)).astype(np.float32)
    av = A.transpose(0, 1, 3, 2)          # ggml [300, 9, 6, 4] with nb0 = 36 B
    bv = B.transpose(0, 1, 3, 2)          # ggml [1, 9, 6, 4] with nb1 = 4 B: broadcast along ne0
    got = gpu_add(A, av, B, bv)
    assert (bits(got) == bits(O.add(av, bv))).all()


def test_add_large_rows_bitwise(hip):
    """Rows longer than a workgroup and more rows than the grid cap."""
    rng = np.random.default_rng(13)
    a = rng.standard_normal((2, 3000, 1037)).astype(np.float32)
    b = rng.standard_normal((2, 1, 1037)).astype(np.float32)
    got = gpu_add(a, a, b, b)
    assert (bits(got) == bits(O.add(a, b))).all()


def gpu_acc(t, b_base, b_view, nb1, nb2, nb3, off, inplace):
    dt, db = Dev(t), Dev(b_base)
    ta = dt.tensor()
    if inplace:
        H.acc_f32(ta, db.tensor(b_view), ta, nb1, nb2, nb3, off, True)
        H.sync()
        r = dt.read()
        src = None
    else:
        out = empty(t.shape)
        H.acc_f32(ta, db.tensor(b_view), out.tensor(), nb1, nb2, nb3, off, False)
        H.sync()
        r = out.read()
        src = dt.read()
        out.free()
    dt.free()
    db.free()
    return r, src


@pytest.mark.parametrize("inplace", [False, True])
def test_acc_regions_bitwise(hip, inplace):
    announce(f"acc inplace={inplace}")
    rng = np.random.default_rng(14)
    t = rng.standard_normal((5, 40, 300)).astype(np.float32)   # ggml [300, 40, 5]
    b = rng.standard_normal((3, 20, 250)).astype(np.float32)   # ggml [250, 20, 3]
    nb1, nb2 = 300 * 4, 12000 * 4
    off = (1 * 12000 + 7 * 300 + 11) * 4
    got, src = gpu_acc(t, b, b, nb1, nb2, nb2 * 5, off, inplace)
    want = O.acc(t.copy(), b, nb1, nb2, nb2 * 5, off, inplace=True)
    assert (bits(got) == bits(want)).all()
    if not inplace:
        assert (bits(src) == bits(t)).all()  # the source target is left untouched
    # a region that skips every other row, and the reference's own KAT shape
    b2 = rng.standard_normal((20, 100)).astype(np.float32)
    got, _ = gpu_acc(t, b2, b2, 2 * nb1, nb2, nb2, 4 * 3, inplace)
    want = O.acc(t.copy(), b2, 2 * nb1, nb2, nb2, 12, inplace=True)
    assert (bits(got) == bits(want)).all()
    tk = np.arange(1, 9, dtype=np.float32).reshape(2, 4)
    bk = np.array([[10, 20], [30, 40]], np.float32)
    got, _ = gpu_acc(tk, bk, bk, 16, 0, 0, 4, inplace)
    assert (got.reshape(-1) == [1, 12, 23, 4, 5, 36, 47, 8]).all()


def test_acc_rejects_bad_regions(hip):
    t = Dev(np.zeros((2, 4), np.float32))
    b = Dev(np.ones((2, 2), np.float32))
    with pytest.raises(H.HipError) as e:
        H.acc_f32(t.tensor(), b.tensor(), t.tensor(), 16, 0, 0, 12, True)  # leaves the target
    assert e.value.code == H.E_SHAPE
    with pytest.raises(H.HipError) as e:
        H.acc_f32(t.tensor(), b.tensor(), t.tensor(), 4, 0, 0, 0, True)  # rows overlap each other
    assert e.value.code == H.E_SHAPE
    t.free()
    b.free()


@pytest.mark.parametrize("d_ne", [[8, 5, 6, 4], [8, 1, 6, 4], [4, 5, 3, 2], [1, 1, 1, 1], [2, 5, 1, 4]])
def test_repeat_back_bitwise(hip, d_ne):
    announce(f"repeat_back {d_ne}")
    rng = np.random.default_rng(15)
    A = rng.standard_normal((4, 6, 5, 8)).astype(np.float32)  # ggml [8, 5, 6, 4]
    for view in (A, A.transpose(0, 1, 3, 2)):
        ne, _ = O.view_meta(view)
        if any(ne[k] % d_ne[k] for k in range(4)):
            continue
        da = Dev(A)
        out = empty(O.ggml_shape(d_ne))
        H.repeat_back_f32(da.tensor(view), out.tensor())
        H.sync()
        got = out.read()
        da.free()
        out.free()
        assert (bits(got) == bits(O.repeat_back(view, d_ne))).all()


@pytest.mark.parametrize("a_shape,d_ne", [((512, 4096), [4096, 1, 1, 1]), ((6, 4, 6, 8), [8, 3, 2, 3]),
                                          ((1000, 64), [64, 1, 1, 1]), ((130, 100), [100, 1, 1, 1]),
                                          ((300, 70), [70, 3, 1, 1]),
                                          ((5, 3, 70, 33), [33, 7, 1, 1]), ((2, 1000, 64), [64, 1, 1, 1])])
def test_repeat_back_columns_bitwise(hip, a_shape, d_ne):
    """ne0 not repeated (the Linear layer's db: [4096, 512] back to [4096, 1]), with
    repeats along one, two or three dims, plain and transposed-plane views."""
    announce(f"repeat_back columns {a_shape} -> {d_ne}")
    rng = np.random.default_rng(17)
    A = rng.standard_normal(a_shape).astype(np.float32)
    views = [A]
    if A.ndim == 4 and A.shape[0] == A.shape[2]:
        views.append(A.transpose(2, 1, 0, 3))  # swap ggml dims 1 and 3 (nb3 < nb1)
    for view in views:
        ne, _ = O.view_meta(view)
        if any(ne[k] % d_ne[k] for k in range(4)):
            continue
        da = Dev(A)
        out = empty(O.ggml_shape(d_ne))
        H.repeat_back_f32(da.tensor(view), out.tensor())
        H.sync()
        got = out.read()
        da.free()
        out.free()
        assert (bits(got) == bits(O.repeat_back(view, d_ne))).all()


def test_repeat_back_mul_mat_broadcast_shape(hip):
    """The shape mul_mat's backward reduces: dA of configuration 4
    ([128, 1024, 32, 4] summed back to src0's [128, 1024, 8, 4])."""
    rng = np.random.default_rng(16)
    A = rng.standard_normal((4, 32, 1024, 128)).astype(np.float32)
    da = Dev(A)
    out = empty((4, 8, 1024, 128))
    H.repeat_back_f32(da.tensor(), out.tensor())
    H.sync()
    got = out.read()
    da.free()
    out.free()
    assert (bits(got) == bits(O.repeat_back(A, [128, 1024, 8, 4]))).all()


# ---------------------------------------------------------------- mul / repeat / sum
# trc_hip_mul_f32 / trc_hip_repeat_f32 / trc_hip_sum_f32 against orc_mul /
# orc_repeat / orc_sum (compute_binary, compute_repeat, compute_sum): bitwise.

def gpu_mul(a_base, a_view, b_base, b_view):
    da, db = Dev(a_base), Dev(b_base)
    ne, _ = O.view_meta(a_view)
    out = empty(O.ggml_shape(ne))
    H.mul_f32(da.tensor(a_view), db.tensor(b_view), out.tensor())
    H.sync()
    r = out.read()
    for d in (da, db, out):
        d.free()
    return r


@pytest.mark.parametrize("bshape", [(3, 5, 7, 33), (1, 5, 7, 33), (3, 1, 7, 1), (1, 1, 1, 33), (1, 1, 1, 1)])
def test_mul_broadcast_bitwise(hip, bshape):
    announce(f"mul bcast {bshape}")
    rng = np.random.default_rng(21)
    a = rng.standard_normal((3, 5, 7, 33)).astype(np.float32)
    b = rng.standard_normal(bshape).astype(np.float32)
    assert (bits(gpu_mul(a, a, b, b)) == bits(O.mul(a, b))).all()


def test_mul_strided_and_linear_loss_shape(hip):
    """The loss product of a Linear layer: y [4096, 512] times a constant of the
    same shape, and a transposed operand."""
    rng = np.random.default_rng(22)
    y = rng.standard_normal((512, 4096)).astype(np.float32)
    g = (rng.standard_normal((512, 4096)) * 1e-2).astype(np.float32)
    assert (bits(gpu_mul(y, y, g, g)) == bits(O.mul(y, g))).all()
    A = rng.standard_normal((40, 30)).astype(np.float32)
    B = rng.standard_normal((30, 40)).astype(np.float32)
    assert (bits(gpu_mul(A, A.T, B, B)) == bits(O.mul(A.T, B))).all()


def gpu_repeat(a_base, a_view, d_ne):
    da = Dev(a_base)
    out = empty(O.ggml_shape(d_ne))
    H.repeat_f32(da.tensor(a_view), out.tensor())
    H.sync()
    r = out.read()
    da.free()
    out.free()
    return r


@pytest.mark.parametrize("ashape,d_ne", [((1, 1, 1, 1), [4096, 512, 1, 1]), ((1, 1, 1, 7), [7, 33, 5, 3]),
                                         ((1, 1, 3, 8), [16, 6, 2, 1]), ((1, 2, 1, 1), [12, 5, 4, 1]),
                                         ((3, 1, 5, 1), [9, 5, 1, 3]), ((1, 1, 1, 1), [1, 1, 1, 1])])
def test_repeat_bitwise(hip, ashape, d_ne):
    announce(f"repeat {ashape} -> {d_ne}")
    rng = np.random.default_rng(23)
    a = rng.standard_normal(ashape).astype(np.float32)
    assert (bits(gpu_repeat(a, a, d_ne)) == bits(O.repeat(a, d_ne))).all()


def test_repeat_strided_source_bitwise(hip):
    rng = np.random.default_rng(24)
    A = rng.standard_normal((6, 1, 9)).astype(np.float32)
    av = A.transpose(1, 2, 0)  # ggml [6, 9, 1] with nb0 = 36 B
    assert (bits(gpu_repeat(A, av, [6, 9, 4, 2])) == bits(O.repeat(av, [6, 9, 4, 2]))).all()


def gpu_sum(a_base, a_view):
    da = Dev(a_base)
    out = empty((1,))
    H.sum_f32(da.tensor(a_view), out.tensor())
    H.sync()
    r = out.read()[0]
    da.free()
    out.free()
    return np.float32(r)


@pytest.mark.parametrize("shape", [(512, 4096), (3, 5, 7, 33), (1, 1, 1, 1), (2, 3, 1500, 5), (1, 1, 2500, 3)])
def test_sum_bitwise(hip, shape):
    """Rows of every length, more rows than the 1024 the kernel sums per pass,
    and the Linear loss shape [4096, 512]."""
    announce(f"sum {shape}")
    rng = np.random.default_rng(25)
    a = (rng.standard_normal(shape) * 10.0 ** rng.integers(-3, 4, shape)).astype(np.float32)
    assert bits(gpu_sum(a, a)) == bits(O.sum_all(a))


@pytest.mark.parametrize("shape,cut", [((300, 36), None), ((100, 4), None), ((65, 8200), None), ((100, 4), 2),
                                       ((9, 1000), None), ((3, 2, 17, 256), None), ((5000, 8), None),
                                       ((4100, 260), None),
                                       ((70, 4096), 4093), ((1_200_000, 1), None)])
def test_sum_row_paths_bitwise(hip, shape, cut):
    """Rows read four floats at a time (16-byte aligned rows) with row lengths that
    leave partial batches and tails, rows cut shorter than their stride, and more
    rows than the row-sum workspace holds (the one-workgroup kernel)."""
    announce(f"sum rows {shape} cut {cut}")
    rng = np.random.default_rng(27)
    a = (rng.standard_normal(shape) * 10.0 ** rng.integers(-3, 4, shape)).astype(np.float32)
    av = a if cut is None else a[..., :cut]
    assert bits(gpu_sum(a, av)) == bits(O.sum_all(av))


def test_sum_order_and_strides_bitwise(hip):
    big = np.float32(2.0 ** 53)
    for arr in (np.array([big, 1, -big], np.float32), np.array([big, 1, -big], np.float32).reshape(3, 1),
                np.array([-big, 1, big], np.float32).reshape(3, 1, 1)):
        assert bits(gpu_sum(arr, arr)) == bits(O.sum_all(arr))
    rng = np.random.default_rng(26)
    A = rng.standard_normal((6, 70, 50)).astype(np.float32)
    av = A.transpose(2, 0, 1)  # strided rows
    assert bits(gpu_sum(A, av)) == bits(O.sum_all(av))


def gpu_unary(a_base, a_view, s=None):
    """sqr (s None) or scale by s of a view of a_base on the device; contiguous result."""
    da = Dev(a_base)
    ne, _ = O.view_meta(a_view)
    out = empty(O.ggml_shape(ne))
    if s is None:
        H.sqr_f32(da.tensor(a_view), out.tensor())
    else:
        H.scale_f32(da.tensor(a_view), out.tensor(), s)
    H.sync()
    r = out.read()
    da.free()
    out.free()
    return r


def _unary_specials():
    """Values whose square or scaled product rounds, overflows, underflows to a
    subnormal or zero, or carries a NaN or an infinity through."""
    return np.array([0.0, -0.0, 1.0, -1.5, 3.4e38, -1.9e19, 1.9e19, 1.2e-38, 1.4e-45, -1e-23, 1e-20,
                     np.inf, -np.inf, np.nan, 1.0000001, 3.0e-3, 7.7, -2.5e5], np.float32)


@pytest.mark.parametrize("shape", [(3, 5, 7, 64), (4, 6, 33), (257,), (1, 1, 1, 1), (2, 3, 4100)])
@pytest.mark.parametrize("s", [None, 2.0, -0.37, 1e-30])
def test_sqr_and_scale_bitwise(hip, shape, s):
    """Contiguous tensors: rows of a multiple of four floats take the kernel that
    reads four floats per lane, the others the one-float kernel."""
    announce(f"{'sqr' if s is None else f'scale {s}'} {shape}")
    rng = np.random.default_rng(31)
    a = (rng.standard_normal(shape) * 10.0 ** rng.integers(-20, 20, shape)).astype(np.float32)
    want = O.sqr(a) if s is None else O.scale(a, s)
    assert (bits(gpu_unary(a, a, s)) == bits(want)).all()


@pytest.mark.parametrize("s", [None, 2.0, 1e-30, 1e30])
def test_sqr_and_scale_special_values_bitwise(hip, s):
    announce(f"{'sqr' if s is None else f'scale {s}'} specials")
    sp = _unary_specials()
    a = np.concatenate([sp, -sp, sp * np.float32(0.5)]).astype(np.float32)
    a = np.tile(a, 8).reshape(6, 72)  # 72-float rows: the four-floats-per-lane kernel
    want = O.sqr(a) if s is None else O.scale(a, s)
    assert (bits(gpu_unary(a, a, s)) == bits(want)).all()
    b = a[:, :71]  # rows cut to 71 floats: the one-float kernel
    want = O.sqr(b) if s is None else O.scale(b, s)
    assert (bits(gpu_unary(a, b, s)) == bits(want)).all()


def test_sqr_and_scale_strided_views_bitwise(hip):
    rng = np.random.default_rng(32)
    A = rng.standard_normal((4, 6, 300, 9)).astype(np.float32)
    for view in (A.transpose(0, 1, 3, 2), A.transpose(3, 2, 1, 0), A[:, ::2, 1:, :]):
        announce(f"sqr/scale view {view.shape} {view.strides}")
        assert (bits(gpu_unary(A, view)) == bits(O.sqr(view))).all()
        assert (bits(gpu_unary(A, view, 2.0)) == bits(O.scale(view, 2.0))).all()


def test_sqr_and_scale_reject_bad_shapes(hip):
    da, out = Dev(np.zeros((4, 8), np.float32)), empty((8, 5))
    with pytest.raises(H.HipError):
        H.sqr_f32(da.tensor(), out.tensor())
    with pytest.raises(H.HipError):
        H.scale_f32(da.tensor(), out.tensor(), 2.0)
    da.free()
    out.free()
