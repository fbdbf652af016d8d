"""Pins the oracle's add / acc / repeat_back (oracle/oracle.cpp) before the HIP
kernels are compared against them:
  - the reference's own known-answer tests (tests/test_ops.cpp:52-95, 1128-1220),
  - its PyTorch goldens for add (tests/golden/add_same_*, add_bcast_*; tolerance
    of tests/test_golden.cpp:190-201),
  - numpy's float32 arithmetic where it performs the same single rounding
    (add, acc) and a float64 bound where the summation order differs
    (repeat_back),
  - the reference library's own CPU kernels (oracle/_ref), bit for bit.
"""
import numpy as np
import pytest

import oracle_lib as O

GOLDEN = O.ROOT / "tests" / "golden"


def _bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------- known answers

def test_add_kats():
    # tests/test_ops.cpp:52-71 and :73-95
    a = np.array([1, 2, 3, 4], np.float32)
    b = np.array([10, 20, 30, 40], np.float32)
    assert (O.add(a, b) == [11, 22, 33, 44]).all()
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)  # ggml [3, 2]
    b = np.array([10, 20, 30], np.float32)             # ggml [3], broadcast along dim 1
    assert (O.add(a, b) == np.array([[11, 22, 33], [14, 25, 36]], np.float32)).all()


def test_repeat_back_kat():
    # tests/test_ops.cpp:1128-1150: a [3,1] repeated to [3,4] then summed back = 4a
    a = np.array([1, 2, 3], np.float32).reshape(1, 3)
    rep = np.repeat(a, 4, axis=0)  # ggml [3, 4]
    assert (O.repeat_back(rep, [3, 1]).reshape(-1) == [4, 8, 12]).all()


def test_acc_kats():
    # tests/test_ops.cpp:1152-1182: b [2,2] into target [4,2] at offset 4 B, nb1 = 16 B
    t = np.arange(1, 9, dtype=np.float32).reshape(2, 4)
    b = np.array([[10, 20], [30, 40]], np.float32)
    r = O.acc(t, b, 16, 0, 0, 4)
    assert (r.reshape(-1) == [1, 12, 23, 4, 5, 36, 47, 8]).all()
    assert (t.reshape(-1) == np.arange(1, 9)).all()  # not inplace: target unchanged
    # :1184-1220: inplace 3D, region at (i0=0, i1=1, i2=1) of a [2,3,4] target
    t = np.arange(24, dtype=np.float32).reshape(4, 3, 2)
    b = np.arange(100, 108, dtype=np.float32).reshape(2, 2, 2)
    want = t.copy()
    want[1:3, 1:3, 0:2] += b
    O.acc(t, b, 8, 24, 96, 8 + 24, inplace=True)
    assert (t == want).all()


# ---------------------------------------------------------------- goldens

@pytest.mark.parametrize("name", ["add_same", "add_bcast"])
def test_add_goldens(name):
    a = np.load(GOLDEN / f"{name}_in0.npy", allow_pickle=False).astype(np.float32)
    b = np.load(GOLDEN / f"{name}_in1.npy", allow_pickle=False).astype(np.float32)
    want = np.load(GOLDEN / f"{name}_out.npy", allow_pickle=False)
    got = O.add(a, b)
    assert np.allclose(got, want, atol=1e-4, rtol=1e-3)


# ---------------------------------------------------------------- numpy closed forms

def test_add_matches_numpy_broadcast_bitwise():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((3, 5, 7, 9)).astype(np.float32)
    for bshape in [(3, 5, 7, 9), (1, 5, 7, 9), (3, 1, 7, 1), (1, 1, 1, 9), (3, 5, 1, 1), (1, 1, 1, 1)]:
        b = rng.standard_normal(bshape).astype(np.float32)
        want = a + b  # numpy float32 add: one IEEE rounding per element, like the reference
        assert (_bits(O.add(a, b)) == _bits(want)).all(), bshape
    # strided (transposed) operands
    at = a.transpose(0, 1, 3, 2)
    b = rng.standard_normal((1, 5, 9, 1)).astype(np.float32)
    assert (_bits(O.add(at, b)) == _bits(at + b)).all()


def test_acc_matches_numpy_slice_add():
    rng = np.random.default_rng(2)
    t = rng.standard_normal((3, 6, 10)).astype(np.float32)  # ggml [10, 6, 3]
    b = rng.standard_normal((2, 4, 5)).astype(np.float32)   # ggml [5, 4, 2]
    nb1, nb2 = 10 * 4, 60 * 4
    off = (1 * 60 + 2 * 10 + 3) * 4                          # start at (i0=3, i1=2, i2=1)
    want = t.copy()
    want[1:3, 2:6, 3:8] += b
    assert (_bits(O.acc(t, b, nb1, nb2, nb2 * 3, off)) == _bits(want)).all()
    # the region's row stride may skip rows: every other row of the target
    b0 = np.ascontiguousarray(b[0, :3])  # ggml [5, 3] onto rows 0, 2, 4
    want = t.copy()
    want[0, 0:6:2, 0:5] += b0
    assert (_bits(O.acc(t, b0, 2 * nb1, nb2, nb2, 0)) == _bits(want)).all()


def test_acc_rejects_out_of_range_region():
    t = np.zeros((2, 4), np.float32)
    b = np.ones((2, 2), np.float32)
    with pytest.raises(AssertionError):
        O.acc(t, b, 16, 0, 0, 12)  # last element would land past the 8 floats


def test_repeat_back_float64_bound():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((4, 6, 5, 8)).astype(np.float32)   # ggml [8, 5, 6, 4]
    for d_ne in ([8, 5, 6, 4], [8, 1, 6, 4], [4, 5, 3, 2], [1, 1, 1, 1], [2, 5, 1, 4]):
        got = O.repeat_back(a, d_ne)
        r = [a.shape[3 - k] // d_ne[k] for k in range(4)]
        t = a.astype(np.float64).reshape(r[3], d_ne[3], r[2], d_ne[2], r[1], d_ne[1], r[0], d_ne[0])
        want = t.sum(axis=(0, 2, 4, 6))
        nsum = int(np.prod(r))
        bound = nsum * 2.0 ** -24 * np.abs(t).sum(axis=(0, 2, 4, 6)) + 1e-30
        assert (np.abs(got - want) <= bound).all(), d_ne


# ---------------------------------------------------------------- reference library

pytestmark_ref = pytest.mark.skipif(not O.have_ref(), reason="oracle/_ref not built (reference checkout absent)")


@pytestmark_ref
@pytest.mark.parametrize("pa,pb,bshape", [
    ((0, 1, 2, 3), (0, 1, 2, 3), None),
    ((1, 0, 2, 3), (1, 0, 2, 3), None),
    ((0, 2, 1, 3), (0, 1, 2, 3), (1,)),
    ((1, 0, 2, 3), (0, 1, 2, 3), (2,)),
])
def test_add_bitwise_vs_reference(pa, pb, bshape):
    rng = np.random.default_rng(4)
    A = rng.standard_normal((3, 4, 5, 6)).astype(np.float32)   # base ggml [6, 5, 4, 3]
    ane = [6, 5, 4, 3]
    ape = [ane[pa[i]] for i in range(4)]
    bne = [ape[O_pb] for O_pb in range(4)]
    if bshape is not None:   # collapse some dims of b to 1 (broadcast)
        for k in bshape:
            bne[k] = 1
    # b base laid out so that permute(b, pb) has shape bne
    inv = [0] * 4
    for i in range(4):
        inv[pb[i]] = i
    b_base_ne = [bne[inv[k]] for k in range(4)]
    B = rng.standard_normal(tuple(b_base_ne[::-1])).astype(np.float32)
    want = O.ref_add(A, pa, B, pb)
    av = np.transpose(A, [3 - pa[3 - k] for k in range(4)])
    bv = np.transpose(B, [3 - pb[3 - k] for k in range(4)])
    got = O.add(av, bv)
    assert (_bits(got) == _bits(want)).all()


@pytestmark_ref
@pytest.mark.parametrize("inplace", [False, True])
def test_acc_bitwise_vs_reference(inplace):
    rng = np.random.default_rng(5)
    t = rng.standard_normal((4, 6, 10)).astype(np.float32)
    b = rng.standard_normal((3, 4, 5)).astype(np.float32)
    args = (10 * 4, 60 * 4, 240 * 4, (1 * 60 + 1 * 10 + 2) * 4)
    want = O.ref_acc(t, b, *args, inplace)
    got = O.acc(t.copy(), b, *args, inplace=inplace)
    assert (_bits(got) == _bits(want)).all()


@pytestmark_ref
@pytest.mark.parametrize("pa,d_ne", [
    ((0, 1, 2, 3), [8, 5, 6, 4]),
    ((0, 1, 2, 3), [8, 1, 3, 1]),
    ((1, 0, 2, 3), [5, 4, 2, 4]),
    ((0, 2, 1, 3), [2, 6, 5, 2]),
])
def test_repeat_back_bitwise_vs_reference(pa, d_ne):
    rng = np.random.default_rng(6)
    A = rng.standard_normal((4, 6, 5, 8)).astype(np.float32)  # base ggml [8, 5, 6, 4]
    want = O.ref_repeat_back(A, pa, d_ne)
    av = np.transpose(A, [3 - pa[3 - k] for k in range(4)])
    got = O.repeat_back(av, d_ne)
    assert (_bits(got) == _bits(want)).all()


# ---------------------------------------------------------------- mul / sum / repeat
# The nodes of a Linear layer's scalar loss (sum(mul(y, g))) and its backward
# (repeat of the loss gradient): tests/test_ops.cpp:98-118, 795-815 and the
# PyTorch goldens mul_same_*, sum_*, repeat_* (tests/golden/cases.txt:3,30,41).

def test_mul_kat():
    # the product step of tests/test_ops.cpp:98-118: (a - b) * a
    a = np.array([4, 6, 8], np.float32)
    b = np.array([2, 3, 4], np.float32)
    assert (O.mul(a - b, a) == [8, 18, 32]).all()


def test_mul_golden():
    a = np.load(GOLDEN / "mul_same_in0.npy", allow_pickle=False).astype(np.float32)
    b = np.load(GOLDEN / "mul_same_in1.npy", allow_pickle=False).astype(np.float32)
    want = np.load(GOLDEN / "mul_same_out.npy", allow_pickle=False)
    assert np.allclose(O.mul(a, b), want, atol=1e-4, rtol=1e-3)


def test_mul_matches_numpy_broadcast_bitwise():
    rng = np.random.default_rng(11)
    a = rng.standard_normal((3, 5, 7, 9)).astype(np.float32)
    for bshape in [(3, 5, 7, 9), (1, 5, 7, 9), (3, 1, 7, 1), (1, 1, 1, 9), (1, 1, 1, 1)]:
        b = rng.standard_normal(bshape).astype(np.float32)
        assert (_bits(O.mul(a, b)) == _bits(a * b)).all(), bshape
    at = a.transpose(0, 2, 1, 3)
    b = rng.standard_normal((1, 7, 1, 9)).astype(np.float32)
    assert (_bits(O.mul(at, b)) == _bits(at * b)).all()


def test_repeat_kat_and_golden():
    # tests/test_ops.cpp:795-815: [1, 2] repeated to ggml [2, 3]
    assert (O.repeat(np.array([1, 2], np.float32), [2, 3]).reshape(-1) == [1, 2, 1, 2, 1, 2]).all()
    a = np.load(GOLDEN / "repeat_in0.npy", allow_pickle=False).astype(np.float32)
    want = np.load(GOLDEN / "repeat_out.npy", allow_pickle=False)
    got = O.repeat(a, [2, 3, 1, 1])  # tests/golden/cases.txt:41 target ne = [2, 3, 1, 1]
    assert np.allclose(got, want.reshape(got.shape), atol=1e-4, rtol=1e-3)


def test_repeat_matches_numpy_tile():
    rng = np.random.default_rng(12)
    for ashape, reps in [((1, 1, 1, 1), (2, 3, 4, 5)), ((1, 3, 1, 5), (2, 1, 4, 1)), ((2, 3, 4, 5), (1, 2, 1, 3))]:
        a = rng.standard_normal(ashape).astype(np.float32)
        want = np.tile(a, reps)
        assert (_bits(O.repeat(a, list(want.shape)[::-1])) == _bits(want)).all()
    a = rng.standard_normal((3, 4)).astype(np.float32).T  # strided source
    assert (_bits(O.repeat(a, [3, 8])) == _bits(np.tile(a, (2, 1)))).all()


def test_sqr_and_scale_goldens():
    """The reference suite's PyTorch goldens unary_sqr and scale (s = 2.5), read
    by its tests/test_golden.cpp (cases tests/golden/reference_suite/cases.txt:9,25)
    at that program's tolerance (tests/test_golden.cpp:190-201)."""
    suite = GOLDEN / "reference_suite"
    a = np.load(suite / "unary_sqr_in0.npy", allow_pickle=False).astype(np.float32)
    want = np.load(suite / "unary_sqr_out.npy", allow_pickle=False)
    assert np.allclose(O.sqr(a), want.reshape(a.shape), atol=1e-4, rtol=1e-3)
    a = np.load(suite / "scale_in0.npy", allow_pickle=False).astype(np.float32)
    want = np.load(suite / "scale_out.npy", allow_pickle=False)
    assert np.allclose(O.scale(a, 2.5), want.reshape(a.shape), atol=1e-4, rtol=1e-3)


def test_sum_golden():
    a = np.load(GOLDEN / "sum_in0.npy", allow_pickle=False).astype(np.float32)
    want = np.load(GOLDEN / "sum_out.npy", allow_pickle=False).reshape(())
    assert np.isclose(O.sum_all(a), want, atol=1e-4, rtol=1e-3)


def test_sum_order_is_revealed():
    big = np.float32(2.0 ** 53)
    # within a row, in double: (2^53 + 1) rounds back to 2^53, so the row is 0
    # (exactly 1 in any other order)
    assert O.sum_all(np.array([big, 1, -big], np.float32)) == 0
    assert O.sum_all(np.array([big, -big, 1], np.float32)) == 1
    # across rows (i1 fastest) and planes (i2, then i3): the same cancellation
    assert O.sum_all(np.array([big, 1, -big], np.float32).reshape(3, 1)) == 0
    assert O.sum_all(np.array([big, 1, -big], np.float32).reshape(3, 1, 1)) == 0
    assert O.sum_all(np.array([big, 1, -big], np.float32).reshape(3, 1, 1, 1)) == 0
    assert O.sum_all(np.array([-big, 1, big], np.float32).reshape(3, 1)) == 1
    # double, not float, accumulation: 2^24 + 16 ones stays exact
    row = np.concatenate([[np.float32(2.0 ** 24)], np.ones(16, np.float32)]).astype(np.float32)
    assert O.sum_all(row) == np.float32(2.0 ** 24 + 16)


def test_sum_within_one_rounding_of_exact():
    import math
    rng = np.random.default_rng(13)
    a = (rng.standard_normal((3, 4, 50, 70)) * 10.0 ** rng.integers(-3, 4, (3, 4, 50, 70))).astype(np.float32)
    exact = math.fsum(a.astype(np.float64).reshape(-1))
    got = float(O.sum_all(a))
    # double partial sums carry ~1e-16 relative error per add over 42000 terms,
    # then one float rounding: within 2 float ulps of the exact sum
    assert abs(got - exact) <= 2 * np.spacing(np.float32(abs(exact))) + 1e-9 * np.abs(a).sum()


@pytestmark_ref
@pytest.mark.parametrize("pa,pb,bshape", [((0, 1, 2, 3), (0, 1, 2, 3), None), ((1, 0, 2, 3), (0, 1, 2, 3), (2,))])
def test_mul_bitwise_vs_reference(pa, pb, bshape):
    rng = np.random.default_rng(14)
    A = rng.standard_normal((3, 4, 5, 6)).astype(np.float32)
    ane = [6, 5, 4, 3]
    ape = [ane[pa[i]] for i in range(4)]
    bne = list(ape)
    if bshape is not None:
        for k in bshape:
            bne[k] = 1
    inv = [0] * 4
    for i in range(4):
        inv[pb[i]] = i
    b_base_ne = [bne[inv[k]] for k in range(4)]
    B = rng.standard_normal(tuple(b_base_ne[::-1])).astype(np.float32)
    want = O.ref_mul(A, pa, B, pb)
    av = np.transpose(A, [3 - pa[3 - k] for k in range(4)])
    bv = np.transpose(B, [3 - pb[3 - k] for k in range(4)])
    assert (_bits(O.mul(av, bv)) == _bits(want)).all()


@pytestmark_ref
@pytest.mark.parametrize("pa", [(0, 1, 2, 3), (1, 0, 2, 3), (0, 2, 1, 3), (2, 3, 0, 1)])
def test_sum_bitwise_vs_reference(pa):
    rng = np.random.default_rng(15)
    A = (rng.standard_normal((4, 6, 5, 300)) * 1e3).astype(np.float32)  # base ggml [300, 5, 6, 4]
    want = O.ref_sum(A, pa)
    av = np.transpose(A, [3 - pa[3 - k] for k in range(4)])
    assert _bits(O.sum_all(av)) == _bits(want)


@pytestmark_ref
@pytest.mark.parametrize("ashape,pa,d_ne", [
    # the reference's repeat broadcasts extent-1 dims only (tensor_can_repeat,
    # src/core/trc_tensor.cpp:81-88)
    ((4, 6, 1, 8), (0, 1, 2, 3), [8, 10, 6, 4]),
    ((4, 6, 1, 8), (1, 0, 2, 3), [10, 8, 6, 4]),
    ((1, 6, 5, 1), (0, 2, 1, 3), [7, 6, 5, 3]),
    ((1, 1, 1, 1), (0, 1, 2, 3), [9, 4, 3, 2]),
])
def test_repeat_bitwise_vs_reference(ashape, pa, d_ne):
    rng = np.random.default_rng(16)
    A = rng.standard_normal(ashape).astype(np.float32)
    want = O.ref_repeat(A, pa, d_ne)
    av = np.transpose(A, [3 - pa[3 - k] for k in range(4)])
    assert (_bits(O.repeat(av, d_ne)) == _bits(want)).all()


# ---------------------------------------------------------------- sqr / scale

def _specials():
    """Finite values over the exponent range, signed zeros, subnormals, infinities,
    NaN, and values whose square or scaled value overflows or underflows."""
    rng = np.random.default_rng(21)
    v = (rng.standard_normal(4000) * 10.0 ** rng.integers(-40, 39, 4000)).astype(np.float32)
    extra = np.array([0.0, -0.0, 1e-45, -1e-45, 1e-38, 3.4e38, -3.4e38, 1.8e19, 1.9e19, np.inf, -np.inf, np.nan,
                      1.0, -1.0, 0.5, 3.0], dtype=np.float32)
    return np.concatenate([v, extra]).reshape(1, 1, 4, 1004)


def test_sqr_is_float32_square():
    a = _specials()
    with np.errstate(over="ignore", invalid="ignore"):
        want = a * a
    assert (_bits(O.sqr(a)) == _bits(want)).all()


@pytest.mark.parametrize("s", [2.0, -0.5, 3.0e-39, 1.0e30, 0.0])
def test_scale_is_float32_product(s):
    a = _specials()
    with np.errstate(over="ignore", invalid="ignore"):
        want = a * np.float32(s)
    assert (_bits(O.scale(a, s)) == _bits(want)).all()


def test_sqr_and_scale_on_strided_views():
    rng = np.random.default_rng(22)
    base = rng.standard_normal((3, 4, 7, 9)).astype(np.float32)
    v = np.transpose(base, (1, 0, 3, 2))  # every stride non-contiguous
    assert (_bits(O.sqr(v)) == _bits(np.ascontiguousarray(v * v))).all()
    assert (_bits(O.scale(v, 1.5)) == _bits(np.ascontiguousarray(v * np.float32(1.5)))).all()


@pytestmark_ref
@pytest.mark.parametrize("pa", [(0, 1, 2, 3), (1, 0, 2, 3), (2, 3, 0, 1)])
def test_sqr_and_scale_bitwise_vs_reference(pa):
    rng = np.random.default_rng(23)
    A = (rng.standard_normal((3, 4, 5, 6)) * 1e3).astype(np.float32)
    av = np.transpose(A, [3 - pa[3 - k] for k in range(4)])
    assert (_bits(O.sqr(av)) == _bits(O.ref_unary(A, pa, True))).all()
    assert (_bits(O.scale(av, 2.0)) == _bits(O.ref_unary(A, pa, False, 2.0))).all()
    assert (_bits(O.scale(av, -0.37)) == _bits(O.ref_unary(A, pa, False, -0.37))).all()
