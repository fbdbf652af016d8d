"""H3 parity: trc_hip_mul_mat_f32 (FP32 MFMA) against the oracle.

Reference semantics: compute_mul_mat (src/backends/cpu/trc_cpu_ops.cpp:182-216).
Bar (written here, from the benchmark's tolerance): for every dst row r (one
ne0-run), max_i |y_ri - yhat_ri| / ||yhat_r||_2 <= 1e-4, where yhat is the oracle.
The reference's own goldens additionally hold at their atol 1e-4 / rtol 1e-3.
"""
import numpy as np
import pytest

import oracle_lib as O
from conftest import GOLDEN, announce
from gpu_util import Dev, Stream, empty, gpu_mul_mat
from traincpp_amd import hip as H
from traincpp_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-4


def g(name):
    return np.load(GOLDEN / f"{name}.npy", allow_pickle=False)


def as4(a):
    return a.reshape((1,) * (4 - a.ndim) + a.shape)


def ramp(n):
    """The conformance tests' input ramp (tests/test_backend_conformance.cpp:130-135)."""
    i = np.arange(n)
    return ((i % 17) - 8).astype(np.float32) * np.float32(0.25)


def t01(x):
    return np.swapaxes(x, 2, 3)


def run_views(A, a_view_fn, B, b_view_fn):
    """Uploads the base arrays, runs the GPU on the views, returns (gpu, oracle)."""
    da, db = Dev(A), Dev(B)
    av, bv = a_view_fn(da.base), b_view_fn(db.base)
    got = gpu_mul_mat(da, av, db, bv)
    want = O.mul_mat(av, bv, threads=8)
    da.free()
    db.free()
    return got, want


@pytest.mark.parametrize("case", ["mul_mat", "mul_mat_batch", "mul_mat_batch_bcast_div", "mul_mat_batch_tile"])
def test_reference_goldens(hip, case):
    announce(f"mul_mat golden {case}")
    a, b, want = as4(g(f"{case}_in0")), as4(g(f"{case}_in1")), g(f"{case}_out")
    got, orc = run_views(a, lambda x: x, b, lambda x: x)
    assert np.all(np.abs(got - want) <= 1e-4 + 1e-3 * np.abs(want))
    assert O.row_l2_error(got, orc) <= TOL


# The conformance suite's mul_mat cases (tests/test_backend_conformance.cpp:455-553,928-934):
# (a base shape in ggml order, transpose a?, b base shape, transpose b?)
CONFORMANCE = {
    "basic": ((5, 3, 1, 1), False, (5, 4, 1, 1), False),
    "transposed_a": ((3, 5, 1, 1), True, (5, 4, 1, 1), False),
    "transposed_b": ((5, 3, 1, 1), False, (4, 5, 1, 1), True),
    "tile_boundary": ((33, 70, 1, 1), False, (33, 66, 1, 1), False),
    "batch": ((5, 3, 1, 1), False, (5, 4, 2, 3), False),
    "batch_bcast_div": ((5, 3, 2, 1), False, (5, 4, 4, 1), False),
    "batch_transposed": ((3, 5, 2, 2), True, (4, 5, 2, 2), True),
    "batch_tile_boundary": ((33, 70, 1, 1), False, (33, 66, 2, 2), False),
    "grid_batch_z": ((8, 4, 1, 1), False, (8, 4, 65, 1), False),
}


@pytest.mark.parametrize("name", list(CONFORMANCE))
def test_conformance_cases(hip, name):
    ane, ta, bne, tb = CONFORMANCE[name]
    announce(f"mul_mat conformance {name}")
    A = ramp(int(np.prod(ane))).reshape(ane[::-1])
    B = ramp(int(np.prod(bne))).reshape(bne[::-1])
    got, want = run_views(A, t01 if ta else (lambda x: x), B, t01 if tb else (lambda x: x))
    # the conformance tolerance (test_backend_conformance.cpp:107) and the benchmark bar
    assert np.all(np.abs(got - want) <= 1e-5 + 2e-4 * np.abs(want))
    assert O.row_l2_error(got, want) <= TOL


@pytest.mark.parametrize("case", ["grad_mul_mat_batch", "grad_mul_mat_batch_div"])
def test_backward_goldens(hip, case):
    """dA = transpose(mul_mat(transpose(dY), transpose(B))) (+ plane sum) and
    dB = mul_mat(transpose(A), dY) (src/core/trc_autograd.cpp:487-503) on the GPU."""
    announce(f"mul_mat backward golden {case}")
    A, B = as4(g(f"{case}_in0")), as4(g(f"{case}_in1"))
    Y, _ = run_views(A, lambda x: x, B, lambda x: x)
    dY = (2.0 * Y).astype(np.float32)
    dA_t, _ = run_views(dY, t01, B, t01)
    dA_full = t01(dA_t)
    a3, a2, b3, b2 = A.shape[0], A.shape[1], B.shape[0], B.shape[1]
    dA = dA_full.reshape(b3 // a3, a3, b2 // a2, a2, *dA_full.shape[2:]).sum(axis=(0, 2))
    dB, _ = run_views(A, t01, dY, lambda x: x)
    for got, name in ((dA, "grad0"), (dB, "grad1")):
        want = g(f"{case}_{name}")
        assert np.all(np.abs(got - want) <= 1e-4 + 1e-3 * np.abs(want)), name


@pytest.mark.parametrize("shape", [
    # K, M, N, b2, b3, a2, a3
    (1, 1, 1, 1, 1, 1, 1), (2, 33, 31, 1, 1, 1, 1), (17, 65, 129, 1, 1, 1, 1), (100, 130, 70, 3, 2, 3, 1),
    (256, 256, 256, 1, 1, 1, 1), (513, 200, 300, 2, 1, 1, 1), (64, 128, 128, 4, 2, 2, 2), (7, 9, 11, 6, 1, 3, 1),
    # 128 or more 128x128 tiles but under 512 and K >= 1024: K in two parts that
    # meet in dst (partial tiles, K not a multiple of the slab, two planes)
    (2500, 2000, 1000, 1, 1, 1, 1), (1030, 1000, 1000, 1, 1, 2, 1),
    # the same with whole tiles and slabs (double-buffered slabs): broadcast
    # planes, and 8 planes (each plane's tiles on one XCD)
    (1024, 1024, 512, 4, 1, 2, 1), (1088, 512, 512, 8, 1, 1, 1),
    # 512 or more whole 128x128 tiles, K whole (double-buffered slabs)
    (64, 4096, 2048, 1, 1, 1, 1),
    # plane counts that are a multiple of 8 (each plane's tiles on one XCD):
    # ragged 64x64 tiles over 8 planes, ragged 128x128 tiles over 64 planes
    (33, 70, 90, 4, 2, 1, 1), (40, 300, 300, 8, 8, 1, 1),
])
@pytest.mark.parametrize("layout", ["kk", "tk", "kt", "tt", "gen"])
def test_random_shapes_and_layouts(hip, shape, layout):
    K, M, N, b2, b3, a2, a3 = shape
    rng = np.random.default_rng(K * 7 + M * 3 + N)
    announce(f"mul_mat random {shape} {layout}")
    if layout == "gen":
        # every-other-element views: nb0 = 8 forces the scalar (generic) loaders
        A = rng.standard_normal((a3, a2, M, 2 * K)).astype(np.float32)
        B = rng.standard_normal((b3 * a3, b2 * a2, N, 2 * K)).astype(np.float32)
        got, want = run_views(A, lambda x: x[..., ::2], B, lambda x: x[..., ::2])
    else:
        ta, tb = layout[0] == "t", layout[1] == "t"
        A = rng.standard_normal((a3, a2, K, M) if ta else (a3, a2, M, K)).astype(np.float32)
        B = rng.standard_normal((b3 * a3, b2 * a2, K, N) if tb else (b3 * a3, b2 * a2, N, K)).astype(np.float32)
        got, want = run_views(A, t01 if ta else (lambda x: x), B, t01 if tb else (lambda x: x))
    assert O.row_l2_error(got, want) <= TOL


def sampled_oracle_cols(av, bv, cols):
    """Oracle values of dst columns `cols` (dst rows in the row-L2 metric)."""
    pa, ane, anb = O.base_ptr_and_meta(av)
    pb, bne, bnb = O.base_ptr_and_meta(bv)
    dne = [ane[1], bne[1], bne[2], bne[3]]
    out = np.zeros((dne[3], dne[2], dne[1], dne[0]), dtype=np.float32)
    _, _, dnb = O.base_ptr_and_meta(out)
    for j in cols:
        rc = O.oracle().orc_mul_mat_cols(pa, O.NE(*ane), O.NB(*anb), pb, O.NE(*bne), O.NB(*bnb), out.ctypes.data,
                                         O.NE(*dne), O.NB(*dnb), int(j), int(j) + 1, 8)
        assert rc == 0
    return out[:, :, cols, :]


def config3_inputs():
    t = 7  # Q5_1 weights, dequantized on the GPU exactly as the oracle does
    n = 4096 * 4096 // 32
    raw = synth.block_bytes(synth.quant_blocks(t, n, synth.config_seed(3, 0)))
    W = O.dequant(t, raw, threads=8).reshape(1, 1, 4096, 4096)
    X = synth.normal(synth.config_seed(3, 1), 4096 * 512).reshape(1, 1, 512, 4096)
    dY = synth.normal(synth.config_seed(3, 2), 4096 * 512, 0.0, 1e-2).reshape(1, 1, 512, 4096)
    return W, X, dY


# sampled dst rows (ne1 indices) at full size: tile edges, both ends and a stride
COLS = sorted({0, 1, 31, 32, 63, 64, 127, 128, 200, 255, 256, 383, 384, 510, 511, *range(5, 512, 37)})


def sums_error(got, av, bv):
    """Every dst element enters two float64 checksums that the operands fix:
    sum_j dst[i, j] = sum_k a[k, i] * (sum_j b[k, j]) and
    sum_i dst[i, j] = sum_k (sum_i a[k, i]) * b[k, j], per plane (a's planes by the
    ggml modulo broadcast). Returns the larger row-L2-normalised error of the two;
    a wrong or missing tile anywhere moves one of them far above FP32 rounding."""
    ne3, ne2 = got.shape[0], got.shape[1]
    worst = 0.0
    for i3 in range(ne3):
        for i2 in range(ne2):
            a = np.asarray(av[i3 % av.shape[0], i2 % av.shape[1]], dtype=np.float64)  # [M, K]
            b = np.asarray(bv[i3, i2], dtype=np.float64)                              # [N, K]
            d = np.asarray(got[i3, i2], dtype=np.float64)                             # [N, M]
            s_i, r_i = d.sum(axis=0), a @ b.sum(axis=0)
            s_j, r_j = d.sum(axis=1), b @ a.sum(axis=0)
            for s, r in ((s_i, r_i), (s_j, r_j)):
                worst = max(worst, float(np.abs(s - r).max() / max(np.linalg.norm(r), 1e-30)))
    return worst


@pytest.fixture(scope="module")
def cfg3():
    return config3_inputs()


@pytest.mark.parametrize("product", ["Y=W.X", "dX=W^T.dY", "dW^T=dY^T.X^T"])
def test_config3_full_size(hip, cfg3, product):
    """The linear layer's three products at 4096 x 4096 x 512, checked on sampled
    dst rows against the oracle."""
    W, X, dY = cfg3
    announce(f"mul_mat cfg3 {product}")
    if product == "Y=W.X":
        A, af, B, bf, cols = W, (lambda x: x), X, (lambda x: x), COLS
    elif product == "dX=W^T.dY":
        A, af, B, bf, cols = W, t01, dY, (lambda x: x), COLS
    else:
        A, af, B, bf, cols = dY, t01, X, t01, [0, 1, 4095, 1000, 2048]
    da, db = Dev(A), Dev(B)
    av, bv = af(da.base), bf(db.base)
    got = gpu_mul_mat(da, av, db, bv)
    want = sampled_oracle_cols(av, bv, cols)
    assert O.row_l2_error(got[:, :, cols, :], want) <= TOL
    assert np.isfinite(got).all()
    assert sums_error(got, av, bv) <= 1e-5
    da.free()
    db.free()


def test_config4_broadcast_permuted(hip):
    """src0 ne=[128,1024,8,4] x src1 = permute(base[128,32,512,4], 0,2,1,3)
    (ne=[128,512,32,4], nb1 > nb2), planes broadcast (i2%8, i3%4)."""
    announce("mul_mat cfg4")
    A = synth.normal(synth.config_seed(4, 0), 128 * 1024 * 8 * 4).reshape(4, 8, 1024, 128)
    base = synth.normal(synth.config_seed(4, 1), 128 * 32 * 512 * 4).reshape(4, 512, 32, 128)
    da, db = Dev(A), Dev(base)
    bv = np.swapaxes(db.base, 1, 2)  # ggml permute(0,2,1,3)
    ne, nb = O.view_meta(bv)
    assert ne == [128, 512, 32, 4] and nb == [4, 16384, 512, 8388608]
    got = gpu_mul_mat(da, da.base, db, bv)
    cols = [0, 7, 31, 32, 255, 256, 300, 480, 511]
    want = sampled_oracle_cols(da.base, bv, cols)
    assert O.row_l2_error(got[:, :, cols, :], want) <= TOL
    assert sums_error(got, da.base, bv) <= 1e-5
    da.free()
    db.free()


def test_split_products_on_two_streams(hip):
    """K split in two (K >= 1024, 128 to 511 tiles of 128 x 128): the waves holding
    one block in the two parts meet in dst through ticket words kept with the
    stream's workspace, which every launch leaves clear. Two such products
    alternate on two streams, 20 calls each, so that they overlap on the GPU and
    each stream needs its own words: one with whole tiles (double-buffered
    slabs), one with ragged tiles. Each result equals, bit for bit, the same
    product run twice more on the null stream, and matches the oracle."""
    streams = [Stream(), Stream()]
    cases = []
    for c, (K, M, N) in enumerate([(1024, 2048, 1024), (1100, 2000, 1000)]):  # 16 x 8 tiles each
        A = synth.normal(940 + c, K * M).reshape(1, 1, M, K)
        B = synth.normal(950 + c, K * N).reshape(1, 1, N, K) * np.float32(10.0 ** c)
        cases.append((A, B, Dev(A), Dev(B), empty((1, 1, N, M))))
    announce("mul_mat K split, two streams")
    for _ in range(20):
        for c, (A, B, da, db, dd) in enumerate(cases):
            H.mul_mat_f32(da.tensor(), db.tensor(), dd.tensor(), streams[c].handle)
    for st in streams:
        H.sync(st.handle)
    for A, B, da, db, dd in cases:
        got = dd.read()
        for _ in range(2):
            alone = gpu_mul_mat(da, da.base, db, db.base)
            assert np.array_equal(got.view(np.uint32), alone.view(np.uint32))
        assert O.row_l2_error(got, O.mul_mat(A, B, threads=8)) <= TOL
        for dv in (da, db, dd):
            dv.free()
    for st in streams:
        st.close()


def test_shape_errors_are_rejected(hip):
    a = empty((1, 1, 4, 8))
    b = empty((1, 1, 4, 6))
    d = empty((1, 1, 4, 4))
    with pytest.raises(H.HipError) as e:
        H.mul_mat_f32(a.tensor(), b.tensor(), d.tensor())  # K 8 vs 6
    assert e.value.code == H.E_SHAPE
    b2 = empty((1, 3, 4, 8))
    a2 = empty((1, 2, 4, 8))
    d2 = empty((1, 3, 4, 4))
    with pytest.raises(H.HipError) as e:
        H.mul_mat_f32(a2.tensor(), b2.tensor(), d2.tensor())  # 3 % 2 != 0
    assert e.value.code == H.E_SHAPE
    # dst sharing bytes with an operand
    buf = empty((1, 1, 8, 8))  # a: K = 8, M = 8
    b3 = empty((1, 1, 6, 8))   # b: K = 8, N = 6
    with pytest.raises(H.HipError) as e:
        H.mul_mat_f32(buf.tensor(), b3.tensor(), H.tensor(buf.ptr + 16, [8, 6, 1, 1], H.contiguous_nb([8, 6, 1, 1])))
    assert e.value.code == H.E_SHAPE
    with pytest.raises(H.HipError) as e:
        H.mul_mat_f32(buf.tensor(), b3.tensor(), H.tensor(b3.ptr, [8, 6, 1, 1], H.contiguous_nb([8, 6, 1, 1])))
    assert e.value.code == H.E_SHAPE
    for t in (buf, b3):
        t.free()


# ---------------------------------------------------------------- few columns (N <= 64)

@pytest.fixture(scope="module")
def cfg0_w():
    """Configuration 0's weight: the Q8_0 blocks of a 4096 x 4096 tensor as the GGUF
    warm start turns them into F32 (src/io/trc_gguf.cpp:1082-1088), here by the oracle."""
    n = 4096 * 4096 // 32
    raw = synth.block_bytes(synth.quant_blocks(H.TYPE_Q8_0, n, synth.config_seed(0, 8)))
    return O.dequant(H.TYPE_Q8_0, raw, threads=8).reshape(1, 1, 4096, 4096)


@pytest.mark.parametrize("N", [1, 2, 3, 5, 7, 8, 16, 32, 64])
@pytest.mark.parametrize("layout", ["contiguous", "transposed"])
def test_config0_f32_few_columns(hip, cfg0_w, N, layout):
    """mul_mat(W F32 [4096, 4096], X [4096, N]) at configuration 0's size, every dst
    element against the oracle: X k-contiguous, or X = transpose(base[N, 4096])
    (k strided, the layout of a transposed activation view)."""
    announce(f"mul_mat cfg0 F32 N={N} {layout}")
    X = synth.normal(synth.config_seed(0, 100 + N), 4096 * N)
    if layout == "contiguous":
        got, want = run_views(cfg0_w, lambda x: x, X.reshape(1, 1, N, 4096), lambda x: x)
    else:
        got, want = run_views(cfg0_w, lambda x: x, X.reshape(1, 1, 4096, N), t01)
    assert got.shape == (1, 1, N, 4096)
    assert O.row_l2_error(got, want) <= TOL


@pytest.mark.parametrize("K,M,N", [(512, 16, 1), (4096, 48, 5), (4096, 4096, 8), (1028, 70, 12), (2048, 33, 40)])
def test_few_columns_one_hot(hip, K, M, N):
    """W rows with a single 1 at k = kmap[i] and X[j, k] = 1000 j + k: every output
    is one X element times 1 plus exact zeros, so it must equal 1000 j + kmap[i]
    bit for bit. A wrong lane-to-(column, k) mapping in the few-column loads shows
    up here as the value of the (column, k) that was read instead."""
    announce(f"mul_mat one-hot K={K} M={M} N={N}")
    kmap = (np.arange(M) * 131 + 7) % K
    W = np.zeros((1, 1, M, K), np.float32)
    W[0, 0, np.arange(M), kmap] = 1.0
    X = (1000.0 * np.arange(N)[:, None] + np.arange(K)[None, :]).astype(np.float32).reshape(1, 1, N, K)
    a, b = Dev(W), Dev(X)
    got = gpu_mul_mat(a, W, b, X)
    want = (1000.0 * np.arange(N)[:, None] + kmap[None, :]).astype(np.float32).reshape(1, 1, N, M)
    assert np.array_equal(got, want)
    a.free()
    b.free()


def test_config0_f32_deterministic(hip, cfg0_w):
    """The waves' partial sums meet in a fixed order: two runs give the same bits."""
    announce("mul_mat cfg0 F32 N=8 twice")
    X = synth.normal(synth.config_seed(0, 108), 4096 * 8).reshape(1, 1, 8, 4096)
    a, _ = run_views(cfg0_w, lambda x: x, X, lambda x: x)
    b, _ = run_views(cfg0_w, lambda x: x, X, lambda x: x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("shape", [
    # K, M, N, b2, b3, a2, a3: ragged row blocks, K not a multiple of the 32-wide chunk,
    # fewer chunks than waves, every column-group count, broadcast planes
    (4, 1, 1, 1, 1, 1, 1), (36, 17, 5, 1, 1, 1, 1), (100, 33, 16, 1, 1, 1, 1), (512, 70, 17, 1, 1, 1, 1),
    (1028, 250, 33, 1, 1, 1, 1), (2048, 300, 48, 1, 1, 1, 1), (260, 129, 64, 1, 1, 1, 1),
    (128, 64, 8, 4, 2, 2, 1), (96, 48, 24, 6, 1, 3, 1), (64, 40, 64, 2, 2, 1, 2),
    (1000, 77, 7, 1, 1, 1, 1), (4100, 33, 6, 2, 1, 1, 1),
])
@pytest.mark.parametrize("layout", ["kk", "kt", "kgen", "kmis"])
def test_few_columns_shapes(hip, shape, layout):
    """The few-column path (N <= 64, W k-contiguous) on ragged shapes and planes, with
    X k-contiguous (kk), transposed (kt), every other element (kgen) or 4 bytes off
    16-byte alignment (kmis: read element by element)."""
    K, M, N, b2, b3, a2, a3 = shape
    rng = np.random.default_rng(K * 11 + M * 5 + N)
    announce(f"mul_mat few columns {shape} {layout}")
    A = rng.standard_normal((a3, a2, M, K)).astype(np.float32)
    if layout == "kk":
        B = rng.standard_normal((b3 * a3, b2 * a2, N, K)).astype(np.float32)
        got, want = run_views(A, lambda x: x, B, lambda x: x)
    elif layout == "kt":
        B = rng.standard_normal((b3 * a3, b2 * a2, K, N)).astype(np.float32)
        got, want = run_views(A, lambda x: x, B, t01)
    elif layout == "kgen":
        B = rng.standard_normal((b3 * a3, b2 * a2, N, 2 * K)).astype(np.float32)
        got, want = run_views(A, lambda x: x, B, lambda x: x[..., ::2])
    else:
        B = rng.standard_normal((b3 * a3, b2 * a2, N, K + 1)).astype(np.float32)
        got, want = run_views(A, lambda x: x, B, lambda x: x[..., 1:])
    assert O.row_l2_error(got, want) <= TOL


# ---------------------------------------------------------------- dst += mul_mat (trc_hip_mul_mat_acc_f32)

def _acc_run(A, a_view_fn, B, b_view_fn, D0):
    """GPU d0 + mul_mat(a, b) through the accumulate entry, and mul_mat(a, b) alone."""
    da, db, dd = Dev(A), Dev(B), Dev(D0)
    av, bv = a_view_fn(da.base), b_view_fn(db.base)
    H.mul_mat_acc_f32(da.tensor(av), db.tensor(bv), dd.tensor())
    H.sync()
    got = dd.read()
    mm = gpu_mul_mat(da, av, db, bv)
    for d in (da, db, dd):
        d.free()
    return got, mm, av, bv


@pytest.mark.parametrize("shape", [
    # (K, M, N, a transposed, b transposed): the gradient of configuration 3's weight as
    # the plugin fuses it (mul_mat(X^T, dY^T) into W's accumulator), smaller transposed
    # products, and the few-column kernel
    (512, 4096, 4096, True, True), (128, 1024, 768, True, True), (300, 130, 70, False, True),
    (4096, 4096, 8, False, False), (1000, 77, 7, False, False), (96, 48, 40, True, False),
    # 512 whole tiles with k-contiguous operands (double-buffered slabs)
    (256, 4096, 2048, False, False), (64, 4096, 2048, False, True), (96, 4096, 2048, True, False),
])
def test_mul_mat_acc_adds_the_product(hip, shape):
    """Each element gets the product's float sum, then one float add into dst: the
    result equals numpy float32 d0 + (the GPU's mul_mat of the same operands) bit for
    bit, on shapes whose plain product keeps K whole, as these do."""
    K, M, N, at, bt = shape
    announce(f"mul_mat_acc K={K} M={M} N={N} a{'T' if at else ''} b{'T' if bt else ''}")
    A = synth.normal(900 + K, K * M).reshape(1, 1, K, M) if at else synth.normal(900 + K, K * M).reshape(1, 1, M, K)
    B = synth.normal(901 + N, K * N).reshape(1, 1, K, N) if bt else synth.normal(901 + N, K * N).reshape(1, 1, N, K)
    D0 = synth.normal(902 + M, M * N).reshape(1, 1, N, M)
    got, mm, av, bv = _acc_run(A, t01 if at else (lambda x: x), B, t01 if bt else (lambda x: x), D0)
    assert np.array_equal(got.view(np.uint32), (D0 + mm).view(np.uint32))
    if K * M * N <= 64 << 20:
        assert O.row_l2_error(mm, O.mul_mat(av, bv, threads=8)) <= TOL


def test_mul_mat_acc_keeps_k_whole(hip):
    """Configuration 3's forward shape, whose plain product sums K in two parts that
    meet in dst: added into dst it keeps K whole (d + a + b would round differently
    from d + (a + b)), and is checked against d0 + the oracle's product."""
    announce("mul_mat_acc configuration 3 forward shape")
    K, M, N = 4096, 4096, 512
    W = synth.normal(910, K * M).reshape(1, 1, M, K)
    X = synth.normal(911, K * N).reshape(1, 1, N, K)
    D0 = synth.normal(912, M * N).reshape(1, 1, N, M)
    got, _, av, bv = _acc_run(W, lambda x: x, X, lambda x: x, D0)
    cols = np.arange(0, N, 37)
    want = D0[:, :, cols, :] + O.mul_mat(av, np.ascontiguousarray(bv[:, :, cols, :]), threads=8)
    assert O.row_l2_error(got[:, :, cols, :], want) <= TOL
    again, _, _, _ = _acc_run(W, lambda x: x, X, lambda x: x, D0)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


def test_mul_mat_acc_rejects_overlap(hip):
    buf = empty((1, 1, 8, 8))
    b3 = empty((1, 1, 6, 8))
    with pytest.raises(H.HipError) as e:
        H.mul_mat_acc_f32(buf.tensor(), b3.tensor(), H.tensor(buf.ptr + 16, [8, 6, 1, 1], H.contiguous_nb([8, 6, 1, 1])))
    assert e.value.code == H.E_SHAPE
    for t in (buf, b3):
        t.free()
