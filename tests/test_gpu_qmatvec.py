"""H2 parity: trc_hip_qmatvec (fused dequant-matvec) against the oracle's
dequantize-then-mul_mat (gguf_tensor_to_f32, src/io/trc_gguf.cpp:966-1049,
followed by compute_mul_mat, src/backends/cpu/trc_cpu_ops.cpp:182-216).

Bar (written here): for every dst row (ne0-run over M), max|y - yhat| / ||yhat||_2 <= 1e-4.
"""
import numpy as np
import pytest

import oracle_lib as O
from conftest import announce
from gpu_util import Dev, Stream, empty, mem_free
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
@pytest.mark.parametrize("N", [1, 2, 3, 4])
@pytest.mark.parametrize("K,M,w_off", [(32 * 130, 3001, 0), (32 * 264, 999, 4), (32 * 264, 999, 0), (512, 20000, 0),
                                       (32 * 200, 777, 0), (16384, 300, 0), (32 * 126, 1000, 0), (4096, 3001, 0),
                                       (4096, 13001, 0), (4096, 14000, 0), (4096, 16384, 0)])
def test_dot_kernel_weight_paths(hip, name, N, K, M, w_off):
    """The one- to four-column kernels' ways of reading W (three and four
    columns only through LDS, four only within one chunk and not for Q4_0; the
    other cases take the matrix-core kernel): into registers (130
    blocks per row, not a multiple of 8; or W 4 bytes off a 16-byte boundary;
    or 126 blocks, K in one chunk), through LDS over two full chunks of 128
    blocks and a short one (264 blocks; one column: one chunk per wave, a fourth
    slot idle), two chunks (200 blocks) and four full ones (512 blocks), through
    LDS with more workgroups than CUs (20000 rows of 8 per wave), and with K in
    one chunk (the instance without the chunk loop, where rows are stored when
    a wave issues its last copies): two rows per wave with one in flight (3001
    rows), seven rows per wave (14000 rows, and 13001: 233 workgroups whose
    last rows lie past M) and eight (16384; Q4_0 with one column keeps three
    rows in flight at all three)."""
    t = TYPES[name]
    announce(f"qmatvec dot paths {name} N={N} K={K} M={M} w_off={w_off}")
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 1000 + K + M))
    X = synth.normal(K + 7 * M, K * N).reshape(1, 1, N, K)
    padded = np.zeros(raw.nbytes + w_off, np.uint8)
    padded[w_off:] = raw
    dw, dx = Dev(padded), Dev(X)
    dy = empty((1, 1, N, M))
    H.qmatvec(t, dw.ptr + w_off, K, M, (K // 32) * H.BLOCK_BYTES[t], dx.ptr, N, K * 4, dy.ptr, M * 4)
    H.sync()
    got = np.ascontiguousarray(dy.read())
    for d in (dw, dx, dy):
        d.free()
    assert O.row_l2_error(got, oracle_qmatvec(t, raw, K, M, X)) <= TOL


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
@pytest.mark.parametrize("N", [2, 4])
def test_edge_shapes_and_padded_columns(hip, name, K, M, N):
    t = TYPES[name]
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
        H.qmatvec(H.TYPE_Q4_0, w.ptr, 64, 4, 36, x.ptr, H.QMATVEC_MAX_N + 1, 256, y.ptr, 16)
    assert e.value.code == H.E_SHAPE
    with pytest.raises(H.HipError) as e:
        H.qmatvec(H.TYPE_Q4_0, w.ptr, 48, 4, 36, x.ptr, 1, 192, y.ptr, 16)  # K % 32
    assert e.value.code == H.E_SHAPE
    with pytest.raises(H.HipError) as e:
        H.qmatvec(H.TYPE_Q4_1, w.ptr + 2, 64, 4, 40, x.ptr, 1, 256, y.ptr, 16)
    assert e.value.code == H.E_ALIGN


# The fp16 matrix-core kernel (qmm.hip) takes 2 <= N <= 16 with a multiple of
# 8 blocks per row (K % 256 == 0), in chunks of 16 blocks; the cases below pin
# its layouts, grid shapes, partial last chunks and numerics. Up to 8 columns it
# packs each column's hi and lo x planes into one 16-column tile, above that it
# gives each plane its own MFMA. Other block counts above exercise the fallback
# kernels.

@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("N", [2, 3, 5, 7, 8, 16])
def test_mfma_path_all_formats(hip, name, N):
    t = TYPES[name]
    K, M = 32 * 40, 301  # 20 pairs: two full chunks and a half one; M not a tile multiple
    announce(f"qmm {name} K={K} M={M} N={N}")
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 211 + t))
    X = synth.normal(31 + N, K * N).reshape(1, 1, N, K)
    got = gpu_qmatvec(t, raw, K, M, X)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert O.row_l2_error(got, want) <= TOL


@pytest.mark.parametrize("name", ["q4_0", "q5_1", "q8_0"])
@pytest.mark.parametrize("M", [1, 5, 16, 250, 3000, 20000])
@pytest.mark.parametrize("N", [8, 16])
def test_mfma_grid_shapes(hip, name, M, N):
    """Rows per workgroup from 8 to 64 (1 to 4 tiles), masked tail rows, K in
    one part or two (up to 24 rows per CU), packed (N = 8) or not."""
    t = TYPES[name]
    K = 256 * 3
    announce(f"qmm grid {name} K={K} M={M} N={N}")
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 3 + M))
    X = synth.normal(17 + M, K * N).reshape(1, 1, N, K)
    got = gpu_qmatvec(t, raw, K, M, X, x_pad=8, y_pad=5)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert O.row_l2_error(got, want) <= TOL


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("K, M, N", [(1024, 7000, 8), (2048, 6500, 5), (768, 9000, 6), (256, 8000, 7),
                                     (512, 14336, 8), (256, 20000, 8)])
def test_mfma_x_in_lds(hip, name, K, M, N):
    """Up to 8 columns with K in one part of at most 4 chunks (M above 24 rows
    per CU): where x fits beside the chunk ring (32 to 56 rows per workgroup, 80
    for Q4_0), every workgroup converts x into LDS itself, with no pre-pass; the
    other formats take the pre-pass. K = 768 ends on a half chunk, K = 256 is one
    chunk of 4 pairs. A NaN in the last column checks that the in-LDS scales
    carry it."""
    t = TYPES[name]
    announce(f"qmm x in LDS {name} K={K} M={M} N={N}")
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 41 + K + N))
    X = synth.normal(43 + M, K * N).reshape(1, 1, N, K).astype(np.float32)
    X[0, 0, 1] *= np.float32(1e-20)  # columns of very different magnitude
    X[0, 0, 2, 32:64] = np.float32(1e-40)  # a denormal block
    X[0, 0, N - 1, K - 7] = np.nan
    got = gpu_qmatvec(t, raw, K, M, X, x_pad=4, y_pad=3)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert not np.isfinite(got[0, 0, N - 1]).any()
    assert O.row_l2_error(got[:, :, : N - 1], want[:, :, : N - 1]) <= TOL


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("N", [8, 9])
def test_mfma_dynamic_range(hip, name, N):
    """Columns of very different magnitude, blocks of very different magnitude
    inside one column, and denormal x: the scale is per block and column, with
    hi and lo packed into one tile (N = 8) or not (N = 9)."""
    t = TYPES[name]
    K, M = 32 * 16, 96
    announce(f"qmm range {name} N={N}")
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 77 + t))
    X = synth.normal(5, K * N).reshape(1, 1, N, K).astype(np.float32)
    scales = [1e-30, 1e-6, 1e-3, 1.0, 1e3, 1e6, 1e20, 3e25, 1.0]
    if N == 8:
        del scales[6]
    col_scale = np.array(scales, np.float32)
    X *= col_scale[None, None, :, None]
    X[0, 0, N - 1, 64:96] *= np.float32(1e12)  # one loud block in an otherwise unit column
    X[0, 0, N - 1, 96:128] *= np.float32(1e-12)  # and a quiet one
    X[0, 0, 3, 0:32] = np.float32(1e-40)  # a block of denormals next to normal blocks
    got = gpu_qmatvec(t, raw, K, M, X)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert np.isfinite(got).all()
    assert O.row_l2_error(got, want) <= TOL


@pytest.mark.parametrize("name", ["q4_0", "q5_1", "q8_0"])
@pytest.mark.parametrize("N", [1, 2, 4, 6, 12])
@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
@pytest.mark.parametrize("K", [256, 32 * 296])
def test_nonfinite_x(hip, name, N, bad, K):
    """A non-finite x element makes its column non-finite, as in the reference
    (the fixed-point kernels return NaN there); the other columns are unaffected.
    Covers the integer-dot (N = 1, 2), one-chunk-per-wave (N = 1, 296 blocks:
    the element sits in the third chunk) and fp16 MFMA (N = 4 for Q4_0, packed
    N = 6, unpacked N = 12) kernels."""
    t = TYPES[name]
    M = 40
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 8))
    X = synth.normal(9, K * N).reshape(1, 1, N, K)
    j = N - 1
    X[0, 0, j, K - 219] = bad
    got = gpu_qmatvec(t, raw, K, M, X)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert not np.isfinite(want[0, 0, j]).any()
    assert not np.isfinite(got[0, 0, j]).any()
    keep = [c for c in range(N) if c != j]
    if keep:
        assert O.row_l2_error(got[:, :, keep], want[:, :, keep]) <= TOL


def test_mfma_q8_0_minus_128(hip):
    """GGUF Q8_0 quants may be -128 (the synthetic draws stop at -127)."""
    t = TYPES["q8_0"]
    K, M, N = 256, 48, 16
    blocks = synth.quant_blocks(t, K * M // 32, 21)
    qs = blocks["qs"].copy()
    qs[::3, ::5] = -128
    qs[1::7, :] = -128  # whole blocks at the extreme
    blocks["qs"] = qs
    raw = synth.block_bytes(blocks)
    X = synth.normal(22, K * N).reshape(1, 1, N, K)
    got = gpu_qmatvec(t, raw, K, M, X)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert O.row_l2_error(got, want) <= TOL


@pytest.mark.parametrize("nblk", [2048, 2056])
def test_mfma_block_limit(hip, nblk):
    """2048 blocks per row is the int8 kernel's limit; 2056 takes the fallback."""
    t = TYPES["q5_0"]
    K, M, N = 32 * nblk, 24, 5
    announce(f"qmm limit nblk={nblk}")
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, nblk))
    X = synth.normal(nblk, K * N).reshape(1, 1, N, K)
    got = gpu_qmatvec(t, raw, K, M, X)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert O.row_l2_error(got, want) <= TOL


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("N", [17, 31, 33, 48, 64])
def test_skinny_gemm_wide(hip, name, N):
    """N up to 64: one fused pass over W per 16 columns (the last slice may be a
    single column, which takes the batch-1 kernel)."""
    t = TYPES[name]
    K, M = 32 * 40, 203
    announce(f"qmatvec wide {name} N={N}")
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 300 + N + t))
    X = synth.normal(400 + N, K * N).reshape(1, 1, N, K)
    got = gpu_qmatvec(t, raw, K, M, X, x_pad=8, y_pad=5)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert O.row_l2_error(got, want) <= TOL


def test_config2_q4_0_n64(hip):
    """Configuration 2's weight (Q4_0 14336 x 4096) against 64 columns."""
    t = TYPES["q4_0"]
    K, M, N = 4096, 14336, 64
    announce("qmatvec cfg2 q4_0 N=64")
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, synth.config_seed(2, t)))
    X = synth.normal(synth.config_seed(2, 164), K * N).reshape(1, 1, N, K)
    got = gpu_qmatvec(t, raw, K, M, X)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert O.row_l2_error(got, want) <= TOL


# Column contents for the dynamic-range cases of the integer-dot kernels (N = 1..4).
def _range_column(p, K, rng):
    x = rng.standard_normal(K).astype(np.float32)
    if p == 0:
        return np.full(K, 1e-41, np.float32) * np.sign(x)      # every element denormal
    if p == 1:
        return x * np.float32(1e-30)
    if p == 2:
        return x * np.float32(3e25)
    if p == 3:
        x[37] = np.float32(1e12)                                # an outlier inside a block
        return x
    if p == 4:
        x[0:32] = np.float32(1e-40)                             # a denormal block beside normal ones
        x[64:96] *= np.float32(1e-12)
        return x
    return x


RANGE_PATTERNS = 6


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("N,p0", [(1, p) for p in range(RANGE_PATTERNS)] + [(2, 0), (2, 3), (3, 0), (3, 3),
                                                                            (4, 0), (4, 2)])
@pytest.mark.parametrize("K,M", [(4096, 96), (32 * 130, 96), (32 * 264, 160)])
def test_dot_dynamic_range(hip, name, N, p0, K, M):
    """The one- to four-column kernels scale x per 32-element block by a power
    of two 2^-s that must stay a float down to all-denormal blocks: column j
    holds pattern (p0 + j) % 6 (all-denormal, scale 1e-30, scale 3e25, a 1e12
    outlier inside a block, a denormal block beside normal ones, unit). Weights
    through LDS (K = 4096), through registers (130 blocks per row) and one chunk
    per wave (264 blocks)."""
    t = TYPES[name]
    announce(f"qmatvec dot range {name} N={N} p0={p0} K={K}")
    rng = np.random.default_rng(1000 * p0 + N + K)
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 50 + t + K))
    X = np.stack([_range_column((p0 + j) % RANGE_PATTERNS, K, rng) for j in range(N)]).reshape(1, 1, N, K)
    got = gpu_qmatvec(t, raw, K, M, X)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert np.isfinite(got).all()
    assert O.row_l2_error(got, want) <= TOL
    for j in range(N):
        if (p0 + j) % RANGE_PATTERNS == 0:
            # the bar's 1e-30 floor makes any tiny column pass, so the denormal
            # column is also held to its own scale: the reference's products are
            # themselves denormal and keep only a few bits, hence the loose 5 %
            g, w = got[0, 0, j].astype(np.float64), want[0, 0, j].astype(np.float64)
            assert np.abs(w).max() > 0
            assert np.abs(g - w).max() <= 0.05 * np.abs(w).max()


def test_two_streams_do_not_share_x(hip):
    """Two different 16-column products (the matrix-core path, whose x planes go
    to a device workspace) enqueued alternately on two streams, so that they
    overlap on the GPU; each stream's calls must use its own workspace. Both
    results match the oracle and equal, bit for bit, the same call run alone."""
    t = TYPES["q4_0"]
    K, M, N = 4096, 2048, 16
    streams = [Stream(), Stream()]
    cases = []
    for c in range(2):
        raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 900 + c))
        X = synth.normal(910 + c, K * N).reshape(1, 1, N, K) * np.float32(10.0 ** (3 * c))
        cases.append((raw, X, Dev(raw), Dev(X), empty((1, 1, N, M))))
    announce("qmatvec two streams, 16 columns each")
    for _ in range(40):
        for c, (raw, X, dw, dx, dy) in enumerate(cases):
            H.qmatvec(t, dw.ptr, K, M, (K // 32) * 18, dx.ptr, N, K * 4, dy.ptr, M * 4, streams[c].handle)
    for s in streams:
        H.sync(s.handle)
    for c, (raw, X, dw, dx, dy) in enumerate(cases):
        got = np.ascontiguousarray(dy.read())
        assert O.row_l2_error(got, oracle_qmatvec(t, raw, K, M, X)) <= TOL
        alone = empty((1, 1, N, M))
        H.qmatvec(t, dw.ptr, K, M, (K // 32) * 18, dx.ptr, N, K * 4, alone.ptr, M * 4)
        H.sync()
        assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(alone.read()).view(np.uint32))
        for d in (dw, dx, dy, alone):
            d.free()
    for s in streams:
        s.close()


def test_stream_workspaces_are_released_and_bounded(hip):
    """The 16-column path converts x into a workspace per stream. 64 streams are
    created and destroyed, each with one call and trc_hip_qmatvec_release_stream
    before hipStreamDestroy: free device memory comes back to within 1 MiB of its
    start. Then 12 streams stay alive without a release: the device keeps at most
    8 workspaces, so memory grows by at most 8 of them. Every result equals the
    null stream's bit for bit."""
    t = TYPES["q4_0"]
    K, M, N = 4096, 2048, 16
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, 930))
    X = synth.normal(931, K * N).reshape(1, 1, N, K)
    dw, dx, dy = Dev(raw), Dev(X), empty((1, 1, N, M))

    def call(stream):
        H.qmatvec(t, dw.ptr, K, M, (K // 32) * 18, dx.ptr, N, K * 4, dy.ptr, M * 4, stream)
        H.sync(stream)
        return np.ascontiguousarray(dy.read())

    announce("qmatvec stream workspaces: 64 streams released, 12 kept")
    ref = call(None)
    assert O.row_l2_error(ref, oracle_qmatvec(t, raw, K, M, X)) <= TOL
    start = mem_free()
    for _ in range(64):
        s = Stream()
        assert np.array_equal(call(s.handle).view(np.uint32), ref.view(np.uint32))
        s.close()  # trc_hip_qmatvec_release_stream, then hipStreamDestroy
    assert abs(mem_free() - start) <= 1 << 20
    live = [Stream() for _ in range(12)]
    before = mem_free()  # after the streams' own allocations
    for s in live:
        assert np.array_equal(call(s.handle).view(np.uint32), ref.view(np.uint32))
    ws_bound = 12 << 20  # one workspace (8.3 MiB) with the allocator's rounding
    grown = before - mem_free()
    print(f"12 live streams: workspaces took {grown / 2**20:.1f} MiB", flush=True)
    assert grown <= 8 * ws_bound
    for s in live:
        s.close()
    H.qmatvec_release_stream(None)
    assert mem_free() >= start - (1 << 20)
    H.qmatvec_release_stream(None)  # nothing left to free: still OK
    for d in (dw, dx, dy):
        d.free()


def _random_cases(n=48, seed=20261202):
    """Seeded shapes across every routing of trc_hip_qmatvec: K with block counts
    that are and are not multiples of 8 (LDS copies or register loads, matrix
    cores or not), one to four chunks, M from a handful of rows to more
    workgroups than CUs (K split or not), N from 1 to 64 (integer-dot kernel,
    packed and unpacked matrix-core tiles, 32-column slices), padded x and y
    strides. Sizes keep the oracle under a few seconds in all."""
    rng = np.random.default_rng(seed)
    names = list(TYPES)
    cases = []
    while len(cases) < n:
        nblk = int(rng.choice([8, 16, 24, 40, 64, 72, 128, 136, 200, 256, 264, 448])) + int(rng.choice([0, 0, 0, 1, 3]))
        K = 32 * nblk
        N = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16, 17, 24, 31, 32, 33, 40, 48, 64]))
        M = int(rng.choice([1, 7, 33, 257, 1000, 2049, 4097, 6200, 9000, 14336, 17000]))
        if K * M * N > 3e8:
            continue
        cases.append((names[int(rng.integers(len(names)))], K, M, N, int(rng.integers(0, 3)) * 4, int(rng.integers(0, 3))))
    return cases


@pytest.mark.parametrize("name, K, M, N, x_pad, y_pad", _random_cases())
def test_random_routes(hip, name, K, M, N, x_pad, y_pad):
    t = TYPES[name]
    announce(f"qmatvec random {name} K={K} M={M} N={N} pads={x_pad},{y_pad}")
    raw = synth.block_bytes(synth.quant_blocks(t, K * M // 32, K + 3 * M + 7 * N))
    X = synth.normal(K * 5 + M + N, K * N).reshape(1, 1, N, K)
    got = gpu_qmatvec(t, raw, K, M, X, x_pad=x_pad, y_pad=y_pad)
    want = oracle_qmatvec(t, raw, K, M, X)
    assert O.row_l2_error(got, want) <= TOL
