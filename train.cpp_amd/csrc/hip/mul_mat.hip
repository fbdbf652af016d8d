// H3: ggml-semantics F32 mul_mat on the gfx950 FP32 matrix cores.
//
//   dst[i,j,i2,i3] = sum_k a[k,i,i2%a2,i3%a3] * b[k,j,i2,i3]
//
// Reference semantics: compute_mul_mat (src/backends/cpu/trc_cpu_ops.cpp:182-216)
// with byte-strided operands (:30-42) and the modulo broadcast of src0 planes
// (src/ops/trc_ops.cpp:366-385). The CPU sums k sequentially; here the sum is
// split across MFMA k-steps, so results agree to rounding (row-L2-normalised
// error <= 1e-4), not bit for bit.
//
// Work decomposition
//   - One workgroup = 4 waves computes a BM x BN tile of one output plane
//     (BM along i = dst ne0, BN along j = dst ne1).
//   - Each wave owns TI x TJ tiles of 32x32, each one v_mfma_f32_32x32x2_f32
//     accumulator (16 floats per lane). MFMA rows run along j and MFMA columns
//     along i, so lanes 0..31 of an accumulator register hold 32 consecutive i:
//     the dst stores are 128-byte runs when dst is ne0-contiguous.
//   - K advances in BK-deep slabs staged in LDS as [k][row] (row = i or j,
//     contiguous), read by the MFMA feed with 32 consecutive floats per half-wave.
//     BK is 16 for 128x128 tiles and 32 for 64x64 tiles, whose waves would
//     otherwise run only 8 MFMAs between two barriers.
//   - Each operand is loaded by one of three loaders chosen on the host from
//     its strides: K_CONTIG (nb0 == 4: float4 along k, the layout of weights and
//     activations), R_CONTIG (nb1 == 4: float4 along i/j, the layout of the
//     transposed views autograd builds, src/core/trc_autograd.cpp:487-503) and
//     GENERIC (scalar loads for any other stride). Out-of-range elements load 0.
//   - The next slab is fetched into registers while the current one is being
//     multiplied, so global latency overlaps MFMA work.
//   - Workgroups go to the 8 XCDs in turn (workgroup b on XCD b % 8), each
//     with its own L2. With a multiple of 8 planes, every tile of plane p is
//     put on XCD p % 8, so each src1 plane (and, under the modulo broadcast,
//     each src0 plane) is read into one L2 only; otherwise tiles follow the
//     grid order, where the tiles sharing one src0 row block meet on one XCD.
//   - When 128x128 tiles would give under two workgroups per CU, K is split in
//     two: 8-wave workgroups (64x32 per wave) each sum half of K for one tile,
//     into a dst cleared beforehand, with float atomic adds. 0 + a + b rounds
//     the same in either order, so results stay deterministic.
#include "common.h"

namespace trc_hip {
namespace {


enum LoadMode { K_CONTIG = 0, R_CONTIG = 1, GENERIC = 2 };

struct MMArgs {
    const uint8_t* a;
    const uint8_t* b;
    uint8_t* d;
    int64_t K, M, N;
    int64_t a_nb0, a_nb1, a_nb2, a_nb3, a_ne2, a_ne3;
    int64_t b_nb0, b_nb1, b_nb2, b_nb3, b_ne2;
    int64_t d_nb0, d_nb1, d_nb2, d_nb3;
    int64_t tiles_i, tiles_j;
    int xcd_planes;  // 1: planes % 8 == 0, tiles of plane p on XCD p % 8
};

// Loads a ROWS x BK slab (rows = i for src0, j for src1) of one operand into
// registers, then stores it to LDS as lds[k * LD + row].
template <int MODE, int ROWS, int BK, int THREADS>
struct SlabLoader {
    static constexpr int LD = ROWS + 4;
    static constexpr int PER = ROWS * BK / THREADS;  // floats per thread
    static_assert(PER % 4 == 0, "slab must give each thread whole float4s");
    float r[PER];

    __device__ __forceinline__ void load(const uint8_t* base, int64_t nb_k, int64_t nb_r, int64_t row0,
                                         int64_t nrows, int64_t k0, int64_t K, int tid) {
        if constexpr (MODE == K_CONTIG) {
#pragma unroll
            for (int u = 0; u < PER / 4; ++u) {
                const int q = tid + THREADS * u;
                const int row = q / (BK / 4);
                const int kq = q % (BK / 4);
                const int64_t gr = row0 + row;
                const int64_t gk = k0 + 4 * kq;
                f4 v = {0.f, 0.f, 0.f, 0.f};
                if (gr < nrows && gk < K) v = *(const f4*) (base + gr * nb_r + gk * 4);
                r[4 * u + 0] = v.x;
                r[4 * u + 1] = v.y;
                r[4 * u + 2] = v.z;
                r[4 * u + 3] = v.w;
            }
        } else if constexpr (MODE == R_CONTIG) {
#pragma unroll
            for (int u = 0; u < PER / 4; ++u) {
                const int q = tid + THREADS * u;
                const int k = q / (ROWS / 4);
                const int rq = q % (ROWS / 4);
                const int64_t gr = row0 + 4 * rq;
                const int64_t gk = k0 + k;
                f4 v = {0.f, 0.f, 0.f, 0.f};
                if (gr < nrows && gk < K) v = *(const f4*) (base + gk * nb_k + gr * 4);
                r[4 * u + 0] = v.x;
                r[4 * u + 1] = v.y;
                r[4 * u + 2] = v.z;
                r[4 * u + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int e = tid + THREADS * u;
                const int row = e % ROWS;
                const int k = e / ROWS;
                const int64_t gr = row0 + row;
                const int64_t gk = k0 + k;
                float v = 0.f;
                if (gr < nrows && gk < K) v = *(const float*) (base + gk * nb_k + gr * nb_r);
                r[u] = v;
            }
        }
    }

    __device__ __forceinline__ void store(float* lds, int tid) const {
        if constexpr (MODE == K_CONTIG) {
#pragma unroll
            for (int u = 0; u < PER / 4; ++u) {
                const int q = tid + THREADS * u;
                const int row = q / (BK / 4);
                const int kq = q % (BK / 4);
#pragma unroll
                for (int c = 0; c < 4; ++c) lds[(4 * kq + c) * LD + row] = r[4 * u + c];
            }
        } else if constexpr (MODE == R_CONTIG) {
#pragma unroll
            for (int u = 0; u < PER / 4; ++u) {
                const int q = tid + THREADS * u;
                const int k = q / (ROWS / 4);
                const int rq = q % (ROWS / 4);
                f4 v = {r[4 * u + 0], r[4 * u + 1], r[4 * u + 2], r[4 * u + 3]};
                *(f4*) (lds + k * LD + 4 * rq) = v;
            }
        } else {
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int e = tid + THREADS * u;
                lds[(e / ROWS) * LD + (e % ROWS)] = r[u];
            }
        }
    }
};

// SPLIT: parts of K (1, or 2 summed into a cleared dst with atomic adds).
template <int WI, int WJ, int TI, int TJ, int BK, int AMODE, int BMODE, int SPLIT>
__global__ __launch_bounds__(WI * WJ * 64) void k_mul_mat(MMArgs p) {
    constexpr int THREADS = WI * WJ * 64;
    static_assert(SPLIT == 1 || SPLIT == 2, "two parts at most keep the atomic sums deterministic");
    constexpr int BM = WI * TI * 32;  // tile extent along i
    constexpr int BN = WJ * TJ * 32;  // tile extent along j
    using LA = SlabLoader<AMODE, BM, BK, THREADS>;
    using LB = SlabLoader<BMODE, BN, BK, THREADS>;
    __shared__ __attribute__((aligned(16))) float As[BK * LA::LD];
    __shared__ __attribute__((aligned(16))) float Bs[BK * LB::LD];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wi = wave % WI;
    const int wj = wave / WI;

    int64_t t = blockIdx.x;
    if (p.xcd_planes) {
        // workgroup b = 8k + x runs on XCD x: give it tile k % tpp of plane 8 (k / tpp) + x
        const int64_t tpp = p.tiles_i * p.tiles_j * SPLIT, x = t & 7, k = t >> 3;
        t = (8 * (k / tpp) + x) * tpp + k % tpp;
    }
    const int part = SPLIT > 1 ? (int) (t % SPLIT) : 0;
    t /= SPLIT;
    const int64_t ti = t % p.tiles_i;
    t /= p.tiles_i;
    const int64_t tj = t % p.tiles_j;
    const int64_t plane = t / p.tiles_j;
    const int64_t i2 = plane % p.b_ne2;
    const int64_t i3 = plane / p.b_ne2;

    const uint8_t* a = p.a + (i2 % p.a_ne2) * p.a_nb2 + (i3 % p.a_ne3) * p.a_nb3;
    const uint8_t* b = p.b + i2 * p.b_nb2 + i3 * p.b_nb3;
    uint8_t* d = p.d + i2 * p.d_nb2 + i3 * p.d_nb3;
    const int64_t i0 = ti * BM;
    const int64_t j0 = tj * BN;

    f16v acc[TI][TJ];
#pragma unroll
    for (int x = 0; x < TI; ++x)
#pragma unroll
        for (int y = 0; y < TJ; ++y)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[x][y][v] = 0.f;

    LA la;
    LB lb;
    // this part's slabs: [kt0, kt0 + nk)
    const int64_t slabs = (p.K + BK - 1) / BK;
    const int64_t per_part = (slabs + SPLIT - 1) / SPLIT;
    const int64_t kt0 = part * per_part;
    const int64_t nk = slabs - kt0 < per_part ? slabs - kt0 : per_part;
    la.load(a, p.a_nb0, p.a_nb1, i0, p.M, kt0 * BK, p.K, tid);
    lb.load(b, p.b_nb0, p.b_nb1, j0, p.N, kt0 * BK, p.K, tid);
    la.store(As, tid);
    lb.store(Bs, tid);
    __syncthreads();

    const int half = lane >> 5;  // which k of the pair this lane feeds
    const int col = lane & 31;
    for (int64_t kt = 0; kt < nk; ++kt) {
        const bool more = kt + 1 < nk;
        if (more) {
            la.load(a, p.a_nb0, p.a_nb1, i0, p.M, (kt0 + kt + 1) * BK, p.K, tid);
            lb.load(b, p.b_nb0, p.b_nb1, j0, p.N, (kt0 + kt + 1) * BK, p.K, tid);
        }
        // Several 4-wave workgroups share a CU without a K split: a wave in its
        // MFMA block issues ahead of the others' loads, stores and barriers
        // (dW 142 -> 136 us, configuration 4 168 -> 161 us, same bits). The split
        // products run one workgroup per CU, where it measured no gain.
        if constexpr (SPLIT == 1) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int s = 0; s < BK / 2; ++s) {
            const int kr = 2 * s + half;
            float av[TI], bv[TJ];
#pragma unroll
            for (int x = 0; x < TI; ++x) av[x] = As[kr * LA::LD + (wi * TI + x) * 32 + col];
#pragma unroll
            for (int y = 0; y < TJ; ++y) bv[y] = Bs[kr * LB::LD + (wj * TJ + y) * 32 + col];
#pragma unroll
            for (int x = 0; x < TI; ++x)
#pragma unroll
                for (int y = 0; y < TJ; ++y)
                    acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(bv[y], av[x], acc[x][y], 0, 0, 0);
        }
        if constexpr (SPLIT == 1) __builtin_amdgcn_s_setprio(0);
        if (more) {
            __syncthreads();
            la.store(As, tid);
            lb.store(Bs, tid);
            __syncthreads();
        }
    }

    // Accumulator register v of lane l holds MFMA row 8*(v/4) + 4*(l/32) + v%4
    // (a j offset) and column l%32 (an i offset).
#pragma unroll
    for (int x = 0; x < TI; ++x) {
        const int64_t i = i0 + (wi * TI + x) * 32 + col;
        if (i >= p.M) continue;
#pragma unroll
        for (int y = 0; y < TJ; ++y) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t j = j0 + (wj * TJ + y) * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                if (j >= p.N) continue;
                float* dst = (float*) (d + i * p.d_nb0 + j * p.d_nb1);
                if constexpr (SPLIT > 1) {
                    __hip_atomic_fetch_add(dst, acc[x][y][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                } else {
                    // Non-temporal: dst is not read again by this launch (dW
                    // 1 % and configuration 4 2 % faster than plain stores).
                    __builtin_nontemporal_store(acc[x][y][v], dst);
                }
            }
        }
    }
}

int pick_mode(const trc_hip_tensor& t, int64_t rows) {
    const uintptr_t base = (uintptr_t) t.data;
    if (t.nb[0] == 4 && t.ne[0] % 4 == 0 && t.nb[1] % 16 == 0 && t.nb[2] % 16 == 0 && t.nb[3] % 16 == 0 &&
        (base & 15u) == 0)
        return K_CONTIG;
    if (t.nb[1] == 4 && rows % 4 == 0 && t.nb[0] % 16 == 0 && t.nb[2] % 16 == 0 && t.nb[3] % 16 == 0 &&
        (base & 15u) == 0)
        return R_CONTIG;
    return GENERIC;
}

template <int WI, int WJ, int TI, int TJ, int BK, int AM, int BMO, int SPLIT>
int launch_cfg(MMArgs& p, int64_t planes, hipStream_t stream) {
    constexpr int BM = WI * TI * 32, BN = WJ * TJ * 32;
    p.tiles_i = (p.M + BM - 1) / BM;
    p.tiles_j = (p.N + BN - 1) / BN;
    const int64_t grid = p.tiles_i * p.tiles_j * planes * SPLIT;
    if (grid > 0x7FFFFFFF) return fail(TRC_HIP_E_SHAPE, "mul_mat: %lld workgroups exceed one launch", (long long) grid);
    p.xcd_planes = planes % 8 == 0 ? 1 : 0;
    hipLaunchKernelGGL((k_mul_mat<WI, WJ, TI, TJ, BK, AM, BMO, SPLIT>), dim3((unsigned) grid), dim3(WI * WJ * 64), 0,
                       stream, p);
    return check_launch("mul_mat_f32");
}

template <int WI, int WJ, int TI, int TJ, int BK, int SPLIT>
int dispatch_modes(MMArgs& p, int am, int bm, int64_t planes, hipStream_t s) {
#define TRC_MM_CASE(A, B) \
    if (am == A && bm == B) return launch_cfg<WI, WJ, TI, TJ, BK, A, B, SPLIT>(p, planes, s);
    TRC_MM_CASE(K_CONTIG, K_CONTIG)
    TRC_MM_CASE(K_CONTIG, R_CONTIG)
    TRC_MM_CASE(K_CONTIG, GENERIC)
    TRC_MM_CASE(R_CONTIG, K_CONTIG)
    TRC_MM_CASE(R_CONTIG, R_CONTIG)
    TRC_MM_CASE(R_CONTIG, GENERIC)
    TRC_MM_CASE(GENERIC, K_CONTIG)
    TRC_MM_CASE(GENERIC, R_CONTIG)
    TRC_MM_CASE(GENERIC, GENERIC)
#undef TRC_MM_CASE
    return fail(TRC_HIP_E_INVALID, "mul_mat: bad load modes");
}

}  // namespace

int launch_mul_mat_f32(const trc_hip_tensor& a, const trc_hip_tensor& b, const trc_hip_tensor& d,
                       hipStream_t stream) {
    MMArgs p;
    p.a = (const uint8_t*) a.data;
    p.b = (const uint8_t*) b.data;
    p.d = (uint8_t*) d.data;
    p.K = a.ne[0];
    p.M = a.ne[1];
    p.N = b.ne[1];
    p.a_nb0 = (int64_t) a.nb[0]; p.a_nb1 = (int64_t) a.nb[1]; p.a_nb2 = (int64_t) a.nb[2]; p.a_nb3 = (int64_t) a.nb[3];
    p.a_ne2 = a.ne[2]; p.a_ne3 = a.ne[3];
    p.b_nb0 = (int64_t) b.nb[0]; p.b_nb1 = (int64_t) b.nb[1]; p.b_nb2 = (int64_t) b.nb[2]; p.b_nb3 = (int64_t) b.nb[3];
    p.b_ne2 = b.ne[2];
    p.d_nb0 = (int64_t) d.nb[0]; p.d_nb1 = (int64_t) d.nb[1]; p.d_nb2 = (int64_t) d.nb[2]; p.d_nb3 = (int64_t) d.nb[3];
    const int am = pick_mode(a, p.M);
    const int bm = pick_mode(b, p.N);
    const int64_t planes = b.ne[2] * b.ne[3];

    // Large tiles when they still give every CU at least two workgroups. With
    // between half and two tiles per CU and a long K, large tiles with K in two
    // parts (into a cleared, contiguous dst); otherwise 64x64 tiles.
    const int64_t big_tiles = ((p.M + 127) / 128) * ((p.N + 127) / 128) * planes;
    if (big_tiles >= 512) return dispatch_modes<2, 2, 2, 2, 16, 1>(p, am, bm, planes, stream);
    const bool dense_dst = p.d_nb0 == 4 && p.d_nb1 == 4 * p.M && p.d_nb2 == p.d_nb1 * p.N &&
                           p.d_nb3 == p.d_nb2 * b.ne[2];
    if (dense_dst && p.K >= 1024 && 2 * big_tiles >= device_cus()) {
        const int rc = launch_fill_f32((float*) d.data, 0.f, p.M * p.N * planes, stream);
        if (rc != TRC_HIP_OK) return rc;
        return dispatch_modes<2, 4, 2, 1, 16, 2>(p, am, bm, planes, stream);
    }
    return dispatch_modes<2, 2, 1, 1, 32, 1>(p, am, bm, planes, stream);
}

}  // namespace trc_hip
