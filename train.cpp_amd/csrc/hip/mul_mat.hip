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
//     two: 8-wave workgroups (64x32 per wave) each sum half of K for one tile.
//     The two waves that hold one 64x32 block meet in dst without a clear: each
//     takes a ticket; the first stores its sums, the second adds its own with
//     float atomics once the first's are in. a + b is the same in either order,
//     so results stay deterministic. With whole tiles and float4 loaders the
//     split products take k_mul_mat_db: two LDS slab buffers, the stores and
//     loads of the next slabs spread between the MFMAs, one barrier per slab.
//   - Up to 64 columns against a k-contiguous src0 (decode-sized batches) take
//     k_mm_skinny below instead: one pass over src0 on every CU.
#include "common.h"

#include <type_traits>

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
    int64_t d_span;  // bytes from a dst plane's first element to past its last
    uint32_t* tickets;  // K split in two: two words per wave of every tile, zero between launches
};

constexpr uint32_t MM_RSRC_WORD3 = 0x00020000u;  // gfx9 buffer resource: raw 32-bit dwords
constexpr uint32_t MM_OUT = 0x80000000u;         // an offset past the resource: loads read 0, stores drop

// Loads a ROWS x BK slab (rows = i for src0, j for src1) of one operand into
// registers, then stores it to LDS as lds[k * LD + row]. The k-contiguous
// loader gives 4 consecutive lanes the 4 float4s of 16 k of one row (64
// contiguous bytes), then the next rows, then the next 16 k, and stores each
// float4 as four floats down four k rows: a half-wave covers 4 k quads of 8
// rows, and a pitch of ROWS + 2 puts the quads 8 of the 32 banks apart, so the
// stores are conflict-free for any BK. (With 8 lanes per row at BK = 32 and a
// pitch of ROWS + 4, 20 % of the forward product's LDS cycles were
// bank-conflict stalls, and 4-way conflicts made 128 x 64 tiles at BK = 32 11 %
// slower.) The other loaders store float4s, whose rows stay 16-byte aligned.
// KI (k-contiguous only): the slab is stored as planes of k pairs, element
// (k, row) at (k / 2) * 2 * LD + 2 * row + k % 2, so one 8-byte read gives a
// lane the two k of a row that two consecutive MFMAs take from it.
template <int MODE, int ROWS, int BK, int THREADS, bool KI = false>
struct SlabLoader {
    static_assert(MODE != K_CONTIG || BK % 16 == 0, "k-contiguous slabs come in 16-k groups");
    static constexpr int LD = MODE == K_CONTIG ? ROWS + 2 : ROWS + 4;
    static constexpr int PER = ROWS * BK / THREADS;  // floats per thread
    static_assert(PER % 4 == 0, "slab must give each thread whole float4s");
    float r[PER];

    __device__ __forceinline__ void load(const uint8_t* base, int64_t nb_k, int64_t nb_r, int64_t row0,
                                         int64_t nrows, int64_t k0, int64_t K, int tid) {
        if constexpr (MODE == K_CONTIG) {
#pragma unroll
            for (int u = 0; u < PER / 4; ++u) {
                const int q = tid + THREADS * u;
                const int row = (q >> 2) % ROWS;
                const int kq = (q & 3) + 4 * (q / (4 * ROWS));
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
                const int row = (q >> 2) % ROWS;
                const int kq = (q & 3) + 4 * (q / (4 * ROWS));
                if constexpr (KI) {
                    *(float2*) (lds + (2 * kq) * 2 * LD + 2 * row) = float2{r[4 * u + 0], r[4 * u + 1]};
                    *(float2*) (lds + (2 * kq + 1) * 2 * LD + 2 * row) = float2{r[4 * u + 2], r[4 * u + 3]};
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) lds[(4 * kq + c) * LD + row] = r[4 * u + c];
                }
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

// SPLIT: parts of K (1, or 2 meeting in dst through the stream's ticket words).
// ACC: dst += the product (K in one part).
template <int WI, int WJ, int TI, int TJ, int BK, int AMODE, int BMODE, int SPLIT, bool ACC = false, bool KI = false>
__global__ __launch_bounds__(WI * WJ * 64) void k_mul_mat(MMArgs p) {
    constexpr int THREADS = WI * WJ * 64;
    static_assert(SPLIT == 1 || SPLIT == 2, "two parts at most keep the atomic sums deterministic");
    static_assert(!ACC || SPLIT == 1, "d + a + b would round differently from d + (a + b)");
    constexpr int BM = WI * TI * 32;  // tile extent along i
    constexpr int BN = WJ * TJ * 32;  // tile extent along j
    using LA = SlabLoader<AMODE, BM, BK, THREADS, KI && AMODE == K_CONTIG>;
    using LB = SlabLoader<BMODE, BN, BK, THREADS, KI && BMODE == K_CONTIG>;
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
    const int64_t tile = t;
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
        if constexpr (KI) {
            // k in groups of 4: the first MFMA of a group takes k = 4t + 2 half, the
            // second 4t + 2 half + 1, from both operands
#pragma unroll
            for (int t4 = 0; t4 < BK / 4; ++t4) {
                const int k0 = 4 * t4 + 2 * half;
                float2 av[TI], bv[TJ];
#pragma unroll
                for (int x = 0; x < TI; ++x) {
                    const int r = (wi * TI + x) * 32 + col;
                    if constexpr (AMODE == K_CONTIG) {
                        av[x] = *(const float2*) (As + (k0 >> 1) * 2 * LA::LD + 2 * r);
                    } else {
                        av[x] = float2{As[k0 * LA::LD + r], As[(k0 + 1) * LA::LD + r]};
                    }
                }
#pragma unroll
                for (int y = 0; y < TJ; ++y) {
                    const int r = (wj * TJ + y) * 32 + col;
                    if constexpr (BMODE == K_CONTIG) {
                        bv[y] = *(const float2*) (Bs + (k0 >> 1) * 2 * LB::LD + 2 * r);
                    } else {
                        bv[y] = float2{Bs[k0 * LB::LD + r], Bs[(k0 + 1) * LB::LD + r]};
                    }
                }
#pragma unroll
                for (int x = 0; x < TI; ++x)
#pragma unroll
                    for (int y = 0; y < TJ; ++y) {
                        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(bv[y].x, av[x].x, acc[x][y], 0, 0, 0);
                        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(bv[y].y, av[x].y, acc[x][y], 0, 0, 0);
                    }
            }
        } else {
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
    if constexpr (ACC) {
        // d + v, the float add acc would make with this product, one 32 x 32
        // block at a time, all 16 old values read before any store (interleaved,
        // each read would wait for the store before it: the compiler cannot tell
        // the addresses apart). Through a buffer resource over the dst plane
        // (under 2 GiB, checked on the host) the 16 addresses are one lane offset
        // plus uniform multiples of nb1, and rows or columns past dst get an
        // offset past the resource (reads 0, stores dropped), so there is no
        // branch and each block's accumulators are read only when it is stored.
        const __amdgpu_buffer_rsrc_t rd =
            __builtin_amdgcn_make_buffer_rsrc((void*) d, (short) 0, (int) p.d_span, MM_RSRC_WORD3);
#pragma unroll
        for (int x = 0; x < TI; ++x) {
            const int64_t i = i0 + (wi * TI + x) * 32 + col;
#pragma unroll
            for (int y = 0; y < TJ; ++y) {
                const int64_t jb = j0 + (wj * TJ + y) * 32 + 4 * half;
                const uint32_t vo = i < p.M ? (uint32_t) (i * p.d_nb0 + jb * p.d_nb1) : MM_OUT;
                float old[16];
                if (j0 + BN <= p.N) {  // every column of the tile exists: one offset
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const uint32_t so = (uint32_t) ((8 * (v >> 2) + (v & 3)) * p.d_nb1);
                        old[v] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rd, vo, so, 0));
                    }
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const uint32_t so = (uint32_t) ((8 * (v >> 2) + (v & 3)) * p.d_nb1);
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, old[v] + acc[x][y][v]), rd,
                                                              vo, so, 0);
                    }
                } else {  // the tile's last columns lie past dst: four at a time (fewer offsets held)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
#pragma unroll
                        for (int v = 4 * q; v < 4 * q + 4; ++v) {
                            const int c = 8 * (v >> 2) + (v & 3);
                            old[v] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                   rd, jb + c < p.N ? vo : MM_OUT, (uint32_t) (c * p.d_nb1), 0));
                        }
#pragma unroll
                        for (int v = 4 * q; v < 4 * q + 4; ++v) {
                            const int c = 8 * (v >> 2) + (v & 3);
                            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, old[v] + acc[x][y][v]),
                                                                  rd, jb + c < p.N ? vo : MM_OUT,
                                                                  (uint32_t) (c * p.d_nb1), 0);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        return;
    }
    if constexpr (SPLIT > 1) {
        // dst element of accumulator register v of tile (x, y), or null past dst
        auto out = [&](int x, int y, int v) -> float* {
            const int64_t i = i0 + (wi * TI + x) * 32 + col;
            const int64_t j = j0 + (wj * TJ + y) * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
            return i < p.M && j < p.N ? (float*) (d + i * p.d_nb0 + j * p.d_nb1) : nullptr;
        };
        // The waves holding this 64 x 32 block in the two parts meet through two
        // ticket words (ticket_first and the protocol it begins, common.h).
        // Against a cleared dst with an atomic add from each part, this leaves
        // out the clearing launch and half of the atomics (configuration 3's
        // forward and dX products 156.7 -> 150.5 and 155.6 -> 149.4 us), with
        // the same sums.
        uint32_t* tk = p.tickets + 2 * (tile * (WI * WJ) + wave);
        if (ticket_first(tk, lane)) {
#pragma unroll
            for (int x = 0; x < TI; ++x)
#pragma unroll
                for (int y = 0; y < TJ; ++y)
#pragma unroll
                    for (int v = 0; v < 16; ++v)
                        if (float* o = out(x, y, v))
                            __hip_atomic_store(o, acc[x][y][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ticket_publish(tk, lane);
            return;
        }
        ticket_wait(tk, lane);
#pragma unroll
        for (int x = 0; x < TI; ++x)
#pragma unroll
            for (int y = 0; y < TJ; ++y)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    if (float* o = out(x, y, v))
                        __hip_atomic_fetch_add(o, acc[x][y][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ticket_clear(tk, lane);
        return;
    }
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
                // Non-temporal: dst is not read again by this launch (dW 1 % and
                // configuration 4 2 % faster than plain stores).
                __builtin_nontemporal_store(acc[x][y][v], (float*) (d + i * p.d_nb0 + j * p.d_nb1));
            }
        }
    }
}

// ------------------------------------------ double-buffered slabs, whole tiles
//
// 128 x 128 tiles on 8-wave workgroups (64 x 32 per wave) when every tile and
// slab is whole (M and N multiples of 128, K of 2 slabs per part) and both
// operands load as float4s (k- or row-contiguous). k_mul_mat stores each slab
// between two barriers while no MFMA runs, with both waves of every SIMD
// waiting together; here two LDS slab buffers take turns: during the MFMAs of
// slab s the registers holding slab s + 1 are stored into the idle buffer (one
// float4 piece per group of 4 k, from group S0 on) and then refilled with slab
// s + 2 (from group L0 on), with one barrier per slab. Whole tiles need no
// bounds checks, which keeps the slab loop free of branches and selects (with
// clamped addresses and selects the split schedule measured 157-160 us, slower
// than k_mul_mat). Both operands are read as k-paired LDS planes where they are
// k-contiguous, so the MFMAs take k in groups of 4 (k = 4t + 2 half, then
// 4t + 2 half + 1). Two uses (interleaved minimums, one box, configuration 3 /
// 4):
//   - K split in two (DbPlan<2, ...>: 32-deep slabs, default priority), the
//     parts meeting in dst through the stream's ticket words as in k_mul_mat:
//     forward 149.5 -> 137.4 us (its sums now group k by pairs, within 6e-5 of
//     281), dX 148.8 -> 146.0 us (same bits);
//   - K whole (DbPlan<1, ...>: 16-deep slabs, two workgroups per CU, the MFMA-block
//     priority of k_mul_mat): dW 135.3 -> 129.7 us, configuration 4 158.5 ->
//     147.2 us; ACC adds the product into dst as k_mul_mat's ACC does.
constexpr int DB_WI = 2, DB_WJ = 4, DB_TI = 2, DB_TJ = 1;
constexpr int DB_THREADS = DB_WI * DB_WJ * 64;
constexpr int DB_BM = DB_WI * DB_TI * 32, DB_BN = DB_WJ * DB_TJ * 32;
// slab depth, the group of 4 k from which a slab's pieces are stored (S0) and
// the next slab's loaded (L0), and the MFMA-block priority, per number of K
// parts and src0 layout. Measured on configuration 3 (µs): the forward product
// (k-contiguous src0) 140.0 with S0 = 1, 137.3-137.5 with S0 = 0 and L0 = 1..4;
// dX (row-contiguous src0) 146.0-146.2 with S0 = 1 and L0 = 3..4, 146.9-149.9
// with S0 = 0 or 2; the priority made both slower (141.0, 153.3), 64-deep slabs
// changed them by under 1 %.
template <int SPLIT, int AMODE>
struct DbPlan;
template <int AMODE>
struct DbPlan<2, AMODE> {
    static constexpr int BK = 32, S0 = AMODE == K_CONTIG ? 0 : 1, L0 = AMODE == K_CONTIG ? 2 : 4;
    static constexpr bool PRIO = false;
};
template <int AMODE>
struct DbPlan<1, AMODE> {
    static constexpr int BK = 16, S0 = 0, L0 = 1;
    static constexpr bool PRIO = true;
};

// One operand's slab as NU float4 pieces per thread: the K_CONTIG mapping of
// SlabLoader (4 lanes per 64 contiguous bytes of a row, then rows, then k) with
// k-paired planes, or the R_CONTIG one (float4s along the rows of one k).
template <int MODE, int ROWS, int BK>
struct SlabPieces {
    static_assert(MODE != K_CONTIG || BK % 16 == 0, "k-contiguous pieces come in 16-k groups");
    static_assert(ROWS * BK % (DB_THREADS * 4) == 0, "whole float4 pieces per thread");
    static constexpr int LD = MODE == K_CONTIG ? ROWS + 2 : ROWS + 4;
    static constexpr int NU = ROWS * BK / DB_THREADS / 4;
    static constexpr int SZ = BK * LD;
    const uint8_t* src[NU];  // piece u of the part's first slab
    int lo[NU];              // its LDS float offset
    int64_t step;            // bytes from one slab to the next
    f4 r[NU];

    __device__ __forceinline__ void init(const uint8_t* base, int64_t nb_k, int64_t nb_r, int64_t row0, int64_t k0,
                                         int tid) {
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int q = tid + DB_THREADS * u;
            if constexpr (MODE == K_CONTIG) {
                const int row = (q >> 2) % ROWS, kq = (q & 3) + 4 * (q / (4 * ROWS));
                src[u] = base + (row0 + row) * nb_r + (k0 + 4 * kq) * 4;
                lo[u] = (2 * kq) * 2 * LD + 2 * row;
            } else {
                const int k = q / (ROWS / 4), rq = q % (ROWS / 4);
                src[u] = base + (row0 + 4 * rq) * 4 + (k0 + k) * nb_k;
                lo[u] = k * LD + 4 * rq;
            }
        }
        step = MODE == K_CONTIG ? (int64_t) BK * 4 : (int64_t) BK * nb_k;
    }
    __device__ __forceinline__ void load(int64_t s, int u) { r[u] = *(const f4*) (src[u] + s * step); }
    __device__ __forceinline__ void store(float* l, int u) const {
        if constexpr (MODE == K_CONTIG) {
            *(float2*) (l + lo[u]) = float2{r[u].x, r[u].y};
            *(float2*) (l + lo[u] + 2 * LD) = float2{r[u].z, r[u].w};
        } else {
            *(f4*) (l + lo[u]) = r[u];
        }
    }
    // the k pair (k0, k0 + 1) of row r, k0 even
    __device__ __forceinline__ static float2 pair(const float* l, int k0, int r) {
        if constexpr (MODE == K_CONTIG) return *(const float2*) (l + (k0 >> 1) * 2 * LD + 2 * r);
        else return float2{l[k0 * LD + r], l[(k0 + 1) * LD + r]};
    }
};

template <int AMODE, int BMODE, int SPLIT, bool ACC = false>
__global__ __launch_bounds__(DB_THREADS) void k_mul_mat_db(MMArgs p) {
    using PL = DbPlan<SPLIT, AMODE>;
    constexpr int BK = PL::BK;
    using PA = SlabPieces<AMODE, DB_BM, BK>;
    using PB = SlabPieces<BMODE, DB_BN, BK>;
    constexpr int NU = PA::NU + PB::NU;
    static_assert(!ACC || SPLIT == 1, "d + a + b would round differently from d + (a + b)");
    static_assert(PL::L0 >= PL::S0, "a piece's registers are stored before the load of the slab after refills them");
    static_assert(PL::S0 + NU <= BK / 4 && PL::L0 + NU <= BK / 4, "every piece is placed within the slab's k groups");
    __shared__ __attribute__((aligned(16))) float As[2][PA::SZ];
    __shared__ __attribute__((aligned(16))) float Bs[2][PB::SZ];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wi = wave % DB_WI, wj = wave / DB_WI;
    const int half = lane >> 5, col = lane & 31;

    int64_t t = blockIdx.x;
    if (p.xcd_planes) {
        const int64_t tpp = p.tiles_i * p.tiles_j * SPLIT, x = t & 7, k = t >> 3;
        t = (8 * (k / tpp) + x) * tpp + k % tpp;
    }
    const int part = SPLIT > 1 ? (int) (t % SPLIT) : 0;
    t /= SPLIT;
    const int64_t tile = t;
    const int64_t ti = t % p.tiles_i;
    t /= p.tiles_i;
    const int64_t tj = t % p.tiles_j;
    const int64_t plane = t / p.tiles_j;
    const int64_t i2 = plane % p.b_ne2, i3 = plane / p.b_ne2;
    const uint8_t* a = p.a + (i2 % p.a_ne2) * p.a_nb2 + (i3 % p.a_ne3) * p.a_nb3;
    const uint8_t* b = p.b + i2 * p.b_nb2 + i3 * p.b_nb3;
    uint8_t* d = p.d + i2 * p.d_nb2 + i3 * p.d_nb3;
    const int64_t i0 = ti * DB_BM, j0 = tj * DB_BN;
    const int64_t nk = p.K / BK / SPLIT;  // slabs per part (at least 2)
    PA pa;
    PB pb;
    pa.init(a, p.a_nb0, p.a_nb1, i0, part * nk * BK, tid);
    pb.init(b, p.b_nb0, p.b_nb1, j0, part * nk * BK, tid);
    auto gload = [&](int64_t s, int u) {
        if (u < PA::NU) pa.load(s, u);
        else pb.load(s, u - PA::NU);
    };
    auto lstore = [&](int buf, int u) {
        if (u < PA::NU) pa.store(As[buf], u);
        else pb.store(Bs[buf], u - PA::NU);
    };

    f16v acc[DB_TI][DB_TJ];
#pragma unroll
    for (int x = 0; x < DB_TI; ++x)
#pragma unroll
        for (int y = 0; y < DB_TJ; ++y)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[x][y][v] = 0.f;
    // slab 0 into buffer 0, slab 1 into the registers
#pragma unroll
    for (int u = 0; u < NU; ++u) gload(0, u);
#pragma unroll
    for (int u = 0; u < NU; ++u) lstore(0, u);
#pragma unroll
    for (int u = 0; u < NU; ++u) gload(1, u);
    __syncthreads();

    // slab kt from buffer kt % 2; STORE: the registers (slab kt + 1) go to the
    // other buffer; LOAD: slab kt + 2 refills them. Compile-time flags keep the
    // k loop one branch-free block.
    auto slab = [&](int64_t kt, auto store_next, auto load_after) {
        constexpr bool STORE = decltype(store_next)::value, LOAD = decltype(load_after)::value;
        const int cur = (int) (kt & 1);
        const float* ac = As[cur];
        const float* bc = Bs[cur];
        if constexpr (PL::PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int t4 = 0; t4 < BK / 4; ++t4) {
            const int k0 = 4 * t4 + 2 * half;
            float2 av[DB_TI], bv[DB_TJ];
#pragma unroll
            for (int x = 0; x < DB_TI; ++x) av[x] = PA::pair(ac, k0, (wi * DB_TI + x) * 32 + col);
#pragma unroll
            for (int y = 0; y < DB_TJ; ++y) bv[y] = PB::pair(bc, k0, (wj * DB_TJ + y) * 32 + col);
#pragma unroll
            for (int x = 0; x < DB_TI; ++x)
#pragma unroll
                for (int y = 0; y < DB_TJ; ++y) {
                    acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(bv[y].x, av[x].x, acc[x][y], 0, 0, 0);
                    acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(bv[y].y, av[x].y, acc[x][y], 0, 0, 0);
                }
            if constexpr (STORE) {
                if (t4 >= PL::S0 && t4 < PL::S0 + NU) lstore(cur ^ 1, t4 - PL::S0);
            }
            if constexpr (LOAD) {
                if (t4 >= PL::L0 && t4 < PL::L0 + NU) gload(kt + 2, t4 - PL::L0);
            }
        }
        if constexpr (PL::PRIO) __builtin_amdgcn_s_setprio(0);
        __syncthreads();
    };
    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
    // (nk >= 2 here; the guards also give the compiler the block layout that
    // measured 146 us for dX against 149 us without them, the loop unchanged)
    for (int64_t kt = 0; kt + 2 < nk; ++kt) slab(kt, yes{}, yes{});
    if (nk >= 2) slab(nk - 2, yes{}, no{});
    if (nk >= 1) slab(nk - 1, no{}, no{});

    // accumulator register v of tile (x, y) holds dst row i = i0 + (wi TI + x) 32
    // + col and column j = j0 + (wj TJ + y) 32 + 8 (v / 4) + 4 half + v % 4
    auto out = [&](int x, int y, int v) -> float* {
        const int64_t i = i0 + (wi * DB_TI + x) * 32 + col;
        const int64_t j = j0 + (wj * DB_TJ + y) * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
        return i < p.M && j < p.N ? (float*) (d + i * p.d_nb0 + j * p.d_nb1) : nullptr;
    };
    if constexpr (SPLIT > 1) {
        // the parts meet in dst (ticket_first and the protocol it begins, common.h)
        uint32_t* tk = p.tickets + 2 * (tile * (DB_WI * DB_WJ) + wave);
        if (ticket_first(tk, lane)) {
#pragma unroll
            for (int x = 0; x < DB_TI; ++x)
#pragma unroll
                for (int y = 0; y < DB_TJ; ++y)
#pragma unroll
                    for (int v = 0; v < 16; ++v)
                        if (float* o = out(x, y, v))
                            __hip_atomic_store(o, acc[x][y][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ticket_publish(tk, lane);
            return;
        }
        ticket_wait(tk, lane);
#pragma unroll
        for (int x = 0; x < DB_TI; ++x)
#pragma unroll
            for (int y = 0; y < DB_TJ; ++y)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    if (float* o = out(x, y, v))
                        __hip_atomic_fetch_add(o, acc[x][y][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ticket_clear(tk, lane);
    } else if constexpr (ACC) {
        // d + v, one 32 x 32 block at a time with its 16 old values read before
        // any store, through a buffer resource over the dst plane (as k_mul_mat's
        // ACC epilogue; the tile is whole, so one lane offset and uniform
        // multiples of nb1 address all 16)
        const __amdgpu_buffer_rsrc_t rd =
            __builtin_amdgcn_make_buffer_rsrc((void*) d, (short) 0, (int) p.d_span, MM_RSRC_WORD3);
#pragma unroll
        for (int x = 0; x < DB_TI; ++x) {
            const int64_t i = i0 + (wi * DB_TI + x) * 32 + col;
#pragma unroll
            for (int y = 0; y < DB_TJ; ++y) {
                const int64_t jb = j0 + (wj * DB_TJ + y) * 32 + 4 * half;
                const uint32_t vo = (uint32_t) (i * p.d_nb0 + jb * p.d_nb1);
                float old[16];
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const uint32_t so = (uint32_t) ((8 * (v >> 2) + (v & 3)) * p.d_nb1);
                    old[v] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rd, vo, so, 0));
                }
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const uint32_t so = (uint32_t) ((8 * (v >> 2) + (v & 3)) * p.d_nb1);
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, old[v] + acc[x][y][v]), rd, vo,
                                                          so, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        // non-temporal: dst is not read again by this launch. The tile is
        // whole, so no element needs a bounds check; with out()'s check (and
        // its branches) dW took 145-148 us instead of 131
#pragma unroll
        for (int x = 0; x < DB_TI; ++x)
#pragma unroll
            for (int y = 0; y < DB_TJ; ++y)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int64_t i = i0 + (wi * DB_TI + x) * 32 + col;
                    const int64_t j = j0 + (wj * DB_TJ + y) * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                    __builtin_nontemporal_store(acc[x][y][v], (float*) (d + i * p.d_nb0 + j * p.d_nb1));
                }
    }
}

// Launches k_mul_mat_db when the shape fits it (whole tiles and slabs, float4
// loaders, the K parts' ticket words in p.tickets when SPLIT is 2); returns
// -1 (launching nothing) otherwise.
template <int SPLIT, bool ACC>
int launch_db(MMArgs& p, int am, int bm, int64_t planes, hipStream_t stream) {
    static_assert(DbPlan<SPLIT, K_CONTIG>::BK == DbPlan<SPLIT, R_CONTIG>::BK, "one slab depth per K split");
    constexpr int BK = DbPlan<SPLIT, K_CONTIG>::BK;
    if (p.M % DB_BM != 0 || p.N % DB_BN != 0 || p.K % (2 * BK * SPLIT) != 0 || am == GENERIC || bm == GENERIC)
        return -1;
    p.tiles_i = p.M / DB_BM;
    p.tiles_j = p.N / DB_BN;
    p.xcd_planes = planes % 8 == 0 ? 1 : 0;
    p.d_span = (p.M - 1) * p.d_nb0 + (p.N - 1) * p.d_nb1 + 4;
    const int64_t grid = p.tiles_i * p.tiles_j * planes * SPLIT;
    if (grid > 0x7FFFFFFF) return fail(TRC_HIP_E_SHAPE, "mul_mat: %lld workgroups exceed one launch", (long long) grid);
#define TRC_MM_DB(A, B) \
    if (am == A && bm == B) \
        hipLaunchKernelGGL((k_mul_mat_db<A, B, SPLIT, ACC>), dim3((unsigned) grid), dim3(DB_THREADS), 0, stream, p);
    TRC_MM_DB(K_CONTIG, K_CONTIG)
    TRC_MM_DB(K_CONTIG, R_CONTIG)
    TRC_MM_DB(R_CONTIG, K_CONTIG)
    TRC_MM_DB(R_CONTIG, R_CONTIG)
#undef TRC_MM_DB
    return check_launch("mul_mat_f32 (double-buffered slabs)");
}

// ---------------------------------------------------------------- few columns
//
// dst = W . X with N <= 64 columns and W k-contiguous (the weight of a Linear
// layer run at decode batch, e.g. the F32 weight a GGUF warm start produces,
// src/io/trc_gguf.cpp:1082-1088, times 8 activation columns): W is read from
// HBM once, so the product is bound by W's bytes, not by MFMA work.
//   - One workgroup per 16 rows of W (one row block of one plane) and all of K;
//     its SK_WAVES waves take the 32-wide k chunks in turn (chunk c to wave
//     c % SK_WAVES), so every wave streams its own part of the 16 rows. Row
//     block rb starts at chunk 37 rb (mod the chunk count), so the workgroups
//     in flight read different offsets of their rows (rows 16 KiB apart would
//     otherwise all start on the same offset: 4 % faster on configuration 0).
//   - Lane l reads row l % 16 of the block at k = 32c + 4g .. +3 and
//     32c + 16 + 4g .. +3 (g = l / 16): two float4 loads, 64 contiguous bytes
//     per row and instruction. It reads X column 16t + l % 16 at the same k.
//   - With 5 to 8 k-contiguous columns, those X loads would fetch half lines for
//     16 column slots, half of them empty. One load of 8 columns x 32 k (full
//     128-byte lines; lane 8j + q holds column j at k = 32c + 4q) replaces
//     the two, and ds_bpermute moves each float to the lane the MFMA wants it
//     in. The texture path's load count per chunk drops from 4 to 3; cfg0's
//     N = 8 product went from 16.2 to 15.2 us.
//   - v_mfma_f32_16x16x4_f32 with X as the A operand (MFMA row = column j of X)
//     and W as the B operand (MFMA column = row i of W); A and B take the same
//     k from the same lane, so any k order within a chunk gives the same dot.
//     Accumulator register v of lane l then holds dst row i = l % 16, column
//     j = 16t + 4 (l / 16) + v.
//   - Loads go through buffer resources (16 rows of W, one plane of X): an
//     element outside the operands gets an offset past its resource, which the
//     hardware reads as 0. No branch or select waits on a load, so AHEAD chunks
//     per wave stay in flight ahead of the MFMAs (the loads for chunk n + AHEAD
//     are issued once chunk n's registers are consumed).
//   - The waves' partial sums meet in LDS and are added in wave order
//     (0 + w0 + w1 + ...), so results do not depend on timing.

struct SkArgs {
    const uint8_t* a;
    const uint8_t* b;
    uint8_t* d;
    int64_t K, M, N;
    int64_t a_nb1, a_nb2, a_nb3, a_ne2, a_ne3;
    int64_t b_nb0, b_nb1, b_nb2, b_nb3, b_ne2;
    int64_t d_nb0, d_nb1, d_nb2, d_nb3;
    int64_t row_blocks;  // ceil(M / 16)
    int64_t x_span;      // bytes from one X plane's first element to past its last
    int chunks;          // ceil(K / 32)
    int accumulate;      // 1: dst += the product
};

constexpr int SK_WAVES = 16;
constexpr int SK_MAX_N = 64;
constexpr uint32_t SK_RSRC_WORD3 = 0x00020000u;  // gfx9 buffer resource: raw 32-bit dwords
constexpr uint32_t SK_OUT = 0x80000000u;         // an offset past every resource: the load returns 0
constexpr int SK_X8 = 3;                          // X mode: k-contiguous, at most 8 columns
typedef int i4 __attribute__((ext_vector_type(4)));

// One chunk's operands in registers: W (two float4) and X (two float4 per
// 16-column group).
template <int NT>
struct SkChunk {
    f4 w0, w1;
    f4 x0[NT], x1[NT];
};

// Loads this wave's n-th chunk (chunk index wave + SK_WAVES * n, rotated by rot).
template <int NT, int BMODE>
__device__ __forceinline__ void sk_load(SkChunk<NT>& c, __amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rx,
                                        uint32_t wrow_off, const SkArgs& p, int wave, int n, int mine, int g, int r,
                                        int rot) {
    const bool chunk_ok = n < mine;
    int chunk = wave + SK_WAVES * n + rot;
    chunk = chunk >= p.chunks ? chunk - p.chunks : chunk;
    const int k0 = chunk * 32 + 4 * g;
    const int k1 = k0 + 16;
    // K % 4 == 0 on this path: a float4 is wholly inside K or wholly past it
    const bool ok0 = chunk_ok && k0 < p.K, ok1 = chunk_ok && k1 < p.K;
    // rows past M lie past rw's range by construction
    c.w0 = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rw, ok0 ? wrow_off + 4u * k0 : SK_OUT, 0, 0));
    c.w1 = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rw, ok1 ? wrow_off + 4u * k1 : SK_OUT, 0, 0));
    if constexpr (BMODE == SK_X8) {
        // up to 8 columns: one load of 8 columns x 32 k, full 128-byte lines; lane
        // 8c + q holds column c at k = 32 chunk + 4q .. +3 (sk_mfma moves it into place)
        const int xl = 16 * g + r;
        const int xc = xl >> 3;
        const int kx = chunk * 32 + 4 * (xl & 7);
        const bool cx = chunk_ok && xc < p.N && kx < p.K;
        const uint32_t off = (uint32_t) xc * (uint32_t) p.b_nb1 + 4u * (uint32_t) kx;
        c.x0[0] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rx, cx ? off : SK_OUT, 0, 0));
        return;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int j = 16 * t + r;
        const bool c0 = ok0 && j < p.N, c1 = ok1 && j < p.N;
        const uint32_t col = (uint32_t) j * (uint32_t) p.b_nb1;
        if constexpr (BMODE == K_CONTIG) {
            c.x0[t] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rx, c0 ? col + 4u * k0 : SK_OUT, 0, 0));
            c.x1[t] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rx, c1 ? col + 4u * k1 : SK_OUT, 0, 0));
        } else {
            const uint32_t nb0 = (uint32_t) p.b_nb0;
            const uint32_t o0 = c0 ? col + nb0 * (uint32_t) k0 : SK_OUT;
            const uint32_t o1 = c1 ? col + nb0 * (uint32_t) k1 : SK_OUT;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                c.x0[t][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, c0 ? o0 + nb0 * e : SK_OUT, 0, 0));
                c.x1[t][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, c1 ? o1 + nb0 * e : SK_OUT, 0, 0));
            }
        }
    }
}

template <int NT, int BMODE>
__device__ __forceinline__ void sk_mfma(const SkChunk<NT>& c, f4 (&acc)[NT], int r, int g) {
    if constexpr (BMODE == SK_X8) {
        // lane (r, g) takes column r % 8 at k = 32 chunk + 4g (+16) from the lane that
        // loaded it. MFMA rows 8..15 get copies of rows 0..7: they only reach output
        // columns 8..15, which do not exist here and are never stored.
        const int src0 = 4 * (8 * (r & 7) + g), src1 = src0 + 16;
        // (the whole vector is cast: clang's __builtin_bit_cast of one element of a
        // vector type reads element 0 whatever the index)
        const i4 xi = __builtin_bit_cast(i4, c.x0[0]);
        f4 a0, a1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            a0[e] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src0, xi[e]));
            a1[e] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src1, xi[e]));
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[s], c.w0[s], acc[0], 0, 0, 0);
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[s], c.w1[s], acc[0], 0, 0, 0);
        return;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(c.x0[t][s], c.w0[s], acc[t], 0, 0, 0);
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(c.x1[t][s], c.w1[s], acc[t], 0, 0, 0);
    }
}

template <int NT, int AHEAD, int BMODE>
__global__ __launch_bounds__(SK_WAVES * 64) void k_mm_skinny(SkArgs p) {
    __shared__ float red[SK_WAVES * NT * 4 * 64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar branches and offsets
    const int r = lane & 15, g = lane >> 4;

    const int64_t rb = blockIdx.x % p.row_blocks;
    const int64_t plane = blockIdx.x / p.row_blocks;
    const int64_t i2 = plane % p.b_ne2;
    const int64_t i3 = plane / p.b_ne2;
    const uint8_t* aplane = p.a + (i2 % p.a_ne2) * p.a_nb2 + (i3 % p.a_ne3) * p.a_nb3;
    const uint8_t* bplane = p.b + i2 * p.b_nb2 + i3 * p.b_nb3;

    // W rows rb*16 .. of this plane up to the last valid byte of the last valid row;
    // X of this plane up to its last element (spans checked below 2^31 on the host)
    const int64_t rows = p.M - rb * 16 < 16 ? p.M - rb * 16 : 16;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void*) (aplane + rb * 16 * p.a_nb1), (short) 0, (int) ((rows - 1) * p.a_nb1 + p.K * 4), SK_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void*) bplane, (short) 0, (int) p.x_span, SK_RSRC_WORD3);
    const uint32_t wrow_off = (uint32_t) r * (uint32_t) p.a_nb1;

    f4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = (f4){0.f, 0.f, 0.f, 0.f};

    // this wave's chunks: wave, wave + SK_WAVES, ... (mine of them). The last
    // batch of AHEAD chunks runs after the loop, with no loads behind it; chunks
    // past `mine` in it were loaded as zeros.
    const int mine = wave < p.chunks ? (p.chunks - 1 - wave) / SK_WAVES + 1 : 0;
    const int rot = (int) ((rb * 37) % p.chunks);
    SkChunk<NT> buf[AHEAD];
#pragma unroll
    for (int u = 0; u < AHEAD; ++u) sk_load<NT, BMODE>(buf[u], rw, rx, wrow_off, p, wave, u, mine, g, r, rot);
    int n0 = 0;
    for (; n0 + AHEAD < mine; n0 += AHEAD) {
#pragma unroll
        for (int u = 0; u < AHEAD; ++u) {
            // a wave with a chunk's MFMAs to issue goes first (W [4096, 11008]^T
            // times 8 columns 3 % faster, other shapes 0-1 %; same bits)
            __builtin_amdgcn_s_setprio(1);
            sk_mfma<NT, BMODE>(buf[u], acc, r, g);
            __builtin_amdgcn_s_setprio(0);
            sk_load<NT, BMODE>(buf[u], rw, rx, wrow_off, p, wave, n0 + AHEAD + u, mine, g, r, rot);
            // with the 8-column X loads the scheduler otherwise sinks the whole
            // batch of refills below the last chunk's wait (1 us slower)
            if constexpr (BMODE == SK_X8) __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int u = 0; u < AHEAD; ++u) sk_mfma<NT, BMODE>(buf[u], acc, r, g);

    // partial sums of every wave, then the sum over waves in wave order
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[(wave * NT * 4 + t * 4 + v) * 64 + lane] = acc[t][v];
    __syncthreads();
    for (int e = threadIdx.x; e < NT * 4 * 64; e += SK_WAVES * 64) {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < SK_WAVES; ++w) s += red[w * NT * 4 * 64 + e];
        const int el = e & 63, tv = e >> 6;  // tv = 4t + v
        const int64_t j = 16 * (tv >> 2) + 4 * (el >> 4) + (tv & 3);
        const int64_t di = rb * 16 + (el & 15);
        if (di < p.M && j < p.N) {
            float* dst = (float*) (p.d + i2 * p.d_nb2 + i3 * p.d_nb3 + di * p.d_nb0 + j * p.d_nb1);
            *dst = p.accumulate ? *dst + s : s;
        }
    }
}

template <int NT, int AHEAD>
int launch_skinny_nt(SkArgs& p, int bmode, int64_t planes, hipStream_t stream) {
    const int64_t grid = p.row_blocks * planes;
    if (grid > 0x7FFFFFFF) return fail(TRC_HIP_E_SHAPE, "mul_mat: %lld workgroups exceed one launch", (long long) grid);
    if (NT == 1 && bmode == K_CONTIG && p.N > 4 && p.N <= 8) {
        // 5..8 columns: X in full lines (at 4 or fewer the 16-column loads are as fast)
        hipLaunchKernelGGL((k_mm_skinny<1, AHEAD, SK_X8>), dim3((unsigned) grid), dim3(SK_WAVES * 64), 0, stream, p);
    } else if (bmode == K_CONTIG) {
        hipLaunchKernelGGL((k_mm_skinny<NT, AHEAD, K_CONTIG>), dim3((unsigned) grid), dim3(SK_WAVES * 64), 0, stream, p);
    } else {
        // element-by-element X loads hold more addresses: half as many chunks ahead
        constexpr int GA = AHEAD > 1 ? AHEAD / 2 : 1;
        hipLaunchKernelGGL((k_mm_skinny<NT, GA, GENERIC>), dim3((unsigned) grid), dim3(SK_WAVES * 64), 0, stream, p);
    }
    return check_launch("mul_mat_f32 (few columns)");
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

template <int WI, int WJ, int TI, int TJ, int BK, int AM, int BMO, int SPLIT, bool ACC, bool KI = false>
int launch_cfg(MMArgs& p, int64_t planes, hipStream_t stream) {
    constexpr int BM = WI * TI * 32, BN = WJ * TJ * 32;
    p.tiles_i = (p.M + BM - 1) / BM;
    p.tiles_j = (p.N + BN - 1) / BN;
    const int64_t grid = p.tiles_i * p.tiles_j * planes * SPLIT;
    if (grid > 0x7FFFFFFF) return fail(TRC_HIP_E_SHAPE, "mul_mat: %lld workgroups exceed one launch", (long long) grid);
    p.xcd_planes = planes % 8 == 0 ? 1 : 0;
    p.d_span = (p.M - 1) * p.d_nb0 + (p.N - 1) * p.d_nb1 + 4;
    hipLaunchKernelGGL((k_mul_mat<WI, WJ, TI, TJ, BK, AM, BMO, SPLIT, ACC, KI>), dim3((unsigned) grid),
                       dim3(WI * WJ * 64), 0, stream, p);
    return check_launch("mul_mat_f32");
}

template <int WI, int WJ, int TI, int TJ, int BK, int SPLIT, bool ACC = false>
int dispatch_modes(MMArgs& p, int am, int bm, int64_t planes, hipStream_t s) {
#define TRC_MM_CASE(A, B) \
    if (am == A && bm == B) return launch_cfg<WI, WJ, TI, TJ, BK, A, B, SPLIT, ACC>(p, planes, s);
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
                       hipStream_t stream, bool accumulate) {
    MMArgs p;
    p.tickets = nullptr;
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

    // Up to 64 columns against a k-contiguous W: one pass over W on every CU.
    // Its loads address 16 rows of W and one plane of X through 32-bit offsets.
    const int64_t x_span = (p.N - 1) * p.b_nb1 + (p.K - 1) * p.b_nb0 + 4;
    if (p.N <= SK_MAX_N && am == K_CONTIG && 16 * p.a_nb1 + 4 * p.K < ((int64_t) 1 << 31) &&
        x_span < ((int64_t) 1 << 31) && p.b_nb0 < ((int64_t) 1 << 31) && p.b_nb1 < ((int64_t) 1 << 31) &&
        (p.K + 31) / 32 < ((int64_t) 1 << 26)) {
        SkArgs s;
        s.a = p.a; s.b = p.b; s.d = p.d;
        s.K = p.K; s.M = p.M; s.N = p.N;
        s.a_nb1 = p.a_nb1; s.a_nb2 = p.a_nb2; s.a_nb3 = p.a_nb3; s.a_ne2 = p.a_ne2; s.a_ne3 = p.a_ne3;
        s.b_nb0 = p.b_nb0; s.b_nb1 = p.b_nb1; s.b_nb2 = p.b_nb2; s.b_nb3 = p.b_nb3; s.b_ne2 = p.b_ne2;
        s.d_nb0 = p.d_nb0; s.d_nb1 = p.d_nb1; s.d_nb2 = p.d_nb2; s.d_nb3 = p.d_nb3;
        s.accumulate = accumulate ? 1 : 0;
        s.row_blocks = (p.M + 15) / 16;
        s.x_span = x_span;
        s.chunks = (int) ((p.K + 31) / 32);
        // K_CONTIG operands are 16-byte aligned with K % 4 == 0; anything else is read element by element
        const int sbm = bm == K_CONTIG ? K_CONTIG : GENERIC;
        if (p.N <= 16) return launch_skinny_nt<1, 4>(s, sbm, planes, stream);
        if (p.N <= 32) return launch_skinny_nt<2, 2>(s, sbm, planes, stream);
        if (p.N <= 48) return launch_skinny_nt<3, 2>(s, sbm, planes, stream);
        return launch_skinny_nt<4, 1>(s, sbm, planes, stream);
    }

    // Large tiles when they still give every CU at least two workgroups. With
    // between half and two tiles per CU and a long K, large tiles with K in two
    // parts (into a contiguous dst; the parts meet through ticket words in the
    // stream's workspace); otherwise 64x64 tiles.
    const int64_t big_tiles = ((p.M + 127) / 128) * ((p.N + 127) / 128) * planes;
    if (accumulate) {
        // K stays in one part: the large tiles when they fill the CUs twice
        // (double-buffered when whole), else 64 x 64
        if (big_tiles >= 512) {
            const int drc = launch_db<1, true>(p, am, bm, planes, stream);
            if (drc >= 0) return drc;
            return dispatch_modes<2, 2, 2, 2, 16, 1, true>(p, am, bm, planes, stream);
        }
        return dispatch_modes<2, 2, 1, 1, 32, 1, true>(p, am, bm, planes, stream);
    }
    if (big_tiles >= 512) {
        const int drc = launch_db<1, false>(p, am, bm, planes, stream);
        if (drc >= 0) return drc;
        return dispatch_modes<2, 2, 2, 2, 16, 1>(p, am, bm, planes, stream);
    }
    const bool dense_dst = p.d_nb0 == 4 && p.d_nb1 == 4 * p.M && p.d_nb2 == p.d_nb1 * p.N &&
                           p.d_nb3 == p.d_nb2 * b.ne[2];
    if (dense_dst && p.K >= 1024 && 2 * big_tiles >= device_cus()) {
        static_assert(511 * 8 * 2 <= MM_TICKETS, "two ticket words per wave of under 512 tiles");
        const int rc = mm_stream_tickets(stream, &p.tickets);
        if (rc != TRC_HIP_OK) return rc;
        // whole tiles and slabs with float4 loaders: double-buffered slabs
        const int drc = launch_db<2, false>(p, am, bm, planes, stream);
        if (drc >= 0) return drc;
        // a transposed src0 against a k-contiguous src1 (the dX product of a
        // Linear layer): k-paired LDS planes for src1, 4 % faster there; 1.5 %
        // slower with both operands k-contiguous (the forward product)
        if (am == R_CONTIG && bm == K_CONTIG) {
            return launch_cfg<2, 4, 2, 1, 32, R_CONTIG, K_CONTIG, 2, false, true>(p, planes, stream);
        }
        return dispatch_modes<2, 4, 2, 1, 32, 2>(p, am, bm, planes, stream);
    }
    return dispatch_modes<2, 2, 1, 1, 32, 1>(p, am, bm, planes, stream);
}

}  // namespace trc_hip
