// F32 element-wise graph ops that a Linear layer's forward and autograd
// backward put around mul_mat on the device: ADD and MUL with ggml broadcast,
// ACC into a strided region, REPEAT_BACK, REPEAT, and SUM (the scalar loss).
// Each output element is produced by the same single float operation, or the
// same ordered sum, as the reference CPU kernels, so the results are
// bit-identical:
//   add, mul     src/ops/trc_ops.cpp:19-32,46,59; compute_binary
//                src/backends/cpu/trc_cpu_ops.cpp:52-78 (offset_broadcast :18-28)
//   acc          src/core/trc_tensor.cpp:322-361; compute_acc trc_cpu_ops.cpp:954-999
//   repeat_back  src/ops/trc_ops.cpp:458-470; compute_repeat_back trc_cpu_ops.cpp:932-952
//   repeat       src/ops/trc_ops.cpp:447-456; compute_repeat trc_cpu_ops.cpp:913-928
//   sum          src/ops/trc_ops.cpp:214-221; compute_sum trc_cpu_ops.cpp:302-315
//                (row_sum_f32 :284-300)
//
// Mapping: one workgroup row-loop per ggml row (ne0-run); lanes stride over the
// row, so loads and stores along ne0 are coalesced whenever nb0 == 4.
#include "common.h"

namespace trc_hip {
namespace {

constexpr int EW_THREADS = 256;

struct Shape4 {
    int64_t ne[4];
    int64_t nb[4];  // bytes
};

Shape4 shape_of(const trc_hip_tensor& t) {
    Shape4 s;
    for (int d = 0; d < 4; ++d) {
        s.ne[d] = t.ne[d];
        s.nb[d] = (int64_t) t.nb[d];
    }
    return s;
}

enum class BinOp { ADD, MUL };

// dst[i] = a[i] (+ or *) b[broadcast(i)], rows of dst distributed over the grid
template <BinOp OP>
__global__ __launch_bounds__(EW_THREADS) void k_binary(const uint8_t* __restrict__ a, Shape4 sa,
                                                       const uint8_t* __restrict__ b, Shape4 sb,
                                                       uint8_t* __restrict__ d, Shape4 sd) {
    const int64_t rows = sd.ne[1] * sd.ne[2] * sd.ne[3];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const int64_t i1 = r % sd.ne[1], i2 = (r / sd.ne[1]) % sd.ne[2], i3 = r / (sd.ne[1] * sd.ne[2]);
        const uint8_t* pa = a + i1 * sa.nb[1] + i2 * sa.nb[2] + i3 * sa.nb[3];
        const uint8_t* pb = b + (sb.ne[1] == 1 ? 0 : i1 * sb.nb[1]) + (sb.ne[2] == 1 ? 0 : i2 * sb.nb[2]) +
                            (sb.ne[3] == 1 ? 0 : i3 * sb.nb[3]);
        uint8_t* pd = d + i1 * sd.nb[1] + i2 * sd.nb[2] + i3 * sd.nb[3];
        const int64_t bnb0 = sb.ne[0] == 1 ? 0 : sb.nb[0];
        for (int64_t i0 = threadIdx.x; i0 < sd.ne[0]; i0 += EW_THREADS) {
            const float va = *(const float*) (pa + i0 * sa.nb[0]), vb = *(const float*) (pb + i0 * bnb0);
            *(float*) (pd + i0 * sd.nb[0]) = OP == BinOp::ADD ? va + vb : va * vb;
        }
    }
}

// k_binary with four floats per lane: rows of a, d (and b, unless b broadcasts
// along ne0) are 16-byte aligned with nb0 == 4 and ne0 % 4 == 0. The same single
// rounding per element.
template <BinOp OP>
__global__ __launch_bounds__(EW_THREADS) void k_binary4(const uint8_t* __restrict__ a, Shape4 sa,
                                                        const uint8_t* __restrict__ b, Shape4 sb,
                                                        uint8_t* __restrict__ d, Shape4 sd) {
    const int64_t rows = sd.ne[1] * sd.ne[2] * sd.ne[3];
    const int64_t n4 = sd.ne[0] / 4;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const int64_t i1 = r % sd.ne[1], i2 = (r / sd.ne[1]) % sd.ne[2], i3 = r / (sd.ne[1] * sd.ne[2]);
        const f4* pa = (const f4*) (a + i1 * sa.nb[1] + i2 * sa.nb[2] + i3 * sa.nb[3]);
        const uint8_t* pb = b + (sb.ne[1] == 1 ? 0 : i1 * sb.nb[1]) + (sb.ne[2] == 1 ? 0 : i2 * sb.nb[2]) +
                            (sb.ne[3] == 1 ? 0 : i3 * sb.nb[3]);
        f4* pd = (f4*) (d + i1 * sd.nb[1] + i2 * sd.nb[2] + i3 * sd.nb[3]);
        for (int64_t q = threadIdx.x; q < n4; q += EW_THREADS) {
            const f4 va = pa[q];
            f4 vb;
            if (sb.ne[0] == 1) {
                const float x = *(const float*) pb;
                vb = (f4){x, x, x, x};
            } else {
                vb = ((const f4*) pb)[q];
            }
            pd[q] = OP == BinOp::ADD ? va + vb : va * vb;
        }
    }
}

enum class UnOp { SQR, SCALE };

// dst[i] = a[i] * a[i] (SQR: fn_sqr, src/backends/cpu/trc_cpu_ops.cpp:86, through
// compute_unary :119-135) or a[i] * s (SCALE: compute_scale :140-150), element i
// of dst from element i of a (same shape, any strides): one float multiply each,
// rows of dst distributed over the grid as in k_binary
template <UnOp OP>
__global__ __launch_bounds__(EW_THREADS) void k_unary(const uint8_t* __restrict__ a, Shape4 sa,
                                                      uint8_t* __restrict__ d, Shape4 sd, float s) {
    const int64_t rows = sd.ne[1] * sd.ne[2] * sd.ne[3];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const int64_t i1 = r % sd.ne[1], i2 = (r / sd.ne[1]) % sd.ne[2], i3 = r / (sd.ne[1] * sd.ne[2]);
        const uint8_t* pa = a + i1 * sa.nb[1] + i2 * sa.nb[2] + i3 * sa.nb[3];
        uint8_t* pd = d + i1 * sd.nb[1] + i2 * sd.nb[2] + i3 * sd.nb[3];
        for (int64_t i0 = threadIdx.x; i0 < sd.ne[0]; i0 += EW_THREADS) {
            const float v = *(const float*) (pa + i0 * sa.nb[0]);
            *(float*) (pd + i0 * sd.nb[0]) = OP == UnOp::SQR ? v * v : v * s;
        }
    }
}

// k_unary with four floats per lane (rows of a and d 16-byte aligned, nb0 == 4,
// ne0 % 4 == 0); the same single rounding per element
template <UnOp OP>
__global__ __launch_bounds__(EW_THREADS) void k_unary4(const uint8_t* __restrict__ a, Shape4 sa,
                                                       uint8_t* __restrict__ d, Shape4 sd, float s) {
    const int64_t rows = sd.ne[1] * sd.ne[2] * sd.ne[3];
    const int64_t n4 = sd.ne[0] / 4;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const int64_t i1 = r % sd.ne[1], i2 = (r / sd.ne[1]) % sd.ne[2], i3 = r / (sd.ne[1] * sd.ne[2]);
        const f4* pa = (const f4*) (a + i1 * sa.nb[1] + i2 * sa.nb[2] + i3 * sa.nb[3]);
        f4* pd = (f4*) (d + i1 * sd.nb[1] + i2 * sd.nb[2] + i3 * sd.nb[3]);
        for (int64_t q = threadIdx.x; q < n4; q += EW_THREADS) {
            const f4 v = pa[q];
            pd[q] = OP == UnOp::SQR ? v * v : v * s;
        }
    }
}

// k_repeat for a dst whose rows are 16-byte aligned with nb0 == 4 and ne0 % 4 ==
// 0: one row of dst per workgroup pass, four floats per lane and store.
__global__ __launch_bounds__(EW_THREADS) void k_repeat4(const uint8_t* __restrict__ a, Shape4 sa,
                                                        uint8_t* __restrict__ d, Shape4 sd) {
    const int64_t rows = sd.ne[1] * sd.ne[2] * sd.ne[3];
    const int64_t n4 = sd.ne[0] / 4;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const int64_t i1 = r % sd.ne[1], i2 = (r / sd.ne[1]) % sd.ne[2], i3 = r / (sd.ne[1] * sd.ne[2]);
        const uint8_t* pa = a + (i1 % sa.ne[1]) * sa.nb[1] + (i2 % sa.ne[2]) * sa.nb[2] + (i3 % sa.ne[3]) * sa.nb[3];
        f4* pd = (f4*) (d + i1 * sd.nb[1] + i2 * sd.nb[2] + i3 * sd.nb[3]);
        if (sa.ne[0] == 1) {  // one value per row of dst (e.g. a loss gradient spread out)
            const float x = *(const float*) pa;
            for (int64_t q = threadIdx.x; q < n4; q += EW_THREADS) pd[q] = (f4){x, x, x, x};
            continue;
        }
        for (int64_t q = threadIdx.x; q < n4; q += EW_THREADS) {
            f4 v;
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = *(const float*) (pa + ((4 * q + c) % sa.ne[0]) * sa.nb[0]);
            pd[q] = v;
        }
    }
}

// dst[i] = a[i mod a.ne, per dim]: every dim of a is 1 (broadcast) or dst's
// extent; one thread per dst element, grid-stride
__global__ __launch_bounds__(EW_THREADS) void k_repeat(const uint8_t* __restrict__ a, Shape4 sa,
                                                       uint8_t* __restrict__ d, Shape4 sd) {
    const int64_t n = sd.ne[0] * sd.ne[1] * sd.ne[2] * sd.ne[3];
    for (int64_t j = (int64_t) blockIdx.x * EW_THREADS + threadIdx.x; j < n; j += (int64_t) gridDim.x * EW_THREADS) {
        int64_t rem = j, oa = 0, od = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t idx = rem % sd.ne[k];
            rem /= sd.ne[k];
            oa += (sa.ne[k] == 1 ? 0 : idx % sa.ne[k]) * sa.nb[k];
            od += idx * sd.nb[k];
        }
        *(float*) (d + od) = *(const float*) (a + oa);
    }
}

// *d = sum of a, as compute_sum forms it: each row (ne0-run) summed from 0 in
// double in element order, the row sums added in double in row order (i1
// fastest, then i2, i3), one rounding to float at the end.
//
// Two launches. k_sum_rows: one lane per row, its row's sequential double sum
// (the chain cannot be split without changing the rounding), with the row's
// next SR_AHEAD loads issued ahead of the adds, from addresses clamped into the
// row so no branch waits on them; the row sums go to a workspace. k_sum_combine:
// one wave adds them in row order. k_sum (one workgroup, no workspace) serves
// the row counts the workspace cannot hold.
constexpr int SR_THREADS = 64;
constexpr int SR_AHEAD = 32;

template <bool VEC>
__global__ __launch_bounds__(SR_THREADS) void k_sum_rows(const uint8_t* __restrict__ a, Shape4 sa,
                                                         double* __restrict__ part) {
    const int64_t rows = sa.ne[1] * sa.ne[2] * sa.ne[3];
    const int64_t r = (int64_t) blockIdx.x * SR_THREADS + threadIdx.x;
    if (r >= rows) return;  // no barrier below
    const int64_t i1 = r % sa.ne[1], i2 = (r / sa.ne[1]) % sa.ne[2], i3 = r / (sa.ne[1] * sa.ne[2]);
    const uint8_t* p = a + i1 * sa.nb[1] + i2 * sa.nb[2] + i3 * sa.nb[3];
    const int64_t n = sa.ne[0];
    double s = 0.0;
    if constexpr (VEC) {  // nb0 == 4, every row 16-byte aligned
        const f4* q = (const f4*) p;
        const int64_t n4 = n / 4;
        if (n4 > 0) {
            f4 buf[SR_AHEAD];
#pragma unroll
            for (int u = 0; u < SR_AHEAD; ++u) buf[u] = q[u < n4 ? u : n4 - 1];
            for (int64_t i = 0; i < n4; i += SR_AHEAD) {
#pragma unroll
                for (int u = 0; u < SR_AHEAD; ++u) {
                    if (i + u < n4) {  // the same for every lane: rows have one length
                        const f4 v = buf[u];
                        s = s + (double) v.x;
                        s = s + (double) v.y;
                        s = s + (double) v.z;
                        s = s + (double) v.w;
                    }
                    const int64_t nx = i + SR_AHEAD + u;
                    buf[u] = q[nx < n4 ? nx : n4 - 1];
                }
            }
        }
        for (int64_t i0 = 4 * n4; i0 < n; ++i0) s = s + (double) ((const float*) p)[i0];
    } else {
        float buf[SR_AHEAD];
#pragma unroll
        for (int u = 0; u < SR_AHEAD; ++u) buf[u] = *(const float*) (p + (u < n ? u : n - 1) * sa.nb[0]);
        for (int64_t i = 0; i < n; i += SR_AHEAD) {
#pragma unroll
            for (int u = 0; u < SR_AHEAD; ++u) {
                if (i + u < n) s = s + (double) buf[u];
                const int64_t nx = i + SR_AHEAD + u;
                buf[u] = *(const float*) (p + (nx < n ? nx : n - 1) * sa.nb[0]);
            }
        }
    }
    part[r] = s;
}

// k_sum_rows for 16-byte aligned rows (nb0 == 4), with the loads spread over a
// whole workgroup: SB_ROWS rows per workgroup stream through an LDS ring of
// SB_D chunks of SB_C floats per row, loaded by all SB_THREADS threads (1 KB
// runs per row) SB_D - 1 chunks ahead of the lanes that hold the rows' sums;
// lane r of wave 0 adds row r's chunk in element order. With SB_D >= 3 one
// barrier per chunk separates a slot's reads from its next fill. The threads
// that stage a chunk convert it to double (exact) as they store it, so the
// lanes on the chain issue only the adds (configuration 3's loss: 29.1 ->
// 27.0 us per launch). What remains is the chain itself: each dependent
// v_add_f64 waits ~15 cycles for the one before, 4096 of them per row.
constexpr int SB_ROWS = 8;
constexpr int SB_THREADS = 256;
constexpr int SB_C = 256;
constexpr int SB_LD = SB_C + 2;  // padded row (in doubles) of an LDS slot: rows 4 banks apart
typedef double sb_d2 __attribute__((ext_vector_type(2)));
constexpr int SB_D = 4;
constexpr int SB_PER = SB_ROWS * SB_C / 4 / SB_THREADS;  // float4 loads per thread and chunk
static_assert(SB_PER * SB_THREADS * 4 == SB_ROWS * SB_C, "a chunk is whole float4s per thread");

__global__ __launch_bounds__(SB_THREADS) void k_sum_rows_lds(const uint8_t* __restrict__ a, Shape4 sa,
                                                             double* __restrict__ part) {
    __shared__ __attribute__((aligned(16))) double ring[SB_D * SB_ROWS * SB_LD];
    const int64_t rows = sa.ne[1] * sa.ne[2] * sa.ne[3];
    const int64_t r0 = (int64_t) blockIdx.x * SB_ROWS;
    const int64_t n = sa.ne[0];
    const int64_t n4 = n / 4;
    const int64_t chunks = (n + SB_C - 1) / SB_C;
    const int tid = threadIdx.x;
    // this thread's float4s of a chunk: row e / (SB_C / 4), float4 e % (SB_C / 4)
    const f4* src[SB_PER];
    int lrow[SB_PER], lq[SB_PER];
#pragma unroll
    for (int u = 0; u < SB_PER; ++u) {
        const int e = tid + SB_THREADS * u;
        lrow[u] = e / (SB_C / 4);
        lq[u] = e % (SB_C / 4);
        int64_t r = r0 + lrow[u];
        r = r < rows ? r : rows - 1;  // rows past the end re-read the last; nobody adds them
        const int64_t i1 = r % sa.ne[1], i2 = (r / sa.ne[1]) % sa.ne[2], i3 = r / (sa.ne[1] * sa.ne[2]);
        src[u] = (const f4*) (a + i1 * sa.nb[1] + i2 * sa.nb[2] + i3 * sa.nb[3]);
    }
    // float4 q of a row covers elements 4q .. 4q + 3 (n % 4 == 0 on this path); a
    // float4 past the row's end is read from the row's last (valid) and never added
    auto load = [&](int64_t c, f4 (&v)[SB_PER]) {
#pragma unroll
        for (int u = 0; u < SB_PER; ++u) {
            const int64_t q = c * (SB_C / 4) + lq[u];
            v[u] = src[u][q < n4 ? q : n4 - 1];
        }
    };
    auto store = [&](int64_t c, const f4 (&v)[SB_PER]) {
        double* slot = ring + (int) (c % SB_D) * SB_ROWS * SB_LD;
#pragma unroll
        for (int u = 0; u < SB_PER; ++u) {
            double* dst = slot + lrow[u] * SB_LD + 4 * lq[u];
            *(sb_d2*) dst = sb_d2{(double) v[u].x, (double) v[u].y};
            *(sb_d2*) (dst + 2) = sb_d2{(double) v[u].z, (double) v[u].w};
        }
    };
    for (int64_t c = 0; c < SB_D - 1 && c < chunks; ++c) {
        f4 v[SB_PER];
        load(c, v);
        store(c, v);
    }
    __syncthreads();
    double s = 0.0;
    const bool chain = tid < SB_ROWS && r0 + tid < rows;
    for (int64_t c = 0; c < chunks; ++c) {
        f4 v[SB_PER];
        const bool more = c + SB_D - 1 < chunks;
        if (more) load(c + SB_D - 1, v);
        if (chain) {
            const double* row = ring + (int) (c % SB_D) * SB_ROWS * SB_LD + tid * SB_LD;
            const int64_t m = n - c * SB_C < SB_C ? n - c * SB_C : SB_C;
            if (m == SB_C) {
                // a whole chunk: the next 16 values are read from LDS while the
                // current 16 are added, so only the adds stay on the chain
                const sb_d2* row2 = (const sb_d2*) row;
                sb_d2 cur[8], nxt[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) cur[k] = row2[k];
#pragma unroll
                for (int g = 0; g < SB_C / 16; ++g) {
                    if (g + 1 < SB_C / 16) {
#pragma unroll
                        for (int k = 0; k < 8; ++k) nxt[k] = row2[8 * (g + 1) + k];
                    }
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        s = s + cur[k].x;
                        s = s + cur[k].y;
                    }
#pragma unroll
                    for (int k = 0; k < 8; ++k) cur[k] = nxt[k];
                }
            } else {
                for (int64_t i = 0; i < m; ++i) s = s + row[i];
            }
        }
        __syncthreads();
        if (more) store(c + SB_D - 1, v);
    }
    if (chain) part[r0 + tid] = s;
}

// *d = (float) (0 + part[0] + part[1] + ...), in row order. Up to SC_BATCH row
// sums at a time are staged in LDS by the whole wave (all loads in flight
// together), then lane 0 adds them, reading the next pair while adding one.
constexpr int SC_BATCH = 4096;
__global__ __launch_bounds__(64) void k_sum_combine(const double* __restrict__ part, int64_t rows,
                                                    float* __restrict__ d) {
    __shared__ __attribute__((aligned(16))) double buf[SC_BATCH];
    double total = 0.0;
    for (int64_t r0 = 0; r0 < rows; r0 += SC_BATCH) {
        const int n = (int) (rows - r0 < SC_BATCH ? rows - r0 : SC_BATCH);
        for (int k = threadIdx.x; k < n; k += 64) buf[k] = part[r0 + k];
        __syncthreads();
        if (threadIdx.x == 0) {
            int k = 0;
            if (n >= 8) {
                typedef double d2 __attribute__((ext_vector_type(2)));
                d2 cur[4], nxt[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) cur[q] = *(const d2*) (buf + 2 * q);
                for (; k + 8 <= n; k += 8) {
                    const bool more = k + 16 <= n;
#pragma unroll
                    for (int q = 0; q < 4; ++q) nxt[q] = more ? *(const d2*) (buf + k + 8 + 2 * q) : cur[q];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        total = total + cur[q].x;
                        total = total + cur[q].y;
                    }
#pragma unroll
                    for (int q = 0; q < 4; ++q) cur[q] = nxt[q];
                }
            }
            for (; k < n; ++k) total = total + buf[k];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) *d = (float) total;
}

// The same sums in one workgroup: each thread sums one row of a block of
// SUM_THREADS rows into LDS, then thread 0 adds the block's row sums in order.
constexpr int SUM_THREADS = 1024;
__global__ __launch_bounds__(SUM_THREADS) void k_sum(const uint8_t* __restrict__ a, Shape4 sa, float* __restrict__ d) {
    __shared__ double row[SUM_THREADS];
    const int64_t rows = sa.ne[1] * sa.ne[2] * sa.ne[3];
    double total = 0.0;
    for (int64_t r0 = 0; r0 < rows; r0 += SUM_THREADS) {
        const int64_t r = r0 + threadIdx.x;
        double s = 0.0;
        if (r < rows) {
            const int64_t i1 = r % sa.ne[1], i2 = (r / sa.ne[1]) % sa.ne[2], i3 = r / (sa.ne[1] * sa.ne[2]);
            const uint8_t* p = a + i1 * sa.nb[1] + i2 * sa.nb[2] + i3 * sa.nb[3];
            for (int64_t i0 = 0; i0 < sa.ne[0]; ++i0) s = s + (double) *(const float*) (p + i0 * sa.nb[0]);
        }
        row[threadIdx.x] = s;
        __syncthreads();
        if (threadIdx.x == 0) {
            const int64_t n = rows - r0 < SUM_THREADS ? rows - r0 : SUM_THREADS;
            for (int64_t k = 0; k < n; ++k) total = total + row[k];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) *d = (float) total;
}

// contiguous copy of n floats (acc with inplace == false starts from a)
__global__ __launch_bounds__(EW_THREADS) void k_copy_f32(const float* __restrict__ src, float* __restrict__ dst,
                                                         int64_t n) {
    for (int64_t i = (int64_t) blockIdx.x * EW_THREADS + threadIdx.x; i < n; i += (int64_t) gridDim.x * EW_THREADS) {
        dst[i] = src[i];
    }
}

// d[offset + i0*4 + i1*nb1 + i2*nb2 + i3*nb3] += b[i]; the launcher has checked
// that no two elements of b land on the same float, so rows run in parallel
__global__ __launch_bounds__(EW_THREADS) void k_acc(const uint8_t* __restrict__ b, Shape4 sb, uint8_t* __restrict__ d,
                                                    int64_t offset, int64_t nb1, int64_t nb2, int64_t nb3) {
    const int64_t rows = sb.ne[1] * sb.ne[2] * sb.ne[3];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const int64_t i1 = r % sb.ne[1], i2 = (r / sb.ne[1]) % sb.ne[2], i3 = r / (sb.ne[1] * sb.ne[2]);
        const uint8_t* pb = b + i1 * sb.nb[1] + i2 * sb.nb[2] + i3 * sb.nb[3];
        uint8_t* pd = d + offset + i1 * nb1 + i2 * nb2 + i3 * nb3;
        for (int64_t i0 = threadIdx.x; i0 < sb.ne[0]; i0 += EW_THREADS) {
            float* t = (float*) (pd + i0 * 4);
            *t = *t + *(const float*) (pb + i0 * sb.nb[0]);
        }
    }
}

// d (contiguous, shape dn) = sum over the repeats of a; every output is summed
// from 0 in a's linear element order: repeat index k3, k2, k1, k0, k0 fastest
__global__ __launch_bounds__(EW_THREADS) void k_repeat_back(const uint8_t* __restrict__ a, Shape4 sa,
                                                            float* __restrict__ d, Shape4 sd) {
    const int64_t n = sd.ne[0] * sd.ne[1] * sd.ne[2] * sd.ne[3];
    const int64_t r0 = sa.ne[0] / sd.ne[0], r1 = sa.ne[1] / sd.ne[1], r2 = sa.ne[2] / sd.ne[2],
                  r3 = sa.ne[3] / sd.ne[3];
    for (int64_t j = (int64_t) blockIdx.x * EW_THREADS + threadIdx.x; j < n; j += (int64_t) gridDim.x * EW_THREADS) {
        const int64_t j0 = j % sd.ne[0], j1 = (j / sd.ne[0]) % sd.ne[1], j2 = (j / (sd.ne[0] * sd.ne[1])) % sd.ne[2],
                      j3 = j / (sd.ne[0] * sd.ne[1] * sd.ne[2]);
        float s = 0.f;
        for (int64_t k3 = 0; k3 < r3; ++k3)
            for (int64_t k2 = 0; k2 < r2; ++k2)
                for (int64_t k1 = 0; k1 < r1; ++k1) {
                    const uint8_t* row = a + (j1 + k1 * sd.ne[1]) * sa.nb[1] + (j2 + k2 * sd.ne[2]) * sa.nb[2] +
                                         (j3 + k3 * sd.ne[3]) * sa.nb[3];
                    for (int64_t k0 = 0; k0 < r0; ++k0) s = s + *(const float*) (row + (j0 + k0 * sd.ne[0]) * sa.nb[0]);
                }
        d[j] = s;
    }
}

// The same sums when ne0 is not repeated (a.ne0 == d.ne0, e.g. a bias gradient
// summed over the tokens): output j's terms are rows k1, k2, k3 (k1 fastest) at
// one column, so their offsets from a's element j follow a counter that is the
// same for every lane. RB_AHEAD loads run ahead of the in-order adds, from
// offsets that stay inside a (terms past the last re-read the first).
constexpr int RB_THREADS = 64;
constexpr int RB_AHEAD = 64;
__global__ __launch_bounds__(RB_THREADS) void k_repeat_back_cols(const uint8_t* __restrict__ a, Shape4 sa,
                                                                 float* __restrict__ d, Shape4 sd) {
    const int64_t n = sd.ne[0] * sd.ne[1] * sd.ne[2] * sd.ne[3];
    const int64_t j = (int64_t) blockIdx.x * RB_THREADS + threadIdx.x;
    if (j >= n) return;  // no barrier below
    const int64_t j0 = j % sd.ne[0], j1 = (j / sd.ne[0]) % sd.ne[1], j2 = (j / (sd.ne[0] * sd.ne[1])) % sd.ne[2],
                  j3 = j / (sd.ne[0] * sd.ne[1] * sd.ne[2]);
    const uint8_t* base = a + j0 * sa.nb[0] + j1 * sa.nb[1] + j2 * sa.nb[2] + j3 * sa.nb[3];
    const int64_t r1 = sa.ne[1] / sd.ne[1], r2 = sa.ne[2] / sd.ne[2], r3 = sa.ne[3] / sd.ne[3];
    const int64_t st1 = sd.ne[1] * sa.nb[1], st2 = sd.ne[2] * sa.nb[2], st3 = sd.ne[3] * sa.nb[3];
    const int64_t terms = r1 * r2 * r3;
    // the counter of the next term to load: (k1, k2, k3) and its byte offset
    int64_t k1 = 0, k2 = 0, k3 = 0, off = 0, next = 0;
    auto advance = [&]() {
        ++next;
        ++k1;
        off += st1;
        if (k1 == r1) {
            k1 = 0;
            off -= r1 * st1;
            ++k2;
            off += st2;
            if (k2 == r2) {
                k2 = 0;
                off -= r2 * st2;
                ++k3;
                off += st3;
            }
        }
    };
    float buf[RB_AHEAD];
#pragma unroll
    for (int u = 0; u < RB_AHEAD; ++u) {
        buf[u] = *(const float*) (base + (next < terms ? off : 0));
        advance();
    }
    float s = 0.f;
    for (int64_t q0 = 0; q0 < terms; q0 += RB_AHEAD) {
#pragma unroll
        for (int u = 0; u < RB_AHEAD; ++u) {
            if (q0 + u < terms) s = s + buf[u];  // the same for every lane
            buf[u] = *(const float*) (base + (next < terms ? off : 0));
            advance();
        }
    }
    d[j] = s;
}

// k_repeat_back_cols when only dim 1 repeats (output j's terms are a's element j
// and every st1 bytes after it), with the loads spread over a workgroup: 64
// consecutive outputs per workgroup, RL_T terms of each per chunk, streamed
// through an LDS ring of RL_D chunks by all RL_THREADS threads, RL_D - 1 chunks
// ahead of wave 0, whose lane o adds output o's terms in order.
constexpr int RL_THREADS = 256;
constexpr int RL_T = 32;
constexpr int RL_D = 4;
constexpr int RL_PER = RL_T * 64 / RL_THREADS;  // loads per thread and chunk
__global__ __launch_bounds__(RL_THREADS) void k_repeat_back_lds(const uint8_t* __restrict__ a, Shape4 sa,
                                                                float* __restrict__ d, Shape4 sd) {
    __shared__ float ring[RL_D * RL_T * 64];
    const int64_t n = sd.ne[0] * sd.ne[1] * sd.ne[2] * sd.ne[3];
    const int tid = threadIdx.x, o = tid % 64;
    int64_t j = (int64_t) blockIdx.x * 64 + o;
    const bool valid = j < n;
    j = valid ? j : n - 1;  // outputs past the end re-read the last; nobody stores them
    const int64_t j0 = j % sd.ne[0], j1 = (j / sd.ne[0]) % sd.ne[1], j2 = (j / (sd.ne[0] * sd.ne[1])) % sd.ne[2],
                  j3 = j / (sd.ne[0] * sd.ne[1] * sd.ne[2]);
    const uint8_t* base = a + j0 * sa.nb[0] + j1 * sa.nb[1] + j2 * sa.nb[2] + j3 * sa.nb[3];
    const int64_t terms = sa.ne[1] / sd.ne[1];
    const int64_t st1 = sd.ne[1] * sa.nb[1];
    const int64_t chunks = (terms + RL_T - 1) / RL_T;
    auto load = [&](int64_t c, float (&v)[RL_PER]) {
#pragma unroll
        for (int u = 0; u < RL_PER; ++u) {
            const int64_t q = c * RL_T + (tid + RL_THREADS * u) / 64;  // this load's term
            v[u] = *(const float*) (base + (q < terms ? q : terms - 1) * st1);
        }
    };
    auto store = [&](int64_t c, const float (&v)[RL_PER]) {
        float* slot = ring + (int) (c % RL_D) * RL_T * 64;
#pragma unroll
        for (int u = 0; u < RL_PER; ++u) slot[tid + RL_THREADS * u] = v[u];  // [term][output]
    };
    for (int64_t c = 0; c < RL_D - 1 && c < chunks; ++c) {
        float v[RL_PER];
        load(c, v);
        store(c, v);
    }
    __syncthreads();
    float s = 0.f;
    for (int64_t c = 0; c < chunks; ++c) {
        float v[RL_PER];
        const bool more = c + RL_D - 1 < chunks;
        if (more) load(c + RL_D - 1, v);
        if (tid < 64) {
            const float* slot = ring + (int) (c % RL_D) * RL_T * 64;
            const int64_t m = terms - c * RL_T < RL_T ? terms - c * RL_T : RL_T;
            if (m == RL_T) {  // a whole chunk: every term read first, then added in order
                float t[RL_T];
#pragma unroll
                for (int q = 0; q < RL_T; ++q) t[q] = slot[q * 64 + o];
#pragma unroll
                for (int q = 0; q < RL_T; ++q) s = s + t[q];
            } else {
                for (int64_t q = 0; q < m; ++q) s = s + slot[q * 64 + o];
            }
        }
        __syncthreads();
        if (more) store(c + RL_D - 1, v);
    }
    if (tid < 64 && valid) d[j] = s;
}

unsigned grid_for(int64_t work, int64_t per_block) {
    int64_t g = (work + per_block - 1) / per_block;
    const int64_t cap = (int64_t) device_cus() * 16;
    if (g > cap) g = cap;
    return (unsigned) (g < 1 ? 1 : g);
}

bool f32_aligned(const trc_hip_tensor& t) {
    if ((((uintptr_t) t.data) & 3u) != 0) return false;
    for (int d = 0; d < 4; ++d) {
        if ((t.nb[d] & 3u) != 0) return false;
    }
    return true;
}

bool contiguous_f32(const trc_hip_tensor& t) {
    size_t nb = 4;
    for (int d = 0; d < 4; ++d) {
        if (t.ne[d] > 1 && t.nb[d] != nb) return false;
        nb *= (size_t) t.ne[d];
    }
    return true;
}

int64_t nelem(const trc_hip_tensor& t) { return t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]; }

// Every row (ne0-run) starts 16-byte aligned and holds whole float4s.
bool rows_vec4(const trc_hip_tensor& t) {
    if (t.nb[0] != 4 || t.ne[0] % 4 != 0 || (((uintptr_t) t.data) & 15u) != 0) return false;
    for (int d = 1; d < 4; ++d) {
        if (t.ne[d] > 1 && t.nb[d] % 16 != 0) return false;
    }
    return true;
}

bool shape_ok(const trc_hip_tensor& t) {
    for (int d = 0; d < 4; ++d) {
        if (t.ne[d] <= 0) return false;
    }
    return true;
}

template <BinOp OP>
int launch_binary(const char* name, const trc_hip_tensor& a, const trc_hip_tensor& b, const trc_hip_tensor& d,
                  hipStream_t s) {
    if (a.type != TRC_HIP_TYPE_F32 || b.type != TRC_HIP_TYPE_F32 || d.type != TRC_HIP_TYPE_F32) {
        return fail(TRC_HIP_E_INVALID, "%s: F32 tensors only", name);
    }
    if (!shape_ok(a) || !shape_ok(b) || !shape_ok(d)) return fail(TRC_HIP_E_SHAPE, "%s: empty or negative extent", name);
    for (int k = 0; k < 4; ++k) {
        if (d.ne[k] != a.ne[k] || (b.ne[k] != a.ne[k] && b.ne[k] != 1)) {
            return fail(TRC_HIP_E_SHAPE, "%s: dst must have a's shape and b must broadcast to it (dim %d)", name, k);
        }
    }
    if (!f32_aligned(a) || !f32_aligned(b) || !f32_aligned(d)) return fail(TRC_HIP_E_ALIGN, "%s: 4-byte alignment", name);
    const int64_t rows = d.ne[1] * d.ne[2] * d.ne[3];
    if (rows_vec4(a) && rows_vec4(d) && (b.ne[0] == 1 || rows_vec4(b))) {
        hipLaunchKernelGGL(k_binary4<OP>, dim3(grid_for(rows, 1)), dim3(EW_THREADS), 0, s, (const uint8_t*) a.data,
                           shape_of(a), (const uint8_t*) b.data, shape_of(b), (uint8_t*) d.data, shape_of(d));
        return check_launch(name);
    }
    hipLaunchKernelGGL(k_binary<OP>, dim3(grid_for(rows, 1)), dim3(EW_THREADS), 0, s, (const uint8_t*) a.data,
                       shape_of(a), (const uint8_t*) b.data, shape_of(b), (uint8_t*) d.data, shape_of(d));
    return check_launch(name);
}

}  // namespace

int launch_add_f32(const trc_hip_tensor& a, const trc_hip_tensor& b, const trc_hip_tensor& d, hipStream_t s) {
    return launch_binary<BinOp::ADD>("add", a, b, d, s);
}

int launch_mul_f32(const trc_hip_tensor& a, const trc_hip_tensor& b, const trc_hip_tensor& d, hipStream_t s) {
    return launch_binary<BinOp::MUL>("mul", a, b, d, s);
}

namespace {

template <UnOp OP>
int launch_unary(const char* name, const trc_hip_tensor& a, const trc_hip_tensor& d, float scale, hipStream_t s) {
    if (a.type != TRC_HIP_TYPE_F32 || d.type != TRC_HIP_TYPE_F32) return fail(TRC_HIP_E_INVALID, "%s: F32 tensors only", name);
    if (!shape_ok(a) || !shape_ok(d)) return fail(TRC_HIP_E_SHAPE, "%s: empty or negative extent", name);
    for (int k = 0; k < 4; ++k) {
        if (d.ne[k] != a.ne[k]) return fail(TRC_HIP_E_SHAPE, "%s: dst must have a's shape (dim %d)", name, k);
    }
    if (!f32_aligned(a) || !f32_aligned(d)) return fail(TRC_HIP_E_ALIGN, "%s: 4-byte alignment", name);
    const int64_t rows = d.ne[1] * d.ne[2] * d.ne[3];
    if (rows_vec4(a) && rows_vec4(d)) {
        hipLaunchKernelGGL(k_unary4<OP>, dim3(grid_for(rows, 1)), dim3(EW_THREADS), 0, s, (const uint8_t*) a.data,
                           shape_of(a), (uint8_t*) d.data, shape_of(d), scale);
        return check_launch(name);
    }
    hipLaunchKernelGGL(k_unary<OP>, dim3(grid_for(rows, 1)), dim3(EW_THREADS), 0, s, (const uint8_t*) a.data,
                       shape_of(a), (uint8_t*) d.data, shape_of(d), scale);
    return check_launch(name);
}

}  // namespace

int launch_sqr_f32(const trc_hip_tensor& a, const trc_hip_tensor& d, hipStream_t s) {
    return launch_unary<UnOp::SQR>("sqr", a, d, 0.f, s);
}

int launch_scale_f32(const trc_hip_tensor& a, const trc_hip_tensor& d, float scale, hipStream_t s) {
    return launch_unary<UnOp::SCALE>("scale", a, d, scale, s);
}

int launch_repeat_f32(const trc_hip_tensor& a, const trc_hip_tensor& d, hipStream_t s) {
    if (a.type != TRC_HIP_TYPE_F32 || d.type != TRC_HIP_TYPE_F32) return fail(TRC_HIP_E_INVALID, "repeat: F32 tensors only");
    if (!shape_ok(a) || !shape_ok(d)) return fail(TRC_HIP_E_SHAPE, "repeat: empty or negative extent");
    for (int k = 0; k < 4; ++k) {
        // ggml_can_repeat(a, dst): every dst extent a multiple of a's
        if (d.ne[k] % a.ne[k] != 0) return fail(TRC_HIP_E_SHAPE, "repeat: dst.ne[%d] is not a multiple of a.ne[%d]", k, k);
    }
    if (!f32_aligned(a) || !f32_aligned(d)) return fail(TRC_HIP_E_ALIGN, "repeat: 4-byte alignment");
    const int64_t n = nelem(d);
    if (rows_vec4(d)) {
        const int64_t rows = d.ne[1] * d.ne[2] * d.ne[3];
        hipLaunchKernelGGL(k_repeat4, dim3(grid_for(rows, 1)), dim3(EW_THREADS), 0, s, (const uint8_t*) a.data,
                           shape_of(a), (uint8_t*) d.data, shape_of(d));
        return check_launch("repeat");
    }
    hipLaunchKernelGGL(k_repeat, dim3(grid_for(n, EW_THREADS)), dim3(EW_THREADS), 0, s, (const uint8_t*) a.data,
                       shape_of(a), (uint8_t*) d.data, shape_of(d));
    return check_launch("repeat");
}

int launch_sum_f32(const trc_hip_tensor& a, const trc_hip_tensor& d, hipStream_t s) {
    if (a.type != TRC_HIP_TYPE_F32 || d.type != TRC_HIP_TYPE_F32) return fail(TRC_HIP_E_INVALID, "sum: F32 tensors only");
    if (!shape_ok(a) || !shape_ok(d)) return fail(TRC_HIP_E_SHAPE, "sum: empty or negative extent");
    if (nelem(d) != 1) return fail(TRC_HIP_E_SHAPE, "sum: dst must hold one element");
    if (!f32_aligned(a) || !f32_aligned(d)) return fail(TRC_HIP_E_ALIGN, "sum: 4-byte alignment");
    const int64_t rows = a.ne[1] * a.ne[2] * a.ne[3];
    if ((size_t) rows * sizeof(double) > qm_workspace_bytes()) {
        hipLaunchKernelGGL(k_sum, dim3(1), dim3(SUM_THREADS), 0, s, (const uint8_t*) a.data, shape_of(a),
                           (float*) d.data);
        return check_launch("sum");
    }
    // the row sums go to this stream's workspace (the one trc_hip_qmatvec uses;
    // work on one stream runs in order, so the two never meet)
    uint8_t* ws = nullptr;
    const int rc = qm_stream_workspace(s, &ws);
    if (rc != TRC_HIP_OK) return rc;
    const bool vec = a.nb[0] == 4 && (((uintptr_t) a.data) & 15u) == 0 && (a.ne[1] == 1 || a.nb[1] % 16 == 0) &&
                     (a.ne[2] == 1 || a.nb[2] % 16 == 0) && (a.ne[3] == 1 || a.nb[3] % 16 == 0);
    const unsigned grid = (unsigned) ((rows + SR_THREADS - 1) / SR_THREADS);
    if (vec && a.ne[0] >= SB_C && a.ne[0] % 4 == 0) {
        hipLaunchKernelGGL(k_sum_rows_lds, dim3((unsigned) ((rows + SB_ROWS - 1) / SB_ROWS)), dim3(SB_THREADS), 0, s,
                           (const uint8_t*) a.data, shape_of(a), (double*) ws);
    } else if (vec) {
        hipLaunchKernelGGL(k_sum_rows<true>, dim3(grid), dim3(SR_THREADS), 0, s, (const uint8_t*) a.data, shape_of(a),
                           (double*) ws);
    } else {
        hipLaunchKernelGGL(k_sum_rows<false>, dim3(grid), dim3(SR_THREADS), 0, s, (const uint8_t*) a.data,
                           shape_of(a), (double*) ws);
    }
    int st = check_launch("sum (rows)");
    if (st != TRC_HIP_OK) return st;
    hipLaunchKernelGGL(k_sum_combine, dim3(1), dim3(64), 0, s, (const double*) ws, rows, (float*) d.data);
    return check_launch("sum (row sums)");
}

int launch_acc_f32(const trc_hip_tensor& a, const trc_hip_tensor& b, const trc_hip_tensor& d, size_t nb1, size_t nb2,
                   size_t nb3, size_t offset, int inplace, hipStream_t s) {
    if (a.type != TRC_HIP_TYPE_F32 || b.type != TRC_HIP_TYPE_F32 || d.type != TRC_HIP_TYPE_F32) {
        return fail(TRC_HIP_E_INVALID, "acc: F32 tensors only");
    }
    if (!shape_ok(a) || !shape_ok(b) || !shape_ok(d)) return fail(TRC_HIP_E_SHAPE, "acc: empty or negative extent");
    for (int k = 0; k < 4; ++k) {
        if (d.ne[k] != a.ne[k]) return fail(TRC_HIP_E_SHAPE, "acc: dst must have a's shape");
    }
    if (!contiguous_f32(a) || !contiguous_f32(d)) return fail(TRC_HIP_E_SHAPE, "acc: a and dst must be contiguous");
    if (!f32_aligned(a) || !f32_aligned(b) || !f32_aligned(d) || (nb1 & 3u) || (nb2 & 3u) || (nb3 & 3u) ||
        (offset & 3u)) {
        return fail(TRC_HIP_E_ALIGN, "acc: 4-byte alignment of pointers, strides and offset");
    }
    // region inside a (src/core/trc_tensor.cpp:331-337)
    const size_t nbytes = (size_t) nelem(a) * 4;
    size_t last = (size_t) (b.ne[0] - 1) * 4;
    last += b.ne[1] > 1 ? (size_t) (b.ne[1] - 1) * nb1 : 0;
    last += b.ne[2] > 1 ? (size_t) (b.ne[2] - 1) * nb2 : 0;
    last += b.ne[3] > 1 ? (size_t) (b.ne[3] - 1) * nb3 : 0;
    if (offset + last + 4 > nbytes) return fail(TRC_HIP_E_SHAPE, "acc: region leaves the target");
    // the region must not overlap itself: with its dims sorted by stride, each
    // stride must clear the span of the smaller ones
    {
        int64_t ne[4] = {b.ne[0], b.ne[1], b.ne[2], b.ne[3]};
        size_t st[4] = {4, nb1, nb2, nb3};
        int idx[4] = {0, 1, 2, 3};
        for (int i = 1; i < 4; ++i)
            for (int j = i; j > 0 && st[idx[j]] < st[idx[j - 1]]; --j) {
                const int t = idx[j];
                idx[j] = idx[j - 1];
                idx[j - 1] = t;
            }
        size_t span = 0;  // bytes covered by the dims already placed
        for (int i = 0; i < 4; ++i) {
            const int k = idx[i];
            if (ne[k] == 1) continue;
            if (st[k] < (span == 0 ? 4 : span)) return fail(TRC_HIP_E_SHAPE, "acc: region overlaps itself");
            span = st[k] * (size_t) (ne[k] - 1) + (span == 0 ? 4 : span);
        }
    }
    if (!inplace && a.data != d.data) {
        const int64_t n = nelem(a);
        hipLaunchKernelGGL(k_copy_f32, dim3(grid_for(n, EW_THREADS)), dim3(EW_THREADS), 0, s, (const float*) a.data,
                           (float*) d.data, n);
        const int rc = check_launch("acc copy");
        if (rc != TRC_HIP_OK) return rc;
    }
    const int64_t rows = b.ne[1] * b.ne[2] * b.ne[3];
    hipLaunchKernelGGL(k_acc, dim3(grid_for(rows, 1)), dim3(EW_THREADS), 0, s, (const uint8_t*) b.data, shape_of(b),
                       (uint8_t*) d.data, (int64_t) offset, (int64_t) nb1, (int64_t) nb2, (int64_t) nb3);
    return check_launch("acc");
}

int launch_repeat_back_f32(const trc_hip_tensor& a, const trc_hip_tensor& d, hipStream_t s) {
    if (a.type != TRC_HIP_TYPE_F32 || d.type != TRC_HIP_TYPE_F32) {
        return fail(TRC_HIP_E_INVALID, "repeat_back: F32 tensors only");
    }
    if (!shape_ok(a) || !shape_ok(d)) return fail(TRC_HIP_E_SHAPE, "repeat_back: empty or negative extent");
    for (int k = 0; k < 4; ++k) {
        if (a.ne[k] % d.ne[k] != 0) return fail(TRC_HIP_E_SHAPE, "repeat_back: a.ne must be a multiple of dst.ne");
    }
    if (!contiguous_f32(d)) return fail(TRC_HIP_E_SHAPE, "repeat_back: dst must be contiguous");
    if (!f32_aligned(a) || !f32_aligned(d)) return fail(TRC_HIP_E_ALIGN, "repeat_back: 4-byte alignment");
    const int64_t n = nelem(d);
    if (a.ne[0] == d.ne[0] && a.ne[2] == d.ne[2] && a.ne[3] == d.ne[3] && a.ne[1] / d.ne[1] >= 2 * RL_T) {
        hipLaunchKernelGGL(k_repeat_back_lds, dim3((unsigned) ((n + 63) / 64)), dim3(RL_THREADS), 0, s,
                           (const uint8_t*) a.data, shape_of(a), (float*) d.data, shape_of(d));
        return check_launch("repeat_back");
    }
    if (a.ne[0] == d.ne[0]) {
        hipLaunchKernelGGL(k_repeat_back_cols, dim3((unsigned) ((n + RB_THREADS - 1) / RB_THREADS)), dim3(RB_THREADS),
                           0, s, (const uint8_t*) a.data, shape_of(a), (float*) d.data, shape_of(d));
        return check_launch("repeat_back");
    }
    hipLaunchKernelGGL(k_repeat_back, dim3(grid_for(n, EW_THREADS)), dim3(EW_THREADS), 0, s, (const uint8_t*) a.data,
                       shape_of(a), (float*) d.data, shape_of(d));
    return check_launch("repeat_back");
}

}  // namespace trc_hip
