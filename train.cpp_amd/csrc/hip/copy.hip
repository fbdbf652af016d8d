// Element-wise memory kernels: F32 fill (Device::fill_tensors) and the strided
// copy behind OP_DUP/OP_CPY/OP_CONT (compute_dup,
// src/backends/cpu/trc_cpu_ops.cpp:219-236). Both are HBM-bound streams; a copy
// is exact whatever order its elements move in.
#include "common.h"

namespace trc_hip {
namespace {

constexpr int CP_THREADS = 256;

__global__ __launch_bounds__(CP_THREADS) void k_fill_f32(float* __restrict__ dst, float value, int64_t n) {
    const int64_t stride = (int64_t) gridDim.x * CP_THREADS;
    for (int64_t i = (int64_t) blockIdx.x * CP_THREADS + threadIdx.x; i < n; i += stride) {
        dst[i] = value;
    }
}

// 16-byte stores for a 16-byte aligned dst; the last n % 4 floats go one by one.
__global__ __launch_bounds__(CP_THREADS) void k_fill_f32x4(f4* __restrict__ dst, float value, int64_t n4,
                                                          float* __restrict__ tail, int ntail) {
    const f4 v = {value, value, value, value};
    const int64_t stride = (int64_t) gridDim.x * CP_THREADS;
    for (int64_t i = (int64_t) blockIdx.x * CP_THREADS + threadIdx.x; i < n4; i += stride) dst[i] = v;
    if (blockIdx.x == 0 && (int) threadIdx.x < ntail) tail[threadIdx.x] = value;
}

// Copies element i of src to element i of dst in ggml linear order
// (tensor_offset_linear, src/core/trc_tensor.cpp:95-103), ne0 fastest. The
// launch covers ne0 x rows with x along ne0, so a run of ne0 is one wave's
// contiguous read (or write) whenever that side has nb0 == element size.
template <typename T>
__global__ __launch_bounds__(CP_THREADS) void k_cpy(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                   int64_t ne0, int64_t ne1, int64_t ne2, int64_t rows,
                                                   int64_t snb0, int64_t snb1, int64_t snb2, int64_t snb3,
                                                   int64_t dnb0, int64_t dnb1, int64_t dnb2, int64_t dnb3) {
    const int64_t total = ne0 * rows;
    const int64_t stride = (int64_t) gridDim.x * CP_THREADS;
    for (int64_t idx = (int64_t) blockIdx.x * CP_THREADS + threadIdx.x; idx < total; idx += stride) {
        const int64_t i0 = idx % ne0;
        const int64_t r = idx / ne0;
        const int64_t i1 = r % ne1;
        const int64_t i2 = (r / ne1) % ne2;
        const int64_t i3 = r / (ne1 * ne2);
        const T v = *(const T*) (src + i0 * snb0 + i1 * snb1 + i2 * snb2 + i3 * snb3);
        *(T*) (dst + i0 * dnb0 + i1 * dnb1 + i2 * dnb2 + i3 * dnb3) = v;
    }
}

// The same copy for 4-byte elements when src runs along dim 1 (nb1 == 4, the
// transposed views autograd builds) and dst along dim 0 (nb0 == 4): 64 x 64
// tiles of (i0, i1) go through LDS, read as 256-byte runs of src along i1 and
// written as 256-byte runs of dst along i0.
constexpr int TT = 64;
__global__ __launch_bounds__(CP_THREADS) void k_cpy_transpose(const uint8_t* __restrict__ src,
                                                             uint8_t* __restrict__ dst, int64_t ne0, int64_t ne1,
                                                             int64_t ne2, int64_t tiles0, int64_t tiles1,
                                                             int64_t snb0, int64_t snb2, int64_t snb3, int64_t dnb1,
                                                             int64_t dnb2, int64_t dnb3) {
    __shared__ uint32_t tile[TT][TT + 1];
    int64_t t = blockIdx.x;
    const int64_t t0 = t % tiles0;
    t /= tiles0;
    const int64_t t1 = t % tiles1;
    const int64_t plane = t / tiles1;
    const int64_t i2 = plane % ne2, i3 = plane / ne2;
    const uint8_t* sp = src + i2 * snb2 + i3 * snb3;
    uint8_t* dp = dst + i2 * dnb2 + i3 * dnb3;
    const int64_t b0 = t0 * TT, b1 = t1 * TT;
    const int lane = threadIdx.x % TT, row = threadIdx.x / TT;  // 4 rows per pass
#pragma unroll
    for (int k = 0; k < TT; k += CP_THREADS / TT) {
        const int64_t i0 = b0 + row + k, i1 = b1 + lane;
        if (i0 < ne0 && i1 < ne1) tile[row + k][lane] = *(const uint32_t*) (sp + i0 * snb0 + i1 * 4);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < TT; k += CP_THREADS / TT) {
        const int64_t i0 = b0 + lane, i1 = b1 + row + k;
        if (i0 < ne0 && i1 < ne1) *(uint32_t*) (dp + i0 * 4 + i1 * dnb1) = tile[lane][row + k];
    }
}

// k_cpy_transpose with 16-byte global accesses, for whole tiles (ne0 and ne1
// multiples of 64) of 16-byte aligned rows: a lane reads four floats along i1
// and writes four along i0; the tile is kept in LDS as [i1][i0].
constexpr int TL = TT + 4;  // LDS row stride in floats (keeps rows 16-byte aligned)
__global__ __launch_bounds__(CP_THREADS) void k_cpy_transpose4(const uint8_t* __restrict__ src,
                                                              uint8_t* __restrict__ dst, int64_t ne2,
                                                              int64_t tiles0, int64_t tiles1, int64_t snb0,
                                                              int64_t snb2, int64_t snb3, int64_t dnb1, int64_t dnb2,
                                                              int64_t dnb3) {
    __shared__ __attribute__((aligned(16))) float tile[TT * TL];
    int64_t t = blockIdx.x;
    const int64_t t0 = t % tiles0;
    t /= tiles0;
    const int64_t t1 = t % tiles1;
    const int64_t plane = t / tiles1;
    const int64_t i2 = plane % ne2, i3 = plane / ne2;
    const uint8_t* sp = src + i2 * snb2 + i3 * snb3 + t0 * TT * snb0 + t1 * TT * 4;
    uint8_t* dp = dst + i2 * dnb2 + i3 * dnb3 + t0 * TT * 4 + t1 * TT * dnb1;
    const int q = threadIdx.x % (TT / 4), row = threadIdx.x / (TT / 4);  // 16 rows per pass
#pragma unroll
    for (int k = 0; k < TT; k += CP_THREADS / (TT / 4)) {
        const f4 v = *(const f4*) (sp + (row + k) * snb0 + q * 16);  // src row i0 = row + k, i1 = 4q .. 4q + 3
#pragma unroll
        for (int c = 0; c < 4; ++c) tile[(4 * q + c) * TL + row + k] = v[c];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < TT; k += CP_THREADS / (TT / 4)) {
        // dst row i1 = row + k, i0 = 4q .. 4q + 3
        *(f4*) (dp + (row + k) * dnb1 + q * 16) = *(const f4*) (tile + (row + k) * TL + 4 * q);
    }
}

unsigned grid_for(int64_t n) {
    const int64_t want = (n + CP_THREADS - 1) / CP_THREADS;
    return (unsigned) (want < 65536 ? (want > 0 ? want : 1) : 65536);
}

}  // namespace

int launch_fill_f32(float* dst, float value, int64_t count, hipStream_t stream) {
    if ((((uintptr_t) dst) & 15u) == 0) {
        const int64_t n4 = count / 4;
        hipLaunchKernelGGL(k_fill_f32x4, dim3(grid_for(n4)), dim3(CP_THREADS), 0, stream, (f4*) dst, value, n4,
                           dst + 4 * n4, (int) (count - 4 * n4));
    } else {
        hipLaunchKernelGGL(k_fill_f32, dim3(grid_for(count)), dim3(CP_THREADS), 0, stream, dst, value, count);
    }
    return check_launch("fill_f32");
}

int launch_cpy(const trc_hip_tensor& s, const trc_hip_tensor& d, size_t es, hipStream_t stream) {
    const int64_t rows = s.ne[1] * s.ne[2] * s.ne[3];
    const int64_t n = s.ne[0] * rows;
    const uint8_t* sp = (const uint8_t*) s.data;
    uint8_t* dp = (uint8_t*) d.data;
    if (es == 4 && s.nb[1] == 4 && d.nb[0] == 4 && s.ne[0] > 1 && s.ne[1] > 1) {
        const int64_t tiles0 = (s.ne[0] + TT - 1) / TT, tiles1 = (s.ne[1] + TT - 1) / TT;
        const int64_t grid = tiles0 * tiles1 * s.ne[2] * s.ne[3];
        const bool whole = s.ne[0] % TT == 0 && s.ne[1] % TT == 0 && (((uintptr_t) sp | (uintptr_t) dp) & 15u) == 0 &&
                           s.nb[0] % 16 == 0 && d.nb[1] % 16 == 0 && s.nb[2] % 16 == 0 && s.nb[3] % 16 == 0 &&
                           d.nb[2] % 16 == 0 && d.nb[3] % 16 == 0;
        if (grid <= 0x7FFFFFFF && whole) {
            hipLaunchKernelGGL(k_cpy_transpose4, dim3((unsigned) grid), dim3(CP_THREADS), 0, stream, sp, dp, s.ne[2],
                               tiles0, tiles1, (int64_t) s.nb[0], (int64_t) s.nb[2], (int64_t) s.nb[3],
                               (int64_t) d.nb[1], (int64_t) d.nb[2], (int64_t) d.nb[3]);
            return check_launch("cpy (transpose)");
        }
        if (grid <= 0x7FFFFFFF) {
            hipLaunchKernelGGL(k_cpy_transpose, dim3((unsigned) grid), dim3(CP_THREADS), 0, stream, sp, dp, s.ne[0],
                               s.ne[1], s.ne[2], tiles0, tiles1, (int64_t) s.nb[0], (int64_t) s.nb[2],
                               (int64_t) s.nb[3], (int64_t) d.nb[1], (int64_t) d.nb[2], (int64_t) d.nb[3]);
            return check_launch("cpy (transpose)");
        }
    }
#define TRC_CPY_ARGS                                                                                        \
    dim3(grid_for(n)), dim3(CP_THREADS), 0, stream, sp, dp, s.ne[0], s.ne[1], s.ne[2], rows,                \
        (int64_t) s.nb[0], (int64_t) s.nb[1], (int64_t) s.nb[2], (int64_t) s.nb[3], (int64_t) d.nb[0],      \
        (int64_t) d.nb[1], (int64_t) d.nb[2], (int64_t) d.nb[3]
    switch (es) {
        case 1: hipLaunchKernelGGL(k_cpy<uint8_t>, TRC_CPY_ARGS); break;
        case 2: hipLaunchKernelGGL(k_cpy<uint16_t>, TRC_CPY_ARGS); break;
        case 4: hipLaunchKernelGGL(k_cpy<uint32_t>, TRC_CPY_ARGS); break;
        default: hipLaunchKernelGGL(k_cpy<uint64_t>, TRC_CPY_ARGS); break;
    }
#undef TRC_CPY_ARGS
    return check_launch("cpy");
}

}  // namespace trc_hip
