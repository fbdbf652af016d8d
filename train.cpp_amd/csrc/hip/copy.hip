// Element-wise memory kernels: F32 fill (Device::fill_tensors) and the strided
// copy behind OP_DUP/OP_CPY/OP_CONT (compute_dup,
// src/backends/cpu/trc_cpu_ops.cpp:219-236). Both are HBM-bound streams.
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
