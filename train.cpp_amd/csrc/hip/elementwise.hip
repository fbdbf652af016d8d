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
// fastest, then i2, i3), one rounding to float at the end. One workgroup: each
// thread sums one row of a block of SUM_THREADS rows into LDS, then thread 0
// adds the block's row sums in order.
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

int launch_repeat_f32(const trc_hip_tensor& a, const trc_hip_tensor& d, hipStream_t s) {
    if (a.type != TRC_HIP_TYPE_F32 || d.type != TRC_HIP_TYPE_F32) return fail(TRC_HIP_E_INVALID, "repeat: F32 tensors only");
    if (!shape_ok(a) || !shape_ok(d)) return fail(TRC_HIP_E_SHAPE, "repeat: empty or negative extent");
    for (int k = 0; k < 4; ++k) {
        // ggml_can_repeat(a, dst): every dst extent a multiple of a's
        if (d.ne[k] % a.ne[k] != 0) return fail(TRC_HIP_E_SHAPE, "repeat: dst.ne[%d] is not a multiple of a.ne[%d]", k, k);
    }
    if (!f32_aligned(a) || !f32_aligned(d)) return fail(TRC_HIP_E_ALIGN, "repeat: 4-byte alignment");
    const int64_t n = nelem(d);
    hipLaunchKernelGGL(k_repeat, dim3(grid_for(n, EW_THREADS)), dim3(EW_THREADS), 0, s, (const uint8_t*) a.data,
                       shape_of(a), (uint8_t*) d.data, shape_of(d));
    return check_launch("repeat");
}

int launch_sum_f32(const trc_hip_tensor& a, const trc_hip_tensor& d, hipStream_t s) {
    if (a.type != TRC_HIP_TYPE_F32 || d.type != TRC_HIP_TYPE_F32) return fail(TRC_HIP_E_INVALID, "sum: F32 tensors only");
    if (!shape_ok(a) || !shape_ok(d)) return fail(TRC_HIP_E_SHAPE, "sum: empty or negative extent");
    if (nelem(d) != 1) return fail(TRC_HIP_E_SHAPE, "sum: dst must hold one element");
    if (!f32_aligned(a) || !f32_aligned(d)) return fail(TRC_HIP_E_ALIGN, "sum: 4-byte alignment");
    hipLaunchKernelGGL(k_sum, dim3(1), dim3(SUM_THREADS), 0, s, (const uint8_t*) a.data, shape_of(a), (float*) d.data);
    return check_launch("sum");
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
    hipLaunchKernelGGL(k_repeat_back, dim3(grid_for(n, EW_THREADS)), dim3(EW_THREADS), 0, s, (const uint8_t*) a.data,
                       shape_of(a), (float*) d.data, shape_of(d));
    return check_launch("repeat_back");
}

}  // namespace trc_hip
