// H2: fused dequant-matvec / skinny GEMM, y = mul_mat(W_quant, x) on gfx950.
//
// There is no reference kernel: the reference CPU path rejects a quantized
// src0 (src/ops/trc_ops.cpp:368), so the result it must reproduce is
// gguf_tensor_to_f32 (src/io/trc_gguf.cpp:966-1049, dequantize_q* :320-417)
// followed by compute_mul_mat (src/backends/cpu/trc_cpu_ops.cpp:182-216).
// Blocks are decoded in registers and never written back as F32. Within a
// block the scale is factored out of the dot product,
//   sum_e (q_e*d + m) * x_e = d * sum_e q_e*x_e + m * sum_e x_e,
// which reorders the reference's arithmetic; parity is by tolerance.
//
// Mapping: a wave owns R consecutive rows of W; its 64 lanes stride over the
// row's blocks (lane l takes blocks l, l+64, ...). Each lane decodes one block
// of each of the R rows once and reuses the decoded values for all N columns
// of x, so x is read once per R rows. Partial sums are reduced across the wave
// at the end and lane 0 writes the R x N outputs.
#include "common.h"

namespace trc_hip {
namespace {

constexpr int QV_THREADS = 256;
constexpr int QV_WAVES = QV_THREADS / 64;

__device__ __forceinline__ uint32_t u16_at(const uint8_t* p) { return *(const uint16_t*) p; }
__device__ __forceinline__ uint32_t u32_at_2(const uint8_t* p) {
    const uint16_t* h = (const uint16_t*) p;
    return (uint32_t) h[0] | ((uint32_t) h[1] << 16);
}
__device__ __forceinline__ uint32_t u32_at_4(const uint8_t* p) { return *(const uint32_t*) p; }

// Integer quants of one block as floats (bias already removed), plus d and m.
template <int TYPE>
__device__ __forceinline__ void decode_block(const uint8_t* blk, float q[32], float& d, float& m) {
    if constexpr (TYPE == TRC_HIP_TYPE_Q8_0) {
        d = half_bits_to_float(u16_at(blk));
        m = 0.f;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t v = u32_at_2(blk + 2 + 4 * w);
#pragma unroll
            for (int c = 0; c < 4; ++c) q[4 * w + c] = (float) (int) (int8_t) ((v >> (8 * c)) & 0xFFu);
        }
        return;
    } else {
        uint32_t qs[4];
        uint32_t qh = 0;
        float bias = 0.f;
        if constexpr (TYPE == TRC_HIP_TYPE_Q4_0) {
            d = half_bits_to_float(u16_at(blk));
            m = 0.f;
            bias = 8.f;
#pragma unroll
            for (int w = 0; w < 4; ++w) qs[w] = u32_at_2(blk + 2 + 4 * w);
        } else if constexpr (TYPE == TRC_HIP_TYPE_Q4_1) {
            const uint32_t dm = u32_at_4(blk);
            d = half_bits_to_float(dm & 0xFFFFu);
            m = half_bits_to_float(dm >> 16);
#pragma unroll
            for (int w = 0; w < 4; ++w) qs[w] = u32_at_4(blk + 4 + 4 * w);
        } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_0) {
            d = half_bits_to_float(u16_at(blk));
            m = 0.f;
            bias = 16.f;
            qh = u32_at_2(blk + 2);
#pragma unroll
            for (int w = 0; w < 4; ++w) qs[w] = u32_at_2(blk + 6 + 4 * w);
        } else {  // Q5_1
            const uint32_t dm = u32_at_4(blk);
            d = half_bits_to_float(dm & 0xFFFFu);
            m = half_bits_to_float(dm >> 16);
            qh = u32_at_4(blk + 4);
#pragma unroll
            for (int w = 0; w < 4; ++w) qs[w] = u32_at_4(blk + 8 + 4 * w);
        }
#pragma unroll
        for (int w = 0; w < 4; ++w) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = 4 * w + c;  // low nibble -> element e, high -> e + 16
                const uint32_t byte = (qs[w] >> (8 * c)) & 0xFFu;
                const uint32_t lo = (byte & 0xFu) | (((qh >> e) & 1u) << 4);
                const uint32_t hi = (byte >> 4) | (((qh >> (e + 16)) & 1u) << 4);
                q[e] = (float) lo - bias;
                q[e + 16] = (float) hi - bias;
            }
        }
    }
}

template <int TYPE, int NB, int R>
__global__ __launch_bounds__(QV_THREADS) void k_qmatvec(const uint8_t* __restrict__ W, int64_t nblk, int64_t M,
                                                        int64_t nb1_w, const float* __restrict__ x, int64_t nb1_x,
                                                        float* __restrict__ y, int64_t nb1_y, int N) {
    constexpr int BYTES = block_bytes(TYPE);
    constexpr bool HAS_MIN = TYPE == TRC_HIP_TYPE_Q4_1 || TYPE == TRC_HIP_TYPE_Q5_1;
    const int lane = threadIdx.x & 63;
    const int64_t row0 = ((int64_t) blockIdx.x * QV_WAVES + (threadIdx.x >> 6)) * R;
    if (row0 >= M) return;

    float acc[R][NB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int n = 0; n < NB; ++n) acc[r][n] = 0.f;

    for (int64_t b = lane; b < nblk; b += 64) {
        float q[R][32];
        float dd[R], mm[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (row0 + r < M) {
                decode_block<TYPE>(W + (row0 + r) * nb1_w + b * BYTES, q[r], dd[r], mm[r]);
            } else {
                dd[r] = 0.f;
                mm[r] = 0.f;
#pragma unroll
                for (int e = 0; e < 32; ++e) q[r][e] = 0.f;
            }
        }
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            if (n < N) {
                const f4* xp = (const f4*) ((const uint8_t*) x + n * nb1_x) + b * 8;
                f4 xv[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) xv[c] = xp[c];
                float xs = 0.f;
                if constexpr (HAS_MIN) {
#pragma unroll
                    for (int c = 0; c < 8; ++c) xs += (xv[c].x + xv[c].y) + (xv[c].z + xv[c].w);
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float s = 0.f;
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        s += q[r][4 * c + 0] * xv[c].x;
                        s += q[r][4 * c + 1] * xv[c].y;
                        s += q[r][4 * c + 2] * xv[c].z;
                        s += q[r][4 * c + 3] * xv[c].w;
                    }
                    acc[r][n] += dd[r] * s;
                    if constexpr (HAS_MIN) acc[r][n] += mm[r] * xs;
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            float v = acc[r][n];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            acc[r][n] = v;
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (row0 + r >= M) break;
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                if (n < N) *(float*) ((uint8_t*) y + n * nb1_y + (row0 + r) * 4) = acc[r][n];
            }
        }
    }
}

template <int TYPE, int NB, int R>
int launch_nb(const void* wq, int64_t K, int64_t M, size_t nb1_w, const float* x, int64_t N, size_t nb1_x, float* y,
              size_t nb1_y, hipStream_t stream) {
    const int64_t waves = (M + R - 1) / R;
    const int64_t grid = (waves + QV_WAVES - 1) / QV_WAVES;
    hipLaunchKernelGGL((k_qmatvec<TYPE, NB, R>), dim3((unsigned) grid), dim3(QV_THREADS), 0, stream,
                       (const uint8_t*) wq, K / QK, M, (int64_t) nb1_w, x, (int64_t) nb1_x, y, (int64_t) nb1_y,
                       (int) N);
    return check_launch("qmatvec");
}

template <int TYPE>
int launch_type(const void* wq, int64_t K, int64_t M, size_t nb1_w, const float* x, int64_t N, size_t nb1_x,
                float* y, size_t nb1_y, hipStream_t s) {
    if (N == 1) return launch_nb<TYPE, 1, 4>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, s);
    if (N == 2) return launch_nb<TYPE, 2, 4>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, s);
    if (N <= 4) return launch_nb<TYPE, 4, 2>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, s);
    if (N <= 8) return launch_nb<TYPE, 8, 2>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, s);
    return launch_nb<TYPE, 16, 2>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, s);
}

}  // namespace

int launch_qmatvec(int type, const void* wq, int64_t K, int64_t M, size_t nb1_w, const float* x, int64_t N,
                   size_t nb1_x, float* y, size_t nb1_y, hipStream_t stream) {
    const bool wide = type == TRC_HIP_TYPE_Q4_1 || type == TRC_HIP_TYPE_Q5_1;
    const unsigned walign = wide ? 3u : 1u;
    if ((((uintptr_t) wq) & walign) != 0 || (nb1_w & walign) != 0) {
        return fail(TRC_HIP_E_ALIGN, "qmatvec: W rows must be %d-byte aligned", wide ? 4 : 2);
    }
    if ((((uintptr_t) x) & 15u) != 0 || (nb1_x & 15u) != 0 || (((uintptr_t) y) & 3u) != 0 || (nb1_y & 3u) != 0) {
        return fail(TRC_HIP_E_ALIGN, "qmatvec: x columns must be 16-byte and y columns 4-byte aligned");
    }
    switch (type) {
        case TRC_HIP_TYPE_Q4_0: return launch_type<TRC_HIP_TYPE_Q4_0>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, stream);
        case TRC_HIP_TYPE_Q4_1: return launch_type<TRC_HIP_TYPE_Q4_1>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, stream);
        case TRC_HIP_TYPE_Q5_0: return launch_type<TRC_HIP_TYPE_Q5_0>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, stream);
        case TRC_HIP_TYPE_Q5_1: return launch_type<TRC_HIP_TYPE_Q5_1>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, stream);
        case TRC_HIP_TYPE_Q8_0: return launch_type<TRC_HIP_TYPE_Q8_0>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, stream);
        default: return fail(TRC_HIP_E_INVALID, "qmatvec: bad type %d", type);
    }
}

}  // namespace trc_hip
