// H2 for 2 <= N <= 16 columns: fused dequant x skinny GEMM on the int8 matrix
// cores (v_mfma_i32_16x16x32_i8).
//
// Result to reproduce: gguf_tensor_to_f32 (src/io/trc_gguf.cpp:966-1049,
// dequantize_q* :320-417) followed by compute_mul_mat
// (src/backends/cpu/trc_cpu_ops.cpp:182-216); parity is by tolerance.
//
// Numerics. Within one 32-element block b of one row m
//   sum_e (q_e*d + mn) * x_e,j = d * sum_e q_e * x_e,j + mn * sum_e x_e,j.
// x is converted once per call (k_qmm_xprep) to block fixed point: for every
// block b and column j, X_e = rint(x_e * 2^s) with s chosen so |X_e| <= 2^21,
// i.e. 22 significant bits for the block's largest |x|. X is split into three
// signed byte digits, X = P0 + 256 P1 + 65536 P2 (P0, P1 in [-128, 127],
// |P2| <= 32). The three MFMAs per block then give the exact integer sums
// sum_e q_e P_p,e; for Q4_0/Q4_1/Q5_0/Q5_1 they combine exactly into one
// int32 (|q| <= 31 keeps it below 2^31), for Q8_0 in float. One conversion and
// two float operations apply 2^-s and d. The only rounding beyond FP32's is
// the 22-bit representation of x (at most 2^-22 of the block maximum per
// element), the same order as the reference's own FP32 sum over 32 products.
// A block of x holding Inf or NaN turns its columns' outputs into NaN.
//
// Operand layout (lane l, m16 = l % 16, g = l / 16):
//   A (16 x 32, i8)  = x digits: row = column j = m16 of x, k = 8g .. 8g+7
//   B (32 x 16, i8)  = quants:   column = row m16 of the W tile, k = 8g .. 8g+7
//   D (16 x 16, i32) = lane holds rows 4g .. 4g+3 (columns j of y), column m16.
// k -> element order. Lane g's 8 k values are 4 low-nibble elements
// E(g, i) = (c + 4g + i) & 15, i = 0..3, and the 4 high-nibble elements
// 16 + E(g, i). For Q4_0, Q5_0 and Q8_0, blocks come in pairs whose second
// block starts on a 4-byte boundary: odd blocks use c = 0 and even blocks c = 2.
// With c = 2 the quant bytes a lane needs are one aligned dword, or
// (lane group 3) one v_perm of two. Q4_1/Q5_1 blocks are 4-byte aligned and
// use c = 0 throughout. k_qmm_xprep writes the x digits in the same order, so
// each lane loads its operand with one 8-byte load per digit plane.
//
// Work split: a workgroup owns up to 64 rows (T tiles of 16). Its QM_WAVES
// waves split the K pairs evenly, and each wave streams its share of the
// pairs of all T tiles with QM_DEPTH pairs of loads in flight. The partial
// sums are added across the waves through LDS in a fixed order, so results
// are deterministic. Rows per workgroup are chosen so the grid covers every
// CU once when M allows.
#include "common.h"

namespace trc_hip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int QM_MAX_BLOCKS = 2048;  // K <= 65536
constexpr int QM_WAVES = 8;
constexpr int QM_DEPTH = 2;

// x in block fixed point, written by k_qmm_xprep and read by k_qmm on the
// same stream. Planes: [block][digit 0..2][lane 0..63] 8 bytes each; scale and
// block sums: [block][column 0..15]. Calls that overlap on one GPU race.
__device__ __attribute__((aligned(256))) uint64_t g_qm_planes[QM_MAX_BLOCKS * 3 * 64];
__device__ __attribute__((aligned(256))) float g_qm_scale[QM_MAX_BLOCKS * 16];
__device__ __attribute__((aligned(256))) float g_qm_xsum[QM_MAX_BLOCKS * 16];

template <int TYPE>
constexpr bool rotated_even() {
    return TYPE == TRC_HIP_TYPE_Q4_0 || TYPE == TRC_HIP_TYPE_Q5_0 || TYPE == TRC_HIP_TYPE_Q8_0;
}

__device__ __forceinline__ uint32_t pack_bytes(const int* v) {
    return (uint32_t) (v[0] & 0xFF) | ((uint32_t) (v[1] & 0xFF) << 8) | ((uint32_t) (v[2] & 0xFF) << 16) |
           ((uint32_t) (v[3] & 0xFF) << 24);
}

// One wave per x block: lane (j, g) converts the 8 elements it feeds to the
// MFMA for column j; lanes j, j+16, j+32, j+48 share the block maximum.
__global__ __launch_bounds__(256) void k_qmm_xprep(const float* __restrict__ x, int64_t ldx, int N, int nblk,
                                                    int rot) {
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblk) return;
    const int l = threadIdx.x & 63, j = l & 15, g = l >> 4;
    const int c = (b & 1) ? 0 : rot;
    const int e0 = (c + 4 * g) & 15, e1 = (c + 4 * g + 2) & 15;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (j < N) {
        const float* col = x + j * ldx + (int64_t) b * QK;
        const float2 a0 = *(const float2*) (col + e0), a1 = *(const float2*) (col + e1);
        const float2 h0 = *(const float2*) (col + 16 + e0), h1 = *(const float2*) (col + 16 + e1);
        v[0] = a0.x; v[1] = a0.y; v[2] = a1.x; v[3] = a1.y;
        v[4] = h0.x; v[5] = h0.y; v[6] = h1.x; v[7] = h1.y;
    }
    float mx = 0.f, sm = 0.f;
    int bad = 0;  // fmaxf drops NaN, so non-finite values are flagged separately
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        mx = fmaxf(mx, fabsf(v[i]));
        sm += v[i];
        bad |= !__builtin_isfinite(v[i]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    sm += __shfl_xor(sm, 16, 64);
    sm += __shfl_xor(sm, 32, 64);
    bad |= __shfl_xor(bad, 16, 64);
    bad |= __shfl_xor(bad, 32, 64);
    const bool finite = bad == 0;
    // mx = f * 2^E, f in [0.5, 1): every |x| * 2^s < 2^21, so |X| <= 2^21
    const int s = (mx > 0.f && finite) ? 21 - __builtin_amdgcn_frexp_expf(mx) : 0;
    int d0[8], d1[8], d2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int X = finite ? (int) __builtin_rintf(__builtin_ldexpf(v[i], s)) : 0;
        const int p0 = (int) (int8_t) (X & 0xFF);
        const int X1 = (X - p0) >> 8;
        const int p1 = (int) (int8_t) (X1 & 0xFF);
        d0[i] = p0;
        d1[i] = p1;
        d2[i] = (X1 - p1) >> 8;
    }
    uint64_t* dst = g_qm_planes + (int64_t) b * 3 * 64 + l;
    dst[0] = (uint64_t) pack_bytes(d0) | ((uint64_t) pack_bytes(d0 + 4) << 32);
    dst[64] = (uint64_t) pack_bytes(d1) | ((uint64_t) pack_bytes(d1 + 4) << 32);
    dst[128] = (uint64_t) pack_bytes(d2) | ((uint64_t) pack_bytes(d2 + 4) << 32);
    if (g == 0) {
        g_qm_scale[b * 16 + j] = finite ? __builtin_ldexpf(1.f, -s) : __builtin_nanf("");
        g_qm_xsum[b * 16 + j] = sm;
    }
}

// Per format: which dwords of a pair each lane loads (NW of them) and how
// they decode into the two blocks' B operands and scales.
template <int TYPE>
struct QmFmt;

// 9 dwords: [d0 qs0.0-1][qs0 2-5]..[qs0 14-15 d1][qs1 0-3]..[qs1 12-15]
template <>
struct QmFmt<TRC_HIP_TYPE_Q4_0> {
    static constexpr int PW = 9, NW = 4;
    __device__ static void offsets(int g, int* o) {
        o[0] = 0; o[1] = 4; o[2] = g < 3 ? 1 + g : 0; o[3] = 5 + g;
    }
};
// 10 dwords: [d0 m0][qs0 x4][d1 m1][qs1 x4]
template <>
struct QmFmt<TRC_HIP_TYPE_Q4_1> {
    static constexpr int PW = 10, NW = 4;
    __device__ static void offsets(int g, int* o) {
        o[0] = 0; o[1] = 5; o[2] = 1 + g; o[3] = 6 + g;
    }
};
// 11 dwords: [d0 qh0.lo][qh0.hi qs0.0-1][qs0 2-5]..[qs0 14-15 d1][qh1][qs1 x4]
template <>
struct QmFmt<TRC_HIP_TYPE_Q5_0> {
    static constexpr int PW = 11, NW = 6;
    __device__ static void offsets(int g, int* o) {
        o[0] = 0; o[1] = 1; o[2] = 5; o[3] = 6; o[4] = g < 3 ? 2 + g : 1; o[5] = 7 + g;
    }
};
// 12 dwords: [d0 m0][qh0][qs0 x4][d1 m1][qh1][qs1 x4]
template <>
struct QmFmt<TRC_HIP_TYPE_Q5_1> {
    static constexpr int PW = 12, NW = 6;
    __device__ static void offsets(int g, int* o) {
        o[0] = 0; o[1] = 1; o[2] = 6; o[3] = 7; o[4] = 2 + g; o[5] = 8 + g;
    }
};
// 17 dwords: [d0 qs0.0-1][qs0 2-5]..[qs0 30-31 d1][qs1 0-3]..[qs1 28-31]
template <>
struct QmFmt<TRC_HIP_TYPE_Q8_0> {
    static constexpr int PW = 17, NW = 7;
    __device__ static void offsets(int g, int* o) {
        o[0] = 0; o[1] = 4; o[2] = 8; o[3] = g < 3 ? 1 + g : 0; o[4] = g < 3 ? 5 + g : 4; o[5] = 9 + g;
        o[6] = 13 + g;
    }
};

// Nibble bytes of a quant dword (low nibbles -> k 0..3, high -> k 4..7 of the
// lane group), with the 5th bits of the 4 low / 4 high elements (bits 0-3 /
// 4-7 of fifth) and the bias subtracted bytewise (no carries: values < 0x90).
template <int BIAS, bool FIVE>
__device__ __forceinline__ long nibbles(uint32_t w, uint32_t fifth) {
    uint32_t lo = w & 0x0F0F0F0Fu;
    uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
    if constexpr (FIVE) {
        lo |= ((fifth & 0xFu) * 0x02040810u) & 0x10101010u;
        hi |= (((fifth >> 4) & 0xFu) * 0x02040810u) & 0x10101010u;
    }
    if constexpr (BIAS == 8) {
        lo = (lo + 0x78787878u) ^ 0x80808080u;
        hi = (hi + 0x78787878u) ^ 0x80808080u;
    } else if constexpr (BIAS == 16) {
        lo = (lo + 0x70707070u) ^ 0x80808080u;
        hi = (hi + 0x70707070u) ^ 0x80808080u;
    }
    return (long) ((uint64_t) lo | ((uint64_t) hi << 32));
}

// 5th bits of lane group g's elements, from a block's qh rotated by c.
__device__ __forceinline__ uint32_t fifth_bits(uint32_t qh, int g) {
    return ((qh >> (4 * g)) & 0xFu) | (((qh >> (16 + 4 * g)) & 0xFu) << 4);
}
__device__ __forceinline__ uint32_t rot2_halves(uint32_t qh) {
    return ((qh >> 2) & 0x3FFF3FFFu) | ((qh << 14) & 0xC000C000u);
}

struct QmBlocks {
    long B[2];       // B operands of the even and odd block
    uint32_t dm[2];  // d (low half) and m (high half, Q4_1/Q5_1) as fp16 bits
};

template <int TYPE>
__device__ __forceinline__ QmBlocks qm_decode(const uint32_t* w, int g, uint32_t sel) {
    QmBlocks r;
    if constexpr (TYPE == TRC_HIP_TYPE_Q4_0) {
        r.B[0] = nibbles<8, false>(__builtin_amdgcn_perm(w[1], w[2], sel), 0);
        r.B[1] = nibbles<8, false>(w[3], 0);
        r.dm[0] = w[0] & 0xFFFFu;
        r.dm[1] = w[1] >> 16;
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q4_1) {
        r.B[0] = nibbles<0, false>(w[2], 0);
        r.B[1] = nibbles<0, false>(w[3], 0);
        r.dm[0] = w[0];
        r.dm[1] = w[1];
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_0) {
        const uint32_t qh0 = __builtin_amdgcn_perm(w[1], w[0], 0x05040302u);
        r.B[0] = nibbles<16, true>(__builtin_amdgcn_perm(w[2], w[4], sel), fifth_bits(rot2_halves(qh0), g));
        r.B[1] = nibbles<16, true>(w[5], fifth_bits(w[3], g));
        r.dm[0] = w[0] & 0xFFFFu;
        r.dm[1] = w[2] >> 16;
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_1) {
        r.B[0] = nibbles<0, true>(w[4], fifth_bits(w[1], g));
        r.B[1] = nibbles<0, true>(w[5], fifth_bits(w[3], g));
        r.dm[0] = w[0];
        r.dm[1] = w[2];
    } else {  // Q8_0
        const uint32_t lo = __builtin_amdgcn_perm(w[1], w[3], sel);
        const uint32_t hi = __builtin_amdgcn_perm(w[2], w[4], sel);
        r.B[0] = (long) ((uint64_t) lo | ((uint64_t) hi << 32));
        r.B[1] = (long) ((uint64_t) w[5] | ((uint64_t) w[6] << 32));
        r.dm[0] = w[0] & 0xFFFFu;
        r.dm[1] = w[2] >> 16;
    }
    return r;
}

template <int TYPE, int T>
struct QmStage {
    uint32_t w[T][QmFmt<TYPE>::NW];
    long xp[2][3];
    f4 sc[2];
    f4 xs[2];
};

template <int TYPE, int T>
__device__ __forceinline__ void qm_load(QmStage<TYPE, T>& st, const uint32_t* const* rowp, const int* off, int p,
                                        int lane, int g) {
    constexpr int PW = QmFmt<TYPE>::PW, NW = QmFmt<TYPE>::NW;
    constexpr bool MIN = TYPE == TRC_HIP_TYPE_Q4_1 || TYPE == TRC_HIP_TYPE_Q5_1;
    // x first: loads return in issue order and the x operands are needed first
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int b = 2 * p + h;
        const uint64_t* xp = g_qm_planes + (int64_t) b * 3 * 64 + lane;
#pragma unroll
        for (int d = 0; d < 3; ++d) st.xp[h][d] = (long) xp[64 * d];
        st.sc[h] = *(const f4*) (g_qm_scale + b * 16 + 4 * g);
        if constexpr (MIN) st.xs[h] = *(const f4*) (g_qm_xsum + b * 16 + 4 * g);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const uint32_t* src = rowp[t] + (int64_t) p * PW;
#pragma unroll
        for (int i = 0; i < NW; ++i) st.w[t][i] = src[off[i]];
    }
}

template <int TYPE, int T>
__device__ __forceinline__ void qm_compute(const QmStage<TYPE, T>& st, int g, uint32_t sel, f4* acc) {
    constexpr bool MIN = TYPE == TRC_HIP_TYPE_Q4_1 || TYPE == TRC_HIP_TYPE_Q5_1;
    const v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const QmBlocks q = qm_decode<TYPE>(st.w[t], g, sel);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const v4i a0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(st.xp[h][0], q.B[h], zero, 0, 0, 0);
            const v4i a1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(st.xp[h][1], q.B[h], zero, 0, 0, 0);
            const v4i a2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(st.xp[h][2], q.B[h], zero, 0, 0, 0);
            const float d = half_bits_to_float(q.dm[h] & 0xFFFFu);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float qx;
                if constexpr (TYPE == TRC_HIP_TYPE_Q8_0) {
                    qx = __builtin_fmaf((float) a2[i], 65536.f, (float) (a0[i] + a1[i] * 256));
                } else {
                    qx = (float) (a0[i] + a1[i] * 256 + a2[i] * 65536);
                }
                acc[t][i] = __builtin_fmaf(qx, d * st.sc[h][i], acc[t][i]);
                if constexpr (MIN) acc[t][i] = __builtin_fmaf(half_bits_to_float(q.dm[h] >> 16), st.xs[h][i], acc[t][i]);
            }
        }
    }
}

template <int TYPE, int T>
__global__ __launch_bounds__(QM_WAVES * 64) void k_qmm(const uint8_t* __restrict__ W, int nblk, int64_t M,
                                                        int64_t nb1_w, float* __restrict__ y, int64_t ldy, int N,
                                                        int rows_per_wg) {
    __shared__ f4 red[QM_WAVES][T][64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, m16 = lane & 15, g = lane >> 4;
    const int64_t r0 = (int64_t) blockIdx.x * rows_per_wg;
    const int64_t rend = r0 + rows_per_wg < M ? r0 + rows_per_wg : M;
    const int np = nblk / 2;
    const int p_begin = (int) ((int64_t) np * wave / QM_WAVES);
    const int p_end = (int) ((int64_t) np * (wave + 1) / QM_WAVES);
    const uint32_t sel = g < 3 ? 0x03020100u : 0x03020504u;

    const uint32_t* rowp[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int64_t m = r0 + 16 * t + m16;
        rowp[t] = (const uint32_t*) (W + (m < rend ? m : r0) * nb1_w);  // masked rows read row r0
    }
    int off[QmFmt<TYPE>::NW];
    QmFmt<TYPE>::offsets(g, off);

    f4 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};

    if (p_begin < p_end) {
        QmStage<TYPE, T> st[QM_DEPTH];
#pragma unroll
        for (int d = 0; d < QM_DEPTH; ++d) {
            const int p = p_begin + d < p_end ? p_begin + d : p_end - 1;
            qm_load<TYPE, T>(st[d], rowp, off, p, lane, g);
        }
        int p = p_begin;
        for (; p + QM_DEPTH <= p_end; p += QM_DEPTH) {
#pragma unroll
            for (int d = 0; d < QM_DEPTH; ++d) {
                const QmStage<TYPE, T> cur = st[d];
                const int pn = p + d + QM_DEPTH < p_end ? p + d + QM_DEPTH : p_end - 1;  // in bounds
                qm_load<TYPE, T>(st[d], rowp, off, pn, lane, g);
                qm_compute<TYPE, T>(cur, g, sel, acc);
            }
        }
#pragma unroll
        for (int d = 0; d < QM_DEPTH; ++d) {
            if (p + d < p_end) qm_compute<TYPE, T>(st[d], g, sel, acc);
        }
    }

#pragma unroll
    for (int t = 0; t < T; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    if (wave >= T) return;
    const int t = wave;
    f4 sum = red[0][t][lane];
#pragma unroll
    for (int w = 1; w < QM_WAVES; ++w) sum += red[w][t][lane];
    const int64_t m = r0 + 16 * t + m16;
    if (m >= rend) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int j = 4 * g + i;
        if (j < N) y[j * ldy + m] = sum[i];
    }
}

template <int TYPE, int T>
int launch_t(const void* wq, int nblk, int64_t M, size_t nb1_w, float* y, size_t nb1_y, int N, int rows,
             hipStream_t s) {
    const int64_t grid = (M + rows - 1) / rows;
    hipLaunchKernelGGL((k_qmm<TYPE, T>), dim3((unsigned) grid), dim3(QM_WAVES * 64), 0, s, (const uint8_t*) wq,
                       nblk, M, (int64_t) nb1_w, y, (int64_t) (nb1_y / sizeof(float)), N, rows);
    return check_launch("qmm");
}

template <int TYPE>
int launch_fmt(const void* wq, int nblk, int64_t M, size_t nb1_w, const float* x, size_t nb1_x, int N, float* y,
               size_t nb1_y, hipStream_t s) {
    hipLaunchKernelGGL(k_qmm_xprep, dim3((unsigned) ((nblk + 3) / 4)), dim3(256), 0, s, x,
                       (int64_t) (nb1_x / sizeof(float)), N, nblk, rotated_even<TYPE>() ? 2 : 0);
    const int rc = check_launch("qmm_xprep");
    if (rc != TRC_HIP_OK) return rc;
    // rows per workgroup: one workgroup per CU when M allows, 8-row granularity, at most 64
    const int64_t cus = device_cus();
    int64_t rows = (M + cus - 1) / cus;
    rows = (rows + 7) / 8 * 8;
    if (rows > 64) rows = 64;
    const int T = (int) ((rows + 15) / 16);
    switch (T) {
        case 1: return launch_t<TYPE, 1>(wq, nblk, M, nb1_w, y, nb1_y, N, (int) rows, s);
        case 2: return launch_t<TYPE, 2>(wq, nblk, M, nb1_w, y, nb1_y, N, (int) rows, s);
        case 3: return launch_t<TYPE, 3>(wq, nblk, M, nb1_w, y, nb1_y, N, (int) rows, s);
        default: return launch_t<TYPE, 4>(wq, nblk, M, nb1_w, y, nb1_y, N, (int) rows, s);
    }
}

}  // namespace

bool qmm_supported(int64_t K, int64_t N, const void* wq, size_t nb1_w) {
    const int64_t nblk = K / QK;
    return N >= 2 && N <= 16 && nblk >= 2 && nblk % 2 == 0 && nblk <= QM_MAX_BLOCKS &&
           (((uintptr_t) wq) & 3u) == 0 && (nb1_w & 3u) == 0;
}

int launch_qmm(int type, const void* wq, int64_t K, int64_t M, size_t nb1_w, const float* x, int64_t N,
               size_t nb1_x, float* y, size_t nb1_y, hipStream_t s) {
    const int nblk = (int) (K / QK);
    switch (type) {
        case TRC_HIP_TYPE_Q4_0: return launch_fmt<TRC_HIP_TYPE_Q4_0>(wq, nblk, M, nb1_w, x, nb1_x, (int) N, y, nb1_y, s);
        case TRC_HIP_TYPE_Q4_1: return launch_fmt<TRC_HIP_TYPE_Q4_1>(wq, nblk, M, nb1_w, x, nb1_x, (int) N, y, nb1_y, s);
        case TRC_HIP_TYPE_Q5_0: return launch_fmt<TRC_HIP_TYPE_Q5_0>(wq, nblk, M, nb1_w, x, nb1_x, (int) N, y, nb1_y, s);
        case TRC_HIP_TYPE_Q5_1: return launch_fmt<TRC_HIP_TYPE_Q5_1>(wq, nblk, M, nb1_w, x, nb1_x, (int) N, y, nb1_y, s);
        case TRC_HIP_TYPE_Q8_0: return launch_fmt<TRC_HIP_TYPE_Q8_0>(wq, nblk, M, nb1_w, x, nb1_x, (int) N, y, nb1_y, s);
        default: return fail(TRC_HIP_E_INVALID, "qmm: bad type %d", type);
    }
}

}  // namespace trc_hip
