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
// Kernels in this file (launch_type picks one per call):
//   - k_qmatvec_dot: N = 1..4 on the packed integer dot instructions (below),
//     weights through LDS when rows are 16-byte aligned;
//   - k_qmatvec_kslots: the same arithmetic for one or two columns when K spans
//     2..4 chunks of 4096 elements, one chunk per wave;
//   - k_qmatvec_n1 / k_qmatvec: FP32 kernels for the shapes the integer-dot
//     kernels do not take (odd block counts, misaligned x). In k_qmatvec a wave
//     owns R consecutive rows of W and its 64 lanes stride over a row's blocks
//     (lane l takes blocks l, l+64, ...); each lane decodes one block of each
//     row once and reuses it for all N columns, and the partial sums are
//     reduced across the wave at the end.
// N from 4 (5 for the formats other than Q4_0) to 32 goes to the fp16 matrix-core
// kernel in qmm.hip.
#include "common.h"

#include <type_traits>

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

// ---------------------------------------------------------------- N = 1 (decode) kernel
//
// The batch-1 product is a pure stream over W, so this kernel is organised
// around moving W at full HBM rate:
//   - W is staged through LDS with fully coalesced dwordx4 loads: a wave copies
//     ROWS row-chunks of CH blocks (CH*BYTES bytes each, a multiple of 16) with
//     every lane issuing all of its loads before its LDS writes.
//   - Each lane then decodes one pair of adjacent blocks per row from LDS.
//     A pair starts on a 4-byte boundary for every format (2*BYTES is a
//     multiple of 4), so the decode uses aligned dword reads and byte-align
//     shifts, never unaligned accesses.
//   - A lane always owns the same pair column, so its 64 x values and their
//     per-block sums stay in registers for every row the wave processes; with
//     K = 32*CH (4096) they are loaded once per wave for the whole launch.
//   - The integer quants are converted with v_cvt_f32_ubyte (1 op per element);
//     the bias (8, 16, or 128 for Q8_0 after flipping the sign bits) is removed
//     once per block through the block's x sum.
// Waves are persistent over tiles of ROWS rows and only synchronise with
// themselves (each wave owns its LDS region).

constexpr int QV1_WAVES = 4;
constexpr int QV1_CH = 128;  // blocks per staged row chunk

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t align2(uint32_t hi, uint32_t lo) {
    return __builtin_amdgcn_alignbyte(hi, lo, 2);  // bytes 2..5 of {hi:lo}
}

__device__ __forceinline__ uint32_t spread4(uint32_t four) {  // bits 0..3 -> bit 4 of bytes 0..3
    return ((four & 1u) << 4) | ((four & 2u) << 11) | ((four & 4u) << 18) | ((four & 8u) << 25);
}

// sum_{c<4} byte_c(q) * x[c]
__device__ __forceinline__ float dot4_ub(uint32_t q, f4 x, float acc) {
    acc += (float) (q & 0xFFu) * x.x;
    acc += (float) ((q >> 8) & 0xFFu) * x.y;
    acc += (float) ((q >> 16) & 0xFFu) * x.z;
    acc += (float) (q >> 24) * x.w;
    return acc;
}

// One decoded block in registers: scale bits, min bits, 5th-bit mask, quant words.
struct Blk {
    uint32_t d, m, qh;
    uint32_t q[8];
};

// Extracts the two blocks of a pair from its aligned dwords (pw = pair start).
template <int TYPE>
__device__ __forceinline__ void read_pair(const uint32_t* pw, Blk& A, Blk& B) {
    if constexpr (TYPE == TRC_HIP_TYPE_Q4_0) {  // 36 B: A at 0, B at 18
        uint32_t w[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) w[i] = pw[i];
        A.d = w[0] & 0xFFFFu;
#pragma unroll
        for (int i = 0; i < 4; ++i) A.q[i] = align2(w[i + 1], w[i]);
        B.d = w[4] >> 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) B.q[i] = w[5 + i];
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q4_1) {  // 40 B: A at 0, B at 20
        uint32_t w[10];
#pragma unroll
        for (int i = 0; i < 10; ++i) w[i] = pw[i];
        A.d = w[0] & 0xFFFFu;
        A.m = w[0] >> 16;
        B.d = w[5] & 0xFFFFu;
        B.m = w[5] >> 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            A.q[i] = w[1 + i];
            B.q[i] = w[6 + i];
        }
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_0) {  // 44 B: A at 0, B at 22
        uint32_t w[11];
#pragma unroll
        for (int i = 0; i < 11; ++i) w[i] = pw[i];
        A.d = w[0] & 0xFFFFu;
        A.qh = align2(w[1], w[0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) A.q[i] = align2(w[i + 2], w[i + 1]);
        B.d = w[5] >> 16;
        B.qh = w[6];
#pragma unroll
        for (int i = 0; i < 4; ++i) B.q[i] = w[7 + i];
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_1) {  // 48 B: A at 0, B at 24
        uint32_t w[12];
#pragma unroll
        for (int i = 0; i < 12; ++i) w[i] = pw[i];
        A.d = w[0] & 0xFFFFu;
        A.m = w[0] >> 16;
        A.qh = w[1];
        B.d = w[6] & 0xFFFFu;
        B.m = w[6] >> 16;
        B.qh = w[7];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            A.q[i] = w[2 + i];
            B.q[i] = w[8 + i];
        }
    } else {  // Q8_0, 68 B: A at 0, B at 34
        uint32_t w[17];
#pragma unroll
        for (int i = 0; i < 17; ++i) w[i] = pw[i];
        A.d = w[0] & 0xFFFFu;
#pragma unroll
        for (int i = 0; i < 8; ++i) A.q[i] = align2(w[i + 1], w[i]);
        B.d = w[8] >> 16;
#pragma unroll
        for (int i = 0; i < 8; ++i) B.q[i] = w[9 + i];
    }
}

// d * sum_e q_e x_e (+ m * sum_e x_e) for one block; xv holds the block's 32 x
// values as 8 float4 (elements 4c..4c+3), xs their sum.
template <int TYPE>
__device__ __forceinline__ float block_dot(const Blk& b, const f4* xv, float xs) {
    float s = 0.f;
    if constexpr (TYPE == TRC_HIP_TYPE_Q8_0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) s = dot4_ub(b.q[i] ^ 0x80808080u, xv[i], s);  // q + 128 as unsigned
        return half_bits_to_float(b.d) * (s - 128.f * xs);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t lo = b.q[i] & 0x0F0F0F0Fu;
            uint32_t hi = (b.q[i] >> 4) & 0x0F0F0F0Fu;
            if constexpr (TYPE == TRC_HIP_TYPE_Q5_0 || TYPE == TRC_HIP_TYPE_Q5_1) {
                lo |= spread4((b.qh >> (4 * i)) & 0xFu);
                hi |= spread4((b.qh >> (16 + 4 * i)) & 0xFu);
            }
            s = dot4_ub(lo, xv[i], s);
            s = dot4_ub(hi, xv[4 + i], s);
        }
        const float d = half_bits_to_float(b.d);
        if constexpr (TYPE == TRC_HIP_TYPE_Q4_0) return d * (s - 8.f * xs);
        if constexpr (TYPE == TRC_HIP_TYPE_Q5_0) return d * (s - 16.f * xs);
        return d * s + half_bits_to_float(b.m) * xs;  // Q4_1, Q5_1
    }
}

template <int TYPE, int ROWS, int HALF>
__global__ __launch_bounds__(QV1_WAVES * 64) void k_qmatvec_n1(const uint8_t* __restrict__ W, int64_t nblk,
                                                              int64_t M, int64_t nb1_w,
                                                              const float* __restrict__ x,
                                                              float* __restrict__ y) {
    constexpr int BYTES = block_bytes(TYPE);
    constexpr int CHB = QV1_CH * BYTES;  // staged bytes per row chunk
    constexpr int F4R = CHB / 16;        // float4s per row chunk
    constexpr int NPH = HALF * F4R / 64; // float4s per lane for HALF rows
    constexpr int PARTS = ROWS / HALF;
    static_assert(CHB % 16 == 0 && (HALF * F4R) % 64 == 0 && ROWS % HALF == 0, "staging must split evenly");
    __shared__ __attribute__((aligned(16))) uint8_t stage[QV1_WAVES * HALF * CHB];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    uint8_t* my = stage + wave * HALF * CHB;
    const int64_t nchunks = (nblk + QV1_CH - 1) / QV1_CH;
    const int64_t ntiles = (M + ROWS - 1) / ROWS;
    const int64_t nwaves = (int64_t) gridDim.x * QV1_WAVES;

    f4 xv[16];
    float xs[2];
    auto load_x = [&](int64_t c) {
        const int64_t b0 = c * QV1_CH + 2 * lane;  // first block of this lane's pair
        if (b0 < nblk) {
            const f4* xp = (const f4*) (x + b0 * QK);
#pragma unroll
            for (int i = 0; i < 16; ++i) xv[i] = xp[i];
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) xv[i] = f4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) s += (xv[8 * h + i].x + xv[8 * h + i].y) + (xv[8 * h + i].z + xv[8 * h + i].w);
            xs[h] = s;
        }
    };

    // rows [r0, r0 + HALF) of the current tile are in LDS: accumulate them
    auto compute_half = [&](float* acc, int64_t row0, int r0, int64_t cb) {
        if (2 * lane < cb) {
#pragma unroll
            for (int r = 0; r < HALF; ++r) {
                if (row0 + r0 + r < M) {
                    Blk A, B;
                    read_pair<TYPE>((const uint32_t*) (my + r * CHB + lane * 2 * BYTES), A, B);
                    acc[r0 + r] += block_dot<TYPE>(A, xv, xs[0]) + block_dot<TYPE>(B, xv + 8, xs[1]);
                }
            }
        }
    };

    for (int64_t tile = (int64_t) blockIdx.x * QV1_WAVES + wave; tile < ntiles; tile += nwaves) {
        const int64_t row0 = tile * ROWS;
        float acc[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) acc[r] = 0.f;

        for (int64_t c = 0; c < nchunks; ++c) {
            const int64_t cb = nblk - c * QV1_CH < QV1_CH ? nblk - c * QV1_CH : QV1_CH;
            const uint8_t* src = W + row0 * nb1_w + c * CHB;
            if (cb == QV1_CH && row0 + ROWS <= M) {
                // whole tile: issue every load of the tile (and x) before using any
                f4 t[PARTS * NPH];
#pragma unroll
                for (int k = 0; k < PARTS * NPH; ++k) {
                    const int i = lane + 64 * k;
                    t[k] = *(const f4*) (src + (i / F4R) * nb1_w + (i % F4R) * 16);
                }
                if (c == 0 || nchunks > 1) {
                    if (tile == (int64_t) blockIdx.x * QV1_WAVES + wave || nchunks > 1) load_x(c);
                }
#pragma unroll
                for (int p = 0; p < PARTS; ++p) {
                    wave_lds_sync();  // every lane is done reading the previous part
#pragma unroll
                    for (int k = 0; k < NPH; ++k) ((f4*) my)[lane + 64 * k] = t[p * NPH + k];
                    wave_lds_sync();  // the staged part is visible to every lane
                    compute_half(acc, row0, p * HALF, cb);
                }
            } else {
                if (tile == (int64_t) blockIdx.x * QV1_WAVES + wave || nchunks > 1) load_x(c);
                const int nf4 = (int) (cb * BYTES / 16);
                for (int p = 0; p < PARTS; ++p) {
                    wave_lds_sync();
                    for (int r = 0; r < HALF; ++r) {
                        if (row0 + p * HALF + r >= M) break;
                        for (int f = lane; f < nf4; f += 64) {
                            ((f4*) (my + r * CHB))[f] = *(const f4*) (src + (p * HALF + r) * nb1_w + f * 16);
                        }
                    }
                    wave_lds_sync();
                    compute_half(acc, row0, p * HALF, cb);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            float v = acc[r];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            acc[r] = v;
        }
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                if (row0 + r < M) y[row0 + r] = acc[r];
            }
        }
    }
}

// ---------------------------------------------------------------- N = 1..4, integer-dot kernels
//
// The FP32 formulation costs about 2.4 VALU operations per weight element
// (convert the nibble, multiply-add, unpack), which makes a batch-1 matvec
// VALU-bound on gfx950 well before it is HBM-bound. This kernel moves the
// multiply-adds onto the packed integer dot instructions instead:
//
//   - Each workgroup converts its chunk of x (4096 elements) once to block
//     fixed point: per 32-element block b, X_e = rint(x_e * 2^s_b) with s_b
//     chosen so |X_e| < 2^22, i.e. a 24-bit two's-complement integer with 22
//     significant bits for the block maximum. Planes, 2^-s_b and the block
//     sums of x go to LDS, then into each lane's registers.
//   - Q4_0 / Q4_1 (4-bit path): X is split into six balanced 4-bit digits, the
//     digit planes are laid out in the quant words' own nibble order, and the
//     quant words XOR 0x88888888 (signed q - 8) go straight into
//     v_dot8_i32_i4: no nibble unpacking and no bias term, and the digit sums
//     combine exactly in int32.
//   - Q5_0 / Q5_1 / Q8_0 (byte path): the three bytes of every X_e are
//     transposed into byte planes; Q5 quant words are split into nibble bytes
//     with the fifth bit added (v_dot4_u32_u8 on the low planes,
//     v_dot4_i32_i8 on the signed top plane); Q8_0 quants meet balanced signed
//     byte digits of X with v_dot4_i32_i8. The plane sums are combined in
//     float; the bias (16) and the min (Q5_1) go through the block sum of x.
//   - The only rounding beyond FP32's is the 24-bit representation of x, whose
//     error per element is at most 2^-23 of the block's largest |x|; the
//     reference's own sequential FP32 sum of 32 products carries an error
//     bound of the same order.
//   - Each lane owns one pair of blocks of the chunk for every row its wave
//     processes (pairs start on 4-byte boundaries for all formats). A wave
//     handles at most QD_RMAX rows strided over all waves, with one or two
//     rows of loads in flight; each row's part of a chunk is reduced across
//     the wave as soon as it is computed and added into lane r, and the wave
//     stores all its rows with one instruction after its last load.

constexpr int QD_CH = 128;        // blocks per chunk of K (one lane = one pair)
constexpr int QD_RMAX = 8;        // rows per wave at most
// Rows whose loads are in flight per wave, as measured (K=4096, M=14336 and
// K=14336, M=4096): two for one column of a 4- or 5-bit format (one row adds
// 0.5 us per call, a third 0.1-0.5 us); one for Q8_0's 34-byte blocks, for two
// columns, and when the grid takes more than one workgroup per CU (the smaller
// LDS ring then lets two workgroups share a CU).
constexpr int qd_prefetch(int type, int nc, bool dma, bool crowded) {
    if (!dma) return type == TRC_HIP_TYPE_Q8_0 ? 1 : 2;
    return crowded || nc > 1 || type == TRC_HIP_TYPE_Q8_0 ? 1 : 2;
}
constexpr int QD_PSTRIDE = 52;    // LDS dwords per pair of planes (48 + 4: conflict-free b128 reads)
constexpr int QD_WAVES = 8;       // waves per workgroup: one x conversion serves 8 waves

template <int TYPE>
struct QdFmt {
    static constexpr int BYTES = block_bytes(TYPE);
    static constexpr int PAIR_WORDS = 2 * BYTES / 4;  // 9, 10, 11, 12, 17
};

// x chunk -> byte planes in LDS. Thread t converts elements [16t, 16t+16) of
// the chunk: half h = t&1 of block b = t>>1 (partner lane t^1 holds the other half).
// x of a chunk through a buffer range of its cb blocks: threads past a short
// (or empty) chunk read zeros from the range check, with no memory access and
// no branch (loads under a branch make the compiler's wait counts fall back to
// full waits, which serialised the x loads of several chunks).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t qd_x_range(const float* xc, int64_t cb) {
    // raw 32-bit dwords (gfx9 buffer resource word 3), cb blocks of 32 floats
    return __builtin_amdgcn_make_buffer_rsrc((void*) xc, (short) 0, (int) cb * QK * 4, 0x00020000u);
}

__device__ __forceinline__ void qd_load_x(const float* __restrict__ xc, int64_t cb, f4* v) {
    const int t = threadIdx.x;
    const __amdgpu_buffer_rsrc_t rs = qd_x_range(xc, cb);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t) (4 * t + i) * 16, 0, 0));
    }
}

// SIGNED: balanced digits X = D0 + 256 D1 + 65536 D2 with every D in [-128, 127]
// (for the signed Q8_0 quants and v_dot4_i32_i8): the bytes of U = X + 0x808080
// (0 < U < 2^24) are D + 128, so the planes of U with each byte's top bit
// flipped are the digits. Otherwise P0, P1 are the unsigned low bytes of X and
// P2 its signed top byte (for the unsigned nibble quants and v_dot4_u32_u8).
// Lane exchange inside a quad (DPP quad_perm; VALU latency, no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float qd_quad_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int qd_quad_i(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}
constexpr int QD_XOR1 = 0xB1;  // quad_perm [1,0,3,2]: lane ^ 1
constexpr int QD_XOR2 = 0x4E;  // quad_perm [2,3,0,1]: lane ^ 2

// PS: LDS dwords per pair of planes (48, or QD_PSTRIDE with the padding that
// makes the once-per-chunk 16-byte reads conflict-free).
template <bool SIGNED, int PS = QD_PSTRIDE>
__device__ __forceinline__ void qd_prologue(const f4* v, int64_t cb, uint32_t* planes, float* scale, float* xsum) {
    const int t = threadIdx.x;
    const int b = t >> 1, h = t & 1;
    const bool active = b < cb;
    float mx = 0.f, sm = 0.f;
    int bad = 0;  // fmaxf drops NaN, so non-finite values are flagged separately
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
        sm += (v[i].x + v[i].y) + (v[i].z + v[i].w);
        bad |= !__builtin_isfinite(v[i].x) | !__builtin_isfinite(v[i].y) | !__builtin_isfinite(v[i].z) |
               !__builtin_isfinite(v[i].w);
    }
    mx = fmaxf(mx, qd_quad_f<QD_XOR1>(mx));
    sm += qd_quad_f<QD_XOR1>(sm);
    bad |= qd_quad_i<QD_XOR1>(bad);
    const bool finite = bad == 0;
    // s = 22 - E with mx = f * 2^E, f in [0.5, 1): every |x| * 2^s < 2^22. At most
    // 149, so that 2^-s stays a float: below 2^-127 every x is a multiple of 2^-149,
    // and x * 2^149 is then an exact integer under 2^22.
    const int s = (mx > 0.f && finite) ? min(22 - __builtin_amdgcn_frexp_expf(mx), 149) : 0;
    uint32_t P[3][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        constexpr uint32_t U = SIGNED ? 0x808080u : 0u;
        const uint32_t a = (uint32_t) (int) __builtin_rintf(__builtin_ldexpf(v[i].x, s)) + U;
        const uint32_t bb = (uint32_t) (int) __builtin_rintf(__builtin_ldexpf(v[i].y, s)) + U;
        const uint32_t c = (uint32_t) (int) __builtin_rintf(__builtin_ldexpf(v[i].z, s)) + U;
        const uint32_t d = (uint32_t) (int) __builtin_rintf(__builtin_ldexpf(v[i].w, s)) + U;
        const uint32_t t_ab = __builtin_amdgcn_perm(bb, a, 0x05010400u);  // a0 b0 a1 b1
        const uint32_t t_cd = __builtin_amdgcn_perm(d, c, 0x05010400u);   // c0 d0 c1 d1
        P[0][i] = __builtin_amdgcn_perm(t_cd, t_ab, 0x05040100u);         // a0 b0 c0 d0
        P[1][i] = __builtin_amdgcn_perm(t_cd, t_ab, 0x07060302u);         // a1 b1 c1 d1
        P[2][i] = __builtin_amdgcn_perm(bb, a, 0x0c0c0602u) | __builtin_amdgcn_perm(d, c, 0x06020c0cu);  // a2 b2 c2 d2
        if constexpr (SIGNED) {
#pragma unroll
            for (int p = 0; p < 3; ++p) P[p][i] ^= 0x80808080u;
        }
    }
    if (active) {
        // pair l = b>>1; within the pair, block (b&1) owns groups 8*(b&1) .. +7:
        // groups 0-3 are elements 0-15 (half 0), groups 4-7 elements 16-31 (half 1)
        uint32_t* dst = planes + (b >> 1) * PS + 8 * (b & 1) + 4 * h;
#pragma unroll
        for (int p = 0; p < 3; ++p) {
            *(uint4*) (dst + 16 * p) = uint4{P[p][0], P[p][1], P[p][2], P[p][3]};
        }
        if (h == 0) {
            scale[b] = finite ? __builtin_ldexpf(1.f, -s) : __builtin_nanf("");
            xsum[b] = sm;
        }
    }
}

// Bytes 0..2 of four 24-bit values, transposed: out[b] = byte b of (a, b_, c, d).
__device__ __forceinline__ void bytes3_of4(uint32_t a, uint32_t b_, uint32_t c, uint32_t d, uint32_t* out) {
    const uint32_t t_ab = __builtin_amdgcn_perm(b_, a, 0x05010400u);  // a0 b0 a1 b1
    const uint32_t t_cd = __builtin_amdgcn_perm(d, c, 0x05010400u);   // c0 d0 c1 d1
    out[0] = __builtin_amdgcn_perm(t_cd, t_ab, 0x05040100u);          // a0 b0 c0 d0
    out[1] = __builtin_amdgcn_perm(t_cd, t_ab, 0x07060302u);          // a1 b1 c1 d1
    out[2] = __builtin_amdgcn_perm(b_, a, 0x0c0c0602u) | __builtin_amdgcn_perm(d, c, 0x06020c0cu);  // a2 b2 c2 d2
}

// 4-bit path (Q4_0, Q4_1): X = D0 + 16 D1 + ... + 16^5 D5 with balanced digits
// D in [-8, 7] (the nibbles of (X + 0x888888) ^ 0x888888), stored as six digit
// planes whose words follow the quant words' own nibble order: quant byte j
// holds element j (low nibble) and j + 16 (high nibble), so plane word g of a
// block pairs element j with its low and j + 16 with its high nibble for the 4
// bytes j of quant word g. Order B: word g = quant bytes 4g..4g+3. Order A (the
// even block of a Q4_0 pair, whose quant bytes start 2 bytes into a dword):
// word 0 = bytes 0, 1, 14, 15 and word g = bytes 4g-2..4g+1. The quant words,
// XOR 0x88888888, become the signed nibbles q - 8, so v_dot8_i32_i4 gives
// sum_e (q_e - 8) * X_e exactly in six digit sums.
//
// All QD_WAVES waves convert: thread t builds plane word g = t&3 of block t>>2
// for the six planes from the 8 elements it needs (two pairs of low elements
// and the same pairs + 16), loaded as float2; the block maximum, sum and
// finiteness are reduced over the 4 threads of the block.
struct QdX4 {
    float2 v[4];  // low pair 0, low pair 1, high pair 0, high pair 1
};
static_assert(QD_WAVES * 64 == 4 * QD_CH, "four converting threads per block of a chunk");

template <bool ORDER_A_EVEN>
__device__ __forceinline__ void qd_load_x_n4(const float* __restrict__ xc, int64_t cb, QdX4& x) {
    const int t = threadIdx.x;
    const int b = t >> 2, g = t & 3;
    const bool order_a = ORDER_A_EVEN && (b & 1) == 0;
    const int j0 = order_a ? (g == 0 ? 0 : 4 * g - 2) : 4 * g;
    const int j1 = order_a ? (g == 0 ? 14 : 4 * g) : 4 * g + 2;
    // zeros past a short chunk from the range check (see qd_load_x)
    const __amdgpu_buffer_rsrc_t rs = qd_x_range(xc, cb);
    const uint32_t base = (uint32_t) (32 * b) * 4;
    const int js[4] = {j0, j1, j0 + 16, j1 + 16};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        x.v[k] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rs, base + (uint32_t) (js[k] >> 1) * 8, 0, 0));
    }
}

template <int PS = QD_PSTRIDE>
__device__ __forceinline__ void qd_prologue_n4(const QdX4& x, int64_t cb, uint32_t* planes, float* scale, float* xsum) {
    const int t = threadIdx.x;
    const int b = t >> 2, g = t & 3;
    float mx = 0.f, sm = 0.f;
    int bad = 0;  // fmaxf drops NaN, so non-finite values are flagged separately
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        mx = fmaxf(mx, fmaxf(fabsf(x.v[i].x), fabsf(x.v[i].y)));
        sm += x.v[i].x + x.v[i].y;
        bad |= !__builtin_isfinite(x.v[i].x) | !__builtin_isfinite(x.v[i].y);
    }
    mx = fmaxf(mx, qd_quad_f<QD_XOR1>(mx));
    sm += qd_quad_f<QD_XOR1>(sm);
    bad |= qd_quad_i<QD_XOR1>(bad);
    mx = fmaxf(mx, qd_quad_f<QD_XOR2>(mx));
    sm += qd_quad_f<QD_XOR2>(sm);
    bad |= qd_quad_i<QD_XOR2>(bad);
    const bool finite = bad == 0;
    // s = 22 - E with mx = f * 2^E, f in [0.5, 1): every |x| * 2^s < 2^22. At most
    // 149, so that 2^-s stays a float: below 2^-127 every x is a multiple of 2^-149,
    // and x * 2^149 is then an exact integer under 2^22.
    const int s = (mx > 0.f && finite) ? min(22 - __builtin_amdgcn_frexp_expf(mx), 149) : 0;
    uint32_t U[8];  // low elements 0-3, high elements 4-7
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int k = (i & 1) * 2 + (i >> 1) * 4;  // v[0] -> U0,1; v[1] -> U2,3; v[2] -> U4,5; v[3] -> U6,7
        const uint32_t a0 = (uint32_t) (int) __builtin_rintf(__builtin_ldexpf(x.v[i].x, s));
        const uint32_t a1 = (uint32_t) (int) __builtin_rintf(__builtin_ldexpf(x.v[i].y, s));
        U[k] = (a0 + 0x888888u) ^ 0x888888u;
        U[k + 1] = (a1 + 0x888888u) ^ 0x888888u;
    }
    if (b < cb) {
        uint32_t BL[3], BH[3];
        bytes3_of4(U[0], U[1], U[2], U[3], BL);
        bytes3_of4(U[4], U[5], U[6], U[7], BH);
        uint32_t* dst = planes + (b >> 1) * PS + 24 * (b & 1) + g;
#pragma unroll
        for (int y = 0; y < 3; ++y) {
            dst[8 * y] = (BL[y] & 0x0F0F0F0Fu) | ((BH[y] & 0x0F0F0F0Fu) << 4);
            dst[8 * y + 4] = ((BL[y] >> 4) & 0x0F0F0F0Fu) | (BH[y] & 0xF0F0F0F0u);
        }
        if (g == 0) {
            scale[b] = finite ? __builtin_ldexpf(1.f, -s) : __builtin_nanf("");
            xsum[b] = sm;
        }
    }
}

template <int TYPE>
__device__ __forceinline__ void qd_unpack(uint32_t w, uint32_t qh_bits8, uint32_t& lo, uint32_t& hi) {
    lo = w & 0x0F0F0F0Fu;
    hi = (w >> 4) & 0x0F0F0F0Fu;
    if constexpr (TYPE == TRC_HIP_TYPE_Q5_0 || TYPE == TRC_HIP_TYPE_Q5_1) {
        // qh_bits8: bits 0-3 = 5th bits of the 4 low elements, bits 4-7 of the 4 high ones
        lo |= ((qh_bits8 & 0xFu) * 0x00204081u & 0x01010101u) << 4;
        hi |= (((qh_bits8 >> 4) & 0xFu) * 0x00204081u & 0x01010101u) << 4;
    }
}

// One block of one row: 4 quant words against this lane's 8 plane groups.
template <int TYPE>
__device__ __forceinline__ float qd_block(const uint32_t* q, uint32_t qh, uint32_t d_bits, uint32_t m_bits,
                                          const uint32_t (*P)[8], float scale, float xs) {
    // six independent accumulation chains (plane x low/high nibble)
    uint32_t s0 = 0, s1 = 0, t0 = 0, t1 = 0;
    int s2 = 0, t2 = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t lo, hi;
        const uint32_t bits = ((qh >> (4 * w)) & 0xFu) | (((qh >> (16 + 4 * w)) & 0xFu) << 4);
        qd_unpack<TYPE>(q[w], bits, lo, hi);
        s0 = __builtin_amdgcn_udot4(lo, P[0][w], s0, false);
        s1 = __builtin_amdgcn_udot4(lo, P[1][w], s1, false);
        s2 = __builtin_amdgcn_sdot4((int) lo, (int) P[2][w], s2, false);
        t0 = __builtin_amdgcn_udot4(hi, P[0][4 + w], t0, false);
        t1 = __builtin_amdgcn_udot4(hi, P[1][4 + w], t1, false);
        t2 = __builtin_amdgcn_sdot4((int) hi, (int) P[2][4 + w], t2, false);
    }
    s0 += t0;
    s1 += t1;
    s2 += t2;
    // sum_e q_e X_e = s0 + 256 s1 + 65536 s2. s0 and s1 stay under 32 * 31 * 255 < 2^18,
    // so both convert exactly and s0 + 256 s1 rounds once, in the first fma.
    const float qx = __builtin_fmaf((float) s2, 65536.f, __builtin_fmaf((float) s1, 256.f, (float) s0)) * scale;
    const float d = half_bits_to_float(d_bits);
    if constexpr (TYPE == TRC_HIP_TYPE_Q4_0) return d * __builtin_fmaf(-8.f, xs, qx);
    if constexpr (TYPE == TRC_HIP_TYPE_Q5_0) return d * __builtin_fmaf(-16.f, xs, qx);
    return __builtin_fmaf(d, qx, half_bits_to_float(m_bits) * xs);
}

// One Q4_0 / Q4_1 block of one row: 4 quant words (already XOR 0x88888888, i.e.
// signed q - 8) against this lane's six 4-bit digit planes P[4*i + g]. Two
// Horner chains (digits 5-4-3 and 2-1-0) carry the digit sums in their
// accumulators, so only two start from zero; the result is exact in int32
// (|sum| <= 32*8*2^22 = 2^30).
template <int TYPE>
__device__ __forceinline__ float qd_block_n4(const uint32_t* q, uint32_t d_bits, uint32_t m_bits, const uint32_t* P,
                                             float scale, float xs) {
    uint32_t hi = 0, lo = 0;
#pragma unroll
    for (int i = 2; i >= 0; --i) {
        if (i < 2) {
            hi <<= 4;
            lo <<= 4;
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            hi = (uint32_t) __builtin_amdgcn_sdot8((int) q[g], (int) P[4 * (i + 3) + g], (int) hi, false);
            lo = (uint32_t) __builtin_amdgcn_sdot8((int) q[g], (int) P[4 * i + g], (int) lo, false);
        }
    }
    const int T = (int) ((hi << 12) + lo);
    const float qx = (float) T * scale;  // sum_e (q_e - 8) x_e
    const float d = half_bits_to_float(d_bits);
    if constexpr (TYPE == TRC_HIP_TYPE_Q4_0) return d * qx;
    // Q4_1: d * sum q x + m * sum x = d * (sum (q-8) x + 8 * sum x) + m * sum x
    return __builtin_fmaf(d, __builtin_fmaf(8.f, xs, qx), half_bits_to_float(m_bits) * xs);
}

// One Q8_0 block of one row: 8 signed quant words against the balanced digit planes.
__device__ __forceinline__ float qd_block_q8(const uint32_t* q, uint32_t d_bits, const uint32_t (*P)[8], float scale) {
    int s0 = 0, s1 = 0, s2 = 0, t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
    for (int w = 0; w < 8; w += 2) {
        s0 = __builtin_amdgcn_sdot4((int) q[w], (int) P[0][w], s0, false);
        s1 = __builtin_amdgcn_sdot4((int) q[w], (int) P[1][w], s1, false);
        s2 = __builtin_amdgcn_sdot4((int) q[w], (int) P[2][w], s2, false);
        t0 = __builtin_amdgcn_sdot4((int) q[w + 1], (int) P[0][w + 1], t0, false);
        t1 = __builtin_amdgcn_sdot4((int) q[w + 1], (int) P[1][w + 1], t1, false);
        t2 = __builtin_amdgcn_sdot4((int) q[w + 1], (int) P[2][w + 1], t2, false);
    }
    s0 += t0;
    s1 += t1;
    s2 += t2;
    // sum_e q_e X_e = s0 + 256 s1 + 65536 s2; |s0 + 256 s1| < 2^27, s2 needs float
    const float qx = __builtin_fmaf((float) s2, 65536.f, (float) (s0 + s1 * 256)) * scale;
    return half_bits_to_float(d_bits) * qx;
}

// Whether a format runs on the 4-bit digit planes (v_dot8) or the byte planes (v_dot4).
template <int TYPE>
constexpr bool qd_nibble_path() {
    return TYPE == TRC_HIP_TYPE_Q4_0 || TYPE == TRC_HIP_TYPE_Q4_1;
}

// Decodes the dwords of a pair (PAIR_WORDS of them) into the fields of its two
// blocks. PA / PB: this lane's 24 plane words of blocks A and B (six 4-bit
// digit planes of 4 words, or three byte planes of 8 words).
template <int TYPE>
__device__ __forceinline__ float qd_pair(const uint32_t* w, const uint32_t* PA, const uint32_t* PB, const float* sc,
                                         const float* xs) {
    // the two block terms are rounded and then added, whatever the compiler
    // would otherwise fuse into a multiply-add
#pragma clang fp contract(off)
    constexpr uint32_t FLIP = 0x88888888u;  // unsigned nibble q -> signed q - 8
    const auto* PA3 = (const uint32_t(*)[8]) PA;
    const auto* PB3 = (const uint32_t(*)[8]) PB;
    uint32_t qa[4], qb[4];
    if constexpr (TYPE == TRC_HIP_TYPE_Q4_0) {
        // 36 B: [dA qA0-1][qA2-5][qA6-9][qA10-13][qA14-15 dB][qB0-3]..[qB12-15]
        qa[0] = __builtin_amdgcn_perm(w[4], w[0], 0x05040302u) ^ FLIP;  // qA 0, 1, 14, 15
#pragma unroll
        for (int i = 1; i < 4; ++i) qa[i] = w[i] ^ FLIP;
#pragma unroll
        for (int i = 0; i < 4; ++i) qb[i] = w[5 + i] ^ FLIP;
        return qd_block_n4<TYPE>(qa, w[0] & 0xFFFFu, 0, PA, sc[0], xs[0]) +
               qd_block_n4<TYPE>(qb, w[4] >> 16, 0, PB, sc[1], xs[1]);
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q4_1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) { qa[i] = w[1 + i] ^ FLIP; qb[i] = w[6 + i] ^ FLIP; }
        return qd_block_n4<TYPE>(qa, w[0] & 0xFFFFu, w[0] >> 16, PA, sc[0], xs[0]) +
               qd_block_n4<TYPE>(qb, w[5] & 0xFFFFu, w[5] >> 16, PB, sc[1], xs[1]);
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) { qa[i] = align2(w[i + 2], w[i + 1]); qb[i] = w[7 + i]; }
        return qd_block<TYPE>(qa, align2(w[1], w[0]), w[0] & 0xFFFFu, 0, PA3, sc[0], xs[0]) +
               qd_block<TYPE>(qb, w[6], w[5] >> 16, 0, PB3, sc[1], xs[1]);
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) { qa[i] = w[2 + i]; qb[i] = w[8 + i]; }
        return qd_block<TYPE>(qa, w[1], w[0] & 0xFFFFu, w[0] >> 16, PA3, sc[0], xs[0]) +
               qd_block<TYPE>(qb, w[7], w[6] & 0xFFFFu, w[6] >> 16, PB3, sc[1], xs[1]);
    } else {  // Q8_0: 17 dwords [d0 q0.0-1][q0 2-5] .. [q0 30-31 d1][q1 0-3] .. [q1 28-31]
        uint32_t a8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) a8[i] = align2(w[i + 1], w[i]);
        (void) xs;
        return qd_block_q8(a8, w[0] & 0xFFFFu, PA3, sc[0]) + qd_block_q8(w + 9, w[8] >> 16, PB3, sc[1]);
    }
}

// Sum over the 64 lanes of a wave with DPP row operations (no LDS traffic);
// the total lands in lane 63.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK,
                                                                  0xF, false));
}

__device__ __forceinline__ float wave_sum_lane63(float v) {
    v += dpp_f32<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x141, 0xF>(v);  // row_half_mirror: sums of 8
    v += dpp_f32<0x140, 0xF>(v);  // row_mirror: sums of 16 in every row
    v += dpp_f32<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_f32<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

// Weight rows through LDS (the DMA form of the kernel). A row's segment of one
// chunk (QD_CH blocks, a multiple of 16 bytes) is copied by 16-byte loads that go
// straight into a per-wave LDS ring (buffer_load ... lds, streaming): consecutive
// lanes read consecutive bytes, so each cache line is read by one instruction
// and need not stay in the caches. Each lane then reads its pair from LDS.
constexpr uint32_t QD_RSRC_WORD3 = 0x00020000u;  // gfx9 buffer resource: raw 32-bit dwords
constexpr int QD_DMA_NT = 2;                      // cache policy bits of the copies: nt

__device__ __forceinline__ void qd_dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*) lds, 16, voff, 0, 0,
                                             QD_DMA_NT);
}

// s_waitcnt immediate with vmcnt = v (bits 3:0 and 15:14), the others at their maximum.
constexpr int qd_vmcnt(int v) { return (v & 0xF) | ((v >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// Wait until at most k rows of NI copies each, and the st store instructions
// issued after the row being waited for, are outstanding. vmcnt counts loads and
// stores together and retires them in issue order, so the count must include
// every store issued after the row's copies, and no more. Callers pass
// compile-time constants, so the switch folds to one wait.
template <int NI>
__device__ __forceinline__ void qd_wait_rows(int k, int st = 0) {
    static_assert(2 * NI + 8 < 64, "vmcnt is 6 bits");
    switch (k * NI + st) {
#define QD_WAIT_CASE(n) case n: __builtin_amdgcn_s_waitcnt(qd_vmcnt(n)); break;
        QD_WAIT_CASE(0) QD_WAIT_CASE(1) QD_WAIT_CASE(2) QD_WAIT_CASE(3) QD_WAIT_CASE(4) QD_WAIT_CASE(5)
        QD_WAIT_CASE(6) QD_WAIT_CASE(7) QD_WAIT_CASE(8) QD_WAIT_CASE(9) QD_WAIT_CASE(10) QD_WAIT_CASE(11)
        QD_WAIT_CASE(12) QD_WAIT_CASE(13) QD_WAIT_CASE(14) QD_WAIT_CASE(15) QD_WAIT_CASE(16) QD_WAIT_CASE(17)
        QD_WAIT_CASE(18)
#undef QD_WAIT_CASE
        default: __builtin_amdgcn_s_waitcnt(qd_vmcnt(0)); break;  // not reached: waits for everything
    }
}

// Workgroup b's place in row order, so that consecutive row slots belong to the
// workgroups of one XCD. The dispatcher deals workgroups to the 8 XCDs round
// robin (b mod 8), and each XCD has its own L2: with this order the rows whose
// results share an output cache line are computed, and their stores merged, in
// one L2. A bijection on [0, nb) for any nb.
__device__ __forceinline__ int64_t qd_xcd_slot(int64_t b, int64_t nb) {
    const int64_t x = b & 7, per = nb >> 3, extra = nb & 7;
    return x * per + (x < extra ? x : extra) + (b >> 3);
}

// The PW dwords of a pair at LDS byte address a, read and waited for in one asm
// block. Plain loads would make the compiler wait for every LDS copy still in
// flight (it cannot tell the ring's slots apart); the row's own copies are
// waited for by qd_wait_rows instead.
typedef uint32_t qd_u2 __attribute__((ext_vector_type(2)));
#define QD_DS2(k, o0, o1) "ds_read2_b32 %" #k ", %[a] offset0:" #o0 " offset1:" #o1 "\n\t"
template <int PW>
__device__ __forceinline__ void qd_lds_words(uint32_t a, uint32_t (&w)[PW]);
template <>
__device__ __forceinline__ void qd_lds_words<9>(uint32_t a, uint32_t (&w)[9]) {
    qd_u2 t[4];
    asm volatile(QD_DS2(0, 0, 1) QD_DS2(1, 2, 3) QD_DS2(2, 4, 5) QD_DS2(3, 6, 7)
                 "ds_read_b32 %4, %[a] offset:32\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]), "=&v"(w[8])
                 : [a] "v"(a));
    for (int i = 0; i < 4; ++i) { w[2 * i] = t[i].x; w[2 * i + 1] = t[i].y; }
}
template <>
__device__ __forceinline__ void qd_lds_words<10>(uint32_t a, uint32_t (&w)[10]) {
    qd_u2 t[5];
    asm volatile(QD_DS2(0, 0, 1) QD_DS2(1, 2, 3) QD_DS2(2, 4, 5) QD_DS2(3, 6, 7) QD_DS2(4, 8, 9)
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]), "=&v"(t[4])
                 : [a] "v"(a));
    for (int i = 0; i < 5; ++i) { w[2 * i] = t[i].x; w[2 * i + 1] = t[i].y; }
}
template <>
__device__ __forceinline__ void qd_lds_words<11>(uint32_t a, uint32_t (&w)[11]) {
    qd_u2 t[5];
    asm volatile(QD_DS2(0, 0, 1) QD_DS2(1, 2, 3) QD_DS2(2, 4, 5) QD_DS2(3, 6, 7) QD_DS2(4, 8, 9)
                 "ds_read_b32 %5, %[a] offset:40\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]), "=&v"(t[4]), "=&v"(w[10])
                 : [a] "v"(a));
    for (int i = 0; i < 5; ++i) { w[2 * i] = t[i].x; w[2 * i + 1] = t[i].y; }
}
template <>
__device__ __forceinline__ void qd_lds_words<12>(uint32_t a, uint32_t (&w)[12]) {
    qd_u2 t[6];
    asm volatile(QD_DS2(0, 0, 1) QD_DS2(1, 2, 3) QD_DS2(2, 4, 5) QD_DS2(3, 6, 7) QD_DS2(4, 8, 9) QD_DS2(5, 10, 11)
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]), "=&v"(t[4]), "=&v"(t[5])
                 : [a] "v"(a));
    for (int i = 0; i < 6; ++i) { w[2 * i] = t[i].x; w[2 * i + 1] = t[i].y; }
}
template <>
__device__ __forceinline__ void qd_lds_words<17>(uint32_t a, uint32_t (&w)[17]) {
    qd_u2 t[8];
    asm volatile(QD_DS2(0, 0, 1) QD_DS2(1, 2, 3) QD_DS2(2, 4, 5) QD_DS2(3, 6, 7) QD_DS2(4, 8, 9) QD_DS2(5, 10, 11)
                     QD_DS2(6, 12, 13) QD_DS2(7, 14, 15) "ds_read_b32 %8, %[a] offset:64\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]), "=&v"(t[4]), "=&v"(t[5]), "=&v"(t[6]),
                   "=&v"(t[7]), "=&v"(w[16])
                 : [a] "v"(a));
    for (int i = 0; i < 8; ++i) { w[2 * i] = t[i].x; w[2 * i + 1] = t[i].y; }
}
#undef QD_DS2

// Workgroup barrier after this wave's LDS writes are done. __syncthreads' fence
// would also wait for every LDS copy in flight, which drains the weight stream.
__device__ __forceinline__ void qd_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// NC columns of x (1 to 4) share one pass over W: each row's quant words are
// decoded once and met by every column's digit planes (48 registers per column).
// DMA: weight rows through LDS (needs 16-byte aligned rows and nblk % 8 == 0);
// otherwise each lane loads its pair into registers.
// PSTORE (in the last chunk): 0 = the wave stores all its rows with one
// instruction per column after its last load; 1 = each row is stored as soon as
// it is reduced, inside the weight stream (lane r stores row r; the wait counts
// of the rows behind it include these stores); 2 = the rows done when the wave
// issues its last copies are stored right then, in one instruction per column
// (no wait for a copy counts them), and the last PF rows at the end.
// ONE: K is one chunk (nblk <= QD_CH), compiled without the chunk loop.
template <int TYPE, int RPW, int NC, bool DMA, int PF_ROWS, int PSTORE, bool ONE = false>
__global__ __launch_bounds__(QD_WAVES * 64) void k_qmatvec_dot(const uint8_t* __restrict__ W, int64_t nblk, int64_t M,
                                                     int64_t nb1_w, const float* __restrict__ x, int64_t ldx,
                                                     float* __restrict__ y, int64_t ldy) {
    constexpr int BYTES = block_bytes(TYPE);
    constexpr int PW = QdFmt<TYPE>::PAIR_WORDS;
    // two-row waves with the early store keep one row in flight, so that row 0 is
    // stored while row 1 streams (M = 4096: 4 % faster than both rows at once)
    constexpr int PF = PSTORE == 2 && RPW == 2 ? 1 : PF_ROWS < RPW ? PF_ROWS : RPW;
    static_assert(RPW <= 64, "each of a wave's rows is stored by one lane");
    constexpr int SEG = QD_CH * BYTES;        // bytes of a row's full chunk
    constexpr int NI = (SEG + 1023) / 1024;   // 16-byte copies per lane and row
    constexpr int SLOTS = PF + 1;             // rows in flight + the row being read
    __shared__ __attribute__((aligned(16))) uint8_t wring[DMA ? QD_WAVES : 1][DMA ? SLOTS : 1][DMA ? NI * 1024 : 16];
    __shared__ __attribute__((aligned(16))) uint32_t planes[NC][(QD_CH / 2) * QD_PSTRIDE];
    __shared__ float scale_l[NC][QD_CH];
    __shared__ float xsum_l[NC][QD_CH];

    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t wave_id = qd_xcd_slot(blockIdx.x, gridDim.x) * QD_WAVES + wv;
    // Rows are strided over the waves (row = wave + r * n_waves), so the loads
    // in flight at any time sweep W in address order rather than starting in
    // every wave's own region.
    const int64_t n_waves = (int64_t) gridDim.x * QD_WAVES;

    // No branches around loads and uses: the wait-count insertion loses track of
    // loads issued under a branch and then waits for every outstanding load
    // before each row. Rows past M re-read row M-1 and lanes past a short last
    // chunk re-read its last pair; their results are dropped.
    int64_t roff[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int64_t row = wave_id + r * n_waves;
        roff[r] = (row < M ? row : M - 1) * nb1_w;
    }

    // lane r: row r's result, the chunks' wave sums added in chunk order (no
    // per-lane accumulators across chunks, which leaves registers for the
    // columns' digit planes)
    float out[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) out[n] = 0.f;

    const int64_t nchunks = (nblk + QD_CH - 1) / QD_CH;
    uint32_t w[DMA ? 1 : RPW][PW];
    // One chunk of K. The last chunk is its own instance (LAST) so that its row
    // stores, and the wait counts that include them, are compile-time constants
    // (under a runtime condition the compiler added a conservative wait after
    // the merge).
    auto chunk = [&](int64_t c, auto last_tag) {
        const int64_t cb = nblk - c * QD_CH < QD_CH ? nblk - c * QD_CH : QD_CH;
        const bool mine = 2 * lane < cb;  // this lane owns a pair of this chunk (cb is even)
        const int pl = mine ? lane : (int) (cb / 2) - 1;
        const uint8_t* base = W + (c * QD_CH + 2 * pl) * BYTES;
        // Prefetching stays within a chunk, so row r of every chunk can use ring
        // slot r % SLOTS: the slot's previous row was read (and waited for) before.
        auto issue = [&](int r) {
            if constexpr (DMA) {
                // lanes past a short last chunk read zeros (the buffer's range check)
                const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                    (void*) (W + roff[r] + c * (int64_t) SEG), (short) 0, (int) cb * BYTES, QD_RSRC_WORD3);
#pragma unroll
                for (int i = 0; i < NI; ++i) qd_dma16(rs, &wring[wv][r % SLOTS][i * 1024], (uint32_t) (i * 1024 + 16 * lane));
            } else {
                const uint32_t* p32 = (const uint32_t*) (base + roff[r]);
#pragma unroll
                for (int i = 0; i < PW; ++i) w[r][i] = p32[i];
            }
        };
        // store instructions issued after row r's copies: one per column for
        // each of the (at most PF) rows before it, in the last chunk only
        constexpr bool LAST = decltype(last_tag)::value;
        // this lane's pair of row r, in registers
        auto pair_words = [&](int r) -> const uint32_t* {
            if constexpr (DMA) {
                constexpr int MID = RPW - 1 - PF;  // PSTORE 2: the row after which the early rows are stored
                const int st = !LAST || PSTORE == 0 ? 0
                               : PSTORE == 1        ? NC * (r < PF ? r : PF)
                                                    : (MID >= 0 && r > MID ? NC : 0);
                qd_wait_rows<NI>(RPW - 1 - r < PF ? RPW - 1 - r : PF, st);
                const uint32_t a = (uint32_t) (uintptr_t) (__attribute__((address_space(3))) uint8_t*) &wring[wv][r % SLOTS][0] +
                                   (uint32_t) pl * (PW * 4);
                qd_lds_words<PW>(a, w[0]);
                return w[0];
            } else {
                return w[r];
            }
        };
        // x is loaded first (vector loads return in issue order), then the
        // weight stream starts so that it overlaps the conversion of x
        f4 xv[NC][4];
        QdX4 xn[NC];
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            if constexpr (qd_nibble_path<TYPE>()) {
                qd_load_x_n4<TYPE == TRC_HIP_TYPE_Q4_0>(x + n * ldx + c * QD_CH * QK, cb, xn[n]);
            } else {
                qd_load_x(x + n * ldx + c * QD_CH * QK, cb, xv[n]);
            }
        }
#pragma unroll
        for (int r = 0; r < PF; ++r) issue(r);
        // keep these loads above the prologue and its barrier
        __builtin_amdgcn_sched_barrier(0);
        if (c > 0) qd_barrier();  // previous chunk's planes are no longer read
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            if constexpr (qd_nibble_path<TYPE>()) {
                qd_prologue_n4(xn[n], cb, planes[n], scale_l[n], xsum_l[n]);
            } else {
                qd_prologue<TYPE == TRC_HIP_TYPE_Q8_0>(xv[n], cb, planes[n], scale_l[n], xsum_l[n]);
            }
        }
        qd_barrier();

        // this lane's pair: the plane words of blocks A and B (24 each) per column.
        // Nibble path: A at dwords 0-23, B at 24-47. Byte path: plane p of A at
        // 16p..16p+7 and of B at 16p+8..16p+15.
        uint32_t PA[NC][24], PB[NC][24];
        float sc[NC][2], xs[NC][2];
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            const uint32_t* src = planes[n] + pl * QD_PSTRIDE;
#pragma unroll
            for (int k = 0; k < 12; ++k) {
                const uint4 v = *(const uint4*) (src + 4 * k);
                uint32_t* dst;
                if constexpr (qd_nibble_path<TYPE>()) {
                    dst = k < 6 ? &PA[n][4 * k] : &PB[n][4 * (k - 6)];
                } else {
                    const int p = k >> 2, g = k & 3;
                    dst = g < 2 ? &PA[n][8 * p + 4 * g] : &PB[n][8 * p + 4 * (g - 2)];
                }
                dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
            }
            sc[n][0] = scale_l[n][2 * pl];
            sc[n][1] = scale_l[n][2 * pl + 1];
            xs[n][0] = xsum_l[n][2 * pl];
            xs[n][1] = xsum_l[n][2 * pl + 1];
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            if (r + PF < RPW) issue(r + PF);
            __builtin_amdgcn_sched_barrier(0);  // row r + PF stays in flight during row r
            const uint32_t* wr = pair_words(r);
            // reduce this chunk's part of row r while the next rows' loads are
            // in flight and add it into lane r
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                const float v = qd_pair<TYPE>(wr, PA[n], PB[n], sc[n], xs[n]);
                const float sum = wave_sum_lane63(mine ? v : 0.f);
                const float s63 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sum), 63));
                out[n] = lane == r ? (c == 0 ? s63 : out[n] + s63) : out[n];
            }
            if constexpr (PSTORE == 1 && LAST) {
                const int64_t row = wave_id + r * n_waves;
#pragma unroll
                for (int n = 0; n < NC; ++n)
                    if (lane == r && row < M) y[n * ldy + row] = out[n];
            }
            if constexpr (PSTORE == 2 && LAST) {
                if (r == RPW - 1 - PF) {
                    const int64_t row = wave_id + (int64_t) lane * n_waves;
#pragma unroll
                    for (int n = 0; n < NC; ++n)
                        if (lane <= r && row < M) y[n * ldy + row] = out[n];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if constexpr (ONE) {
        chunk(0, std::true_type{});
    } else if constexpr (PSTORE != 0) {
        for (int64_t c = 0; c + 1 < nchunks; ++c) chunk(c, std::false_type{});
        chunk(nchunks - 1, std::true_type{});
    } else {
        for (int64_t c = 0; c < nchunks; ++c) chunk(c, std::false_type{});
    }
    if constexpr (PSTORE != 1) {
        // one store per column for the wave's rows not stored yet, after the last load
        constexpr int FIRST = PSTORE == 2 ? (RPW - PF > 0 ? RPW - PF : 0) : 0;
        const int64_t row = wave_id + (int64_t) lane * n_waves;
#pragma unroll
        for (int n = 0; n < NC; ++n)
            if (lane >= FIRST && lane < RPW && row < M) y[n * ldy + row] = out[n];
    }
}

// One or two columns with K in 2..CS chunks of QD_CH blocks (the weights
// through LDS). The 8 waves of a workgroup are QD_WAVES / CS groups of CS
// waves: wave (g, c) takes chunk c of the rows of group g. All of x is
// converted once, each wave's digit planes stay in registers, and no wave meets
// a chunk boundary, so its copies stream without the drain k_qmatvec_dot has at
// every boundary. A row's partial sums meet in LDS and are added in chunk
// order (deterministic). Waves whose chunk is past the end copy nothing (an
// empty buffer range reads zeros) and add zeros. Two columns' planes of four
// chunks fit only without the plane rows' padding (48 dwords per pair).
template <int TYPE, int RPW, int CS, int PF_ROWS, int NC>
__global__ __launch_bounds__(QD_WAVES * 64) void k_qmatvec_kslots(const uint8_t* __restrict__ W, int64_t nblk,
                                                                   int64_t M, int64_t nb1_w,
                                                                   const float* __restrict__ x, int64_t ldx,
                                                                   float* __restrict__ y, int64_t ldy) {
    constexpr int BYTES = block_bytes(TYPE);
    constexpr int PW = QdFmt<TYPE>::PAIR_WORDS;
    constexpr int PF = PF_ROWS < RPW ? PF_ROWS : RPW;
    constexpr int SEG = QD_CH * BYTES;
    constexpr int NI = (SEG + 1023) / 1024;
    constexpr int SLOTS = PF + 1;
    constexpr int G = QD_WAVES / CS;  // row groups per workgroup
    constexpr int PS = NC > 1 ? 48 : QD_PSTRIDE;
    static_assert(QD_WAVES % CS == 0 && RPW <= 64, "chunk slots divide the waves; one lane per row");
    __shared__ __attribute__((aligned(16))) uint8_t wring[QD_WAVES][SLOTS][NI * 1024];
    __shared__ __attribute__((aligned(16))) uint32_t planes[CS][NC][(QD_CH / 2) * PS];
    __shared__ float scale_l[CS][NC][QD_CH];
    __shared__ float xsum_l[CS][NC][QD_CH];
    __shared__ float part[QD_WAVES][NC][RPW];

    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = wv / CS, ch = wv % CS;
    // rows strided over all groups, as the waves of k_qmatvec_dot
    const int64_t group = (int64_t) blockIdx.x * G + g;
    const int64_t n_groups = (int64_t) gridDim.x * G;
    const int64_t nchunks = (nblk + QD_CH - 1) / QD_CH;
    auto chunk_blocks = [&](int64_t c) -> int64_t {
        return c < nchunks ? (nblk - c * QD_CH < QD_CH ? nblk - c * QD_CH : QD_CH) : 0;
    };
    const int64_t cb = chunk_blocks(ch);
    const bool mine = 2 * lane < cb;
    const int pl = mine ? lane : (cb > 0 ? (int) (cb / 2) - 1 : 0);

    int64_t roff[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int64_t row = group + r * n_groups;
        roff[r] = (row < M ? row : M - 1) * nb1_w;
    }
    auto issue = [&](int r) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*) (W + roff[r] + ch * (int64_t) SEG), (short) 0, (int) cb * BYTES, QD_RSRC_WORD3);
#pragma unroll
        for (int i = 0; i < NI; ++i) qd_dma16(rs, &wring[wv][r % SLOTS][i * 1024], (uint32_t) (i * 1024 + 16 * lane));
    };

    // x of every chunk and column (chunks past the end re-point at chunk 0 and
    // convert as empty), then the first rows' copies, then the conversion
    f4 xv[CS][NC][4];
    QdX4 xn[CS][NC];
#pragma unroll
    for (int c = 0; c < CS; ++c) {
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            const float* xc = x + n * ldx + (c < nchunks ? c * QD_CH * QK : 0);
            if constexpr (qd_nibble_path<TYPE>()) {
                qd_load_x_n4<TYPE == TRC_HIP_TYPE_Q4_0>(xc, chunk_blocks(c), xn[c][n]);
            } else {
                qd_load_x(xc, chunk_blocks(c), xv[c][n]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < PF; ++r) issue(r);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < CS; ++c) {
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            if constexpr (qd_nibble_path<TYPE>()) {
                qd_prologue_n4<PS>(xn[c][n], chunk_blocks(c), planes[c][n], scale_l[c][n], xsum_l[c][n]);
            } else {
                qd_prologue<TYPE == TRC_HIP_TYPE_Q8_0, PS>(xv[c][n], chunk_blocks(c), planes[c][n], scale_l[c][n],
                                                          xsum_l[c][n]);
            }
        }
    }
    qd_barrier();

    // this wave's pair of its chunk, per column (layout as in k_qmatvec_dot)
    uint32_t PA[NC][24], PB[NC][24];
    float sc[NC][2], xs[NC][2];
#pragma unroll
    for (int n = 0; n < NC; ++n) {
        const uint32_t* src = planes[ch][n] + pl * PS;
#pragma unroll
        for (int k = 0; k < 12; ++k) {
            const uint4 v = *(const uint4*) (src + 4 * k);
            uint32_t* dst;
            if constexpr (qd_nibble_path<TYPE>()) {
                dst = k < 6 ? &PA[n][4 * k] : &PB[n][4 * (k - 6)];
            } else {
                const int p = k >> 2, gg = k & 3;
                dst = gg < 2 ? &PA[n][8 * p + 4 * gg] : &PB[n][8 * p + 4 * (gg - 2)];
            }
            dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
        }
        sc[n][0] = scale_l[ch][n][2 * pl];
        sc[n][1] = scale_l[ch][n][2 * pl + 1];
        xs[n][0] = xsum_l[ch][n][2 * pl];
        xs[n][1] = xsum_l[ch][n][2 * pl + 1];
    }

    uint32_t w[PW];
    float out[NC];  // lane r: this chunk's part of row r
#pragma unroll
    for (int n = 0; n < NC; ++n) out[n] = 0.f;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        if (r + PF < RPW) issue(r + PF);
        __builtin_amdgcn_sched_barrier(0);  // row r + PF stays in flight during row r
        qd_wait_rows<NI>(RPW - 1 - r < PF ? RPW - 1 - r : PF);
        const uint32_t a = (uint32_t) (uintptr_t) (__attribute__((address_space(3))) uint8_t*) &wring[wv][r % SLOTS][0] +
                           (uint32_t) pl * (PW * 4);
        qd_lds_words<PW>(a, w);
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            const float v = qd_pair<TYPE>(w, PA[n], PB[n], sc[n], xs[n]);
            const float sum = wave_sum_lane63(mine ? v : 0.f);
            const float s63 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sum), 63));
            out[n] = lane == r ? s63 : out[n];
        }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int n = 0; n < NC; ++n)
        if (lane < RPW) part[wv][n][lane] = out[n];
    qd_barrier();
    if (ch == 0) {
        const int r = lane < RPW ? lane : 0;
        const int64_t row = group + (int64_t) lane * n_groups;
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            float s = part[g * CS][n][r];
#pragma unroll
            for (int c = 1; c < CS; ++c) s += part[g * CS + c][n][r];
            if (lane < RPW && row < M) y[n * ldy + row] = s;
        }
    }
}

// Where k_qmatvec_dot stores its rows (PSTORE), as measured against one store
// per column after the last load (configuration 2, M = 14336, graph replays):
// with K in one chunk through LDS, storing the rows done at the last copy issue
// right then (2) is 2-3.4 % faster for one column of every format (per-row
// stores: Q5_0 1 % slower) and within 0.5 % for two to four columns; for Q8_0
// over four chunks (K = 14336) and on the register path per-row stores (1) are
// 2 % faster, and Q4_0 on the register path 3 % slower.
constexpr int qd_pstore(int type, int nc, bool dma, bool one) {
    if (dma && one) return 2;
    return type == TRC_HIP_TYPE_Q8_0 && nc <= 3 ? 1 : 0;
}

template <int TYPE, int RPW, int NC, bool ONE>
int launch_dot_one(const uint8_t* w, int64_t nblk, int64_t M, size_t nb1_w, const float* x, int64_t ldx, float* y,
                   int64_t ldy, bool dma, int64_t grid, hipStream_t s) {
    const dim3 g((unsigned) grid), b(QD_WAVES * 64);
    // only the largest row count per wave can leave more workgroups than CUs
    if constexpr (RPW == QD_RMAX) {
        if (dma && grid > device_cus()) {
            constexpr int PF = qd_prefetch(TYPE, NC, true, true);
            hipLaunchKernelGGL((k_qmatvec_dot<TYPE, RPW, NC, true, PF, qd_pstore(TYPE, NC, true, ONE), ONE>), g, b, 0, s,
                               w, nblk, M, (int64_t) nb1_w, x, ldx, y, ldy);
            return check_launch("qmatvec_dot");
        }
    }
    if (dma) {
        // Q4_0, one column, K of exactly one 4096-element chunk, 7 or 8 rows per
        // wave: three rows in flight measured 0.3-0.8 % faster than two (M = 13000,
        // 14336, 16384; same bits), but 5 % slower at 4 rows per wave and 0.7 %
        // slower at K = 2048, so only there
        if constexpr (ONE && NC == 1 && TYPE == TRC_HIP_TYPE_Q4_0 && RPW >= 7) {
            if (nblk == QD_CH) {
                hipLaunchKernelGGL((k_qmatvec_dot<TYPE, RPW, NC, true, 3, qd_pstore(TYPE, NC, true, ONE), ONE>), g, b,
                                   0, s, w, nblk, M, (int64_t) nb1_w, x, ldx, y, ldy);
                return check_launch("qmatvec_dot");
            }
        }
        constexpr int PF = qd_prefetch(TYPE, NC, true, false);
        hipLaunchKernelGGL((k_qmatvec_dot<TYPE, RPW, NC, true, PF, qd_pstore(TYPE, NC, true, ONE), ONE>), g, b, 0, s, w,
                           nblk, M, (int64_t) nb1_w, x, ldx, y, ldy);
    } else if constexpr (NC <= 2) {
        constexpr int PF = qd_prefetch(TYPE, NC, false, false);
        hipLaunchKernelGGL((k_qmatvec_dot<TYPE, RPW, NC, false, PF, qd_pstore(TYPE, NC, false, ONE), ONE>), g, b, 0, s,
                           w, nblk, M, (int64_t) nb1_w, x, ldx, y, ldy);
    } else {
        return fail(TRC_HIP_E_INVALID, "qmatvec: %d columns need the LDS path", NC);
    }
    return check_launch("qmatvec_dot");
}

template <int TYPE, int RPW, int NC>
int launch_dot_rpw(const void* wq, int64_t nblk, int64_t M, size_t nb1_w, const float* x, size_t nb1_x, float* y,
                   size_t nb1_y, hipStream_t s) {
    const int64_t waves = (M + RPW - 1) / RPW;
    const int64_t grid = (waves + QD_WAVES - 1) / QD_WAVES;
    // the LDS copies need 16-byte aligned row chunks (8 blocks are a multiple of 16 bytes)
    const bool dma = nblk % 8 == 0 && (((uintptr_t) wq) & 15u) == 0 && (nb1_w & 15u) == 0;
    const int64_t ldx = (int64_t) (nb1_x / sizeof(float)), ldy = (int64_t) (nb1_y / sizeof(float));
    const auto* w = (const uint8_t*) wq;
    // K in one chunk (every decode shape with K <= 4096) runs an instance
    // without the chunk loop: 1-5 % faster, measured over the five formats and
    // one to four columns
    if (nblk <= QD_CH) return launch_dot_one<TYPE, RPW, NC, true>(w, nblk, M, nb1_w, x, ldx, y, ldy, dma, grid, s);
    return launch_dot_one<TYPE, RPW, NC, false>(w, nblk, M, nb1_w, x, ldx, y, ldy, dma, grid, s);
}

template <int TYPE, int NC>
int launch_qmatvec_dot(const void* wq, int64_t nblk, int64_t M, size_t nb1_w, const float* x, size_t nb1_x, float* y,
                       size_t nb1_y, hipStream_t s) {
    // spread the rows evenly over 8 waves per CU (2 per SIMD), at most QD_RMAX each
    const int64_t target_waves = (int64_t) device_cus() * 8;
    int64_t rpw = (M + target_waves - 1) / target_waves;
    if (rpw > QD_RMAX) rpw = QD_RMAX;
    if (rpw < 1) rpw = 1;
    switch (rpw) {
        case 1: return launch_dot_rpw<TYPE, 1, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 2: return launch_dot_rpw<TYPE, 2, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 3: return launch_dot_rpw<TYPE, 3, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 4: return launch_dot_rpw<TYPE, 4, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 5: return launch_dot_rpw<TYPE, 5, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 6: return launch_dot_rpw<TYPE, 6, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 7: return launch_dot_rpw<TYPE, 7, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        default: return launch_dot_rpw<TYPE, 8, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
    }
}

template <int TYPE, int RPW, int CS, int NC>
int launch_kslots_rpw(const void* wq, int64_t nblk, int64_t M, size_t nb1_w, const float* x, size_t nb1_x, float* y,
                      size_t nb1_y, hipStream_t s) {
    constexpr int G = QD_WAVES / CS;
    // two rows in flight for one column; one for two columns, as in
    // k_qmatvec_dot (and their planes leave room for no more)
    constexpr int PF = NC > 1 ? 1 : 2;
    const int64_t grid = (M + (int64_t) G * RPW - 1) / ((int64_t) G * RPW);
    hipLaunchKernelGGL((k_qmatvec_kslots<TYPE, RPW, CS, PF, NC>), dim3((unsigned) grid), dim3(QD_WAVES * 64), 0, s,
                       (const uint8_t*) wq, nblk, M, (int64_t) nb1_w, x, (int64_t) (nb1_x / sizeof(float)), y,
                       (int64_t) (nb1_y / sizeof(float)));
    return check_launch("qmatvec_kslots");
}

// Rows per wave of k_qmatvec_kslots at most (its waves hold one chunk's planes
// and one row's words, so more rows cost only their row offsets).
constexpr int QK_RMAX = 16;

template <int TYPE, int CS, int NC>
int launch_kslots(const void* wq, int64_t nblk, int64_t M, size_t nb1_w, const float* x, size_t nb1_x, float* y,
                  size_t nb1_y, hipStream_t s) {
    // spread the rows evenly over the row groups of one workgroup per CU, at most QK_RMAX each
    const int64_t groups = (int64_t) device_cus() * (QD_WAVES / CS);
    int64_t rpw = (M + groups - 1) / groups;
    if (rpw > QK_RMAX) rpw = QK_RMAX;
    if (rpw < 1) rpw = 1;
    switch (rpw) {
        case 1: return launch_kslots_rpw<TYPE, 1, CS, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 2: return launch_kslots_rpw<TYPE, 2, CS, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 3: return launch_kslots_rpw<TYPE, 3, CS, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 4: return launch_kslots_rpw<TYPE, 4, CS, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 5: return launch_kslots_rpw<TYPE, 5, CS, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 6: return launch_kslots_rpw<TYPE, 6, CS, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 7: return launch_kslots_rpw<TYPE, 7, CS, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 8: return launch_kslots_rpw<TYPE, 8, CS, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 9: case 10: return launch_kslots_rpw<TYPE, 10, CS, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 11: case 12: return launch_kslots_rpw<TYPE, 12, CS, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        case 13: case 14: return launch_kslots_rpw<TYPE, 14, CS, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
        default: return launch_kslots_rpw<TYPE, 16, CS, NC>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
    }
}

int qv1_grid(int64_t M, int rows) {
    const int cus = device_cus();
    const int64_t tiles = (M + rows - 1) / rows;
    const int64_t want = (tiles + QV1_WAVES - 1) / QV1_WAVES;
    const int64_t cap = (int64_t) cus * 2;
    return (int) (want < cap ? want : cap);
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
                float* y, size_t nb1_y, hipStream_t s, QmScratch where) {
    const int64_t nblk = K / QK;
    // N = 1..4: integer-dot kernel (one pass over W for all columns; each
    // column's digit planes take 48 registers, so a third and fourth column fit
    // only when the weights come through LDS); pairs of blocks start on 4-byte
    // boundaries and x columns on 16-byte ones
    const bool dot_ok = nblk % 2 == 0 && (((uintptr_t) wq) & 3u) == 0 && (nb1_w & 3u) == 0 &&
                        (((uintptr_t) x) & 15u) == 0 && (nb1_x & 15u) == 0;
    // N = 1 with K in 2..4 chunks of 128 blocks, weights through LDS: one chunk
    // per wave, when one workgroup per CU covers M with up to 16 rows per wave
    // (measured: K = 8192..16384 at M = 4096 8-19 % faster for the 4- and 5-bit
    // formats, K = 13824 at M = 5120 22 %, K = 14336 at M = 8192 6 %; with more
    // workgroups than CUs 27-39 % slower, as each holds ~130 KB of LDS; Q8_0,
    // with one row in flight, no faster)
    const int64_t nchunks = (nblk + QD_CH - 1) / QD_CH;
    const bool lds_ok = nblk % 8 == 0 && (((uintptr_t) wq) & 15u) == 0 && (nb1_w & 15u) == 0;
    // two columns only over four chunks (K = 13824 at M = 5120: 17 % faster,
    // K = 14336 at M = 4096: 7 %; over two or three chunks 2-20 % slower)
    if constexpr (TYPE != TRC_HIP_TYPE_Q8_0) {
        if (dot_ok && lds_ok && (N == 1 || (N == 2 && nchunks == 4)) && nchunks >= 2 && nchunks <= 4) {
            const int cs = nchunks == 2 ? 2 : 4;
            if (M <= (int64_t) device_cus() * (QD_WAVES / cs) * QK_RMAX) {
                if (N == 1) {
                    return cs == 2 ? launch_kslots<TYPE, 2, 1>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s)
                                   : launch_kslots<TYPE, 4, 1>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
                }
                return cs == 2 ? launch_kslots<TYPE, 2, 2>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s)
                               : launch_kslots<TYPE, 4, 2>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
            }
        }
    }
    if (dot_ok && N == 1) return launch_qmatvec_dot<TYPE, 1>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
    if (dot_ok && N == 2) return launch_qmatvec_dot<TYPE, 2>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
    // three columns: 21-33 % faster than the fp16 matrix-core kernel (measured,
    // all formats at K = 4096, M = 14336)
    if (dot_ok && lds_ok && N == 3) return launch_qmatvec_dot<TYPE, 3>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
    // four columns fill the registers (Q5_1 spills 8 bytes per lane, Q4_0 44):
    // 9-24 % faster than the matrix-core kernel for Q4_1, Q5_0, Q5_1 and Q8_0
    // with K in one chunk; Q4_0 10 % slower, and 45 % slower over three chunks
    if (dot_ok && lds_ok && N == 4 && TYPE != TRC_HIP_TYPE_Q4_0 && nchunks == 1) {
        return launch_qmatvec_dot<TYPE, 4>(wq, nblk, M, nb1_w, x, nb1_x, y, nb1_y, s);
    }
    // 3 <= N <= 32 (and N = 2 off the dot kernel's alignment): fp16 matrix-core kernel (qmm.hip)
    if (qmm_supported(K, N, wq, nb1_w)) return launch_qmm(TYPE, wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, s, where);
    // N = 1 streaming kernel: needs 16-byte aligned rows and row chunks
    if (N == 1 && nblk % 8 == 0 && (((uintptr_t) wq) & 15u) == 0 && (nb1_w & 15u) == 0) {
        // Q8_0 blocks are twice as large: a 4-row tile already fills the registers.
        constexpr int ROWS = TYPE == TRC_HIP_TYPE_Q8_0 ? 4 : 8;
        hipLaunchKernelGGL((k_qmatvec_n1<TYPE, ROWS, 4>), dim3(qv1_grid(M, ROWS)), dim3(QV1_WAVES * 64), 0, s,
                           (const uint8_t*) wq, nblk, M, (int64_t) nb1_w, x, y);
        return check_launch("qmatvec_n1");
    }
    if (N == 1) return launch_nb<TYPE, 1, 4>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, s);
    if (N == 2) return launch_nb<TYPE, 2, 4>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, s);
    if (N <= 4) return launch_nb<TYPE, 4, 2>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, s);
    if (N <= 8) return launch_nb<TYPE, 8, 2>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, s);
    return launch_nb<TYPE, 16, 2>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, s);
}

}  // namespace

int launch_qmatvec(int type, const void* wq, int64_t K, int64_t M, size_t nb1_w, const float* x, int64_t N,
                   size_t nb1_x, float* y, size_t nb1_y, hipStream_t stream, QmScratch where) {
    if (N > 16 && !(N <= 32 && qmm_supported(K, N, wq, nb1_w))) {
        // skinny GEMM beyond the columns one launch carries: one fused pass over W
        // per 32 columns on the matrix-core kernel, else per 16 (the launches run
        // in order on the stream, so they can share the x workspace)
        const int64_t step = qmm_supported(K, 32, wq, nb1_w) ? 32 : 16;
        for (int64_t c0 = 0; c0 < N; c0 += step) {
            const int64_t n = N - c0 < step ? N - c0 : step;
            const int rc = launch_qmatvec(type, wq, K, M, nb1_w, (const float*) ((const uint8_t*) x + c0 * nb1_x), n,
                                          nb1_x, (float*) ((uint8_t*) y + c0 * nb1_y), nb1_y, stream, where);
            if (rc != TRC_HIP_OK) return rc;
        }
        return TRC_HIP_OK;
    }
    const bool wide = type == TRC_HIP_TYPE_Q4_1 || type == TRC_HIP_TYPE_Q5_1;
    const unsigned walign = wide ? 3u : 1u;
    if ((((uintptr_t) wq) & walign) != 0 || (nb1_w & walign) != 0) {
        return fail(TRC_HIP_E_ALIGN, "qmatvec: W rows must be %d-byte aligned", wide ? 4 : 2);
    }
    if ((((uintptr_t) x) & 15u) != 0 || (nb1_x & 15u) != 0 || (((uintptr_t) y) & 3u) != 0 || (nb1_y & 3u) != 0) {
        return fail(TRC_HIP_E_ALIGN, "qmatvec: x columns must be 16-byte and y columns 4-byte aligned");
    }
    switch (type) {
        case TRC_HIP_TYPE_Q4_0: return launch_type<TRC_HIP_TYPE_Q4_0>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, stream, where);
        case TRC_HIP_TYPE_Q4_1: return launch_type<TRC_HIP_TYPE_Q4_1>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, stream, where);
        case TRC_HIP_TYPE_Q5_0: return launch_type<TRC_HIP_TYPE_Q5_0>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, stream, where);
        case TRC_HIP_TYPE_Q5_1: return launch_type<TRC_HIP_TYPE_Q5_1>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, stream, where);
        case TRC_HIP_TYPE_Q8_0: return launch_type<TRC_HIP_TYPE_Q8_0>(wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, stream, where);
        default: return fail(TRC_HIP_E_INVALID, "qmatvec: bad type %d", type);
    }
}

}  // namespace trc_hip
