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
// |P2| <= 32). The quants enter the MFMAs unsigned (0..31) or as int8 (Q8_0);
// the Q4_0/Q5_0 bias goes into the first MFMA's accumulator input as
// -bias * sum_e X_e. The three MFMAs per block then give exact integer sums
// that combine into one int32 for Q4_0/Q4_1/Q5_0/Q5_1 (the exact result is
// below 2^31 since |q - bias| <= 31), and in float for Q8_0. One conversion
// and two float operations apply 2^-s and d. The only rounding beyond FP32's is
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
// Work split: a workgroup (8 waves) owns up to 64 rows (T tiles of 16) and
// walks K in chunks of 8 pairs. Each chunk is copied by the whole workgroup
// with coalesced 16-byte buffer loads (loads landing in MFMA layout directly
// would touch 16 rows per instruction and swamp the L1 with tag lookups),
// three chunks ahead in registers, into a 3-buffer LDS ring; wave w computes
// pair w of the chunk for all T tiles, so its x operands are loaded once per
// chunk and reused over the tiles. The partial sums are added across the
// waves through LDS in a fixed order, so results are deterministic. Rows per
// workgroup are chosen so the grid covers every CU once when M allows.
#include "common.h"

namespace trc_hip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int QM_MAX_BLOCKS = 2048;  // K <= 65536
constexpr int QM_WAVES = 8;
constexpr int QM_PLANES = 3;          // byte digits of x per element (2 would give 15-bit x: too coarse
                                      // for the 1e-4 bar on short rows)
constexpr int QM_XBITS = QM_PLANES == 3 ? 21 : 14;  // |X| <= 2^QM_XBITS
constexpr uint32_t QM_RSRC_WORD3 = 0x00020000u;  // gfx9 buffer resource: raw 32-bit dwords

// x in block fixed point, written by k_qmm_xprep and read by k_qmm on the
// same stream. Planes: [block][digit][lane 0..63] 8 bytes each. Meta:
// [block][field][column 0..15] with fields 2^-s (f32), sum of x (f32) and
// -bias * sum of X (i32; bias 8 for Q4_0, 16 for Q5_0, else 0). Calls that overlap on one GPU race.
__device__ __attribute__((aligned(256))) uint64_t g_qm_planes[QM_MAX_BLOCKS * QM_PLANES * 64];
__device__ __attribute__((aligned(256))) uint32_t g_qm_meta[QM_MAX_BLOCKS * 3 * 16];

template <int TYPE>
constexpr bool rotated_even() {
    return TYPE == TRC_HIP_TYPE_Q4_0 || TYPE == TRC_HIP_TYPE_Q5_0 || TYPE == TRC_HIP_TYPE_Q8_0;
}

__device__ __forceinline__ uint32_t pack_bytes(const int* v) {
    return (uint32_t) (v[0] & 0xFF) | ((uint32_t) (v[1] & 0xFF) << 8) | ((uint32_t) (v[2] & 0xFF) << 16) |
           ((uint32_t) (v[3] & 0xFF) << 24);
}

// One thread per (block b, column j): it reads the block's 32 values, finds the
// scale and writes the digit bytes of all four MFMA lanes j + 16g that carry
// column j (no cross-lane traffic, so the kernel is one load and one store deep).
__global__ __launch_bounds__(256) void k_qmm_xprep(const float* __restrict__ x, int64_t ldx, int N, int nblk,
                                                    int rot, int bias) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    const int b = t >> 4, j = t & 15;
    if (b >= nblk) return;
    float v[32];
    if (j < N) {
        const f4* col = (const f4*) (x + j * ldx + (int64_t) b * QK);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const f4 w = col[q];
            v[4 * q] = w.x; v[4 * q + 1] = w.y; v[4 * q + 2] = w.z; v[4 * q + 3] = w.w;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 32; ++e) v[e] = 0.f;
    }
    float mx = 0.f, sm = 0.f;
    int bad = 0;  // fmaxf drops NaN, so non-finite values are flagged separately
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        mx = fmaxf(mx, fabsf(v[e]));
        sm += v[e];
        bad |= !__builtin_isfinite(v[e]);
    }
    const bool finite = bad == 0;
    // mx = f * 2^E, f in [0.5, 1): every |x| * 2^s < 2^QM_XBITS
    const int s = (mx > 0.f && finite) ? QM_XBITS - __builtin_amdgcn_frexp_expf(mx) : 0;
    int dg[QM_PLANES][32];
    int sx = 0;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        const int X = finite ? (int) __builtin_rintf(__builtin_ldexpf(v[e], s)) : 0;
        sx += X;
        // balanced base-256 digits: X = d0 + 256 d1 (+ 65536 d2), d0, d1 in [-128, 127]
        const int X1 = (X + 128) >> 8;
        dg[0][e] = X - (X1 << 8);
        if constexpr (QM_PLANES == 2) {
            dg[1][e] = X1;  // |X1| <= 64
        } else {
            const int X2 = (X1 + 128) >> 8;
            dg[1][e] = X1 - (X2 << 8);
            dg[2][e] = X2;  // |X2| <= 32
        }
    }
    // lane group g feeds k = 8g..8g+7: elements E = (c + 4g + i) & 15 (i < 4), then 16 + E
    const int c = (b & 1) ? 0 : rot;
    uint64_t* dst = g_qm_planes + (int64_t) b * QM_PLANES * 64 + j;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int p = 0; p < QM_PLANES; ++p) {
            int lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // c is 0 or 2: select between two constant indices (no dynamic register indexing)
                lo[i] = c ? dg[p][(2 + 4 * g + i) & 15] : dg[p][(4 * g + i) & 15];
                hi[i] = c ? dg[p][16 + ((2 + 4 * g + i) & 15)] : dg[p][16 + ((4 * g + i) & 15)];
            }
            dst[64 * p + 16 * g] = (uint64_t) pack_bytes(lo) | ((uint64_t) pack_bytes(hi) << 32);
        }
    }
    uint32_t* meta = g_qm_meta + b * 48 + j;
    meta[0] = __builtin_bit_cast(uint32_t, finite ? __builtin_ldexpf(1.f, -s) : __builtin_nanf(""));
    meta[16] = __builtin_bit_cast(uint32_t, sm);
    meta[32] = (uint32_t) (-bias * sx);  // |.| <= 16 * 32 * 2^21 = 2^30
}

// Per format: which dwords of a pair each lane loads (NW of them), in bytes
// from the pair start.
template <int TYPE>
struct QmFmt;

// 9 dwords: [d0 qs0.0-1][qs0 2-5]..[qs0 14-15 d1][qs1 0-3]..[qs1 12-15]
template <>
struct QmFmt<TRC_HIP_TYPE_Q4_0> {
    static constexpr int PW = 9, NW = 4, BIAS = 8;
    __device__ static void offsets(int g, int* o) {
        o[0] = 0; o[1] = 4; o[2] = g < 3 ? 1 + g : 0; o[3] = 5 + g;
    }
};
// 10 dwords: [d0 m0][qs0 x4][d1 m1][qs1 x4]
template <>
struct QmFmt<TRC_HIP_TYPE_Q4_1> {
    static constexpr int PW = 10, NW = 4, BIAS = 0;
    __device__ static void offsets(int g, int* o) {
        o[0] = 0; o[1] = 5; o[2] = 1 + g; o[3] = 6 + g;
    }
};
// 11 dwords: [d0 qh0.lo][qh0.hi qs0.0-1][qs0 2-5]..[qs0 14-15 d1][qh1][qs1 x4]
template <>
struct QmFmt<TRC_HIP_TYPE_Q5_0> {
    static constexpr int PW = 11, NW = 6, BIAS = 16;
    __device__ static void offsets(int g, int* o) {
        o[0] = 0; o[1] = 1; o[2] = 5; o[3] = 6; o[4] = g < 3 ? 2 + g : 1; o[5] = 7 + g;
    }
};
// 12 dwords: [d0 m0][qh0][qs0 x4][d1 m1][qh1][qs1 x4]
template <>
struct QmFmt<TRC_HIP_TYPE_Q5_1> {
    static constexpr int PW = 12, NW = 6, BIAS = 0;
    __device__ static void offsets(int g, int* o) {
        o[0] = 0; o[1] = 1; o[2] = 6; o[3] = 7; o[4] = 2 + g; o[5] = 8 + g;
    }
};
// 17 dwords: [d0 qs0.0-1][qs0 2-5]..[qs0 30-31 d1][qs1 0-3]..[qs1 28-31]
template <>
struct QmFmt<TRC_HIP_TYPE_Q8_0> {
    static constexpr int PW = 17, NW = 7, BIAS = 0;
    __device__ static void offsets(int g, int* o) {
        o[0] = 0; o[1] = 4; o[2] = 8; o[3] = g < 3 ? 1 + g : 0; o[4] = g < 3 ? 5 + g : 4; o[5] = 9 + g;
        o[6] = 13 + g;
    }
};

// Nibble bytes of a quant dword (low nibbles -> k 0..3, high -> k 4..7 of the
// lane group), with the 5th bits of the 4 low / 4 high elements (bits 0-3 /
// 4-7 of fifth). Values stay unsigned (0..31); a bias goes into the MFMA's
// accumulator input instead.
template <bool FIVE>
__device__ __forceinline__ long nibbles(uint32_t w, uint32_t fifth) {
    uint32_t lo = w & 0x0F0F0F0Fu;
    uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
    if constexpr (FIVE) {
        // bit i of a 4-bit field -> bit 8i with one full-rate 24-bit multiply (a plain
        // multiply would be folded with the shift into a quarter-rate 32-bit one),
        // then to bit 4 of byte i
        lo |= (__umul24(fifth & 0xFu, 0x00204081u) & 0x01010101u) << 4;
        hi |= (__umul24((fifth >> 4) & 0xFu, 0x00204081u) & 0x01010101u) << 4;
    }
    return (long) ((uint64_t) lo | ((uint64_t) hi << 32));
}

// 5th bits of lane group g's elements, from a block's qh (rotated for c = 2).
__device__ __forceinline__ uint32_t fifth_bits(uint32_t qh, int g) {
    return ((qh >> (4 * g)) & 0xFu) | (((qh >> (16 + 4 * g)) & 0xFu) << 4);
}
__device__ __forceinline__ uint32_t rot2_halves(uint32_t qh) {
    return ((qh >> 2) & 0x3FFF3FFFu) | ((qh << 14) & 0xC000C000u);
}

// Digit combination a0 + 256 a1 + 65536 a2 as two v_lshl_add_u32: the empty
// asm keeps the compiler from folding it into two shifts and a three-way add.
// (A real inline-asm v_lshl_add would read the MFMA results without the wait
// states the compiler inserts for its own instructions.)
__device__ __forceinline__ uint32_t combine3(int a0, int a1, int a2) {
    uint32_t t = (uint32_t) a0 + ((uint32_t) a1 << 8);
    asm("" : "+v"(t));
    return t + ((uint32_t) a2 << 16);
}

struct QmBlocks {
    long B[2];       // B operands of the even and odd block
    uint32_t dm[2];  // d (low half) and m (high half, Q4_1/Q5_1) as fp16 bits
};

template <int TYPE>
__device__ __forceinline__ QmBlocks qm_decode(const uint32_t* w, int g, uint32_t sel) {
    QmBlocks r;
    if constexpr (TYPE == TRC_HIP_TYPE_Q4_0) {
        r.B[0] = nibbles<false>(__builtin_amdgcn_perm(w[1], w[2], sel), 0);
        r.B[1] = nibbles<false>(w[3], 0);
        r.dm[0] = w[0] & 0xFFFFu;
        r.dm[1] = w[1] >> 16;
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q4_1) {
        r.B[0] = nibbles<false>(w[2], 0);
        r.B[1] = nibbles<false>(w[3], 0);
        r.dm[0] = w[0];
        r.dm[1] = w[1];
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_0) {
        const uint32_t qh0 = __builtin_amdgcn_perm(w[1], w[0], 0x05040302u);
        r.B[0] = nibbles<true>(__builtin_amdgcn_perm(w[2], w[4], sel), fifth_bits(rot2_halves(qh0), g));
        r.B[1] = nibbles<true>(w[5], fifth_bits(w[3], g));
        r.dm[0] = w[0] & 0xFFFFu;
        r.dm[1] = w[2] >> 16;
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_1) {
        r.B[0] = nibbles<true>(w[4], fifth_bits(w[1], g));
        r.B[1] = nibbles<true>(w[5], fifth_bits(w[3], g));
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

constexpr int QM_CP = 8;       // pairs per K chunk (one per wave)
constexpr int QM_RING = 3;     // chunks in flight: registers -> LDS ring depth

// The x operands of one pair (two blocks) for this lane.
struct QmX {
    long xp[2][QM_PLANES];
    f4 sc[2];
    v4i aux[2];  // -BIAS * sum X (int, the first MFMA's accumulator input) or the block sums of x (float bits)
};

template <int TYPE>
__device__ __forceinline__ void qm_load_x(QmX& x, __amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t rm, uint32_t xo,
                                          uint32_t mo, int p) {
    constexpr bool MIN = TYPE == TRC_HIP_TYPE_Q4_1 || TYPE == TRC_HIP_TYPE_Q5_1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int b = 2 * p + h;
#pragma unroll
        for (int d = 0; d < QM_PLANES; ++d) {
            x.xp[h][d] = __builtin_bit_cast(
                long, __builtin_amdgcn_raw_buffer_load_b64(rx, xo, (b * QM_PLANES + d) * 512, 0));
        }
        x.sc[h] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rm, mo, b * 192, 0));
        if constexpr (MIN || QmFmt<TYPE>::BIAS != 0) {
            x.aux[h] = __builtin_bit_cast(
                v4i, __builtin_amdgcn_raw_buffer_load_b128(rm, mo, b * 192 + (MIN ? 64 : 128), 0));
        }
    }
}

// One pair of all T tiles: quant dwords from the LDS chunk, x from registers.
template <int TYPE, int T>
__device__ __forceinline__ void qm_compute(const uint8_t* lds_pair, const uint32_t (*lo)[QmFmt<TYPE>::NW],
                                           const QmX& x, int g, uint32_t sel, f4* acc) {
    constexpr int NW = QmFmt<TYPE>::NW;
    constexpr bool MIN = TYPE == TRC_HIP_TYPE_Q4_1 || TYPE == TRC_HIP_TYPE_Q5_1;
    constexpr int BIAS = QmFmt<TYPE>::BIAS;
    const v4i zero = {0, 0, 0, 0};
    v4i c0[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) c0[h] = BIAS != 0 ? x.aux[h] : zero;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        uint32_t w[NW];
#pragma unroll
        for (int i = 0; i < NW; ++i) w[i] = *(const uint32_t*) (lds_pair + lo[t][i]);
        const QmBlocks q = qm_decode<TYPE>(w, g, sel);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // sum_e (q_e - BIAS) X_e = [sum_e q_e P0_e - BIAS sum_e X_e] + 256 sum_e q_e P1_e + 65536 sum_e q_e P2_e
            const v4i a0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(x.xp[h][0], q.B[h], c0[h], 0, 0, 0);
            const v4i a1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(x.xp[h][1], q.B[h], zero, 0, 0, 0);
            v4i a2 = zero;
            if constexpr (QM_PLANES == 3) a2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(x.xp[h][2], q.B[h], zero, 0, 0, 0);
            const float d = half_bits_to_float(q.dm[h] & 0xFFFFu);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float qx;
                if constexpr (QM_PLANES == 3 && TYPE == TRC_HIP_TYPE_Q8_0) {
                    qx = __builtin_fmaf((float) a2[i], 65536.f, (float) (a0[i] + a1[i] * 256));
                } else if constexpr (QM_PLANES == 3) {
                    // modulo 2^32: the exact result fits in int32 (|q - bias| <= 31, |X| <= 2^21)
                    // even where the partial sums with the bias term would not
                    qx = (float) (int) combine3(a0[i], a1[i], a2[i]);
                } else {
                    qx = (float) (int) ((uint32_t) a0[i] + (uint32_t) a1[i] * 256u);
                }
                acc[t][i] = __builtin_fmaf(qx, d * x.sc[h][i], acc[t][i]);
                if constexpr (MIN) {
                    // the element is copied out first: __builtin_bit_cast applied to a
                    // vector-element lvalue reads element 0 with this compiler
                    const int xs_bits = x.aux[h][i];
                    acc[t][i] = __builtin_fmaf(half_bits_to_float(q.dm[h] >> 16), __builtin_bit_cast(float, xs_bits),
                                               acc[t][i]);
                }
            }
        }
    }
}

template <int TYPE, int T>
struct QmTile {
    static constexpr int PW = QmFmt<TYPE>::PW;
    static constexpr int RB = QM_CP * PW * 4;         // bytes of one row in a chunk (a multiple of 16)
    static constexpr int PITCH = RB + 16;             // LDS row pitch: rows start 4 banks apart
    static constexpr int ROWS = 16 * T;
    static constexpr int BUF = ROWS * PITCH;          // one chunk in LDS
    static constexpr int PIECES = ROWS * (RB / 16);   // 16-byte pieces of a chunk
    static constexpr int PPT = (PIECES + QM_WAVES * 64 - 1) / (QM_WAVES * 64);  // pieces per thread
};

template <int TYPE, int T>
__global__ __launch_bounds__(QM_WAVES * 64) void k_qmm(const uint8_t* __restrict__ W, int nblk, int64_t M,
                                                        int64_t nb1_w, float* __restrict__ y, int64_t ldy, int N,
                                                        int rows_per_wg) {
    using TL = QmTile<TYPE, T>;
    constexpr int NW = QmFmt<TYPE>::NW, PW = TL::PW;
    static_assert(QM_RING * TL::BUF >= QM_WAVES * T * 64 * 16, "reduction buffer aliases the chunk ring");
    __shared__ __attribute__((aligned(16))) uint8_t lds[QM_RING * TL::BUF];

    // wave index as a scalar: the pair a wave computes and its buffer offsets are wave-uniform
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, m16 = lane & 15, g = lane >> 4;
    const int64_t r0 = (int64_t) blockIdx.x * rows_per_wg;
    const int64_t rend = r0 + rows_per_wg < M ? r0 + rows_per_wg : M;
    const int np = nblk / 2;
    const int nch = (np + QM_CP - 1) / QM_CP;
    const uint32_t sel = g < 3 ? 0x03020100u : 0x03020504u;

    // The workgroup's rows as one buffer (the launcher keeps it below 2^31 bytes):
    // loads of rows past M return zeros.
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void*) (W + r0 * nb1_w), (short) 0, (int) ((rend - r0) * nb1_w), QM_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        (void*) g_qm_planes, (short) 0, (int) sizeof(g_qm_planes), QM_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rm =
        __builtin_amdgcn_make_buffer_rsrc((void*) g_qm_meta, (short) 0, (int) sizeof(g_qm_meta), QM_RSRC_WORD3);

    // cooperative chunk copy: thread piece k -> row k / (RB/16), 16 bytes at (k % (RB/16)) * 16
    uint32_t go[TL::PPT], so[TL::PPT];
    bool pv[TL::PPT];
#pragma unroll
    for (int k = 0; k < TL::PPT; ++k) {
        const int q = (int) threadIdx.x + k * QM_WAVES * 64;
        const int row = q / (TL::RB / 16), pc = q % (TL::RB / 16);
        pv[k] = q < TL::PIECES;
        go[k] = (uint32_t) (row * nb1_w) + pc * 16;
        so[k] = row * TL::PITCH + pc * 16;
    }
    // this lane's quant dwords of its wave's pair, per tile, as LDS byte offsets within a chunk
    int off[NW];
    QmFmt<TYPE>::offsets(g, off);
    uint32_t lo[T][NW];
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int i = 0; i < NW; ++i) lo[t][i] = (16 * t + m16) * TL::PITCH + wave * PW * 4 + 4 * off[i];
    }
    const uint32_t xo = lane * 8, mo = 16 * g;

    f4 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};

    uint4 wr[QM_RING][TL::PPT];
    QmX xr[QM_RING];
    auto load_chunk = [&](int s, int c) {
        const int cc = c < nch ? c : nch - 1;  // past the end: repeat the last chunk (unused)
#pragma unroll
        for (int k = 0; k < TL::PPT; ++k) {
            if (pv[k]) {
                wr[s][k] = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, go[k], cc * TL::RB, 0));
            }
        }
        const int p = cc * QM_CP + wave;
        qm_load_x<TYPE>(xr[s], rx, rm, xo, mo, p < np ? p : np - 1);
    };
    auto store_chunk = [&](int s, int buf) {
#pragma unroll
        for (int k = 0; k < TL::PPT; ++k) {
            if (pv[k]) *(uint4*) (lds + buf * TL::BUF + so[k]) = wr[s][k];
        }
    };
    auto step = [&](int c, int s) {
        // chunk c sits in LDS buffer s and its x in xr[s]; chunk c+1 goes to LDS, c+3 is fetched
        if (c * QM_CP + wave < np) qm_compute<TYPE, T>(lds + s * TL::BUF, lo, xr[s], g, sel, acc);
        store_chunk((s + 1) % QM_RING, (s + 1) % QM_RING);
        load_chunk(s, c + QM_RING);
        __syncthreads();
    };

#pragma unroll
    for (int s = 0; s < QM_RING; ++s) load_chunk(s, s);
    store_chunk(0, 0);
    __syncthreads();
    int c = 0;
    for (; c + QM_RING <= nch; c += QM_RING) {
        step(c, 0);
        step(c + 1, 1);
        step(c + 2, 2);
    }
    if (c < nch) step(c, 0);
    if (c + 1 < nch) step(c + 1, 1);

    // sum over the waves (fixed order) through the now idle chunk ring
    f4* red = (f4*) lds;
#pragma unroll
    for (int t = 0; t < T; ++t) red[(wave * T + t) * 64 + lane] = acc[t];
    __syncthreads();
    if (wave >= T) return;
    const int t = wave;
    f4 sum = red[t * 64 + lane];
#pragma unroll
    for (int w = 1; w < QM_WAVES; ++w) sum += red[(w * T + t) * 64 + lane];
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
    hipLaunchKernelGGL(k_qmm_xprep, dim3((unsigned) ((nblk * 16 + 255) / 256)), dim3(256), 0, s, x,
                       (int64_t) (nb1_x / sizeof(float)), N, nblk, rotated_even<TYPE>() ? 2 : 0,
                       QmFmt<TYPE>::BIAS);
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
    // K chunks are copied in 16-byte pieces (a multiple of 4 pairs per row keeps them
    // aligned); a workgroup's 64 rows are addressed through one buffer resource (< 2^31 bytes)
    return N >= 2 && N <= 16 && nblk >= 8 && nblk % 8 == 0 && nblk <= QM_MAX_BLOCKS &&
           (((uintptr_t) wq) & 15u) == 0 && (nb1_w & 15u) == 0 && nb1_w <= ((size_t) 1 << 24);
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
