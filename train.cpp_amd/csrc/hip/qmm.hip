// H2 for 2 <= N <= 32 columns: fused dequant x skinny GEMM on the fp16 matrix
// cores (v_mfma_f32_16x16x32_f16). Columns come in tiles of 16; one launch
// carries one or two tiles (NT), so every weight is read and decoded once per
// 32 columns.
//
// Result to reproduce: gguf_tensor_to_f32 (src/io/trc_gguf.cpp:966-1049,
// dequantize_q* :320-417) followed by compute_mul_mat
// (src/backends/cpu/trc_cpu_ops.cpp:182-216); parity is by tolerance.
//
// Numerics. Within one 32-element block b of one row m
//   sum_e (q_e*d + mn) * x_e,j = d * sum_e (q_e - bias) * x_e,j + mn * sum_e x_e,j.
// The integer quants q_e - bias (|.| <= 128) are exact in fp16. x is converted
// once per call (k_qmm_xprep): every chunk of 16 blocks of every column j is
// scaled by a power of two 2^s so that its max|x'| < 2^14, and x' = x * 2^s is
// split into two fp16 planes, hi = fp16(x') and lo = fp16(x' - hi), about 22
// significant bits. Both planes go through the MFMA into one fp32 accumulator
// (every product of an 11-bit and a 9-bit integer is exact), so a block needs
// one fused multiply-add by d per output, and each pair's sum is scaled back by
// its chunk's 2^-s once. Up to 8 columns, hi and lo share one 16-column tile
// instead (packed: rows 0..7 of the A operand hold hi of columns 0..7, rows
// 8..15 their lo), so each block takes one MFMA and one x load; rows j and
// j + 8 of the result are added once at the end. An element keeps ~22 bits of
// its own magnitude down to 2^17 below its chunk's largest |x|; below that its
// absolute error stays under 2^-39 of that largest |x|, so outputs carry
// FP32-level error. A chunk holding Inf or NaN makes its column come out NaN. (One scale per column would save
// the per-pair rescaling, but finding a column's largest |x| takes one
// workgroup per column, which made the pre-pass ~2 us slower than the
// rescaling saves.)
//
// Quants to fp16 without a conversion instruction: a nibble n OR'ed into the
// mantissa of 1024.0 (0x6400) is the fp16 value 1024 + n, and at bits 4-7 it
// is 1024 + 16n; one packed fp16 add (or fma by 1/16) then gives n - bias
// exactly. Q8_0 bytes go the same way after their sign bits are flipped.
//
// Operand layout (lane l, m16 = l % 16, g = l / 16):
//   A (16 x 32, f16) = x planes: row = column j = m16 of x, k = 8g .. 8g+7
//   B (32 x 16, f16) = quants:   column = row m16 of the W tile, k = 8g .. 8g+7
//   D (16 x 16, f32) = lane holds rows 4g .. 4g+3 (columns j of y), column m16.
// k -> element order. Lane group g's quant bytes hold the elements
// e_p = (c + 4g + p) & 15 (low nibble or Q8_0 low dword) and e_p + 16, p = 0..3,
// and its 8 k values are, in order, e0, e2, e0+16, e2+16, e1, e3, e1+16, e3+16.
// For Q4_0, Q5_0 and Q8_0, blocks come in pairs whose second block starts on a
// 4-byte boundary: odd blocks use c = 0 and even blocks c = 2, so the quant
// bytes a lane needs are one aligned dword or (lane group 3) one v_perm of two.
// Q4_1/Q5_1 blocks are 4-byte aligned and use c = 0 throughout. k_qmm_xprep
// writes the x planes in the same order, so each lane loads its A operand of a
// block with one 16-byte load per plane.
//
// Work split: a workgroup (8 waves) owns up to 112 rows (T tiles of 16) and
// walks K in chunks of 8 pairs. Each chunk is copied by the whole workgroup
// with coalesced 16-byte buffer loads straight into LDS (loads landing in MFMA
// layout directly would touch 16 rows per instruction and swamp the L1 with
// tag lookups), 1 or 2 chunks ahead, into a ring of R + 1 buffers whose rows
// are padded to an odd number of 16-byte pieces (conflict-free reads); wave w
// computes pair w of the chunk for all T row tiles and NT column tiles, so its
// x operands are loaded once per chunk and reused over the row tiles. The partial sums are added across
// the waves through LDS in a fixed order, so results are deterministic. Rows
// per workgroup are chosen so the grid covers every CU once when M allows;
// up to 24 rows per CU, K is split in two parts whose sums meet in y by float
// atomic adds (0 + a + b, the same in either order). Up to 8 columns with K in
// one part of at most 4 chunks, each workgroup converts x into LDS itself and
// the pre-pass does not run.
#include "common.h"

namespace trc_hip {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int QM_MAX_BLOCKS = 2048;  // K <= 65536
constexpr int QM_WAVES = 8;
constexpr int QM_CHB = 16;            // blocks per K chunk (8 pairs, one per wave)
constexpr int QM_LDS = 160 * 1024;      // LDS per workgroup
constexpr int QM_XBITS = 14;          // max|x'| < 2^14 keeps hi and its rounding inside fp16
constexpr int QM_NT = 2;               // column tiles of 16 that one pass over W can carry
constexpr int QM_COLS = 16 * QM_NT;    // columns per chunk and block in the x metadata
constexpr int QM_META_XS = QM_MAX_BLOCKS / QM_CHB * QM_COLS;  // block sums follow the chunk scales
constexpr uint32_t QM_RSRC_WORD3 = 0x00020000u;  // gfx9 buffer resource: raw 32-bit dwords

// x in fp16 planes, written by k_qmm_xprep and read by k_qmm on the same stream,
// in a workspace of QM_WS_BYTES: the A operands, [column tile u][block][plane hi,
// lo][lane 0..63] 16 bytes each (tile u holds columns 16u .. 16u + 15), then the
// meta floats: 2^-s per (chunk, column j) (NaN for a chunk with a non-finite
// value) at [chunk * QM_COLS + j], then the block sums of x' = x * 2^s at
// [QM_META_XS + block * QM_COLS + j] (read for Q4_1/Q5_1). k_qmm_xprep writes
// every entry k_qmm reads, so a workspace needs no clearing between calls.
constexpr int QM_A_BYTES = QM_NT * QM_MAX_BLOCKS * 2 * 64 * 16;
constexpr int QM_META_BYTES = (QM_META_XS + QM_MAX_BLOCKS * QM_COLS) * 4;
static_assert(QM_A_BYTES % 256 == 0, "the meta floats start 256-byte aligned");

template <int TYPE>
constexpr bool rotated_even() {
    return TYPE == TRC_HIP_TYPE_Q4_0 || TYPE == TRC_HIP_TYPE_Q5_0 || TYPE == TRC_HIP_TYPE_Q8_0;
}

// Wave-wide reductions with DPP row operations (VALU latency, no LDS
// round trips): within rows of 16, then into lane 63 with the row broadcasts,
// whose masked-out rows keep 0 (the identity here: values are >= 0, flags 0/1).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int qm_dpp(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, ROW_MASK, 0xF, false);
}
__device__ __forceinline__ float qm_wave_max(float v) {  // every lane: max over the wave (v >= 0)
    auto m = [](float a, int b) { return fmaxf(a, __builtin_bit_cast(float, b)); };
    v = m(v, qm_dpp<0xB1, 0xF>(__builtin_bit_cast(int, v)));   // quad_perm [1,0,3,2]
    v = m(v, qm_dpp<0x4E, 0xF>(__builtin_bit_cast(int, v)));   // quad_perm [2,3,0,1]
    v = m(v, qm_dpp<0x141, 0xF>(__builtin_bit_cast(int, v)));  // row_half_mirror
    v = m(v, qm_dpp<0x140, 0xF>(__builtin_bit_cast(int, v)));  // row_mirror
    v = m(v, qm_dpp<0x142, 0xA>(__builtin_bit_cast(int, v)));  // row_bcast:15
    v = m(v, qm_dpp<0x143, 0xC>(__builtin_bit_cast(int, v)));  // row_bcast:31
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ int qm_wave_or(int v) {  // every lane: OR over the wave
    v |= qm_dpp<0xB1, 0xF>(v);
    v |= qm_dpp<0x4E, 0xF>(v);
    v |= qm_dpp<0x141, 0xF>(v);
    v |= qm_dpp<0x140, 0xF>(v);
    v |= qm_dpp<0x142, 0xA>(v);
    v |= qm_dpp<0x143, 0xC>(v);
    return __builtin_amdgcn_readlane(v, 63);
}

// The 8 x elements lane (block bl = l / 4 of chunk ch, lane group g = l % 4)
// of the wave for column j converts, in slot order (zeros past N or nblk).
__device__ __forceinline__ void qm_xload(const float* __restrict__ x, int64_t ldx, int N, int nblk, int rot, int ch,
                                         int j, int l, float2 (&v)[4]) {
    const int bl = l >> 2, g = l & 3;
    const int b = ch * QM_CHB + bl;
    const bool live = j < N && b < nblk;
    const int c = ((b & 1) == 0 && rot) ? 2 : 0;
    const int e0 = (c + 4 * g) & 15, e2 = (c + 4 * g + 2) & 15;  // e1 = e0 + 1, e3 = e2 + 1
    const float2* blk = (const float2*) (x + (int64_t) (live ? j : 0) * ldx + (int64_t) (live ? b : 0) * QK);
    const float2 z = {0.f, 0.f};
    v[0] = live ? blk[e0 >> 1] : z;
    v[1] = live ? blk[e2 >> 1] : z;
    v[2] = live ? blk[(e0 + 16) >> 1] : z;
    v[3] = live ? blk[(e2 + 16) >> 1] : z;
}

// One chunk of one column, converted by one wave from the values qm_xload gave
// each lane: the chunk's scale 2^-s (NaN for a chunk with a non-finite value),
// the lane's hi and lo A entries and its block's sum of x' (in every lane of the block).
struct QmXConv {
    h8 hi, lo;
    float sm, sc;
};
__device__ __forceinline__ QmXConv qm_xconv(const float2 (&w)[4]) {
    const float v[8] = {w[0].x, w[1].x, w[2].x, w[3].x, w[0].y, w[1].y, w[2].y, w[3].y};  // slot order
    float mx = 0.f;
    int bad = 0;  // fmaxf drops NaN, so non-finite values are flagged separately
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        mx = fmaxf(mx, fabsf(v[k]));
        bad |= !__builtin_isfinite(v[k]);
    }
    mx = qm_wave_max(mx);
    bad = qm_wave_or(bad);
    const bool finite = bad == 0;
    // mx = f * 2^E, f in [0.5, 1): every |x| * 2^s < 2^QM_XBITS. At most 149, so that
    // 2^-s stays a float: below 2^-135 every x is a multiple of 2^-149, and
    // x * 2^149 is then an exact integer under 2^14.
    const int s = (mx > 0.f && finite) ? min(QM_XBITS - __builtin_amdgcn_frexp_expf(mx), 149) : 0;
    QmXConv r;
    float sm = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float e = finite ? __builtin_ldexpf(v[k], s) : 0.f;
        sm += e;
        const _Float16 h = (_Float16) e;
        r.hi[k] = h;
        r.lo[k] = (_Float16) (e - (float) h);
    }
    // the 4 lanes of a block (a quad): sum, in every one of them
    sm += __builtin_bit_cast(float, qm_dpp<0xB1, 0xF>(__builtin_bit_cast(int, sm)));
    sm += __builtin_bit_cast(float, qm_dpp<0x4E, 0xF>(__builtin_bit_cast(int, sm)));
    r.sm = sm;
    r.sc = finite ? __builtin_ldexpf(1.f, -s) : __builtin_nanf("");
    return r;
}

// One wave per (chunk of QM_CHB blocks, column j < ncol = 16 or 32): lane l carries block
// b = l / 4 of the chunk and lane group g = l % 4. It loads exactly the 8
// elements of A entry (b, g) (the low elements e_p and e_p + 16), the wave's
// largest |x| and finiteness give the chunk's scale 2^s, and the lane writes its
// hi and lo entries. The block sums of x' (for Q4_1/Q5_1) are added over the
// four lanes of a block. No reduction spans more than one wave.
//
// Packed (pk = 1, N <= 8, ncol = 8): the wave of column j writes hi to A row j
// and lo to A row j + 8 of one plane, the chunk scale to both, and the block
// sums to row j only (row j + 8 gets 0, so Q4_1/Q5_1 add m * sum x once).
//
// A launch split over K adds two partial sums into y, so then (y0 != nullptr)
// the wave also clears its share of column j of y: rows
// [ch * per, (ch + 1) * per) with per = ceil(M / chunks).
__global__ __launch_bounds__(64) void k_qmm_xprep(const float* __restrict__ x, int64_t ldx, int N, int nblk, int rot,
                                                   int ncol, int pk, float* __restrict__ y0, int64_t ldy, int64_t M,
                                                   uint8_t* __restrict__ ws) {
    uint4* const xa = (uint4*) ws;
    float* const meta = (float*) (ws + QM_A_BYTES);
    const int ch = blockIdx.x / ncol, j = blockIdx.x % ncol;  // columns past N get zeros
    const int l = threadIdx.x, bl = l >> 2, g = l & 3;
    if (y0 != nullptr && j < N) {
        const int64_t nchunks = gridDim.x / ncol, per = (M + nchunks - 1) / nchunks;
        const int64_t a = ch * per, e = a + per < M ? a + per : M;
        for (int64_t m = a + l; m < e; m += 64) y0[j * ldy + m] = 0.f;
    }
    float2 v[4];
    qm_xload(x, ldx, N, nblk, rot, ch, j, l, v);
    const QmXConv r = qm_xconv(v);
    const int b = ch * QM_CHB + bl;
    if (b < nblk) {
        uint4* dst = xa + ((int64_t) (j >> 4) * QM_MAX_BLOCKS + b) * 2 * 64 + (j & 15) + 16 * g;
        dst[0] = __builtin_bit_cast(uint4, r.hi);
        dst[pk ? 8 : 64] = __builtin_bit_cast(uint4, r.lo);
        if (g == 0) meta[QM_META_XS + b * QM_COLS + j] = r.sm;
        if (pk && g == 0) meta[QM_META_XS + b * QM_COLS + j + 8] = 0.f;
    }
    if (l == 0) meta[ch * QM_COLS + j] = r.sc;
    if (pk && l == 0) meta[ch * QM_COLS + j + 8] = r.sc;
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

// fp16 B operand of one block for lane group g, in the k order e0, e2, e0+16,
// e2+16, e1, e3, e1+16, e3+16 (e_p = element of quant byte p of the lane's dword).
//   nibble formats: w = the lane's quant dword (byte p: low nibble e_p, high e_p+16),
//     f5 = the 5th bits as bit p (e_p) and bit 4+p (e_p+16) (Q5_0/Q5_1),
//     value q - BIAS with q = nibble (+ 16 * 5th bit);
//   Q8_0: lo / hi = the lane's quant bytes of e_p / e_p + 16 (signed).
// Masks and the fp16 magic number kept in VGPRs: gfx9 VOP3 encodes no literal,
// so v_and_or_b32 needs its constants in registers (otherwise and + or).
struct QmK {
    uint32_t lo4, hi4, lo8, magic;
};
__device__ __forceinline__ QmK qm_consts() {
    QmK k{0x000F000Fu, 0x00F000F0u, 0x00FF00FFu, 0x64006400u};
    asm volatile("" : "+v"(k.lo4), "+v"(k.hi4), "+v"(k.lo8), "+v"(k.magic));
    return k;
}

template <int BIAS, bool FIVE>
__device__ __forceinline__ h8 qm_nibbles_f16(uint32_t w, uint32_t f5, const QmK& k) {
    const uint32_t w8 = w >> 8;
    uint32_t t0 = (w & k.lo4) | k.magic;   // 1024 + n: bytes 0, 2 low nibbles  (e0, e2)
    uint32_t t1 = (w & k.hi4) | k.magic;   // 1024 + 16n: bytes 0, 2 high       (e0+16, e2+16)
    uint32_t t2 = (w8 & k.lo4) | k.magic;  // bytes 1, 3 low                      (e1, e3)
    uint32_t t3 = (w8 & k.hi4) | k.magic;  // bytes 1, 3 high                     (e1+16, e3+16)
    if constexpr (FIVE) {
        // 5th bit of e_p -> bit 4 (+16 for the high half); of e_p+16 -> bit 8 (x16 scale)
        // with one full-rate 24-bit multiply per pair: bits 0 and 2 of a field land
        // on bits 4 and 20 (x 0x40010), bits 4 and 6 on bits 8 and 24 (x 0x40010 >> ...)
        t0 |= __umul24(f5 & 0x5u, 0x40010u) & 0x00100010u;          // bits 0, 2 -> 4, 20
        t2 |= __umul24((f5 >> 1) & 0x5u, 0x40010u) & 0x00100010u;   // bits 1, 3 -> 4, 20
        t1 |= __umul24((f5 >> 4) & 0x5u, 0x40010u) << 4 & 0x01000100u;  // bits 4, 6 -> 8, 24
        t3 |= __umul24((f5 >> 5) & 0x5u, 0x40010u) << 4 & 0x01000100u;  // bits 5, 7 -> 8, 24
    }
    constexpr _Float16 LOW = (_Float16) (-(1024 + BIAS));        // 1024 + q  -> q - BIAS
    constexpr _Float16 HIGH = (_Float16) (-(64 + BIAS));         // (1024 + 16q) / 16 -> q - BIAS
    const h2 r0 = __builtin_bit_cast(h2, t0) + h2{LOW, LOW};
    const h2 r1 = __builtin_bit_cast(h2, t1) * h2{(_Float16) 0.0625f, (_Float16) 0.0625f} + h2{HIGH, HIGH};
    const h2 r2 = __builtin_bit_cast(h2, t2) + h2{LOW, LOW};
    const h2 r3 = __builtin_bit_cast(h2, t3) * h2{(_Float16) 0.0625f, (_Float16) 0.0625f} + h2{HIGH, HIGH};
    return h8{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
}

__device__ __forceinline__ h8 qm_bytes_f16(uint32_t lo, uint32_t hi, const QmK& k) {
    const uint32_t ul = lo ^ 0x80808080u, uh = hi ^ 0x80808080u;  // q + 128 in every byte
    const uint32_t t0 = (ul & k.lo8) | k.magic;         // bytes 0, 2 of lo (e0, e2)
    const uint32_t t1 = (uh & k.lo8) | k.magic;         // bytes 0, 2 of hi (e0+16, e2+16)
    const uint32_t t2 = ((ul >> 8) & k.lo8) | k.magic;  // bytes 1, 3 of lo (e1, e3)
    const uint32_t t3 = ((uh >> 8) & k.lo8) | k.magic;  // bytes 1, 3 of hi (e1+16, e3+16)
    constexpr _Float16 OFF = (_Float16) -1152.f;               // 1024 + 128 + q -> q
    const h2 r0 = __builtin_bit_cast(h2, t0) + h2{OFF, OFF};
    const h2 r1 = __builtin_bit_cast(h2, t1) + h2{OFF, OFF};
    const h2 r2 = __builtin_bit_cast(h2, t2) + h2{OFF, OFF};
    const h2 r3 = __builtin_bit_cast(h2, t3) + h2{OFF, OFF};
    return h8{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
}

// 5th bits of lane group g's elements, from a block's qh (rotated for c = 2).
__device__ __forceinline__ uint32_t fifth_bits(uint32_t qh, int g) {
    return ((qh >> (4 * g)) & 0xFu) | (((qh >> (16 + 4 * g)) & 0xFu) << 4);
}
__device__ __forceinline__ uint32_t rot2_halves(uint32_t qh) {
    return ((qh >> 2) & 0x3FFF3FFFu) | ((qh << 14) & 0xC000C000u);
}

struct QmBlocks {
    h8 B[2];         // B operands of the even and odd block
    uint32_t dm[2];  // d (low half) and m (high half, Q4_1/Q5_1) as fp16 bits
};

template <int TYPE>
__device__ __forceinline__ QmBlocks qm_decode(const uint32_t* w, int g, uint32_t sel, const QmK& k) {
    QmBlocks r;
    if constexpr (TYPE == TRC_HIP_TYPE_Q4_0) {
        r.B[0] = qm_nibbles_f16<8, false>(__builtin_amdgcn_perm(w[1], w[2], sel), 0, k);
        r.B[1] = qm_nibbles_f16<8, false>(w[3], 0, k);
        r.dm[0] = w[0] & 0xFFFFu;
        r.dm[1] = w[1] >> 16;
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q4_1) {
        r.B[0] = qm_nibbles_f16<0, false>(w[2], 0, k);
        r.B[1] = qm_nibbles_f16<0, false>(w[3], 0, k);
        r.dm[0] = w[0];
        r.dm[1] = w[1];
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_0) {
        const uint32_t qh0 = __builtin_amdgcn_perm(w[1], w[0], 0x05040302u);
        r.B[0] = qm_nibbles_f16<16, true>(__builtin_amdgcn_perm(w[2], w[4], sel), fifth_bits(rot2_halves(qh0), g), k);
        r.B[1] = qm_nibbles_f16<16, true>(w[5], fifth_bits(w[3], g), k);
        r.dm[0] = w[0] & 0xFFFFu;
        r.dm[1] = w[2] >> 16;
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_1) {
        r.B[0] = qm_nibbles_f16<0, true>(w[4], fifth_bits(w[1], g), k);
        r.B[1] = qm_nibbles_f16<0, true>(w[5], fifth_bits(w[3], g), k);
        r.dm[0] = w[0];
        r.dm[1] = w[2];
    } else {  // Q8_0
        r.B[0] = qm_bytes_f16(__builtin_amdgcn_perm(w[1], w[3], sel), __builtin_amdgcn_perm(w[2], w[4], sel), k);
        r.B[1] = qm_bytes_f16(w[5], w[6], k);
        r.dm[0] = w[0] & 0xFFFFu;
        r.dm[1] = w[2] >> 16;
    }
    return r;
}

constexpr int QM_CP = 8;       // pairs per K chunk (one per wave)
static_assert(2 * QM_CP == QM_CHB, "the x scales follow the K chunks");

// The x operands of one pair (two blocks) of one column tile for this lane.
struct QmXT {
    h8 a[2][2];  // [block][plane hi, lo]
    f4 sc;       // 2^-s of the pair's chunk for the lane's 4 columns
    f4 xs[2];    // block sums of x' for the lane's 4 columns (Q4_1/Q5_1)
};
template <int NT>
struct QmX {
    QmXT u[NT];  // column tiles
};

// PK: packed hi/lo (one tile, N <= 8): only plane 0 of each block.
template <int TYPE, int NT, bool PK>
__device__ __forceinline__ void qm_load_x(QmX<NT>& x, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rm,
                                          uint32_t ao, uint32_t mo, int p) {
    constexpr bool MIN = TYPE == TRC_HIP_TYPE_Q4_1 || TYPE == TRC_HIP_TYPE_Q5_1;
#pragma unroll
    for (int u = 0; u < NT; ++u) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int b = 2 * p + h;
#pragma unroll
            for (int pl = 0; pl < (PK ? 1 : 2); ++pl) {
                x.u[u].a[h][pl] = __builtin_bit_cast(
                    h8, __builtin_amdgcn_raw_buffer_load_b128(ra, ao, ((u * QM_MAX_BLOCKS + b) * 2 + pl) * 1024, 0));
            }
            if constexpr (MIN) {
                x.u[u].xs[h] = __builtin_bit_cast(
                    f4, __builtin_amdgcn_raw_buffer_load_b128(rm, mo, (QM_META_XS + b * QM_COLS + 16 * u) * 4, 0));
            }
        }
        x.u[u].sc = __builtin_bit_cast(
            f4, __builtin_amdgcn_raw_buffer_load_b128(rm, mo, ((2 * p / QM_CHB) * QM_COLS + 16 * u) * 4, 0));
    }
}

// The scaled sums of one tile's pair: per block d * sum_e (q_e - BIAS) x'_e (+ m *
// sum_e x'_e for Q4_1/Q5_1) in units of x' = x * 2^s, then back to units of x.
template <int TYPE>
__device__ __forceinline__ void qm_scale(const f4 (&c)[2], const uint32_t (&dm)[2], const QmXT& x, f4& acc) {
    constexpr bool MIN = TYPE == TRC_HIP_TYPE_Q4_1 || TYPE == TRC_HIP_TYPE_Q5_1;
    f4 part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float d = half_bits_to_float(dm[h] & 0xFFFFu);
#pragma unroll
        for (int i = 0; i < 4; ++i) part[i] = __builtin_fmaf(d, c[h][i], part[i]);
        if constexpr (MIN) {
            const float mn = half_bits_to_float(dm[h] >> 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // the element is copied out first: __builtin_bit_cast applied to a
                // vector-element lvalue reads element 0 with this compiler
                const float xs = x.xs[h][i];
                part[i] = __builtin_fmaf(mn, xs, part[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float sc = x.sc[i];
        acc[i] = __builtin_fmaf(sc, part[i], acc[i]);
    }
}

// One pair of all T row tiles and NT column tiles: quant dwords from the LDS
// chunk, x from registers. Each row tile's quants are decoded once for all
// column tiles. Software-pipelined over the row tiles: every quant dword is read
// first, then step t issues tile t's MFMAs and, while they run, decodes tile
// t + 1 and scales tile t - 1, whose MFMA results are one step old. The
// scheduling barriers keep the compiler from folding the steps back into a
// dependent chain.
template <int TYPE, int T, int NT, bool PK>
__device__ __forceinline__ void qm_compute(const uint8_t* lds_pair, const uint32_t* lo, const QmX<NT>& x, int g,
                                           uint32_t sel, const QmK& kc, f4 (*acc)[NT]) {
    constexpr int NW = QmFmt<TYPE>::NW, RB = QM_CP * QmFmt<TYPE>::PW * 4;  // bytes of one row in a chunk
    const f4 zero = {0.f, 0.f, 0.f, 0.f};
    uint32_t w[T][NW];
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int i = 0; i < NW; ++i) w[t][i] = *(const uint32_t*) (lds_pair + lo[i] + t * 16 * (RB + 16));
    }
    QmBlocks q[T];
    f4 c[T][NT][2];
    q[0] = qm_decode<TYPE>(w[0], g, sel, kc);
#pragma unroll
    for (int t = 0; t < T; ++t) {
        // sum_e (q_e - BIAS) x'_e over both planes: exact products, fp32 sums
#pragma unroll
        for (int u = 0; u < NT; ++u)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                c[t][u][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.u[u].a[h][0], q[t].B[h], zero, 0, 0, 0);
        if constexpr (!PK) {  // packed: plane 0 already carries lo in rows 8..15
#pragma unroll
            for (int u = 0; u < NT; ++u)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    c[t][u][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.u[u].a[h][1], q[t].B[h], c[t][u][h], 0, 0, 0);
        }
        if (t + 1 < T) q[t + 1] = qm_decode<TYPE>(w[t + 1], g, sel, kc);
        if (t >= 1) {
#pragma unroll
            for (int u = 0; u < NT; ++u) qm_scale<TYPE>(c[t - 1][u], q[t - 1].dm, x.u[u], acc[t - 1][u]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int u = 0; u < NT; ++u) qm_scale<TYPE>(c[T - 1][u], q[T - 1].dm, x.u[u], acc[T - 1][u]);
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at their maximum).
template <int VM>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(VM >= 0 && VM < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((VM & 0xF) | ((VM >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// 16 bytes per lane from a buffer straight into LDS at lds + 16 * lane
// (buffer_load_dwordx4 ... lds; the LDS base goes through M0).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*) lds, 16, voff, soff, 0, 0);
}

template <int TYPE, int T, int ROUNDS>
struct QmTile {
    static constexpr int PW = QmFmt<TYPE>::PW;
    static constexpr int RB = QM_CP * PW * 4;             // bytes of one row in a chunk (a multiple of 16)
    static constexpr int LS = RB + 16;                     // LDS row stride: the row and one spare piece
    static constexpr int FILL = ROUNDS * QM_WAVES * 64 * 16;  // bytes the copy of one chunk writes
    // one chunk buffer in LDS: the copied pieces, and at least all 16T rows, so
    // that the reads of the last tile's rows past the workgroup's stay inside it
    static constexpr int BUF = FILL > 16 * T * LS ? FILL : 16 * T * LS;
};

// k_qmm's LDS: the chunk ring (reused at the end for the sums of every wave),
// then with LXC > 0 the part's x in LDS: the A entries [block of the part][lane]
// (16 bytes each), the chunk scales [chunk][slot] and (Q4_1/Q5_1) the block
// sums [block of the part][slot].
template <int TYPE, int T, int ROUNDS, int R, int NT, int LXC>
struct QmLdsX {
    static constexpr bool MIN = TYPE == TRC_HIP_TYPE_Q4_1 || TYPE == TRC_HIP_TYPE_Q5_1;
    static constexpr int RING = (R + 1) * QmTile<TYPE, T, ROUNDS>::BUF;
    static constexpr int RED = QM_WAVES * T * NT * 64 * 16;
    static constexpr int X0 = RING > RED ? RING : RED;                 // A entries
    static constexpr int SC0 = X0 + LXC * QM_CHB * 1024;               // chunk scales
    static constexpr int XS0 = SC0 + LXC * 16 * 4;                     // block sums
    static constexpr int BYTES = XS0 + (MIN ? LXC * QM_CHB * 16 * 4 : 0);
};

// R chunks of W stream from HBM straight into an LDS ring of R + 1 buffers
// (buffer_load ... lds: no registers, no VALU), each chunk with the x operands
// it needs loaded R chunks ahead into a register ring. Per chunk every wave
// issues exactly ROUNDS + NA vector loads, so one vmcnt wait covers both: the
// counter retires loads in issue order. Lanes past the workgroup's rows and the
// chunks past the end re-read valid data; nothing reads their results.
//
// K split: blockIdx.y selects chunks [c0, c0 + part_chunks) of K. With more than
// one part (gridDim.y == 2) the parts' sums meet in y, which k_qmm_xprep
// cleared, by float atomic adds; 0 + a + b rounds the same in either order.
//
// PK: packed hi/lo x (NT = 1, N <= 8): one x load and one MFMA per block, and
// result rows j + 8 (the lo products) are added into rows j at the end.
//
// LXC > 0 (packed, K in one part of at most LXC chunks): the workgroup converts
// x (xsrc, columns ldx floats apart) into LDS before the main loop, in the
// workspace's layout: wave w takes column w, one chunk at a time, as
// k_qmm_xprep does, and the main loop reads its x operands from LDS. Its x
// loads are issued before the first W copies, so the in-order vmcnt does not
// hold them behind the copies. ws is then not read and no pre-pass runs.
template <int TYPE, int T, int ROUNDS, int R, int NT, bool PK, int LXC>
__global__ __launch_bounds__(QM_WAVES * 64) void k_qmm(const uint8_t* __restrict__ W, int nblk, int64_t M,
                                                        int64_t nb1_w, float* __restrict__ y, int64_t ldy, int N,
                                                        int rows_per_wg, int part_chunks,
                                                        const uint8_t* __restrict__ ws, const float* __restrict__ xsrc,
                                                        int64_t ldx) {
    using TL = QmTile<TYPE, T, ROUNDS>;
    using LL = QmLdsX<TYPE, T, ROUNDS, R, NT, LXC>;
    constexpr int NW = QmFmt<TYPE>::NW, PW = TL::PW;
    constexpr bool MIN = TYPE == TRC_HIP_TYPE_Q4_1 || TYPE == TRC_HIP_TYPE_Q5_1;
    constexpr bool LX = LXC > 0;
    // x loads per chunk and wave: per column tile two blocks x two planes, scales, block sums
    static_assert(!PK || NT == 1, "packed x is one tile of 8 columns");
    static_assert(!LX || PK, "x in LDS is the packed layout");
    static_assert(!LX || QM_WAVES == 8, "one wave per packed column");
    constexpr int NA = LX ? 0 : NT * ((PK ? 1 : 2) * 2 + 1 + (MIN ? 2 : 0));
    static_assert(LL::BYTES <= QM_LDS, "LDS");
    __shared__ __attribute__((aligned(16))) uint8_t lds[LL::BYTES];

    // wave index as a scalar: the pair a wave computes and its buffer offsets are wave-uniform
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, m16 = lane & 15, g = lane >> 4;
    const int64_t r0 = (int64_t) blockIdx.x * rows_per_wg;
    const int64_t rend = r0 + rows_per_wg < M ? r0 + rows_per_wg : M;
    const int rows = (int) (rend - r0);
    const int np = nblk / 2;
    const int nch = (np + QM_CP - 1) / QM_CP;
    const int c0 = blockIdx.y * part_chunks;                             // this part's first chunk
    const int nl = part_chunks < nch - c0 ? part_chunks : nch - c0;      // and its chunk count (>= 1)
    const uint32_t sel = g < 3 ? 0x03020100u : 0x03020504u;

    // The workgroup's rows as one buffer (the launcher keeps it below 2^31 bytes).
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void*) (W + r0 * nb1_w), (short) 0, (int) ((int64_t) rows * nb1_w), QM_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void*) ws, (short) 0, QM_A_BYTES, QM_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rm =
        __builtin_amdgcn_make_buffer_rsrc((void*) (ws + QM_A_BYTES), (short) 0, QM_META_BYTES, QM_RSRC_WORD3);

    // LDS slot k * 512 + thread = row q / LS16, piece q % LS16 of a chunk: rows
    // sit TL::LS = RB + 16 bytes apart, an odd number of 16-byte pieces, so the
    // 16 rows a lane group reads in one instruction fall on 16 different 4-bank
    // groups (64 banks of 4 bytes) and every tile has the same layout at a fixed
    // offset. The spare piece of a row re-reads the row's last piece, and slots
    // past the rows re-read piece 0; nothing reads either.
    constexpr int RB16 = TL::RB / 16, LS16 = RB16 + 1;
    uint32_t go[ROUNDS];
#pragma unroll
    for (int k = 0; k < ROUNDS; ++k) {
        int q = k * QM_WAVES * 64 + (int) threadIdx.x;
        if (q >= rows * LS16) q = 0;
        const int r = q / LS16, slot = q % LS16;
        go[k] = (uint32_t) (r * nb1_w) + (uint32_t) (slot < RB16 ? slot : RB16 - 1) * 16;
    }
    // this lane's quant dwords of its wave's pair in tile 0, as LDS byte offsets
    // within a chunk (tile t adds 16 * t rows)
    int off[NW];
    QmFmt<TYPE>::offsets(g, off);
    uint32_t lo[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int d = wave * PW + off[i];  // dword of the row chunk
        lo[i] = m16 * TL::LS + d * 4;
    }
    const uint32_t xo = lane * 16, mo = 16 * g;
    const QmK kc = qm_consts();

    f4 acc[T][NT];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int u = 0; u < NT; ++u) acc[t][u] = f4{0.f, 0.f, 0.f, 0.f};

    QmX<NT> xr[R];
    // W of the part's chunk c (or of its last one past the end) -> LDS buffer b
    auto load_w = [&](int c, int b) {
        const int cc = c0 + (c < nl ? c : nl - 1);
        uint8_t* dst = lds + b * TL::BUF + wave * 1024;
#pragma unroll
        for (int k = 0; k < ROUNDS; ++k) {
            dma16(rw, dst + k * QM_WAVES * 1024, go[k], cc * TL::RB);
        }
    };
    // x operands of this wave's pair of the part's chunk c -> xr[xs]
    auto load_x = [&](int c, int xs) {
        const int p = (c0 + (c < nl ? c : nl - 1)) * QM_CP + wave;
        qm_load_x<TYPE, NT, PK>(xr[xs], rx, rm, xo, mo, p < np ? p : np - 1);
    };
    // Step c. Loads go out per chunk as W then x, so once at most (R - 1) chunks'
    // loads are outstanding, chunk c's W (this wave's part) and x have landed;
    // the barrier makes every wave's part of the W chunk visible. Chunk c + R's W
    // goes to the buffer of chunk c - 1, which every wave finished before the
    // barrier; its x goes to xr[c % R] once chunk c is computed.
    auto step = [&](int c, int xs) {
        wait_vmcnt<(R - 1) * (ROUNDS + NA)>();
        // a bare s_barrier: __syncthreads' workgroup fence would also wait for
        // every LDS-bound load in flight, i.e. drain the ring each step. The
        // empty asm keeps the compiler from moving LDS accesses across it.
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        load_w(c + R, (c + R) % (R + 1));
        if (c < nl && (c0 + c) * QM_CP + wave < np) {
            if constexpr (LX) {
                // this wave's pair of local chunk c: blocks c * 16 + 2 * wave + h of the part
                QmX<NT> xq;
                const int bq = c * QM_CHB + 2 * wave;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    xq.u[0].a[h][0] = *(const h8*) (lds + LL::X0 + ((bq + h) * 64 + lane) * 16);
                    if constexpr (MIN) xq.u[0].xs[h] = *(const f4*) (lds + LL::XS0 + ((bq + h) * 16 + 4 * g) * 4);
                }
                xq.u[0].sc = *(const f4*) (lds + LL::SC0 + (c * 16 + 4 * g) * 4);
                qm_compute<TYPE, T, NT, PK>(lds + (c % (R + 1)) * TL::BUF, lo, xq, g, sel, kc, acc);
            } else {
                qm_compute<TYPE, T, NT, PK>(lds + (c % (R + 1)) * TL::BUF, lo, xr[xs], g, sel, kc, acc);
            }
        }
        if constexpr (!LX) load_x(c + R, xs);
    };
    // x of the part into LDS: loads first, then the W copies, then the conversion
    float2 xv[LX ? LXC : 1][4];
    if constexpr (LX) {
#pragma unroll
        for (int c = 0; c < LXC; ++c) {
            if (c < nl) qm_xload(xsrc, ldx, N, nblk, rotated_even<TYPE>() ? 2 : 0, c0 + c, wave, lane, xv[c]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // prologue in chunk order (the first wait counts on chunk 0's loads being the oldest)
#pragma unroll
    for (int i = 0; i < R; ++i) {
        load_w(i, i);
        if constexpr (!LX) load_x(i, i);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (LX) {
        const int bl = lane >> 2, gq = lane & 3, j = wave;
#pragma unroll
        for (int c = 0; c < LXC; ++c) {
            if (c < nl) {
                const QmXConv r = qm_xconv(xv[c]);
                uint4* xa = (uint4*) (lds + LL::X0) + (c * QM_CHB + bl) * 64 + j + 16 * gq;
                xa[0] = __builtin_bit_cast(uint4, r.hi);
                xa[8] = __builtin_bit_cast(uint4, r.lo);
                if (lane == 0) {
                    float* sc = (float*) (lds + LL::SC0) + c * 16;
                    sc[j] = r.sc;
                    sc[j + 8] = r.sc;
                }
                if constexpr (MIN) {
                    if (gq == 0) {
                        float* xs = (float*) (lds + LL::XS0) + (c * QM_CHB + bl) * 16;
                        xs[j] = r.sm;
                        xs[j + 8] = 0.f;
                    }
                }
            }
        }
        // the LDS writes complete (lgkmcnt; the W copies stay in flight), then every wave's are visible
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }
    // whole groups of R steps, so that every path issues the same loads (steps
    // past the last chunk compute nothing) and the compiler's own wait counts
    // for the x registers stay exact
    for (int c = 0; c < nl; c += R) {
#pragma unroll
        for (int i = 0; i < R; ++i) step(c + i, i);
    }
    wait_vmcnt<0>();
    __syncthreads();

    // sum over the waves (fixed order) through the now idle chunk ring; wave
    // w then finishes the (row tile, column tile) pairs w, w + 8, ...
    f4* red = (f4*) lds;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int u = 0; u < NT; ++u) red[((wave * T + t) * NT + u) * 64 + lane] = acc[t][u];
    __syncthreads();
    for (int tu = wave; tu < T * NT; tu += QM_WAVES) {
        const int t = tu % T, u = tu / T;
        f4 sum = red[(t * NT + u) * 64 + lane];
#pragma unroll
        for (int w = 1; w < QM_WAVES; ++w) sum += red[((w * T + t) * NT + u) * 64 + lane];
        if constexpr (PK) {
            // lane groups 2 and 3 hold the lo products of lane groups 0 and 1's columns
            if (lane < 32) {
#pragma unroll
                for (int w = 0; w < QM_WAVES; ++w) sum += red[((w * T + t) * NT + u) * 64 + lane + 32];
            }
        }
        const int64_t m = r0 + 16 * t + m16;
        if (m >= rend) continue;
        if (gridDim.y == 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = 16 * u + 4 * g + i;
                if (j < N) y[j * ldy + m] = sum[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = 16 * u + 4 * g + i;
                if (j < N) {
                    __hip_atomic_fetch_add(y + j * ldy + m, sum[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
    }
}

// One call's arguments on their way to the launch.
struct QmCall {
    const void* wq;
    int nblk;
    int64_t M;
    size_t nb1_w;
    float* y;
    size_t nb1_y;
    int N;
    int rows, parts, part_chunks;
    const uint8_t* ws;
    const float* x;  // read by the kernel only when it converts x itself
    size_t nb1_x;
    hipStream_t s;
};

template <int TYPE, int T, int ROUNDS, int R, int NT, bool PK, int LXC>
int launch_t(const QmCall& q) {
    if constexpr (QmLdsX<TYPE, T, ROUNDS, R, NT, LXC>::BYTES > QM_LDS) {
        // not reached: qm_lx_fits keeps such plans on the pre-pass path
        return fail(TRC_HIP_E_INVALID, "qmm: %d rows per workgroup and x exceed the LDS", q.rows);
    } else {
        const int64_t grid = (q.M + q.rows - 1) / q.rows;
        hipLaunchKernelGGL((k_qmm<TYPE, T, ROUNDS, R, NT, PK, LXC>), dim3((unsigned) grid, (unsigned) q.parts),
                           dim3(QM_WAVES * 64), 0, q.s, (const uint8_t*) q.wq, q.nblk, q.M, (int64_t) q.nb1_w, q.y,
                           (int64_t) (q.nb1_y / sizeof(float)), q.N, q.rows, q.part_chunks, q.ws, q.x,
                           (int64_t) (q.nb1_x / sizeof(float)));
        return check_launch("qmm");
    }
}

// 16-byte LDS pieces of one row's chunk: the row and one spare.
template <int TYPE>
constexpr int qm_ls16() {
    return QM_CP * QmFmt<TYPE>::PW * 4 / 16 + 1;
}
// One chunk buffer (QmTile's BUF) for T tiles and ROUNDS pieces per thread, and
// the ring depth R: chunks copied ahead of the one being computed.
template <int TYPE>
constexpr int qm_buf(int t, int rounds) {
    const int fill = rounds * QM_WAVES * 64 * 16, pad = 16 * t * qm_ls16<TYPE>() * 16;
    return fill > pad ? fill : pad;
}
// Measured on configuration 2 (every format, one or two column tiles): two
// chunks ahead beats three or four by 5-15 %; more loads in flight slow the
// weight stream more than they hide its latency. With 6 or more row tiles a
// step's arithmetic is long enough that one chunk ahead is best. The ring of
// R + 1 buffers always fits: qm_max_rows keeps 4 of them within the LDS.
template <int TYPE, int NT>
constexpr int qm_ring(int t, int rounds) {
    return t >= 6 ? 1 : 2;
}
constexpr int qm_rounds(int rows, int ls16) {
    return (rows * ls16 + QM_WAVES * 64 - 1) / (QM_WAVES * 64);
}
// The most rows per workgroup (a multiple of 8) whose ring of 4 buffers fits;
// the buffer grows with the rows, so every smaller count fits too. At most 112
// rows with one column tile, 64 with two (their x operands and sums double the
// registers a row tile needs).
template <int TYPE, int NT>
constexpr int qm_max_rows() {
    int r = NT == 1 ? 112 : 64;
    while (4 * qm_buf<TYPE>((r + 15) / 16, qm_rounds(r, qm_ls16<TYPE>())) > QM_LDS) r -= 8;
    return r;
}

// ROUNDS = 16-byte LDS pieces of a chunk per thread, rounded up. Rows come in
// multiples of 8, so T tiles hold 16T - 8 or 16T rows and ROUNDS takes one of
// two values.
template <int TYPE, int T>
constexpr int qm_rounds_used(int rows) {
    return qm_rounds(rows, qm_ls16<TYPE>()) <= qm_rounds(16 * T - 8, qm_ls16<TYPE>()) ? qm_rounds(16 * T - 8, qm_ls16<TYPE>())
                                                                                   : qm_rounds(16 * T, qm_ls16<TYPE>());
}
template <int TYPE, int T, int NT, bool PK, int LXC>
int launch_rounds(const QmCall& q) {
    constexpr int LS16 = qm_ls16<TYPE>();
    constexpr int LO = qm_rounds(16 * T - 8, LS16), HI = qm_rounds(16 * T, LS16);
    if (qm_rounds(q.rows, LS16) <= LO) return launch_t<TYPE, T, LO, qm_ring<TYPE, NT>(T, LO), NT, PK, LXC>(q);
    if constexpr (16 * T <= qm_max_rows<TYPE, NT>()) {  // 16T rows is within the cap
        return launch_t<TYPE, T, HI, qm_ring<TYPE, NT>(T, HI), NT, PK, LXC>(q);
    } else {
        return fail(TRC_HIP_E_INVALID, "qmm: %d rows per workgroup exceed the LDS plan", q.rows);
    }
}

template <int TYPE, int T, int NT, bool PK, int LXC>
int launch_tiles(int t, const QmCall& q) {
    if constexpr (T > (qm_max_rows<TYPE, NT>() + 15) / 16) {
        return fail(TRC_HIP_E_INVALID, "qmm: %d rows per workgroup exceed the LDS plan", q.rows);
    } else {
        if (t == T) return launch_rounds<TYPE, T, NT, PK, LXC>(q);
        return launch_tiles<TYPE, T + 1, NT, PK, LXC>(t, q);
    }
}

// Work split. Rows per workgroup: one workgroup per CU when M allows, in
// multiples of 8, at most qm_max_rows. Up to 24 rows per CU, K is split in two
// parts, which doubles the rows per workgroup and halves the chunks each one
// walks (and the x operands each one reads).
struct QmPlan {
    int rows, parts, part_chunks;
};
template <int TYPE, int NT>
QmPlan qm_plan(int nblk, int64_t M) {
    const int nch = (nblk / 2 + QM_CP - 1) / QM_CP;
    const int64_t cus = device_cus();
    QmPlan p;
    // measured at K = 4096, N = 8 and 16: the split is faster from M = 2048
    // (-15 %) to 6144 (-1 %), slower from 8192
    p.parts = nch >= 2 && (M + cus - 1) / cus <= 24 ? 2 : 1;
    p.part_chunks = (nch + p.parts - 1) / p.parts;
    p.parts = (nch + p.part_chunks - 1) / p.part_chunks;
    int64_t rows = (M * p.parts + cus - 1) / cus;
    rows = (rows + 7) / 8 * 8;
    if (rows > qm_max_rows<TYPE, NT>()) rows = qm_max_rows<TYPE, NT>();
    p.rows = (int) rows;
    return p;
}

// x converted inside k_qmm (packed calls with K in one part): at most QM_LXC
// chunks, i.e. 64 KB of A entries per workgroup beside the chunk ring. With a
// K split the parts would need y cleared by a launch of its own, which measured
// slower than the pre-pass (configuration 0 10.8 -> 11.5 us).
constexpr int QM_LXC = 4;

// Whether the plan's kernel fits the LDS with the part's x beside its ring
// (QmLdsX with LXC = QM_LXC, at the ROUNDS and ring depth launch_rounds picks).
template <int TYPE, int T>
bool qm_lx_fits_t(int rows) {
    constexpr bool MIN = TYPE == TRC_HIP_TYPE_Q4_1 || TYPE == TRC_HIP_TYPE_Q5_1;
    const int ro = qm_rounds_used<TYPE, T>(rows);
    const int ring = (qm_ring<TYPE, 1>(T, ro) + 1) * qm_buf<TYPE>(T, ro);
    const int red = QM_WAVES * T * 64 * 16;
    const int bytes = (ring > red ? ring : red) + QM_LXC * QM_CHB * 1024 + QM_LXC * 16 * 4 +
                      (MIN ? QM_LXC * QM_CHB * 16 * 4 : 0);
    return bytes <= QM_LDS;
}
template <int TYPE>
bool qm_lx_fits(const QmPlan& p) {
    if (p.parts != 1 || p.part_chunks > QM_LXC) return false;
    switch ((p.rows + 15) / 16) {
        case 1: return qm_lx_fits_t<TYPE, 1>(p.rows);
        case 2: return qm_lx_fits_t<TYPE, 2>(p.rows);
        case 3: return qm_lx_fits_t<TYPE, 3>(p.rows);
        case 4: return qm_lx_fits_t<TYPE, 4>(p.rows);
        case 5: return qm_lx_fits_t<TYPE, 5>(p.rows);
        case 6: return qm_lx_fits_t<TYPE, 6>(p.rows);
        case 7: return qm_lx_fits_t<TYPE, 7>(p.rows);
        default: return false;
    }
}

// NT = 1 for N <= 16, 2 for 17 <= N <= 32: every column tile shares one pass over W.
// PK (N <= 8): x hi and lo packed into one tile; with K in one part whose x fits
// beside the ring, each workgroup converts x itself and no pre-pass runs.
template <int TYPE, int NT, bool PK>
int launch_fmt(const void* wq, int nblk, int64_t M, size_t nb1_w, const float* x, size_t nb1_x, int N, float* y,
               size_t nb1_y, QmScratch where, hipStream_t s) {
    const QmPlan p = qm_plan<TYPE, NT>(nblk, M);
    const int tiles = (p.rows + 15) / 16;
    if constexpr (PK) {
        if (qm_lx_fits<TYPE>(p)) {  // x converted in the kernel: no workspace
            const QmCall q{wq, nblk, M, nb1_w, y, nb1_y, N, p.rows, p.parts, p.part_chunks, nullptr, x, nb1_x, s};
            return launch_tiles<TYPE, 1, NT, PK, QM_LXC>(tiles, q);
        }
    }
    uint8_t* ws = nullptr;
    const int wrc = where == QmScratch::STATIC ? qm_static_scratch(&ws) : qm_stream_workspace(s, &ws);
    if (wrc != TRC_HIP_OK) return wrc;
    const QmCall q{wq, nblk, M, nb1_w, y, nb1_y, N, p.rows, p.parts, p.part_chunks, ws, x, nb1_x, s};
    const int nchunks = (nblk + QM_CHB - 1) / QM_CHB;
    const int ncol = PK ? 8 : 16 * NT;  // one pre-pass wave per chunk and column
    hipLaunchKernelGGL(k_qmm_xprep, dim3((unsigned) (nchunks * ncol)), dim3(64), 0, s, x,
                       (int64_t) (nb1_x / sizeof(float)), N, nblk, rotated_even<TYPE>() ? 2 : 0, ncol, PK ? 1 : 0,
                       p.parts > 1 ? y : nullptr, (int64_t) (nb1_y / sizeof(float)), M, ws);
    const int rc = check_launch("qmm_xprep");
    if (rc != TRC_HIP_OK) return rc;
    return launch_tiles<TYPE, 1, NT, PK, 0>(tiles, q);
}

template <int TYPE>
int launch_cols(const void* wq, int nblk, int64_t M, size_t nb1_w, const float* x, size_t nb1_x, int N, float* y,
                size_t nb1_y, QmScratch where, hipStream_t s) {
    if (N > 16) return launch_fmt<TYPE, 2, false>(wq, nblk, M, nb1_w, x, nb1_x, N, y, nb1_y, where, s);
    if (N > 8) return launch_fmt<TYPE, 1, false>(wq, nblk, M, nb1_w, x, nb1_x, N, y, nb1_y, where, s);
    return launch_fmt<TYPE, 1, true>(wq, nblk, M, nb1_w, x, nb1_x, N, y, nb1_y, where, s);
}

}  // namespace

bool qmm_supported(int64_t K, int64_t N, const void* wq, size_t nb1_w) {
    const int64_t nblk = K / QK;
    // K chunks are copied in 16-byte pieces (a multiple of 4 pairs per row keeps them
    // aligned); a workgroup's rows (at most 112) are addressed through one buffer
    // resource (< 2^31 bytes)
    return N >= 2 && N <= 16 * QM_NT && nblk >= 8 && nblk % 8 == 0 && nblk <= QM_MAX_BLOCKS &&
           (((uintptr_t) wq) & 15u) == 0 && (nb1_w & 15u) == 0 && nb1_w <= ((size_t) 1 << 24);
}

int launch_qmm(int type, const void* wq, int64_t K, int64_t M, size_t nb1_w, const float* x, int64_t N,
               size_t nb1_x, float* y, size_t nb1_y, hipStream_t s, QmScratch where) {
    const int nblk = (int) (K / QK);
    if (nblk > QM_MAX_BLOCKS) {
        return fail(TRC_HIP_E_SHAPE, "qmm: K = %lld exceeds the %d the x workspace holds", (long long) K,
                    QM_MAX_BLOCKS * QK);
    }
    switch (type) {
        case TRC_HIP_TYPE_Q4_0: return launch_cols<TRC_HIP_TYPE_Q4_0>(wq, nblk, M, nb1_w, x, nb1_x, (int) N, y, nb1_y, where, s);
        case TRC_HIP_TYPE_Q4_1: return launch_cols<TRC_HIP_TYPE_Q4_1>(wq, nblk, M, nb1_w, x, nb1_x, (int) N, y, nb1_y, where, s);
        case TRC_HIP_TYPE_Q5_0: return launch_cols<TRC_HIP_TYPE_Q5_0>(wq, nblk, M, nb1_w, x, nb1_x, (int) N, y, nb1_y, where, s);
        case TRC_HIP_TYPE_Q5_1: return launch_cols<TRC_HIP_TYPE_Q5_1>(wq, nblk, M, nb1_w, x, nb1_x, (int) N, y, nb1_y, where, s);
        case TRC_HIP_TYPE_Q8_0: return launch_cols<TRC_HIP_TYPE_Q8_0>(wq, nblk, M, nb1_w, x, nb1_x, (int) N, y, nb1_y, where, s);
        default: return fail(TRC_HIP_E_INVALID, "qmm: bad type %d", type);
    }
}

}  // namespace trc_hip

// ---------------------------------------------------------------- x workspaces
//
// trc_hip_qmatvec: one workspace per (device, stream), allocated by the first
// call on that stream whose shape runs the x pre-pass, and kept for later calls
// on the stream. Work on one stream runs in order, so calls on different
// streams never share x planes. hipStreamPerThread names a different stream in
// every host thread, so its workspaces are also keyed by thread. At most
// QM_STREAM_WS workspaces are kept per device: a new stream past that waits for
// the device to go idle and takes over the least recently used one.
// trc_hip_qmatvec_release_stream frees a stream's workspace after its work.
// Past its QM_WS_BYTES the workspace holds the ticket words of the K-split
// mul_mat (MM_TICKETS words, cleared by a fill kernel on the stream when the
// workspace is made; every launch that takes a ticket leaves it zero again, so
// a workspace handed to another stream after the device went idle is clear).
//
// trc_hip_qmatvec_noalloc: the file-scope device array `scratch` below. Each GPU
// holds its own copy at its own address, found once per device with
// hipGetSymbolAddress; host code uses only that address, never the array's
// name. Every call of that entry on one GPU shares the array, so such calls
// that overlap on one GPU (other streams, concurrent graph replays) race.
namespace trc_hip {
namespace {
constexpr size_t QM_WS_BYTES = (size_t) QM_A_BYTES + (size_t) QM_META_BYTES;
}  // namespace
}  // namespace trc_hip

static __device__ __attribute__((aligned(256))) uint8_t scratch[trc_hip::QM_WS_BYTES];

#include <mutex>
#include <thread>
#include <vector>

namespace trc_hip {
namespace {

constexpr int QM_MAX_DEV = 64;
constexpr int QM_STREAM_WS = 8;  // per-stream workspaces kept per device
std::mutex g_ws_mutex;
uint8_t* g_scratch_dev[QM_MAX_DEV] = {};  // address of `scratch` on each device, once resolved

struct StreamWs {
    int dev;
    hipStream_t stream;
    std::thread::id thread;  // only for hipStreamPerThread
    uint8_t* ptr;
    uint64_t last_use;
};
std::vector<StreamWs>& stream_workspaces() {
    static std::vector<StreamWs> v;
    return v;
}
uint64_t g_ws_clock = 0;

int current_device(int* dev) {
    const hipError_t e = hipGetDevice(dev);
    if (e != hipSuccess) return hip_error(e, "hipGetDevice");
    if (*dev < 0 || *dev >= QM_MAX_DEV) return fail(TRC_HIP_E_NO_DEVICE, "device %d out of range", *dev);
    return TRC_HIP_OK;
}

std::thread::id stream_thread(hipStream_t s) {
    return s == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
}

}  // namespace

size_t qm_workspace_bytes() {
    return QM_WS_BYTES;
}

int qm_scratch_setup() {
    int dev = 0;
    const int rc = current_device(&dev);
    if (rc != TRC_HIP_OK) return rc;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if (g_scratch_dev[dev] != nullptr) return TRC_HIP_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(TRC_HIP_E_INVALID, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_dev[dev] = (uint8_t*) p;
    return TRC_HIP_OK;
}

int qm_static_scratch(uint8_t** ws) {
    int rc = qm_scratch_setup();
    if (rc != TRC_HIP_OK) return rc;
    int dev = 0;
    rc = current_device(&dev);
    if (rc != TRC_HIP_OK) return rc;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    *ws = g_scratch_dev[dev];
    return TRC_HIP_OK;
}

int qm_stream_workspace(hipStream_t s, uint8_t** ws) {
    int dev = 0;
    const int rc = current_device(&dev);
    if (rc != TRC_HIP_OK) return rc;
    const std::thread::id tid = stream_thread(s);
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    std::vector<StreamWs>& v = stream_workspaces();
    int on_dev = 0;
    StreamWs* lru = nullptr;
    for (StreamWs& w : v) {
        if (w.dev != dev) continue;
        if (w.stream == s && w.thread == tid) {
            w.last_use = ++g_ws_clock;
            *ws = w.ptr;
            return TRC_HIP_OK;
        }
        ++on_dev;
        if (lru == nullptr || w.last_use < lru->last_use) lru = &w;
    }
    if (on_dev >= QM_STREAM_WS) {
        // the least recently used stream's last call may still be running: wait
        // for the device, then hand its workspace to this stream
        const hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) return hip_error(e, "qmatvec: waiting for the device to reuse an x workspace");
        lru->stream = s;
        lru->thread = tid;
        lru->last_use = ++g_ws_clock;
        *ws = lru->ptr;
        return TRC_HIP_OK;
    }
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, QM_WS_BYTES + MM_TICKETS * sizeof(uint32_t));
    if (e != hipSuccess) return hip_error(e, "qmatvec: x workspace for a new stream (hipMalloc)");
    const int frc = launch_fill_f32((float*) ((uint8_t*) p + QM_WS_BYTES), 0.f, MM_TICKETS, s);
    if (frc != TRC_HIP_OK) {
        (void) hipFree(p);
        return frc;
    }
    v.push_back({dev, s, tid, (uint8_t*) p, ++g_ws_clock});
    *ws = (uint8_t*) p;
    return TRC_HIP_OK;
}

int mm_stream_tickets(hipStream_t s, uint32_t** tickets) {
    uint8_t* ws = nullptr;
    const int rc = qm_stream_workspace(s, &ws);
    if (rc != TRC_HIP_OK) return rc;
    *tickets = (uint32_t*) (ws + QM_WS_BYTES);
    return TRC_HIP_OK;
}

int qm_release_stream(hipStream_t s) {
    int dev = 0;
    int rc = current_device(&dev);
    if (rc != TRC_HIP_OK) return rc;
    const std::thread::id tid = stream_thread(s);
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    std::vector<StreamWs>& v = stream_workspaces();
    for (size_t i = 0; i < v.size(); ++i) {
        if (v[i].dev != dev || v[i].stream != s || v[i].thread != tid) continue;
        // the stream's last calls may still read the workspace
        rc = hip_error(hipStreamSynchronize(s), "qmatvec_release_stream: hipStreamSynchronize");
        if (rc != TRC_HIP_OK) return rc;
        rc = hip_error(hipFree(v[i].ptr), "qmatvec_release_stream: hipFree");
        v.erase(v.begin() + (long) i);
        return rc;
    }
    return TRC_HIP_OK;
}

}  // namespace trc_hip
