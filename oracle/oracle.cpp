// CPU oracle: restatement of the reference CPU path for GGUF legacy-quant
// dequantization and ggml F32 mul_mat. TEST INFRASTRUCTURE ONLY (the checker);
// see oracle.h for who may load it and how each function is pinned.
//
// Build flags follow the reference build: -O3 -std=c++20 -ffp-contract=off and
// no -march (CMakeLists.txt:32-40), so float expressions round exactly as the
// reference's serial loops do: one rounding per * and per +, no FMA.
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline uint32_t bits_of(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

inline float float_of(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

inline uint16_t load_u16le(const uint8_t* p) {
    return (uint16_t) (p[0] | (p[1] << 8));
}

inline uint32_t load_u32le(const uint8_t* p) {
    return (uint32_t) p[0] | ((uint32_t) p[1] << 8) | ((uint32_t) p[2] << 16) |
           ((uint32_t) p[3] << 24);
}

// Run fn(begin, end) over [0, n) split into `threads` contiguous ranges.
template <typename Fn>
void parallel_ranges(int64_t n, int threads, Fn fn) {
    if (threads <= 1 || n < 2) {
        fn((int64_t) 0, n);
        return;
    }
    const int64_t parts = std::min<int64_t>(threads, n);
    std::vector<std::thread> pool;
    pool.reserve((size_t) parts);
    for (int64_t p = 0; p < parts; ++p) {
        const int64_t b = n * p / parts;
        const int64_t e = n * (p + 1) / parts;
        pool.emplace_back([=] { fn(b, e); });
    }
    for (auto& t : pool) {
        t.join();
    }
}

// ---------------------------------------------------------------- dequant
// Block layouts and element formulas: src/io/trc_gguf.cpp:320-417.
//   Q4_0 {f16 d; u8 qs[16]}            y = (float)(nib - 8) * d
//   Q4_1 {f16 d; f16 m; u8 qs[16]}     y = (float)nib * d + m
//   Q5_0 {f16 d; u32 qh; u8 qs[16]}    y = (float)((nib | bit5) - 16) * d
//   Q5_1 {f16 d; f16 m; u32 qh; qs}    y = (float)(nib | bit5) * d + m
//   Q8_0 {f16 d; i8 qs[32]}            y = (float)q * d
// Element e < 16 takes the low nibble of qs[e], element e >= 16 the high nibble
// of qs[e-16]; the 5th bit of element e is bit e of qh (:370-371, :394-395).

struct Layout {
    int bytes;    // block size in bytes
    int min_off;  // byte offset of the f16 min, or -1
    int qh_off;   // byte offset of the u32 high-bit mask, or -1
    int qs_off;   // byte offset of the quant bytes
    int bias;     // subtracted from the integer quant
    bool q8;      // 32 signed bytes instead of 16 nibble pairs
};

Layout layout_of(int type) {
    switch (type) {
        case ORC_TYPE_Q4_0: return {18, -1, -1, 2, 8, false};
        case ORC_TYPE_Q4_1: return {20, 2, -1, 4, 0, false};
        case ORC_TYPE_Q5_0: return {22, -1, 2, 6, 16, false};
        case ORC_TYPE_Q5_1: return {24, 2, 4, 8, 0, false};
        case ORC_TYPE_Q8_0: return {34, -1, -1, 2, 0, true};
        default: return {0, -1, -1, 0, 0, false};
    }
}

// The 32 integer quants of one block, in output order.
void block_ints(const Layout& L, const uint8_t* blk, int q[32]) {
    const uint8_t* qs = blk + L.qs_off;
    if (L.q8) {
        for (int e = 0; e < 32; ++e) {
            q[e] = (int) (int8_t) qs[e];
        }
        return;
    }
    const uint32_t qh = L.qh_off >= 0 ? load_u32le(blk + L.qh_off) : 0u;
    for (int e = 0; e < 32; ++e) {
        const int nib = e < 16 ? (qs[e] & 0x0F) : (qs[e - 16] >> 4);
        const int hi  = (int) ((qh >> e) & 1u) << 4;
        q[e] = (nib | hi) - L.bias;
    }
}

void dequant_range(const Layout& L, const uint8_t* src, int64_t b0, int64_t b1, float* out) {
    int q[32];
    for (int64_t b = b0; b < b1; ++b) {
        const uint8_t* blk = src + b * L.bytes;
        const float d = orc_fp16_to_fp32(load_u16le(blk));
        block_ints(L, blk, q);
        float* y = out + b * 32;
        if (L.min_off >= 0) {
            const float m = orc_fp16_to_fp32(load_u16le(blk + L.min_off));
            for (int e = 0; e < 32; ++e) {
                const float p = (float) q[e] * d;  // rounded product ...
                y[e] = p + m;                      // ... then rounded sum (no FMA)
            }
        } else {
            for (int e = 0; e < 32; ++e) {
                y[e] = (float) q[e] * d;
            }
        }
    }
}

// ---------------------------------------------------------------- mul_mat
// src/backends/cpu/trc_cpu_ops.cpp:182-216: loop order i3, i2, j, i, k with a
// float accumulator that starts at 0 and adds each rounded product in k order;
// byte-strided loads (:30-42); src0 plane (i2 % a2, i3 % a3) (src/ops/trc_ops.cpp:366-385).

inline float ld(const void* base, size_t off) {
    float v;
    std::memcpy(&v, (const uint8_t*) base + off, 4);
    return v;
}

bool mm_shapes_ok(const int64_t a_ne[4], const int64_t b_ne[4], const int64_t d_ne[4]) {
    for (int i = 0; i < 4; ++i) {
        if (a_ne[i] <= 0 || b_ne[i] <= 0 || d_ne[i] <= 0) return false;
    }
    return a_ne[0] == b_ne[0] && b_ne[2] % a_ne[2] == 0 && b_ne[3] % a_ne[3] == 0 &&
           d_ne[0] == a_ne[1] && d_ne[1] == b_ne[1] && d_ne[2] == b_ne[2] && d_ne[3] == b_ne[3];
}

void mm_outputs(const void* a, const int64_t a_ne[4], const size_t a_nb[4],
                const void* b, const int64_t b_ne[4], const size_t b_nb[4],
                void* d, const size_t d_nb[4], int64_t j_begin, int64_t j_end,
                int64_t o0, int64_t o1) {
    // o enumerates the outputs (i3, i2, jj, i) with i fastest, then jj in
    // [0, j_end - j_begin). Each output is one sequential k-sum, so any split of
    // the range over threads gives the same bits.
    const int64_t K = a_ne[0], M = a_ne[1];
    const int64_t nj = j_end - j_begin;
    for (int64_t o = o0; o < o1; ++o) {
        const int64_t i = o % M, c = o / M;
        const int64_t jj = c % nj;
        const int64_t i2 = (c / nj) % b_ne[2];
        const int64_t i3 = c / (nj * b_ne[2]);
        const int64_t j  = j_begin + jj;
        const size_t oa = (size_t) (i2 % a_ne[2]) * a_nb[2] + (size_t) (i3 % a_ne[3]) * a_nb[3];
        const size_t ob = (size_t) i2 * b_nb[2] + (size_t) i3 * b_nb[3] + (size_t) j * b_nb[1];
        const size_t od = (size_t) i2 * d_nb[2] + (size_t) i3 * d_nb[3] + (size_t) j * d_nb[1];
        const size_t oai = oa + (size_t) i * a_nb[1];
        float acc = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            const float p = ld(a, oai + (size_t) k * a_nb[0]) * ld(b, ob + (size_t) k * b_nb[0]);
            acc = acc + p;
        }
        std::memcpy((uint8_t*) d + od + (size_t) i * d_nb[0], &acc, 4);
    }
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------- fp16
// src/core/trc_float.h:23-40 decodes IEEE binary16 exactly (normals, subnormals,
// signed zeros, Inf). Its NaN path multiplies a signalling pattern by 2^-112,
// which on x86 SSE quiets it; the field decode below reproduces that.
float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t exp  = (h >> 10) & 0x1Fu;
    const uint32_t man  = h & 0x3FFu;
    if (exp == 0x1Fu) {
        return float_of(sign | 0x7F800000u | (man << 13) | (man != 0 ? 0x00400000u : 0u));
    }
    if (exp != 0) {
        return float_of(sign | ((exp + 112u) << 23) | (man << 13));
    }
    // zero or subnormal: man * 2^-24 is exact in binary32
    return float_of(sign | bits_of((float) man * 0x1p-24f));
}

// Round-to-nearest-even binary32 -> binary16 (src/core/trc_float.h:42-63 on
// finite inputs). NaN maps to the canonical quiet NaN 0x7E00.
uint16_t orc_fp32_to_fp16(float f) {
    const uint32_t x    = bits_of(f);
    const uint16_t sign = (uint16_t) ((x >> 16) & 0x8000u);
    const uint32_t ax   = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t) (sign | 0x7E00u);
    if (ax >= 0x477FF000u) return (uint16_t) (sign | 0x7C00u);  // rounds to >= 65520 -> Inf
    if (ax < 0x33000001u) return sign;                          // <= 2^-25 rounds to 0
    const int32_t e = (int32_t) (ax >> 23) - 127;
    uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;  // 24-bit significand
    int shift;
    uint32_t base;
    if (e < -14) {  // subnormal half: value / 2^-24 = mant * 2^(e-23+24)
        shift = -e - 1;  // bits to drop from the 24-bit significand: 23 - (e + 24)
        base  = 0;
    } else {
        shift = 13;
        base  = (uint32_t) (e + 15) << 10;
        mant &= 0x7FFFFFu;
    }
    const uint32_t keep = mant >> shift;
    const uint32_t rem  = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    uint32_t r = base + keep;  // carry from the mantissa rolls into the exponent
    if (rem > half || (rem == half && (keep & 1u))) ++r;
    return (uint16_t) (sign | r);
}

void orc_fp16_to_fp32_n(const uint16_t* h, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_fp16_to_fp32(h[i]);
}

void orc_fp32_to_fp16_n(const float* f, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_fp32_to_fp16(f[i]);
}

int64_t orc_block_bytes(int type) {
    return layout_of(type).bytes;
}

// gguf_tensor_to_f32's quant branch (src/io/trc_gguf.cpp:1040-1044): n/32
// contiguous blocks from the tensor's data offset.
int orc_dequant(int type, const void* blocks, int64_t n_blocks, float* out, int threads) {
    const Layout L = layout_of(type);
    if (L.bytes == 0 || n_blocks < 0) return -1;
    const uint8_t* src = (const uint8_t*) blocks;
    parallel_ranges(n_blocks, threads,
                    [&](int64_t b0, int64_t b1) { dequant_range(L, src, b0, b1, out); });
    return 0;
}

int orc_mul_mat_cols(const void* a, const int64_t a_ne[4], const size_t a_nb[4],
                     const void* b, const int64_t b_ne[4], const size_t b_nb[4],
                     void* d, const int64_t d_ne[4], const size_t d_nb[4],
                     int64_t j_begin, int64_t j_end, int threads) {
    if (!mm_shapes_ok(a_ne, b_ne, d_ne)) return -1;
    if (j_begin < 0 || j_end > b_ne[1] || j_begin >= j_end) return -1;
    const int64_t nout = (j_end - j_begin) * b_ne[2] * b_ne[3] * a_ne[1];
    parallel_ranges(nout, threads, [&](int64_t o0, int64_t o1) {
        mm_outputs(a, a_ne, a_nb, b, b_ne, b_nb, d, d_nb, j_begin, j_end, o0, o1);
    });
    return 0;
}

int orc_mul_mat(const void* a, const int64_t a_ne[4], const size_t a_nb[4],
                const void* b, const int64_t b_ne[4], const size_t b_nb[4],
                void* d, const int64_t d_ne[4], const size_t d_nb[4], int threads) {
    if (!mm_shapes_ok(a_ne, b_ne, d_ne)) return -1;
    return orc_mul_mat_cols(a, a_ne, a_nb, b, b_ne, b_nb, d, d_ne, d_nb, 0, b_ne[1], threads);
}

// ---------------------------------------------------------------- element-wise ops
// Shared helpers: byte offset of linear element i of a strided tensor
// (tensor_offset_linear, src/core/trc_tensor.cpp:94-102) and of the broadcast
// source element for dst element i (offset_broadcast,
// src/backends/cpu/trc_cpu_ops.cpp:18-28).
static size_t lin_offset(const int64_t ne[4], const size_t nb[4], int64_t i) {
    size_t off = 0;
    for (int d = 0; d < 4; ++d) {
        off += (size_t) (i % ne[d]) * nb[d];
        i /= ne[d];
    }
    return off;
}

static size_t bcast_offset(const int64_t t_ne[4], const size_t t_nb[4], const int64_t shape_ne[4], int64_t i) {
    size_t off = 0;
    for (int d = 0; d < 4; ++d) {
        const int64_t idx = i % shape_ne[d];
        i /= shape_ne[d];
        if (t_ne[d] != 1) off += (size_t) idx * t_nb[d];
    }
    return off;
}

static int64_t nelem(const int64_t ne[4]) { return ne[0] * ne[1] * ne[2] * ne[3]; }

// compute_binary's general path (src/backends/cpu/trc_cpu_ops.cpp:52-78): a and
// dst walked in linear order, b through the broadcast offset; one float
// operation per element (fn_add / fn_mul, :47-49).
}  // extern "C"

template <typename Fn>
static int binary_f32(const void* a, const int64_t a_ne[4], const size_t a_nb[4], const void* b,
                      const int64_t b_ne[4], const size_t b_nb[4], void* d, const int64_t d_ne[4],
                      const size_t d_nb[4], Fn fn) {
    for (int k = 0; k < 4; ++k) {
        if (d_ne[k] != a_ne[k] || (b_ne[k] != a_ne[k] && b_ne[k] != 1)) return -1;
    }
    const uint8_t* pa = (const uint8_t*) a;
    const uint8_t* pb = (const uint8_t*) b;
    uint8_t* pd = (uint8_t*) d;
    const int64_t n = nelem(d_ne);
    for (int64_t i = 0; i < n; ++i) {
        const float va = *(const float*) (pa + lin_offset(a_ne, a_nb, i));
        const float vb = *(const float*) (pb + bcast_offset(b_ne, b_nb, d_ne, i));
        *(float*) (pd + lin_offset(d_ne, d_nb, i)) = fn(va, vb);
    }
    return 0;
}

extern "C" {

int orc_add(const void* a, const int64_t a_ne[4], const size_t a_nb[4],
            const void* b, const int64_t b_ne[4], const size_t b_nb[4],
            void* d, const int64_t d_ne[4], const size_t d_nb[4]) {
    return binary_f32(a, a_ne, a_nb, b, b_ne, b_nb, d, d_ne, d_nb, [](float x, float y) { return x + y; });
}

int orc_mul(const void* a, const int64_t a_ne[4], const size_t a_nb[4],
            const void* b, const int64_t b_ne[4], const size_t b_nb[4],
            void* d, const int64_t d_ne[4], const size_t d_nb[4]) {
    return binary_f32(a, a_ne, a_nb, b, b_ne, b_nb, d, d_ne, d_nb, [](float x, float y) { return x * y; });
}

// compute_unary with fn_sqr (src/backends/cpu/trc_cpu_ops.cpp:86, 119-135) and
// compute_scale (:140-150): dst element i (linear order) from a's element i,
// one float multiply each.
static int unary_f32(const void* a, const int64_t a_ne[4], const size_t a_nb[4], void* d, const size_t d_nb[4],
                     int sqr, float s) {
    const uint8_t* pa = (const uint8_t*) a;
    uint8_t* pd = (uint8_t*) d;
    const int64_t n = nelem(a_ne);
    for (int64_t i = 0; i < n; ++i) {
        const float v = *(const float*) (pa + lin_offset(a_ne, a_nb, i));
        *(float*) (pd + lin_offset(a_ne, d_nb, i)) = sqr ? v * v : v * s;
    }
    return 0;
}

int orc_sqr(const void* a, const int64_t a_ne[4], const size_t a_nb[4], void* d, const size_t d_nb[4]) {
    return unary_f32(a, a_ne, a_nb, d, d_nb, 1, 0.f);
}

int orc_scale(const void* a, const int64_t a_ne[4], const size_t a_nb[4], void* d, const size_t d_nb[4], float s) {
    return unary_f32(a, a_ne, a_nb, d, d_nb, 0, s);
}

// compute_sum (src/backends/cpu/trc_cpu_ops.cpp:302-315): rows in the order i3,
// i2, i1; each row summed in double from 0 along i0 (row_sum_f32 :284-300); the
// row sums added in double; one rounding to float.
int orc_sum(const void* a, const int64_t a_ne[4], const size_t a_nb[4], float* out) {
    const uint8_t* pa = (const uint8_t*) a;
    double sum = 0.0;
    for (int64_t i3 = 0; i3 < a_ne[3]; ++i3) {
        for (int64_t i2 = 0; i2 < a_ne[2]; ++i2) {
            for (int64_t i1 = 0; i1 < a_ne[1]; ++i1) {
                const uint8_t* row = pa + (size_t) i1 * a_nb[1] + (size_t) i2 * a_nb[2] + (size_t) i3 * a_nb[3];
                double rs = 0.0;
                for (int64_t i0 = 0; i0 < a_ne[0]; ++i0) rs += *(const float*) (row + (size_t) i0 * a_nb[0]);
                sum += rs;
            }
        }
    }
    *out = (float) sum;
    return 0;
}

// compute_repeat (src/backends/cpu/trc_cpu_ops.cpp:913-928): dst element i (linear
// order over d_ne) takes a's element at index (i_k % a_ne[k]), extent-1 dims at 0.
int orc_repeat(const void* a, const int64_t a_ne[4], const size_t a_nb[4], void* d, const int64_t d_ne[4],
               const size_t d_nb[4]) {
    for (int k = 0; k < 4; ++k) {
        if (a_ne[k] <= 0 || d_ne[k] % a_ne[k] != 0) return -1;
    }
    const uint8_t* pa = (const uint8_t*) a;
    uint8_t* pd = (uint8_t*) d;
    const int64_t n = nelem(d_ne);
    for (int64_t i = 0; i < n; ++i) {
        int64_t rem = i;
        size_t oa = 0;
        for (int k = 0; k < 4; ++k) {
            const int64_t idx = rem % d_ne[k];
            rem /= d_ne[k];
            oa += (size_t) (a_ne[k] == 1 ? 0 : idx % a_ne[k]) * a_nb[k];
        }
        *(float*) (pd + lin_offset(d_ne, d_nb, i)) = *(const float*) (pa + oa);
    }
    return 0;
}

int orc_acc(const void* a, const int64_t a_ne[4], const void* b, const int64_t b_ne[4], const size_t b_nb[4],
            void* d, size_t nb1, size_t nb2, size_t nb3, size_t offset, int inplace) {
    const size_t nbytes = (size_t) nelem(a_ne) * sizeof(float);
    // region bound check of the acc constructor (src/core/trc_tensor.cpp:331-337)
    size_t last = (size_t) (b_ne[0] - 1) * sizeof(float);
    last += b_ne[1] > 1 ? (size_t) (b_ne[1] - 1) * nb1 : 0;
    last += b_ne[2] > 1 ? (size_t) (b_ne[2] - 1) * nb2 : 0;
    last += b_ne[3] > 1 ? (size_t) (b_ne[3] - 1) * nb3 : 0;
    if (offset + last + sizeof(float) > nbytes) return -1;
    if (!inplace) std::memcpy(d, a, nbytes);
    const uint8_t* pb = (const uint8_t*) b;
    uint8_t* pd = (uint8_t*) d;
    const int64_t n = nelem(b_ne);
    for (int64_t i = 0; i < n; ++i) {
        int64_t rem = i, idx[4];
        for (int k = 0; k < 4; ++k) {
            idx[k] = rem % b_ne[k];
            rem /= b_ne[k];
        }
        const size_t od = offset + (size_t) idx[0] * sizeof(float) + (size_t) idx[1] * nb1 + (size_t) idx[2] * nb2 +
                          (size_t) idx[3] * nb3;
        float* t = (float*) (pd + od);
        *t = *t + *(const float*) (pb + lin_offset(b_ne, b_nb, i));
    }
    return 0;
}

int orc_repeat_back(const void* a, const int64_t a_ne[4], const size_t a_nb[4], void* d, const int64_t d_ne[4]) {
    for (int k = 0; k < 4; ++k) {
        if (d_ne[k] <= 0 || a_ne[k] % d_ne[k] != 0) return -1;
    }
    const size_t d_nb[4] = {sizeof(float), sizeof(float) * (size_t) d_ne[0],
                            sizeof(float) * (size_t) (d_ne[0] * d_ne[1]),
                            sizeof(float) * (size_t) (d_ne[0] * d_ne[1] * d_ne[2])};
    std::memset(d, 0, (size_t) nelem(d_ne) * sizeof(float));
    const uint8_t* pa = (const uint8_t*) a;
    uint8_t* pd = (uint8_t*) d;
    const int64_t n = nelem(a_ne);
    for (int64_t i = 0; i < n; ++i) {
        int64_t rem = i;
        size_t od = 0;
        for (int k = 0; k < 4; ++k) {
            const int64_t idx = rem % a_ne[k];
            rem /= a_ne[k];
            od += (size_t) (idx % d_ne[k]) * d_nb[k];
        }
        float* t = (float*) (pd + od);
        *t = *t + *(const float*) (pa + lin_offset(a_ne, a_nb, i));
    }
    return 0;
}

// ---------------------------------------------------------------- rng
// splitmix64 and its float draws: src/core/trc_rng.cpp:38-68.
uint64_t orc_rng_next_u64(uint64_t* state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

float orc_rng_uniform01(uint64_t* state) {
    const uint32_t top24 = (uint32_t) (orc_rng_next_u64(state) >> 40);
    return (float) top24 * 0x1p-24f;
}

float orc_rng_normal(uint64_t* state, float mean, float stddev) {
    float u1 = orc_rng_uniform01(state);
    const float u2 = orc_rng_uniform01(state);
    u1 = std::max(u1, 1e-7f);
    const float radius = std::sqrt(-2.0f * std::log(u1));
    return mean + stddev * radius * std::cos(6.28318530717958647692f * u2);
}

}  // extern "C"
