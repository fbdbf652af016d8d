/*
 * CPU oracle for the GGUF legacy-quant dequant / fused matvec / F32 mul_mat path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: it restates the
 * reference CPU algorithms so that the HIP kernels can be compared against them.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it. The product (libtrc_hip.so, libtraincpp_hip.so) never links or calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the reference checkout of Chui-Las/train.cpp v0.4.0).
 *
 * Pinning (how each function is checked before it is trusted):
 *   orc_fp16_to_fp32   - all 65,536 bit patterns vs the reference's own
 *                        fp16_to_fp32 compiled from src/core/trc_float.h
 *                        (oracle/_ref) and vs numpy float16 on finite values.
 *   orc_fp32_to_fp16   - vs numpy float32->float16 (IEEE RNE) on 2^20+ values and
 *                        vs the reference fp32_to_fp16 (oracle/_ref).
 *   orc_dequant        - the hand-computed KATs of tests/test_gguf.cpp:355-444,
 *                        an exhaustive (q, d, m) sweep against a double-precision
 *                        closed form, one-hot qh masks for the Q5 bit mapping, and
 *                        the reference's gguf_tensor_to_f32 on random blocks
 *                        (oracle/_ref).
 *   orc_mul_mat        - the KATs of tests/test_ops.cpp:185-275, the PyTorch
 *                        goldens tests/golden/mul_mat*.npy and
 *                        grad_mul_mat*.npy (backward compositions), a double-
 *                        precision brute force with an fp32 error bound, and the
 *                        reference's compute_mul_mat through its CPU Device on
 *                        permuted views (oracle/_ref), compared bit for bit.
 *   orc_add            - tests/test_ops.cpp:52-95 (same shape, broadcast), the
 *                        PyTorch goldens tests/golden/add_same_* / add_bcast_*,
 *                        numpy's float32 a + b with broadcasting, and the
 *                        reference's compute_binary on strided views (oracle/_ref).
 *   orc_acc            - tests/test_ops.cpp:1152-1220 (strided region, inplace 3D),
 *                        a numpy slice-add on the same region, and the reference's
 *                        compute_acc (oracle/_ref), bit for bit.
 *   orc_repeat_back    - tests/test_ops.cpp:1128-1150, numpy's reshape-and-sum
 *                        (float64 bound), and the reference's compute_repeat_back
 *                        (oracle/_ref), bit for bit.
 *   orc_mul            - the product step of tests/test_ops.cpp:98-118, the PyTorch
 *                        golden tests/golden/mul_same_*, numpy's float32 a * b with
 *                        broadcasting, and the reference's compute_binary
 *                        (oracle/_ref), bit for bit.
 *   orc_sum            - the PyTorch golden tests/golden/sum_*, order-revealing
 *                        cases whose double sums differ by summation order (within
 *                        a row, across rows and planes) or by accumulating in float,
 *                        math.fsum within one float rounding on random data, and
 *                        the reference's compute_sum (oracle/_ref), bit for bit.
 *   orc_repeat         - tests/test_ops.cpp:795-815, the PyTorch golden
 *                        tests/golden/repeat_*, numpy's tile, and the reference's
 *                        compute_repeat (oracle/_ref), bit for bit.
 *   orc_sqr, orc_scale - numpy's float32 x * x and x * s (finite, signed zeros,
 *                        subnormals, inf and NaN inputs) and the reference's
 *                        compute_unary / compute_scale (oracle/_ref) on strided
 *                        views, bit for bit.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (src/core/trc_types.cpp:22-48). */
enum {
    ORC_TYPE_F32  = 0,
    ORC_TYPE_Q4_0 = 2,
    ORC_TYPE_Q4_1 = 3,
    ORC_TYPE_Q5_0 = 6,
    ORC_TYPE_Q5_1 = 7,
    ORC_TYPE_Q8_0 = 8,
};

float    orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16(float f);
void     orc_fp16_to_fp32_n(const uint16_t* h, float* out, int64_t n);
void     orc_fp32_to_fp16_n(const float* f, uint16_t* out, int64_t n);

/* Block size in bytes for a legacy quant type, 0 if not one of the five. */
int64_t orc_block_bytes(int type);

/* Dequantize n_blocks contiguous blocks of `type` into 32*n_blocks floats.
 * threads <= 1 runs the serial loop; more threads split the block range, which
 * leaves every output value unchanged. Returns 0, or -1 for an unknown type. */
int orc_dequant(int type, const void* blocks, int64_t n_blocks, float* out, int threads);

/* ggml mul_mat on byte-strided F32 operands:
 *   d[i,j,i2,i3] = sum_k a[k,i,i2%a2,i3%a3] * b[k,j,i2,i3]
 * ne/nb are ggml order (ne0 innermost, nb in bytes). threads > 1 splits the
 * outputs (rows i of every (i3,i2,j) column) into ranges; each output keeps the
 * serial k order, so the bits do not depend on the thread count. Returns 0, or
 * -1 when the shapes are not a valid mul_mat. */
int orc_mul_mat(const void* a, const int64_t a_ne[4], const size_t a_nb[4],
                const void* b, const int64_t b_ne[4], const size_t b_nb[4],
                void* d, const int64_t d_ne[4], const size_t d_nb[4], int threads);

/* Same as orc_mul_mat restricted to output columns [j_begin, j_end) of every
 * plane: used to time a bounded slice of a large product. */
int orc_mul_mat_cols(const void* a, const int64_t a_ne[4], const size_t a_nb[4],
                     const void* b, const int64_t b_ne[4], const size_t b_nb[4],
                     void* d, const int64_t d_ne[4], const size_t d_nb[4],
                     int64_t j_begin, int64_t j_end, int threads);

/* ggml add, dst = a + b with b broadcast over dst's shape (dst has a's shape;
 * every b dim equals dst's or is 1). Element order and the single rounding of
 * a + b follow compute_binary (src/backends/cpu/trc_cpu_ops.cpp:52-78, with
 * offset_broadcast :18-28); shape rule src/ops/trc_ops.cpp:19-32. Returns 0, or
 * -1 on shapes add does not accept. */
int orc_add(const void* a, const int64_t a_ne[4], const size_t a_nb[4],
            const void* b, const int64_t b_ne[4], const size_t b_nb[4],
            void* d, const int64_t d_ne[4], const size_t d_nb[4]);
/* ggml acc: d = a (skipped when inplace, then d must alias a) and, for every
 * element i of b in linear order, d[offset + i0*4 + i1*nb1 + i2*nb2 + i3*nb3] +=
 * b[i] (src/core/trc_tensor.cpp:322-361, compute_acc
 * src/backends/cpu/trc_cpu_ops.cpp:954-999). a and d contiguous F32 of one
 * shape. Returns 0, or -1 when the region leaves a. */
int orc_acc(const void* a, const int64_t a_ne[4], const void* b, const int64_t b_ne[4], const size_t b_nb[4],
            void* d, size_t nb1, size_t nb2, size_t nb3, size_t offset, int inplace);
/* ggml repeat_back: d (contiguous, d_ne dividing a_ne) = sums of a over its
 * repeats, each output accumulated from 0 in a's linear element order
 * (src/ops/trc_ops.cpp:458-470, compute_repeat_back
 * src/backends/cpu/trc_cpu_ops.cpp:932-952). Returns 0, or -1 on bad shapes. */
int orc_repeat_back(const void* a, const int64_t a_ne[4], const size_t a_nb[4], void* d, const int64_t d_ne[4]);

/* mul: d = a * b with a's shape, b broadcast (src/ops/trc_ops.cpp:59-61,
 * compute_binary src/backends/cpu/trc_cpu_ops.cpp:52-78). */
int orc_mul(const void* a, const int64_t a_ne[4], const size_t a_nb[4],
            const void* b, const int64_t b_ne[4], const size_t b_nb[4],
            void* d, const int64_t d_ne[4], const size_t d_nb[4]);

/* sum of all elements of a strided F32 tensor (src/ops/trc_ops.cpp:214-221,
 * compute_sum src/backends/cpu/trc_cpu_ops.cpp:302-315). */
int orc_sum(const void* a, const int64_t a_ne[4], const size_t a_nb[4], float* out);

/* repeat of a to d's shape (src/ops/trc_ops.cpp:447-456, compute_repeat
 * src/backends/cpu/trc_cpu_ops.cpp:913-928). */
int orc_repeat(const void* a, const int64_t a_ne[4], const size_t a_nb[4], void* d, const int64_t d_ne[4],
               const size_t d_nb[4]);

/* sqr: d = a * a; scale: d = a * s. d has a's shape (own strides d_nb)
 * (src/ops/trc_ops.cpp:75-77, 107-115; compute_unary / compute_scale
 * src/backends/cpu/trc_cpu_ops.cpp:86, 119-150). */
int orc_sqr(const void* a, const int64_t a_ne[4], const size_t a_nb[4], void* d, const size_t d_nb[4]);
int orc_scale(const void* a, const int64_t a_ne[4], const size_t a_nb[4], void* d, const size_t d_nb[4], float s);

/* splitmix64 stream (src/core/trc_rng.cpp:38-68). */
uint64_t orc_rng_next_u64(uint64_t* state);
float    orc_rng_uniform01(uint64_t* state);
float    orc_rng_normal(uint64_t* state, float mean, float stddev);

#ifdef __cplusplus
}
#endif
