/*
 * trc_hip_abi.h - C ABI of the MI355X (gfx950) HIP backend for traincpp.
 *
 * This is the drop-in boundary. libtrc_hip.so exports exactly these symbols:
 * plain C types, device pointers, byte sizes and an opaque stream handle. It
 * exposes no HIP, torch or C++ types. The C++ Device/BufferType/Buffer
 * implementation (libtraincpp_hip.so, built from
 * train.cpp_amd/csrc/backend/hip_device.cpp) sits on top of these calls, just
 * as the reference's CPU and Vulkan backends sit under the same plugin
 * interface. Each entry point names the reference interface it serves
 * (paths are relative to the reference checkout of Chui-Las/train.cpp v0.4.0).
 *
 * Conventions
 *  - Return value: 0 on success. A positive value is the hipError_t the HIP
 *    runtime reported. A negative value is one of the TRC_HIP_E_* codes below.
 *    On failure trc_hip_last_error() describes the problem; the text is
 *    per-thread and stays valid until the next failing call on that thread.
 *  - Streams are hipStream_t passed as void*; NULL means the null stream. Kernel
 *    entry points only enqueue work, so call trc_hip_sync() before reading results
 *    on the host. Buffer::set_tensor/get_tensor are synchronous in the reference,
 *    and trc_hip_h2d/trc_hip_d2h are synchronous too.
 *  - Tensor layout follows ggml: ne[0] is innermost; nb[] are strides in bytes
 *    (include/traincpp/trc_tensor.h:1-10). `data` is the device address of element
 *    [0,0,0,0], i.e. buffer base + Tensor::data_offset (trc_tensor.h:58).
 *  - Setting the environment variable TRC_HIP_FORCE_ERROR=<entry name> makes
 *    that entry point fail with TRC_HIP_E_FORCED before it touches the device,
 *    so error paths can be tested without a GPU fault.
 *  - Not thread-safe for concurrent calls on one stream, like the reference
 *    (README.md:109).
 */
#ifndef TRC_HIP_ABI_H
#define TRC_HIP_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRC_HIP_ABI_VERSION 1

enum trc_hip_status {
    TRC_HIP_OK          = 0,
    TRC_HIP_E_INVALID   = -1, /* null pointer, negative count, unknown type   */
    TRC_HIP_E_SHAPE     = -2, /* shapes are not a valid (supported) operation */
    TRC_HIP_E_ALIGN     = -3, /* pointer or stride alignment a kernel needs   */
    TRC_HIP_E_NO_DEVICE = -4, /* no HIP device, or ordinal out of range       */
    TRC_HIP_E_FORCED    = -5  /* injected through TRC_HIP_FORCE_ERROR         */
};

/* ggml type ids used by this ABI (include/traincpp/trc_types.h:11-49). */
enum trc_hip_type {
    TRC_HIP_TYPE_F32  = 0,
    TRC_HIP_TYPE_Q4_0 = 2,
    TRC_HIP_TYPE_Q4_1 = 3,
    TRC_HIP_TYPE_Q5_0 = 6,
    TRC_HIP_TYPE_Q5_1 = 7,
    TRC_HIP_TYPE_Q8_0 = 8
};

/* Largest activation batch (columns of src1) the fused quantized matvec takes
 * (skinny GEMM up to 64 columns; W is read once per 32 columns). */
#define TRC_HIP_QMATVEC_MAX_N 64

/* Fields of DeviceProps (include/traincpp/trc_backend.h:14-28) plus what the
 * kernels' launch heuristics need. */
typedef struct trc_hip_props {
    char    name[256];       /* marketing name, e.g. "AMD Instinct MI355X"   */
    char    arch[64];        /* gcnArchName, e.g. "gfx950:sramecc+:xnack-"   */
    int32_t ordinal;
    int32_t compute_units;
    size_t  memory_free;
    size_t  memory_total;
    int32_t unified_memory;  /* 1 for APUs; 0 on MI355X                      */
    int32_t abi_version;     /* TRC_HIP_ABI_VERSION of the loaded library     */
} trc_hip_props;

/* A ggml tensor view on the device: the fields of traincpp::Tensor that the
 * kernels read (include/traincpp/trc_tensor.h:37-70). */
typedef struct trc_hip_tensor {
    void*   data;   /* device address of element [0,0,0,0]         */
    int32_t type;   /* trc_hip_type                                 */
    int32_t flags;  /* reserved, must be 0                          */
    int64_t ne[4];  /* elements per dimension, ne[0] innermost      */
    size_t  nb[4];  /* byte strides                                 */
} trc_hip_tensor;

/* ------------------------------------------------------------------ device */

/* Number of visible HIP devices; device_count()/device_get()
 * (include/traincpp/trc_backend.h:95-101) enumerate one Device per ordinal. */
int trc_hip_device_count(int* count);

/* Selects `ordinal` as the calling thread's current device and fills *props
 * (props may be NULL). Serves Device::props() (trc_backend.h:72). */
int trc_hip_init(int ordinal, trc_hip_props* props);

/* Blocks until all work queued on `stream` has finished. Device::graph_compute
 * is synchronous (trc_backend.h:77-78), so the C++ Device ends each graph here. */
int trc_hip_sync(void* stream);

/* Description of the last failure on the calling thread ("" if none). */
const char* trc_hip_last_error(void);

/* ------------------------------------------------------------------ memory */

/* Device allocation for BufferType::alloc_buffer (trc_backend.h:38-45).
 * *ptr is 256-byte aligned. bytes == 0 yields *ptr == NULL. */
int trc_hip_malloc(void** ptr, size_t bytes);

/* Releases memory from trc_hip_malloc (Buffer destructor, trc_backend.h:49). */
int trc_hip_free(void* ptr);

/* Host -> device copy for Buffer::set_tensor (trc_backend.h:56-57).
 * Synchronous with respect to the host buffer: it may be reused on return. */
int trc_hip_h2d(void* dst, const void* src, size_t bytes, void* stream);

/* Device -> host copy for Buffer::get_tensor (trc_backend.h:58). Synchronous. */
int trc_hip_d2h(void* dst, const void* src, size_t bytes, void* stream);

/* Fills `bytes` bytes with `value` for Buffer::clear (trc_backend.h:59). */
int trc_hip_memset(void* dst, int value, size_t bytes, void* stream);

/* Fills count floats with `value` for Device::fill_tensors
 * (trc_backend.h:66-85). Uses a kernel, not hipMemset, so it is safe to capture. */
int trc_hip_fill_f32(float* dst, float value, int64_t count, void* stream);

/* ------------------------------------------------------------------ compute */

/* Bulk dequantization of n_blocks contiguous GGUF legacy-quant blocks of
 * `type` (Q4_0, Q4_1, Q5_0, Q5_1 or Q8_0) into 32*n_blocks floats.
 * Bit-identical to gguf_tensor_to_f32's quant branch
 * (src/io/trc_gguf.cpp:966-1049 -> dequantize_q* :320-417).
 * `blocks` must be 2-byte aligned (4-byte for Q4_1/Q5_1); `dst` 16-byte aligned. */
int trc_hip_dequant(int type, const void* blocks, int64_t n_blocks, float* dst, void* stream);

/* ggml F32 mul_mat on the MFMA cores: dst[i,j,i2,i3] =
 *   sum_k a[k,i,i2%a.ne2,i3%a.ne3] * b[k,j,i2,i3]
 * for any byte strides (views, transposes, permutes) and the ne2/ne3 modulo
 * broadcast of src0. Serves OP_MUL_MAT (src/ops/trc_ops.cpp:366-385) as
 * computed by compute_mul_mat (src/backends/cpu/trc_cpu_ops.cpp:182-216).
 * All three tensors are TRC_HIP_TYPE_F32 with 4-byte aligned data and strides.
 * The sum is reordered, so results match the CPU to rounding, not bit for bit;
 * they are the same from run to run. dst must not overlap a or b: for some
 * shapes (K >= 1024, between half and two 128 x 128 output tiles per CU, a
 * contiguous dst) the two halves of the sum over k meet in dst, one stored and
 * the other added, ordered through 32 KiB of ticket words kept past the end of
 * the stream's workspace of trc_hip_qmatvec. The first such call on a stream
 * allocates that workspace (make it before capturing the stream into a graph
 * in global capture mode); the rules for that workspace below hold here too:
 * calls on different streams may overlap, a captured graph keeps the words of
 * the stream it was captured on, and trc_hip_qmatvec_release_stream frees them. */
int trc_hip_mul_mat_f32(const trc_hip_tensor* a, const trc_hip_tensor* b,
                        const trc_hip_tensor* dst, void* stream);

/* dst += mul_mat(a, b): each element of the product is summed as
 * trc_hip_mul_mat_f32 sums it (K is never split in parts here), then added to
 * dst with one float add, the add OP_ACC makes (compute_acc,
 * src/backends/cpu/trc_cpu_ops.cpp:954-999). No single reference op: it serves
 * the fusion, in the plugin's graph_compute, of the chain autograd builds for a
 * matrix gradient, mul_mat -> transpose -> cont -> inplace acc into the
 * parameter's accumulator (src/core/trc_autograd.cpp:487-503 and
 * grad_accumulate_inplace :58-77), computed as
 * cont(transpose(mul_mat(x, y))) = mul_mat(y, x) added into the accumulator.
 * Same argument rules as trc_hip_mul_mat_f32; one dst plane (ne0 x ne1) may span
 * at most 2 GiB (TRC_HIP_E_SHAPE beyond). */
int trc_hip_mul_mat_acc_f32(const trc_hip_tensor* a, const trc_hip_tensor* b,
                            const trc_hip_tensor* dst, void* stream);

/* Fused quantized matvec / skinny GEMM: y = mul_mat(W, x) with W quantized.
 *   W : `type` blocks, ne = [K, M]; row m starts at wq + m*nb1_w bytes
 *       (2-byte aligned rows; 4-byte for Q4_1/Q5_1)
 *   x : F32, ne = [K, N]; column n starts at x + n*nb1_x bytes (x[k] contiguous;
 *       x and nb1_x 16-byte aligned)
 *   y : F32, ne = [M, N]; column n starts at y + n*nb1_y bytes (y[m] contiguous;
 *       4-byte aligned)
 * with K % 32 == 0 and 1 <= N <= TRC_HIP_QMATVEC_MAX_N. The address span y covers
 * (from its first to its last element) must not intersect the spans of W and x,
 * even where no byte is shared, as with interleaved columns (TRC_HIP_E_SHAPE
 * otherwise). The blocks are decoded in registers
 * and never written out as F32. There is no counterpart in the reference: its
 * CPU path rejects quantized mul_mat (src/ops/trc_ops.cpp:368) and the
 * equivalent result is gguf_tensor_to_f32 followed by F32 mul_mat.
 * Streams: calls on different streams may overlap. Shapes that run the x
 * pre-pass (most of 2 <= N <= 32 and the 32-column slices of wider N) convert x
 * into a device workspace of about 8.3 MiB that belongs to the (device, stream)
 * pair: the first such call on a stream allocates it (hipMalloc; make that call
 * before capturing the stream into a graph in global capture mode). Each device
 * keeps at most 8 such workspaces; the first call on a ninth stream waits for
 * the device to go idle (hipDeviceSynchronize) and takes over the least recently
 * used one. Call trc_hip_qmatvec_release_stream before destroying a stream to
 * free its workspace. A captured graph keeps using the workspace of the stream
 * it was captured on, so do not replay it concurrently with other work on that
 * stream's workspace, and do not release that stream while the graph is live. */
int trc_hip_qmatvec(int type, const void* wq, int64_t K, int64_t M, size_t nb1_w,
                    const float* x, int64_t N, size_t nb1_x,
                    float* y, size_t nb1_y, void* stream);

/* Frees the x workspace trc_hip_qmatvec keeps for `stream` on the current
 * device, after waiting for the stream's queued work (hipStreamSynchronize).
 * Call it before hipStreamDestroy; a later call on the stream allocates a new
 * workspace. trc_hip_sum_f32 keeps its row sums in the same workspace, and
 * trc_hip_mul_mat_f32 its ticket words past its end.
 * hipStreamPerThread is keyed by the calling thread. Returns TRC_HIP_OK when
 * the stream has no workspace. No counterpart in the reference:
 * it bounds the memory of trc_hip_qmatvec's per-stream workspaces, like the
 * ownership rule of Buffer (include/traincpp/trc_backend.h:33-88). */
int trc_hip_qmatvec_release_stream(void* stream);

/* trc_hip_qmatvec without any allocation, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). No counterpart in the reference. Same arguments,
 * results (bit for bit) and errors as trc_hip_qmatvec. Where trc_hip_qmatvec
 * converts x into its per-stream workspace, this entry uses instead one fixed
 * device array of about 8.3 MiB (the x planes of 32 columns of up to 65536
 * elements, the most any call converts), which each GPU holds from library
 * load until the process ends. Every call of this entry on one GPU shares that
 * array, so calls that overlap on one GPU (on different streams, or in graphs
 * replayed concurrently) race; serialise them. Nothing in it needs clearing
 * between calls. */
int trc_hip_qmatvec_noalloc(int type, const void* wq, int64_t K, int64_t M, size_t nb1_w,
                            const float* x, int64_t N, size_t nb1_x,
                            float* y, size_t nb1_y, void* stream);

/* Strided copy between two tensors of the same type and shape, in ggml linear
 * element order (OP_DUP/OP_CPY/OP_CONT: src/ops/trc_ops.cpp:124-134, computed by
 * compute_dup src/backends/cpu/trc_cpu_ops.cpp:219-236). Element size 1, 2, 4 or 8 B. */
int trc_hip_cpy(const trc_hip_tensor* src, const trc_hip_tensor* dst, void* stream);

/* ggml add, dst = a + b: dst has a's shape, b broadcasts (each b->ne[d] equals
 * a->ne[d] or is 1); any 4-byte aligned strides. OP_ADD (src/ops/trc_ops.cpp:46,
 * shape rule :19-32) as computed by compute_binary
 * (src/backends/cpu/trc_cpu_ops.cpp:52-78): one rounding per element, so the
 * result is bit-identical to the CPU's. F32 only. */
int trc_hip_add_f32(const trc_hip_tensor* a, const trc_hip_tensor* b, const trc_hip_tensor* dst, void* stream);

/* ggml mul, dst = a * b, with the broadcast and layouts of trc_hip_add_f32.
 * OP_MUL (src/ops/trc_ops.cpp:59-61) as computed by compute_binary with fn_mul
 * (src/backends/cpu/trc_cpu_ops.cpp:49, 52-78): one rounding per element, so the
 * result is bit-identical to the CPU's. F32 only. */
int trc_hip_mul_f32(const trc_hip_tensor* a, const trc_hip_tensor* b, const trc_hip_tensor* dst, void* stream);

/* ggml repeat: dst[i0..i3] = a[i0 % a.ne0, .., i3 % a.ne3] for any strides; every
 * dst->ne[d] a multiple of a->ne[d]. OP_REPEAT (src/ops/trc_ops.cpp:447-456) as
 * computed by compute_repeat (src/backends/cpu/trc_cpu_ops.cpp:913-928): an F32
 * copy, bit-identical. */
int trc_hip_repeat_f32(const trc_hip_tensor* a, const trc_hip_tensor* dst, void* stream);

/* ggml sqr: dst = a * a element by element, dst with a's shape, any strides.
 * OP_SQR (src/ops/trc_ops.cpp:75-77) as computed by compute_unary with fn_sqr
 * (src/backends/cpu/trc_cpu_ops.cpp:86, 119-135): one float multiply per element,
 * bit-identical. The square of a loss term, as in the reference's gradient tests
 * of mul_mat (tests/test_grad.cpp:343-373). F32 only. */
int trc_hip_sqr_f32(const trc_hip_tensor* a, const trc_hip_tensor* dst, void* stream);

/* ggml scale: dst = a * s element by element, dst with a's shape, any strides.
 * OP_SCALE (src/ops/trc_ops.cpp:107-115, s in op_params) as computed by
 * compute_scale (src/backends/cpu/trc_cpu_ops.cpp:140-150): one float multiply,
 * bit-identical. Autograd builds it for sqr's gradient, 2 * (x * grad)
 * (src/core/trc_autograd.cpp:288-292). F32 only. */
int trc_hip_scale_f32(const trc_hip_tensor* a, const trc_hip_tensor* dst, float s, void* stream);

/* ggml sum: the one element of dst = the sum of every element of a (any strides).
 * OP_SUM (src/ops/trc_ops.cpp:214-221) as computed by compute_sum
 * (src/backends/cpu/trc_cpu_ops.cpp:302-315, row_sum_f32 :284-300): each row
 * (ne0-run) is summed in double from 0 in element order, the row sums are added
 * in double in row order, and the total is rounded to float once; the same
 * operations in the same order, so the result is bit-identical. Rows are summed
 * in parallel (each row's own sum stays sequential) into the stream's x
 * workspace of trc_hip_qmatvec, which the first such call on a stream allocates
 * (make it before capturing that stream in global mode); more rows than that
 * workspace holds (about a million) are summed by one workgroup. */
int trc_hip_sum_f32(const trc_hip_tensor* a, const trc_hip_tensor* dst, void* stream);

/* ggml acc: dst = a, then dst[offset + i0*4 + i1*nb1 + i2*nb2 + i3*nb3] += b[i]
 * for every element of b. OP_ACC (src/core/trc_tensor.cpp:322-361, computed by
 * compute_acc src/backends/cpu/trc_cpu_ops.cpp:954-999). a and dst contiguous
 * F32 of one shape; with inplace != 0 the copy is skipped (dst is a's storage,
 * as in the reference's inplace view). The region must lie inside a and must
 * not overlap itself (TRC_HIP_E_SHAPE otherwise). Bit-identical to the CPU. */
int trc_hip_acc_f32(const trc_hip_tensor* a, const trc_hip_tensor* b, const trc_hip_tensor* dst, size_t nb1,
                    size_t nb2, size_t nb3, size_t offset, int inplace, void* stream);

/* ggml repeat_back: dst (contiguous, every dst->ne[d] dividing a->ne[d]) = the
 * sums of a over its repeats. OP_REPEAT_BACK (src/ops/trc_ops.cpp:458-470) as
 * computed by compute_repeat_back (src/backends/cpu/trc_cpu_ops.cpp:932-952):
 * each output is summed from 0 in a's linear element order, so the result is
 * bit-identical to the CPU's. F32 only. */
int trc_hip_repeat_back_f32(const trc_hip_tensor* a, const trc_hip_tensor* dst, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRC_HIP_ABI_H */
