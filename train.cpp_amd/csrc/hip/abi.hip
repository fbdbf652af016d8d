// extern "C" entry points of libtrc_hip.so (declared in include/trc_hip_abi.h):
// argument validation, error reporting and the HIP runtime calls. Kernels live
// in dequant.hip, qmatvec.hip, qmm.hip, mul_mat.hip, elementwise.hip and copy.hip.
#include "common.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace trc_hip {

namespace {
thread_local char g_last_error[512] = "";

// TRC_HIP_FORCE_ERROR=<entry> makes that entry point fail before any device work.
bool forced(const char* entry) {
    const char* v = std::getenv("TRC_HIP_FORCE_ERROR");
    return v != nullptr && std::strcmp(v, entry) == 0;
}

bool is_quant(int type) {
    return block_bytes(type) != 0;
}

size_t basic_type_size(int type) {
    switch (type) {
        case 0: return 4;   // F32
        case 1: return 2;   // F16
        case 24: return 1;  // I8
        case 25: return 2;  // I16
        case 26: return 4;  // I32
        case 27: return 8;  // I64
        case 28: return 8;  // F64
        case 30: return 2;  // BF16
        default: return 0;
    }
}
}  // namespace

int hip_error(hipError_t e, const char* what) {
    if (e == hipSuccess) return TRC_HIP_OK;
    std::snprintf(g_last_error, sizeof(g_last_error), "%s: %s (hipError_t %d)", what,
                  hipGetErrorString(e), (int) e);
    // The runtime also keeps the failure as its "last error"; clear it so that
    // the launch check of a later kernel does not report this stale error.
    (void) hipGetLastError();
    return (int) e;
}

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    return hip_error(hipGetLastError(), what);
}

int device_cus() {
    constexpr int MAX_DEV = 64;
    static int cached[MAX_DEV] = {};  // 0 = not queried yet; a benign race stores the same value
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
    if (dev < MAX_DEV && cached[dev] > 0) return cached[dev];
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (dev < MAX_DEV) cached[dev] = cus;
    return cus;
}

}  // namespace trc_hip

using namespace trc_hip;

#define TRC_FORCED(name)                                                               \
    do {                                                                               \
        if (forced(name)) return fail(TRC_HIP_E_FORCED, "%s: forced failure (TRC_HIP_FORCE_ERROR)", name); \
    } while (0)

extern "C" {

const char* trc_hip_last_error(void) {
    return g_last_error;
}

int trc_hip_device_count(int* count) {
    if (count == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_device_count: count is NULL");
    *count = 0;
    TRC_FORCED("trc_hip_device_count");
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice) return TRC_HIP_OK;
    if (e != hipSuccess) return hip_error(e, "hipGetDeviceCount");
    *count = n;
    return TRC_HIP_OK;
}

int trc_hip_init(int ordinal, trc_hip_props* props) {
    TRC_FORCED("trc_hip_init");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        (void) hipGetLastError();
        return fail(TRC_HIP_E_NO_DEVICE, "trc_hip_init: no HIP device is visible");
    }
    if (ordinal < 0 || ordinal >= n) {
        return fail(TRC_HIP_E_NO_DEVICE, "trc_hip_init: ordinal %d out of range (%d devices)", ordinal, n);
    }
    int st = hip_error(hipSetDevice(ordinal), "hipSetDevice");
    if (st != TRC_HIP_OK) return st;
    // the address of trc_hip_qmatvec_noalloc's fixed workspace on this device
    st = qm_scratch_setup();
    if (st != TRC_HIP_OK) return st;
    if (props == nullptr) return TRC_HIP_OK;
    hipDeviceProp_t p;
    st = hip_error(hipGetDeviceProperties(&p, ordinal), "hipGetDeviceProperties");
    if (st != TRC_HIP_OK) return st;
    std::memset(props, 0, sizeof(*props));
    std::snprintf(props->name, sizeof(props->name), "%s", p.name[0] ? p.name : "AMD GPU");
    std::snprintf(props->arch, sizeof(props->arch), "%s", p.gcnArchName);
    props->ordinal = ordinal;
    props->compute_units = p.multiProcessorCount;
    size_t free_b = 0, total_b = 0;
    st = hip_error(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo");
    if (st != TRC_HIP_OK) return st;
    props->memory_free = free_b;
    props->memory_total = total_b;
    props->unified_memory = p.integrated ? 1 : 0;
    props->abi_version = TRC_HIP_ABI_VERSION;
    return TRC_HIP_OK;
}

int trc_hip_sync(void* stream) {
    TRC_FORCED("trc_hip_sync");
    return hip_error(hipStreamSynchronize((hipStream_t) stream), "hipStreamSynchronize");
}

int trc_hip_malloc(void** ptr, size_t bytes) {
    if (ptr == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_malloc: ptr is NULL");
    *ptr = nullptr;
    TRC_FORCED("trc_hip_malloc");
    if (bytes == 0) return TRC_HIP_OK;
    return hip_error(hipMalloc(ptr, bytes), "hipMalloc");
}

int trc_hip_free(void* ptr) {
    TRC_FORCED("trc_hip_free");
    if (ptr == nullptr) return TRC_HIP_OK;
    return hip_error(hipFree(ptr), "hipFree");
}

int trc_hip_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    TRC_FORCED("trc_hip_h2d");
    if (bytes == 0) return TRC_HIP_OK;
    if (dst == nullptr || src == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_h2d: NULL pointer");
    int st = hip_error(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t) stream),
                       "hipMemcpyAsync(H2D)");
    if (st != TRC_HIP_OK) return st;
    return hip_error(hipStreamSynchronize((hipStream_t) stream), "hipStreamSynchronize(H2D)");
}

int trc_hip_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    TRC_FORCED("trc_hip_d2h");
    if (bytes == 0) return TRC_HIP_OK;
    if (dst == nullptr || src == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_d2h: NULL pointer");
    int st = hip_error(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t) stream),
                       "hipMemcpyAsync(D2H)");
    if (st != TRC_HIP_OK) return st;
    return hip_error(hipStreamSynchronize((hipStream_t) stream), "hipStreamSynchronize(D2H)");
}

int trc_hip_memset(void* dst, int value, size_t bytes, void* stream) {
    TRC_FORCED("trc_hip_memset");
    if (bytes == 0) return TRC_HIP_OK;
    if (dst == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_memset: NULL pointer");
    return hip_error(hipMemsetAsync(dst, value, bytes, (hipStream_t) stream), "hipMemsetAsync");
}

int trc_hip_fill_f32(float* dst, float value, int64_t count, void* stream) {
    TRC_FORCED("trc_hip_fill_f32");
    if (count < 0) return fail(TRC_HIP_E_INVALID, "trc_hip_fill_f32: negative count");
    if (count == 0) return TRC_HIP_OK;
    if (dst == nullptr || ((uintptr_t) dst & 3u) != 0) {
        return fail(TRC_HIP_E_INVALID, "trc_hip_fill_f32: dst must be a non-NULL 4-byte aligned pointer");
    }
    return launch_fill_f32(dst, value, count, (hipStream_t) stream);
}

int trc_hip_dequant(int type, const void* blocks, int64_t n_blocks, float* dst, void* stream) {
    TRC_FORCED("trc_hip_dequant");
    if (!is_quant(type)) return fail(TRC_HIP_E_INVALID, "trc_hip_dequant: type %d is not Q4_0/Q4_1/Q5_0/Q5_1/Q8_0", type);
    if (n_blocks < 0) return fail(TRC_HIP_E_INVALID, "trc_hip_dequant: negative block count");
    if (n_blocks > 0 && (blocks == nullptr || dst == nullptr)) {
        return fail(TRC_HIP_E_INVALID, "trc_hip_dequant: NULL pointer");
    }
    return launch_dequant(type, blocks, n_blocks, dst, (hipStream_t) stream);
}

}  // extern "C"

namespace {

// The argument rules of both mul_mat entries; `who` names the entry in messages.
int check_mul_mat_args(const char* who, const trc_hip_tensor* a, const trc_hip_tensor* b, const trc_hip_tensor* dst) {
    if (a == nullptr || b == nullptr || dst == nullptr) {
        return fail(TRC_HIP_E_INVALID, "%s: NULL tensor", who);
    }
    const trc_hip_tensor* ts[3] = {a, b, dst};
    for (const trc_hip_tensor* t : ts) {
        if (t->type != TRC_HIP_TYPE_F32) return fail(TRC_HIP_E_INVALID, "%s: tensors must be F32", who);
        for (int i = 0; i < 4; ++i) {
            if (t->ne[i] <= 0) return fail(TRC_HIP_E_SHAPE, "%s: ne[%d] = %lld", who, i, (long long) t->ne[i]);
            if (t->nb[i] % 4 != 0) return fail(TRC_HIP_E_ALIGN, "%s: nb[%d] = %zu is not a multiple of 4", who, i, t->nb[i]);
        }
        if (t->data == nullptr || ((uintptr_t) t->data & 3u) != 0) {
            return fail(TRC_HIP_E_ALIGN, "%s: data must be non-NULL and 4-byte aligned", who);
        }
    }
    // ggml_can_mul_mat (src/ops/trc_ops.cpp:369-375) and the output shape (:380).
    if (a->ne[0] != b->ne[0] || b->ne[2] % a->ne[2] != 0 || b->ne[3] % a->ne[3] != 0 ||
        dst->ne[0] != a->ne[1] || dst->ne[1] != b->ne[1] || dst->ne[2] != b->ne[2] || dst->ne[3] != b->ne[3]) {
        return fail(TRC_HIP_E_SHAPE,
                    "%s: shapes a[%lld,%lld,%lld,%lld] b[%lld,%lld,%lld,%lld] dst[%lld,%lld,%lld,%lld] "
                    "are not a mul_mat",
                    who, (long long) a->ne[0], (long long) a->ne[1], (long long) a->ne[2], (long long) a->ne[3],
                    (long long) b->ne[0], (long long) b->ne[1], (long long) b->ne[2], (long long) b->ne[3],
                    (long long) dst->ne[0], (long long) dst->ne[1], (long long) dst->ne[2], (long long) dst->ne[3]);
    }
    // dst may be cleared before the sums are added into it (and is read and
    // written while the operands are read), so it must not share bytes with an
    // operand (compared by the byte spans the views cover)
    auto span_end = [](const trc_hip_tensor* t) {
        uintptr_t e = (uintptr_t) t->data + 4;
        for (int i = 0; i < 4; ++i) e += (uintptr_t) (t->ne[i] - 1) * t->nb[i];
        return e;
    };
    for (const trc_hip_tensor* t : {a, b}) {
        if ((uintptr_t) dst->data < span_end(t) && (uintptr_t) t->data < span_end(dst)) {
            return fail(TRC_HIP_E_SHAPE, "%s: dst overlaps an operand", who);
        }
    }
    return TRC_HIP_OK;
}

}  // namespace

extern "C" {

int trc_hip_mul_mat_f32(const trc_hip_tensor* a, const trc_hip_tensor* b, const trc_hip_tensor* dst,
                        void* stream) {
    TRC_FORCED("trc_hip_mul_mat_f32");
    const int rc = check_mul_mat_args("trc_hip_mul_mat_f32", a, b, dst);
    if (rc != TRC_HIP_OK) return rc;
    return launch_mul_mat_f32(*a, *b, *dst, (hipStream_t) stream);
}

int trc_hip_mul_mat_acc_f32(const trc_hip_tensor* a, const trc_hip_tensor* b, const trc_hip_tensor* dst,
                            void* stream) {
    TRC_FORCED("trc_hip_mul_mat_acc_f32");
    const int rc = check_mul_mat_args("trc_hip_mul_mat_acc_f32", a, b, dst);
    if (rc != TRC_HIP_OK) return rc;
    // the kernels address one dst plane through 32-bit buffer offsets
    const uint64_t plane = (uint64_t) (dst->ne[0] - 1) * dst->nb[0] + (uint64_t) (dst->ne[1] - 1) * dst->nb[1] + 4;
    if (plane >= (1ull << 31)) {
        return fail(TRC_HIP_E_SHAPE, "trc_hip_mul_mat_acc_f32: a dst plane spans %llu bytes (2 GiB at most)",
                    (unsigned long long) plane);
    }
    return launch_mul_mat_f32(*a, *b, *dst, (hipStream_t) stream, true);
}

}  // extern "C"

namespace {

// Argument checks shared by trc_hip_qmatvec and trc_hip_qmatvec_noalloc.
int qmatvec_args(const char* entry, int type, const void* wq, int64_t K, int64_t M, size_t nb1_w, const float* x,
                 int64_t N, size_t nb1_x, const float* y, size_t nb1_y) {
    if (!is_quant(type)) return fail(TRC_HIP_E_INVALID, "%s: type %d is not a legacy quant type", entry, type);
    if (K <= 0 || M <= 0 || N <= 0 || K % QK != 0) {
        return fail(TRC_HIP_E_SHAPE, "%s: need K > 0, K %% 32 == 0, M > 0, N > 0 (K=%lld M=%lld N=%lld)", entry,
                    (long long) K, (long long) M, (long long) N);
    }
    if (N > TRC_HIP_QMATVEC_MAX_N) {
        return fail(TRC_HIP_E_SHAPE, "%s: N=%lld exceeds %d", entry, (long long) N, TRC_HIP_QMATVEC_MAX_N);
    }
    if (wq == nullptr || x == nullptr || y == nullptr) return fail(TRC_HIP_E_INVALID, "%s: NULL pointer", entry);
    const size_t row_bytes = (size_t) (K / QK) * (size_t) block_bytes(type);
    if (nb1_w < row_bytes && M > 1) return fail(TRC_HIP_E_SHAPE, "%s: nb1_w %zu < row size %zu", entry, nb1_w, row_bytes);
    if ((N > 1 && (nb1_x < (size_t) K * 4 || nb1_y < (size_t) M * 4))) {
        return fail(TRC_HIP_E_SHAPE, "%s: columns of x or y overlap", entry);
    }
    // y is written (and, for some shapes, cleared first) while W and x are read,
    // so it must share no byte with either (compared by the spans they cover)
    const uintptr_t w0 = (uintptr_t) wq, w1 = w0 + (uintptr_t) (M - 1) * nb1_w + row_bytes;
    const uintptr_t x0 = (uintptr_t) x, x1 = x0 + (uintptr_t) (N - 1) * nb1_x + (uintptr_t) K * 4;
    const uintptr_t y0 = (uintptr_t) y, y1 = y0 + (uintptr_t) (N - 1) * nb1_y + (uintptr_t) M * 4;
    if ((y0 < w1 && w0 < y1) || (y0 < x1 && x0 < y1)) {
        return fail(TRC_HIP_E_SHAPE, "%s: y overlaps W or x", entry);
    }
    return TRC_HIP_OK;
}

}  // namespace

extern "C" {

int trc_hip_qmatvec(int type, const void* wq, int64_t K, int64_t M, size_t nb1_w, const float* x, int64_t N,
                    size_t nb1_x, float* y, size_t nb1_y, void* stream) {
    TRC_FORCED("trc_hip_qmatvec");
    const int rc = qmatvec_args("trc_hip_qmatvec", type, wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y);
    if (rc != TRC_HIP_OK) return rc;
    return launch_qmatvec(type, wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, (hipStream_t) stream, QmScratch::PER_STREAM);
}

int trc_hip_qmatvec_noalloc(int type, const void* wq, int64_t K, int64_t M, size_t nb1_w, const float* x, int64_t N,
                            size_t nb1_x, float* y, size_t nb1_y, void* stream) {
    TRC_FORCED("trc_hip_qmatvec_noalloc");
    const int rc = qmatvec_args("trc_hip_qmatvec_noalloc", type, wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y);
    if (rc != TRC_HIP_OK) return rc;
    return launch_qmatvec(type, wq, K, M, nb1_w, x, N, nb1_x, y, nb1_y, (hipStream_t) stream, QmScratch::STATIC);
}

int trc_hip_qmatvec_release_stream(void* stream) {
    TRC_FORCED("trc_hip_qmatvec_release_stream");
    return qm_release_stream((hipStream_t) stream);
}

int trc_hip_cpy(const trc_hip_tensor* src, const trc_hip_tensor* dst, void* stream) {
    TRC_FORCED("trc_hip_cpy");
    if (src == nullptr || dst == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_cpy: NULL tensor");
    if (src->type != dst->type) return fail(TRC_HIP_E_INVALID, "trc_hip_cpy: types differ (%d vs %d)", src->type, dst->type);
    const size_t es = basic_type_size(src->type);
    if (es == 0) return fail(TRC_HIP_E_INVALID, "trc_hip_cpy: type %d has no per-element size", src->type);
    for (int i = 0; i < 4; ++i) {
        if (src->ne[i] != dst->ne[i] || src->ne[i] <= 0) return fail(TRC_HIP_E_SHAPE, "trc_hip_cpy: shapes differ");
        if (src->nb[i] % es != 0 || dst->nb[i] % es != 0) return fail(TRC_HIP_E_ALIGN, "trc_hip_cpy: strides not element aligned");
    }
    if (src->data == nullptr || dst->data == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_cpy: NULL data");
    if (((uintptr_t) src->data % es) != 0 || ((uintptr_t) dst->data % es) != 0) {
        return fail(TRC_HIP_E_ALIGN, "trc_hip_cpy: data not element aligned");
    }
    return launch_cpy(*src, *dst, es, (hipStream_t) stream);
}

int trc_hip_add_f32(const trc_hip_tensor* a, const trc_hip_tensor* b, const trc_hip_tensor* dst, void* stream) {
    TRC_FORCED("trc_hip_add_f32");
    if (a == nullptr || b == nullptr || dst == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_add_f32: NULL tensor");
    if (a->data == nullptr || b->data == nullptr || dst->data == nullptr) {
        return fail(TRC_HIP_E_INVALID, "trc_hip_add_f32: NULL data");
    }
    return launch_add_f32(*a, *b, *dst, (hipStream_t) stream);
}

int trc_hip_mul_f32(const trc_hip_tensor* a, const trc_hip_tensor* b, const trc_hip_tensor* dst, void* stream) {
    TRC_FORCED("trc_hip_mul_f32");
    if (a == nullptr || b == nullptr || dst == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_mul_f32: NULL tensor");
    if (a->data == nullptr || b->data == nullptr || dst->data == nullptr) {
        return fail(TRC_HIP_E_INVALID, "trc_hip_mul_f32: NULL data");
    }
    return launch_mul_f32(*a, *b, *dst, (hipStream_t) stream);
}

int trc_hip_repeat_f32(const trc_hip_tensor* a, const trc_hip_tensor* dst, void* stream) {
    TRC_FORCED("trc_hip_repeat_f32");
    if (a == nullptr || dst == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_repeat_f32: NULL tensor");
    if (a->data == nullptr || dst->data == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_repeat_f32: NULL data");
    return launch_repeat_f32(*a, *dst, (hipStream_t) stream);
}

int trc_hip_sqr_f32(const trc_hip_tensor* a, const trc_hip_tensor* dst, void* stream) {
    TRC_FORCED("trc_hip_sqr_f32");
    if (a == nullptr || dst == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_sqr_f32: NULL tensor");
    if (a->data == nullptr || dst->data == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_sqr_f32: NULL data");
    return launch_sqr_f32(*a, *dst, (hipStream_t) stream);
}

int trc_hip_scale_f32(const trc_hip_tensor* a, const trc_hip_tensor* dst, float s, void* stream) {
    TRC_FORCED("trc_hip_scale_f32");
    if (a == nullptr || dst == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_scale_f32: NULL tensor");
    if (a->data == nullptr || dst->data == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_scale_f32: NULL data");
    return launch_scale_f32(*a, *dst, s, (hipStream_t) stream);
}

int trc_hip_sum_f32(const trc_hip_tensor* a, const trc_hip_tensor* dst, void* stream) {
    TRC_FORCED("trc_hip_sum_f32");
    if (a == nullptr || dst == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_sum_f32: NULL tensor");
    if (a->data == nullptr || dst->data == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_sum_f32: NULL data");
    return launch_sum_f32(*a, *dst, (hipStream_t) stream);
}

int trc_hip_acc_f32(const trc_hip_tensor* a, const trc_hip_tensor* b, const trc_hip_tensor* dst, size_t nb1,
                    size_t nb2, size_t nb3, size_t offset, int inplace, void* stream) {
    TRC_FORCED("trc_hip_acc_f32");
    if (a == nullptr || b == nullptr || dst == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_acc_f32: NULL tensor");
    if (a->data == nullptr || b->data == nullptr || dst->data == nullptr) {
        return fail(TRC_HIP_E_INVALID, "trc_hip_acc_f32: NULL data");
    }
    return launch_acc_f32(*a, *b, *dst, nb1, nb2, nb3, offset, inplace, (hipStream_t) stream);
}

int trc_hip_repeat_back_f32(const trc_hip_tensor* a, const trc_hip_tensor* dst, void* stream) {
    TRC_FORCED("trc_hip_repeat_back_f32");
    if (a == nullptr || dst == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_repeat_back_f32: NULL tensor");
    if (a->data == nullptr || dst->data == nullptr) return fail(TRC_HIP_E_INVALID, "trc_hip_repeat_back_f32: NULL data");
    return launch_repeat_back_f32(*a, *dst, (hipStream_t) stream);
}

}  // extern "C"
