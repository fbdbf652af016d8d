// Shared definitions for the gfx950 kernels of libtrc_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "trc_hip_abi.h"

namespace trc_hip {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

// GGUF legacy block sizes in bytes (include/traincpp/trc_types.h values,
// src/core/trc_types.cpp:27-31). Every block holds 32 elements.
constexpr int QK = 32;

__host__ __device__ constexpr int block_bytes(int type) {
    return type == TRC_HIP_TYPE_Q4_0   ? 18
           : type == TRC_HIP_TYPE_Q4_1 ? 20
           : type == TRC_HIP_TYPE_Q5_0 ? 22
           : type == TRC_HIP_TYPE_Q5_1 ? 24
           : type == TRC_HIP_TYPE_Q8_0 ? 34
                                       : 0;
}

// IEEE binary16 -> binary32 (v_cvt_f32_f16). Exact on every finite input,
// subnormals included, as is the reference's bit-trick decode
// (src/core/trc_float.h:23-40).
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return (float) __builtin_bit_cast(_Float16, (uint16_t) h);
}

// Two parts of a sum split in two meet in dst without a cleared dst. For each
// block of outputs, the wave holding it in each part takes a ticket from
// tk[0]. The first stores its sums with agent-scope stores (written through to
// where every XCD reads them), waits until all of them are done and raises the
// flag tk[1]. The second waits for the flag, adds its sums with float atomics
// (performed where the stores landed) and clears both words for the next
// launch. a + b is the same in either order, so results do not depend on which
// part comes first. The wait is only for a wave that already holds its ticket
// and has nothing left to wait for, so it ends; a cap on the polls (seconds,
// against the microseconds it takes) bounds it regardless.
constexpr int TICKET_FLAG_POLLS = 1 << 20;

// Whether this wave is the first of the two (lane 0 takes the ticket).
__device__ __forceinline__ bool ticket_first(uint32_t* tk, int lane) {
    uint32_t first = 0;
    if (lane == 0) first = __hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __builtin_amdgcn_readfirstlane(first) == 0;
}
// The first, after its agent-scope stores: waits for them, then raises the flag.
__device__ __forceinline__ void ticket_publish(uint32_t* tk, int lane) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0) __hip_atomic_store(tk + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The second, before its atomic adds: waits for the flag.
__device__ __forceinline__ void ticket_wait(uint32_t* tk, int lane) {
    if (lane == 0) {
        for (int n = 0; n < TICKET_FLAG_POLLS; ++n) {
            if (__hip_atomic_load(tk + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
            __builtin_amdgcn_s_sleep(1);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
// The second, after its adds: both words back to zero.
__device__ __forceinline__ void ticket_clear(uint32_t* tk, int lane) {
    if (lane == 0) {
        __hip_atomic_store(tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(tk + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Launch-side error reporting, implemented in abi.hip.
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
// hipSuccess -> TRC_HIP_OK; otherwise records "what: <HIP message>" and returns e.
int hip_error(hipError_t e, const char* what);
// Compute units of the current device (cached per device).
int device_cus();

// Kernel launchers (one per kernel family). They validate what the kernels
// assume, enqueue on `stream` and return a trc_hip_status / hipError_t.
int launch_dequant(int type, const void* blocks, int64_t n_blocks, float* dst, hipStream_t stream);
// accumulate: dst += the product (each element's float sum, then one add)
int launch_mul_mat_f32(const trc_hip_tensor& a, const trc_hip_tensor& b, const trc_hip_tensor& d,
                       hipStream_t stream, bool accumulate = false);
// Where the fp16 matrix-core path of the fused matvec keeps x's planes and
// scales (qmm.hip): a workspace per (device, stream), allocated by the first
// such call on that stream (trc_hip_qmatvec), or the fixed device array of the
// current GPU (trc_hip_qmatvec_noalloc: no allocation, shared by every such call
// on that GPU).
enum class QmScratch { PER_STREAM, STATIC };
int launch_qmatvec(int type, const void* wq, int64_t K, int64_t M, size_t nb1_w, const float* x,
                   int64_t N, size_t nb1_x, float* y, size_t nb1_y, hipStream_t stream, QmScratch where);
// Fused quant x skinny GEMM on the fp16 matrix cores for 2 <= N <= 32 (N = 2, 3
// only off the integer-dot kernel's alignment)
// (qmm.hip); qmm_supported says whether the shape and alignment fit it.
bool qmm_supported(int64_t K, int64_t N, const void* wq, size_t nb1_w);
int launch_qmm(int type, const void* wq, int64_t K, int64_t M, size_t nb1_w, const float* x, int64_t N,
               size_t nb1_x, float* y, size_t nb1_y, hipStream_t stream, QmScratch where);
// The x workspaces (qmm.hip). qm_scratch_setup finds the address of the fixed
// array on the current device (once per device; it allocates nothing).
size_t qm_workspace_bytes();
int qm_scratch_setup();
int qm_static_scratch(uint8_t** ws);
int qm_stream_workspace(hipStream_t stream, uint8_t** ws);
// Waits for `stream` and frees its workspace on the current device (if any).
int qm_release_stream(hipStream_t stream);
// The ticket words of the K-split mul_mat (two per wave of every tile, at most
// MM_TICKETS of them), kept past the end of the stream's workspace: zero when
// the workspace is made, and left zero by every launch that uses them.
constexpr int MM_TICKETS = 512 * 8 * 2;
int mm_stream_tickets(hipStream_t stream, uint32_t** tickets);
int launch_add_f32(const trc_hip_tensor& a, const trc_hip_tensor& b, const trc_hip_tensor& d, hipStream_t stream);
int launch_mul_f32(const trc_hip_tensor& a, const trc_hip_tensor& b, const trc_hip_tensor& d, hipStream_t stream);
int launch_repeat_f32(const trc_hip_tensor& a, const trc_hip_tensor& d, hipStream_t stream);
int launch_sqr_f32(const trc_hip_tensor& a, const trc_hip_tensor& d, hipStream_t stream);
int launch_scale_f32(const trc_hip_tensor& a, const trc_hip_tensor& d, float scale, hipStream_t stream);
int launch_sum_f32(const trc_hip_tensor& a, const trc_hip_tensor& d, hipStream_t stream);
int launch_acc_f32(const trc_hip_tensor& a, const trc_hip_tensor& b, const trc_hip_tensor& d, size_t nb1, size_t nb2,
                   size_t nb3, size_t offset, int inplace, hipStream_t stream);
int launch_repeat_back_f32(const trc_hip_tensor& a, const trc_hip_tensor& d, hipStream_t stream);
int launch_fill_f32(float* dst, float value, int64_t count, hipStream_t stream);
int launch_cpy(const trc_hip_tensor& src, const trc_hip_tensor& dst, size_t elem_size,
               hipStream_t stream);

}  // namespace trc_hip
