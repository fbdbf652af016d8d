// H1: bulk dequantization of the GGUF legacy block formats to F32 on gfx950.
//
// Semantics: src/io/trc_gguf.cpp:320-417 (dequantize_q4_0 .. dequantize_q8_0),
// reached from gguf_tensor_to_f32 (:966-1049). Every output is computed as the
// reference computes it: the integer quant converted to float, times d, plus m
// for Q4_1/Q5_1, each operation rounded on its own (contraction is off in this
// file). Because q has at most 8 significant bits and d (a binary16) at most 11,
// q*d is exact in binary32, so the only rounding is the "+ m", as on the CPU.
//
// Mapping: the output of one block is 32 floats = 8 quads of 4 floats. One lane
// produces one quad, so 8 lanes cover a block and a wave64 writes 8 blocks
// (1 KiB) as one contiguous run of dwordx4 stores. Each lane loads only the
// bytes its quad needs (scale, min, 4 quant bytes and the 5th-bit mask word);
// lanes of the same block read the same scale, which the L1 serves once.
// One quad per lane and 512 lanes per workgroup: on configuration 1
// (4096 x 11008) this measured 89-91 % of HBM peak against 85-86 % for 4 quads
// per lane at 256 lanes, and 88-89 % for 1 quad at 256 or 1024 lanes. Plain
// stores in place of the non-temporal ones measured 55-68 %.
#pragma clang fp contract(off)

#include "common.h"

namespace trc_hip {
namespace {

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return *(const uint16_t*) p;
}

__device__ __forceinline__ uint32_t ld_u32_from_u16(const uint8_t* p) {
    const uint16_t* h = (const uint16_t*) p;
    return (uint32_t) h[0] | ((uint32_t) h[1] << 16);
}

__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {
    return *(const uint32_t*) p;
}

// Moves bits 0..3 of `four` to bit 4 of bytes 0..3.
__device__ __forceinline__ uint32_t spread_bit4(uint32_t four) {
    return ((four & 1u) << 4) | ((four & 2u) << 11) | ((four & 4u) << 18) | ((four & 8u) << 25);
}

__device__ __forceinline__ f4 bytes_times(uint32_t q, float bias, float d) {
    // (float)(byte - bias) == (float)byte - bias exactly: both are small integers.
    f4 r;
    r.x = ((float) (q & 0xFFu) - bias) * d;
    r.y = ((float) ((q >> 8) & 0xFFu) - bias) * d;
    r.z = ((float) ((q >> 16) & 0xFFu) - bias) * d;
    r.w = ((float) (q >> 24) - bias) * d;
    return r;
}

__device__ __forceinline__ f4 bytes_times_plus(uint32_t q, float d, float m) {
    f4 r;
    r.x = (float) (q & 0xFFu) * d + m;
    r.y = (float) ((q >> 8) & 0xFFu) * d + m;
    r.z = (float) ((q >> 16) & 0xFFu) * d + m;
    r.w = (float) (q >> 24) * d + m;
    return r;
}

// Quad s (0..7) of the block at `blk`: outputs 4s .. 4s+3.
// Outputs 0..15 use the low nibbles of qs[0..15]; 16..31 the high nibbles
// (src/io/trc_gguf.cpp:331-334). For Q5 the 5th bit of output e is qh bit e
// (:370-371, :394-395).
template <int TYPE>
__device__ __forceinline__ f4 dequant_quad(const uint8_t* blk, int s) {
    const int j = 4 * (s & 3);           // first quant byte of this quad
    const int sh = (s & 4) ? 4 : 0;      // high nibbles for the second half
    if constexpr (TYPE == TRC_HIP_TYPE_Q4_0) {
        const float d = half_bits_to_float(ld_u16(blk));
        const uint32_t q = (ld_u32_from_u16(blk + 2 + j) >> sh) & 0x0F0F0F0Fu;
        return bytes_times(q, 8.0f, d);
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q4_1) {
        const uint32_t dm = ld_u32(blk);
        const float d = half_bits_to_float(dm & 0xFFFFu);
        const float m = half_bits_to_float(dm >> 16);
        const uint32_t q = (ld_u32(blk + 4 + j) >> sh) & 0x0F0F0F0Fu;
        return bytes_times_plus(q, d, m);
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_0) {
        const float d = half_bits_to_float(ld_u16(blk));
        const uint32_t qh = ld_u32_from_u16(blk + 2);
        uint32_t q = (ld_u32_from_u16(blk + 6 + j) >> sh) & 0x0F0F0F0Fu;
        q |= spread_bit4((qh >> (4 * s)) & 0xFu);
        return bytes_times(q, 16.0f, d);
    } else if constexpr (TYPE == TRC_HIP_TYPE_Q5_1) {
        const uint32_t dm = ld_u32(blk);
        const float d = half_bits_to_float(dm & 0xFFFFu);
        const float m = half_bits_to_float(dm >> 16);
        const uint32_t qh = ld_u32(blk + 4);
        uint32_t q = (ld_u32(blk + 8 + j) >> sh) & 0x0F0F0F0Fu;
        q |= spread_bit4((qh >> (4 * s)) & 0xFu);
        return bytes_times_plus(q, d, m);
    } else {  // Q8_0: 32 signed bytes, quad s = bytes 4s .. 4s+3
        const float d = half_bits_to_float(ld_u16(blk));
        const uint32_t q = ld_u32_from_u16(blk + 2 + 4 * s);
        f4 r;
        r.x = (float) (int) (int8_t) (q & 0xFFu) * d;
        r.y = (float) (int) (int8_t) ((q >> 8) & 0xFFu) * d;
        r.z = (float) (int) (int8_t) ((q >> 16) & 0xFFu) * d;
        r.w = (float) (int) (int8_t) (q >> 24) * d;
        return r;
    }
}

constexpr int DQ_THREADS = 512;

template <int TYPE, int ITEMS>
__global__ __launch_bounds__(DQ_THREADS) void k_dequant(const uint8_t* __restrict__ src,
                                                        int64_t n_quads, f4* __restrict__ dst) {
    constexpr int BYTES = block_bytes(TYPE);
    const int64_t first = (int64_t) blockIdx.x * (ITEMS * DQ_THREADS) + threadIdx.x;
    f4 v[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t qd = first + (int64_t) it * DQ_THREADS;
        if (qd < n_quads) {
            v[it] = dequant_quad<TYPE>(src + (qd >> 3) * BYTES, (int) (qd & 7));
        }
    }
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t qd = first + (int64_t) it * DQ_THREADS;
        if (qd < n_quads) {
            __builtin_nontemporal_store(v[it], dst + qd);
        }
    }
}

template <int TYPE>
int launch_type(const void* blocks, int64_t n_blocks, float* dst, hipStream_t stream) {
    constexpr int ITEMS = 1;
    const int64_t n_quads = n_blocks * 8;
    const int64_t grid = (n_quads + ITEMS * DQ_THREADS - 1) / (ITEMS * DQ_THREADS);
    if (grid > 0x7FFFFFFF) return fail(TRC_HIP_E_INVALID, "dequant: %lld blocks exceed one launch", (long long) n_blocks);
    hipLaunchKernelGGL((k_dequant<TYPE, ITEMS>), dim3((unsigned) grid), dim3(DQ_THREADS), 0, stream,
                       (const uint8_t*) blocks, n_quads, (f4*) dst);
    return check_launch("dequant");
}

}  // namespace

int launch_dequant(int type, const void* blocks, int64_t n_blocks, float* dst, hipStream_t stream) {
    if (n_blocks == 0) return TRC_HIP_OK;
    const uintptr_t sa = (uintptr_t) blocks;
    const bool wide = type == TRC_HIP_TYPE_Q4_1 || type == TRC_HIP_TYPE_Q5_1;
    if ((sa & (wide ? 3u : 1u)) != 0 || ((uintptr_t) dst & 15u) != 0) {
        return fail(TRC_HIP_E_ALIGN, "dequant: blocks must be %d-byte and dst 16-byte aligned",
                    wide ? 4 : 2);
    }
    switch (type) {
        case TRC_HIP_TYPE_Q4_0: return launch_type<TRC_HIP_TYPE_Q4_0>(blocks, n_blocks, dst, stream);
        case TRC_HIP_TYPE_Q4_1: return launch_type<TRC_HIP_TYPE_Q4_1>(blocks, n_blocks, dst, stream);
        case TRC_HIP_TYPE_Q5_0: return launch_type<TRC_HIP_TYPE_Q5_0>(blocks, n_blocks, dst, stream);
        case TRC_HIP_TYPE_Q5_1: return launch_type<TRC_HIP_TYPE_Q5_1>(blocks, n_blocks, dst, stream);
        case TRC_HIP_TYPE_Q8_0: return launch_type<TRC_HIP_TYPE_Q8_0>(blocks, n_blocks, dst, stream);
        default: return fail(TRC_HIP_E_INVALID, "dequant: type %d is not a legacy quant type", type);
    }
}

}  // namespace trc_hip
