// Internal hooks between the core and the HIP backend in libtraincpp_hip.so.
#pragma once

#include "traincpp/traincpp.h"

namespace traincpp {

// If dst lives in a HIP buffer: uploads n_blocks raw blocks of `type` and
// dequantizes them on the GPU straight into dst (contiguous F32). Returns false
// when dst is not in a HIP buffer (nothing done); aborts on a HIP error.
bool hip_dequant_into(Tensor* dst, Type type, const void* host_blocks, int64_t n_blocks);

// Dequantizes host blocks into host floats through the GPU (device 0).
// Returns false if no HIP device is available.
bool hip_dequant_host(Type type, const void* host_blocks, int64_t n_blocks, float* out);

}  // namespace traincpp
