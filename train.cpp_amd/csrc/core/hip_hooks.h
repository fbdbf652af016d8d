// Internal hooks between the core and the HIP backend in libtraincpp_hip.so.
#pragma once

#include "traincpp/traincpp.h"

namespace traincpp {

// hip_dequant_into (declared in traincpp/trc_hip.h) serves gguf_load_tensor.

// Dequantizes host blocks into host floats through the GPU (device 0).
// Returns false if no HIP device is available.
bool hip_dequant_host(Type type, const void* host_blocks, int64_t n_blocks, float* out);

}  // namespace traincpp
