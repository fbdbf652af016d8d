// Entry points of the MI355X HIP backend (libtraincpp_hip.so, or hip_device.cpp
// built into a traincpp tree). hip_device() is a new sibling of the reference's
// cpu_device()/vulkan_device() (src/core/trc_backends.h:14-22): it returns the
// Device of HIP ordinal `ordinal`, or nullptr when that GPU is not visible.
// Devices are process-lifetime singletons; register them with
// backend_register_device (include/traincpp/trc_backend.h:105) or the
// compile-time device list.
//
// The includes name the traincpp/ directory so that, built inside a traincpp
// tree, they resolve to that tree's own headers.
#pragma once

#include "traincpp/trc_backend.h"
#include "traincpp/trc_gguf.h"

#include <cstdint>

namespace traincpp {

Device* hip_device(int ordinal = 0);
int     hip_device_count();

// Warm-start load of one GGUF tensor in a legacy quant format (Q4_0, Q4_1,
// Q5_0, Q5_1, Q8_0) into a contiguous F32 tensor held in a HIP buffer, with the
// dequantization on the GPU (bit-identical to gguf_tensor_to_f32,
// src/io/trc_gguf.cpp:966-1049). Only the tensor's raw blocks cross PCIe (a
// quarter to a ninth of the F32 bytes); they are read by mmap straight from
// `path`, the file `f` was opened from, at the offsets the public reader
// reports (gguf_data_offset + GgufTensorInfo::offset). f may therefore be
// opened with load_data = false, so the data section is never read into host
// memory. Returns false, having done nothing, when the tensor is not a legacy
// quant type or dst is not such a tensor (use gguf_load_tensor then); prints
// an error and returns false when the name or the file is wrong; aborts on a
// device error.
bool hip_gguf_load_tensor(const char* path, const GgufFile* f, const char* name, Tensor* dst);

// Uploads n_blocks raw blocks of a legacy quant `type` from host memory and
// dequantizes them on the GPU straight into dst (a contiguous F32 tensor in a
// HIP buffer). Returns false, doing nothing, when dst is not in a HIP buffer;
// aborts on a device error. This is the call a reader that already holds the
// blocks makes: the quant branch of the reference's gguf_load_tensor
// (src/io/trc_gguf.cpp:1082-1088) can hand its blocks here instead of
// dequantizing on the host.
bool hip_dequant_into(Tensor* dst, Type type, const void* host_blocks, int64_t n_blocks);

}  // namespace traincpp
