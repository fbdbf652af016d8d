// traincpp-compatible backend plugin interface. Interface of
// include/traincpp/trc_backend.h in the reference (Device / BufferType / Buffer /
// supports_op / graph_compute / fill_tensors, the device registry and the
// buffer helpers). The HIP backend implements these classes; graphs built with
// the traincpp API run on it unchanged.
#pragma once

#include "trc_graph.h"
#include "trc_tensor.h"

#include <cstddef>
#include <string>

namespace traincpp {

enum class DeviceType : int32_t {
    CPU = 0,
    GPU = 1,
    IGPU = 2,
    ACCEL = 3,
};

struct DeviceProps {
    std::string name;
    std::string description;
    DeviceType  type = DeviceType::CPU;
    size_t      memory_free = 0;
    size_t      memory_total = 0;
    bool        unified_memory = false;
};

class Device;

class BufferType {
public:
    virtual ~BufferType() = default;
    virtual Device*     device() const = 0;
    virtual const char* name() const = 0;
    virtual size_t      alignment() const = 0;
    virtual Buffer*     alloc_buffer(size_t size) = 0;  // nullptr on failure
};

class Buffer {
public:
    virtual ~Buffer() = default;
    virtual BufferType* buffer_type() const = 0;
    virtual size_t      size() const = 0;
    virtual void*       base() = 0;          // host mapping, nullptr for device memory
    virtual bool        is_host() const = 0;
    // offset is relative to the start of the tensor
    virtual void set_tensor(Tensor* t, size_t offset, const void* data, size_t size) = 0;
    virtual void get_tensor(const Tensor* t, size_t offset, void* data, size_t size) const = 0;
    virtual void clear() = 0;
};

struct TensorFill {
    Tensor* tensor = nullptr;
    float   value = 0.0f;
};

class Device {
public:
    virtual ~Device() = default;
    virtual const DeviceProps& props() const = 0;
    virtual BufferType*        default_buffer_type() = 0;
    virtual Buffer*            alloc_buffer(size_t size) { return default_buffer_type()->alloc_buffer(size); }
    virtual bool               supports_op(const Tensor* t) const = 0;
    virtual bool               graph_compute(Graph* graph) = 0;  // synchronous
    virtual bool               fill_tensors(const TensorFill* fills, size_t count);
    bool fill_tensor(Tensor* t, float value) {
        TensorFill f{t, value};
        return fill_tensors(&f, 1);
    }
};

const Tensor* graph_first_unsupported(const Graph* graph, const Device* dev);

size_t  device_count();
Device* device_get(size_t index);
Device* device_by_type(DeviceType type);
Device* device_cpu();
void    backend_register_device(Device* device);

Buffer* buffer_alloc_ctx_tensors(Context* ctx, BufferType* buft);
void    buffer_free(Buffer* buf);

struct AllocStats {
    size_t current_bytes = 0;
    size_t peak_bytes = 0;
    size_t n_allocations = 0;
};
AllocStats backend_alloc_stats();
void       backend_alloc_stats_reset();

void tensor_set(Tensor* t, const void* data, size_t offset, size_t size);
void tensor_get(const Tensor* t, void* data, size_t offset, size_t size);
// Fills contiguous F32 tensors through their owning devices (batched per device).
void tensor_fill_values(const TensorFill* fills, size_t count);

}  // namespace traincpp
