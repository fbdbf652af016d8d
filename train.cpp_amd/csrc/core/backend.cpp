// Device registry, context buffer allocation and host<->buffer transfers
// (behaviour of the reference's src/core/trc_backend_reg.cpp for this subset).
#include "impl.h"

#include <algorithm>
#include <cstring>
#include <utility>
#include <vector>

namespace traincpp {

namespace {

std::vector<Device*>& registry() {
    static std::vector<Device*> devices = [] {
        std::vector<Device*> v;
        const int n = hip_device_count();
        for (int i = 0; i < n; ++i) {
            if (Device* d = hip_device(i)) v.push_back(d);
        }
        return v;
    }();
    return devices;
}

struct Owner {
    Buffer*  buffer;
    Context* ctx;
    size_t   bytes;
    bool     counted;
};

std::vector<Owner>& owners() {
    static std::vector<Owner> v;
    return v;
}

AllocStats& stats() {
    static AllocStats s;
    return s;
}

size_t align_up(size_t v, size_t a) {
    return a == 0 ? v : (v + a - 1) / a * a;
}

}  // namespace

// Called by context_free: the context's tensors are gone, so a later
// buffer_free must not touch them.
void backend_forget_context(Context* ctx) {
    for (Owner& o : owners()) {
        if (o.ctx == ctx) o.ctx = nullptr;
    }
}

void backend_register_device(Device* device) {
    TRC_CHECK(device != nullptr, "backend_register_device: device is NULL");
    registry().push_back(device);
}

size_t device_count() {
    return registry().size();
}

Device* device_get(size_t index) {
    return index < registry().size() ? registry()[index] : nullptr;
}

Device* device_by_type(DeviceType type) {
    for (Device* d : registry()) {
        if (d->props().type == type) return d;
    }
    return nullptr;
}

Device* device_cpu() {
    return device_by_type(DeviceType::CPU);
}

const Tensor* graph_first_unsupported(const Graph* graph, const Device* dev) {
    TRC_CHECK(graph != nullptr && dev != nullptr, "graph_first_unsupported: NULL argument");
    for (Tensor* n : graph->nodes) {
        if (n != nullptr && !dev->supports_op(n)) return n;
    }
    return nullptr;
}

bool Device::fill_tensors(const TensorFill* fills, size_t count) {
    for (size_t i = 0; i < count; ++i) {
        Tensor* t = fills[i].tensor;
        TRC_CHECK(t != nullptr && t->type == TYPE_F32 && tensor_is_contiguous(t),
                  "fill_tensors: target must be a contiguous F32 tensor");
        std::vector<float> v((size_t) tensor_nelements(t), fills[i].value);
        tensor_set(t, v.data(), 0, v.size() * sizeof(float));
    }
    return true;
}

Buffer* buffer_alloc_ctx_tensors(Context* ctx, BufferType* buft) {
    TRC_CHECK(ctx != nullptr && buft != nullptr, "buffer_alloc_ctx_tensors: NULL argument");
    const size_t align = std::max<size_t>(buft->alignment(), 1);
    const int n = context_tensor_count(ctx);
    size_t total = 0;
    for (int i = 0; i < n; ++i) {
        const Tensor* t = context_tensor(ctx, i);
        if (t->view_src == nullptr && t->data == nullptr && t->buffer == nullptr) {
            total += align_up(tensor_nbytes(t), align);
        }
    }
    const size_t request = std::max(total, align);
    Buffer* buf = buft->alloc_buffer(request);
    if (buf == nullptr) {
        const DeviceProps& p = buft->device()->props();
        TRC_FAIL("buffer_alloc_ctx_tensors: buffer allocation failed: need %zu bytes (%.2f MiB), device '%s' "
                 "has %zu bytes free of %zu (reduce the batch or split the work)",
                 request, request / 1048576.0, p.name.c_str(), p.memory_free, p.memory_total);
    }
    uint8_t* base = (uint8_t*) buf->base();
    size_t off = 0;
    for (int i = 0; i < n; ++i) {
        Tensor* t = context_tensor(ctx, i);
        if (t->view_src != nullptr || t->data != nullptr || t->buffer != nullptr) continue;
        t->buffer = buf;
        t->data_offset = off;
        t->data = base != nullptr ? base + off : nullptr;
        off += align_up(tensor_nbytes(t), align);
    }
    // views were created after their sources, so one pass in creation order resolves chains
    for (int i = 0; i < n; ++i) {
        Tensor* t = context_tensor(ctx, i);
        if (t->view_src == nullptr) continue;
        const Tensor* s = t->view_src;
        t->data_offset = s->data_offset + t->view_offs;
        t->data = s->data != nullptr ? (uint8_t*) s->data + t->view_offs : nullptr;
    }
    owners().push_back({buf, ctx, request, true});
    AllocStats& st = stats();
    st.current_bytes += request;
    st.peak_bytes = std::max(st.peak_bytes, st.current_bytes);
    st.n_allocations += 1;
    return buf;
}

void buffer_free(Buffer* buf) {
    if (buf == nullptr) return;
    auto& v = owners();
    for (auto it = v.begin(); it != v.end(); ++it) {
        if (it->buffer != buf) continue;
        if (it->ctx != nullptr) {
            const int n = context_tensor_count(it->ctx);
            for (int i = 0; i < n; ++i) {
                Tensor* t = context_tensor(it->ctx, i);
                if (owning_buffer(t) == buf) {
                    t->data = nullptr;
                    if (t->buffer == buf) t->buffer = nullptr;
                }
            }
        }
        if (it->counted) stats().current_bytes -= std::min(stats().current_bytes, it->bytes);
        v.erase(it);
        break;
    }
    delete buf;
}

AllocStats backend_alloc_stats() {
    return stats();
}

void backend_alloc_stats_reset() {
    stats() = AllocStats{};
    for (Owner& o : owners()) o.counted = false;
}

void tensor_set(Tensor* t, const void* data, size_t offset, size_t size) {
    TRC_CHECK(t != nullptr && (data != nullptr || size == 0), "tensor_set: NULL argument");
    TRC_CHECK(offset + size <= tensor_nbytes(t), "tensor_set: %zu bytes at %zu exceed %s (%zu bytes)", size, offset,
              t->name, tensor_nbytes(t));
    if (size == 0) return;
    if (Buffer* b = owning_buffer(t)) {
        b->set_tensor(t, offset, data, size);
        return;
    }
    TRC_CHECK(t->data != nullptr, "tensor_set: tensor %s has no storage", t->name);
    std::memcpy((uint8_t*) t->data + offset, data, size);
}

void tensor_get(const Tensor* t, void* data, size_t offset, size_t size) {
    TRC_CHECK(t != nullptr && (data != nullptr || size == 0), "tensor_get: NULL argument");
    TRC_CHECK(offset + size <= tensor_nbytes(t), "tensor_get: %zu bytes at %zu exceed %s (%zu bytes)", size, offset,
              t->name, tensor_nbytes(t));
    if (size == 0) return;
    if (const Buffer* b = owning_buffer(t)) {
        b->get_tensor(t, offset, data, size);
        return;
    }
    TRC_CHECK(t->data != nullptr, "tensor_get: tensor %s has no storage", t->name);
    std::memcpy(data, (const uint8_t*) t->data + offset, size);
}

void tensor_fill_values(const TensorFill* fills, size_t count) {
    // batch the requests per owning device, as the reference does for device fills
    std::vector<std::pair<Device*, std::vector<TensorFill>>> groups;
    for (size_t i = 0; i < count; ++i) {
        Tensor* t = fills[i].tensor;
        TRC_CHECK(t != nullptr && t->type == TYPE_F32 && tensor_is_contiguous(t),
                  "tensor_fill_values: target must be a contiguous F32 tensor");
        Buffer* b = owning_buffer(t);
        if (b == nullptr) {
            TRC_CHECK(t->data != nullptr, "tensor_fill_values: tensor %s has no storage", t->name);
            std::fill((float*) t->data, (float*) t->data + tensor_nelements(t), fills[i].value);
            continue;
        }
        Device* d = b->buffer_type()->device();
        auto it = std::find_if(groups.begin(), groups.end(), [d](const auto& g) { return g.first == d; });
        if (it == groups.end()) {
            groups.push_back({d, {}});
            it = groups.end() - 1;
        }
        it->second.push_back(fills[i]);
    }
    for (auto& g : groups) {
        TRC_CHECK(g.first->fill_tensors(g.second.data(), g.second.size()), "tensor_fill_values: device fill failed");
    }
}

}  // namespace traincpp
