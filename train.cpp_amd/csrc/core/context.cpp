// Metadata arena: tensors (and host data when no_alloc is false) are carved
// from growing arenas and released together by context_free.
#include "impl.h"

#include <cstdlib>

namespace traincpp {

namespace {

size_t round_up(size_t v, size_t a) {
    return (v + a - 1) / a * a;
}

Context::Arena new_arena(size_t size) {
    Context::Arena a;
    a.size = size;
    a.data = (uint8_t*) std::aligned_alloc(64, round_up(size, 64));
    TRC_CHECK(a.data != nullptr, "context: cannot allocate an arena of %zu bytes", size);
    return a;
}

}  // namespace

Context* context_new(size_t mem_size) {
    ContextParams p;
    p.mem_size = mem_size;
    p.no_alloc = true;
    return context_new(p);
}

Context* context_new(const ContextParams& params) {
    TRC_CHECK(params.mem_size > 0, "context_new: mem_size must be > 0");
    Context* ctx = new Context();
    ctx->no_alloc = params.no_alloc;
    if (params.mem_buffer != nullptr) {
        Context::Arena a;
        a.data = (uint8_t*) params.mem_buffer;
        a.size = params.mem_size;
        a.owned = false;
        ctx->arenas.push_back(a);
        ctx->fixed = true;
    } else {
        ctx->arenas.push_back(new_arena(params.mem_size));
    }
    return ctx;
}

void backend_forget_context(Context* ctx);

void context_free(Context* ctx) {
    if (ctx == nullptr) return;
    backend_forget_context(ctx);
    for (Tensor* t : ctx->tensors) t->~Tensor();
    for (Context::Arena& a : ctx->arenas) {
        if (a.owned) std::free(a.data);
    }
    delete ctx;
}

size_t context_mem_size(const Context* ctx) {
    size_t s = 0;
    for (const Context::Arena& a : ctx->arenas) s += a.size;
    return s;
}

size_t context_mem_used(const Context* ctx) {
    return ctx->used_total;
}

size_t context_mem_available(const Context* ctx) {
    const Context::Arena& a = ctx->arenas.back();
    return a.size - a.used;
}

bool context_no_alloc(const Context* ctx) {
    return ctx->no_alloc;
}

void context_set_no_alloc(Context* ctx, bool no_alloc) {
    ctx->no_alloc = no_alloc;
}

void* context_alloc(Context* ctx, size_t size, size_t align) {
    Context::Arena* a = &ctx->arenas.back();
    size_t start = round_up(a->used, align);
    if (start + size > a->size) {
        TRC_CHECK(!ctx->fixed, "context_alloc: fixed arena exhausted (%zu bytes requested)", size);
        ctx->arenas.push_back(new_arena(size + align > a->size ? size + align : a->size));
        a = &ctx->arenas.back();
        start = 0;
    }
    ctx->used_total += start + size - a->used;
    a->used = start + size;
    return a->data + start;
}

int context_tensor_count(const Context* ctx) {
    return (int) ctx->tensors.size();
}

Tensor* context_tensor(const Context* ctx, int index) {
    TRC_CHECK(index >= 0 && index < (int) ctx->tensors.size(), "context_tensor: index %d out of range", index);
    return ctx->tensors[(size_t) index];
}

}  // namespace traincpp
