// traincpp-compatible context (tensor metadata arena). Interface of
// include/traincpp/trc_context.h in the reference.
#pragma once

#include "trc_tensor.h"

#include <cstddef>

namespace traincpp {

struct Context;

struct ContextParams {
    size_t mem_size = 0;         // bytes of the first arena
    void*  mem_buffer = nullptr; // caller-provided arena (nullptr: allocate)
    bool   no_alloc = true;      // true: tensor data comes from a backend buffer
};

Context* context_new(size_t mem_size);
Context* context_new(const ContextParams& params);
void     context_free(Context* ctx);

size_t context_mem_size(const Context* ctx);
size_t context_mem_used(const Context* ctx);
size_t context_mem_available(const Context* ctx);
bool   context_no_alloc(const Context* ctx);
void   context_set_no_alloc(Context* ctx, bool no_alloc);

void* context_alloc(Context* ctx, size_t size, size_t align = MEM_ALIGN);

int     context_tensor_count(const Context* ctx);
Tensor* context_tensor(const Context* ctx, int index);

}  // namespace traincpp
