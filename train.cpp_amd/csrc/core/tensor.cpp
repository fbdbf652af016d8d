// Tensor metadata, shape helpers and view construction, following the
// reference's ggml layout rules (src/core/trc_tensor.cpp).
#include "impl.h"

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>

namespace traincpp {

int tensor_n_dims(const Tensor* t) {
    int n = 1;
    for (int i = 1; i < MAX_DIMS; ++i) {
        if (t->ne[i] > 1) n = i + 1;
    }
    return n;
}

int64_t tensor_nelements(const Tensor* t) {
    return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3];
}

int64_t tensor_nrows(const Tensor* t) {
    return t->ne[1] * t->ne[2] * t->ne[3];
}

size_t tensor_nbytes(const Tensor* t) {
    const int64_t blck = type_blck_size(t->type);
    TRC_CHECK(blck > 0 && t->ne[0] % blck == 0, "tensor_nbytes: invalid type %d / ne0 %lld", (int) t->type,
              (long long) t->ne[0]);
    // extent of the last element: first row plus (ne[i]-1) strides per outer dim
    size_t n = (size_t) (t->ne[0] / blck) * type_size(t->type);
    for (int i = 1; i < MAX_DIMS; ++i) {
        if (t->ne[i] > 1) n += (size_t) (t->ne[i] - 1) * t->nb[i];
    }
    return n;
}

size_t tensor_element_size(const Tensor* t) {
    return type_size(t->type);
}

size_t tensor_row_size(const Tensor* t) {
    return type_row_size(t->type, t->ne[0]);
}

bool tensor_is_contiguous(const Tensor* t) {
    const int64_t blck = type_blck_size(t->type);
    TRC_CHECK(blck > 0, "tensor_is_contiguous: type %d has no layout", (int) t->type);
    size_t want = type_size(t->type);
    if (t->nb[0] != want) return false;
    want *= (size_t) (t->ne[0] / blck);
    for (int i = 1; i < MAX_DIMS; ++i) {
        if (t->nb[i] != want) return false;
        want *= (size_t) t->ne[i];
    }
    return true;
}

bool tensor_are_same_shape(const Tensor* a, const Tensor* b) {
    for (int i = 0; i < MAX_DIMS; ++i) {
        if (a->ne[i] != b->ne[i]) return false;
    }
    return true;
}

bool tensor_can_repeat(const Tensor* b, const Tensor* a) {
    for (int i = 0; i < MAX_DIMS; ++i) {
        if (b->ne[i] != 1 && b->ne[i] != a->ne[i]) return false;
    }
    return true;
}

bool tensor_is_view(const Tensor* t) {
    return t->view_src != nullptr;
}

size_t tensor_offset_linear(const Tensor* t, int64_t i) {
    size_t off = 0;
    for (int d = 0; d < MAX_DIMS; ++d) {
        off += (size_t) (i % t->ne[d]) * t->nb[d];
        i /= t->ne[d];
    }
    return off;
}

namespace {

size_t last_byte_extent(const Tensor* t) {
    size_t off = 0;
    for (int d = 0; d < MAX_DIMS; ++d) off += (size_t) (t->ne[d] - 1) * t->nb[d];
    return off + type_size(t->type);
}

Tensor* make_tensor(Context* ctx, Type type, int n_dims, const int64_t* ne, const size_t* nb, bool with_data) {
    TRC_CHECK(ctx != nullptr, "new_tensor: ctx is NULL");
    TRC_CHECK(n_dims >= 1 && n_dims <= MAX_DIMS, "new_tensor: %d dimensions", n_dims);
    TRC_CHECK(type_is_storable(type), "new_tensor: type %s cannot be allocated", type_name(type));
    const int64_t blck = type_blck_size(type);
    Tensor* t = new (context_alloc(ctx, sizeof(Tensor), MEM_ALIGN)) Tensor();
    t->type = type;
    for (int i = 0; i < MAX_DIMS; ++i) {
        t->ne[i] = i < n_dims ? ne[i] : 1;
        TRC_CHECK(t->ne[i] > 0, "new_tensor: ne[%d] = %lld", i, (long long) t->ne[i]);
    }
    TRC_CHECK(t->ne[0] % blck == 0, "new_tensor: ne0 %lld is not a multiple of the block size %lld of %s",
              (long long) t->ne[0], (long long) blck, type_name(type));
    if (nb != nullptr) {
        for (int i = 0; i < MAX_DIMS; ++i) t->nb[i] = nb[i];
    } else {
        t->nb[0] = type_size(type);
        t->nb[1] = t->nb[0] * (size_t) (t->ne[0] / blck);
        for (int i = 2; i < MAX_DIMS; ++i) t->nb[i] = t->nb[i - 1] * (size_t) t->ne[i - 1];
    }
    if (with_data && !context_no_alloc(ctx)) t->data = context_alloc(ctx, tensor_nbytes(t), MEM_ALIGN);
    ctx->tensors.push_back(t);
    return t;
}

}  // namespace

// A view shares a's storage: same buffer, offset `offset` bytes from a's start.
Tensor* make_view(Context* ctx, Tensor* a, Op op, int n_dims, const int64_t* ne, const size_t* nb, size_t offset) {
    TRC_CHECK(a != nullptr, "view: source is NULL");
    TRC_CHECK(!type_is_quantized(a->type), "view: quantized source %s", type_name(a->type));
    Tensor* v = make_tensor(ctx, a->type, n_dims, ne, nb, false);
    v->op = op;
    v->view_src = a;
    v->view_offs = offset;
    v->src[0] = a;
    v->nsrc = 1;
    TRC_CHECK(offset + last_byte_extent(v) <= last_byte_extent(a), "view: out of range of its source");
    if (a->data != nullptr || a->buffer != nullptr || a->view_src != nullptr) {
        v->data_offset = a->data_offset + offset;
        v->data = a->data != nullptr ? (uint8_t*) a->data + offset : nullptr;
    }
    return v;
}

Tensor* new_tensor_nd(Context* ctx, Type type, int n_dims, const int64_t* ne) {
    return make_tensor(ctx, type, n_dims, ne, nullptr, true);
}

Tensor* new_tensor_1d(Context* ctx, Type type, int64_t ne0) {
    const int64_t ne[4] = {ne0, 1, 1, 1};
    return new_tensor_nd(ctx, type, 1, ne);
}

Tensor* new_tensor_2d(Context* ctx, Type type, int64_t ne0, int64_t ne1) {
    const int64_t ne[4] = {ne0, ne1, 1, 1};
    return new_tensor_nd(ctx, type, 2, ne);
}

Tensor* new_tensor_3d(Context* ctx, Type type, int64_t ne0, int64_t ne1, int64_t ne2) {
    const int64_t ne[4] = {ne0, ne1, ne2, 1};
    return new_tensor_nd(ctx, type, 3, ne);
}

Tensor* new_tensor_4d(Context* ctx, Type type, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    return new_tensor_nd(ctx, type, 4, ne);
}

Tensor* tensor_dup_meta(Context* ctx, const Tensor* src) {
    Tensor* t = new_tensor_nd(ctx, src->type, MAX_DIMS, src->ne);
    std::memcpy(t->name, src->name, MAX_NAME);
    return t;
}

void tensor_set_name(Tensor* t, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(t->name, MAX_NAME, fmt, ap);
    va_end(ap);
}

float* tensor_data_f32(Tensor* t) {
    TRC_CHECK(t->type == TYPE_F32, "tensor_data_f32: tensor is %s", type_name(t->type));
    return (float*) t->data;
}

const float* tensor_data_f32(const Tensor* t) {
    TRC_CHECK(t->type == TYPE_F32, "tensor_data_f32: tensor is %s", type_name(t->type));
    return (const float*) t->data;
}

}  // namespace traincpp
