// Operator constructors of the HIP path (graph nodes only). Shape rules follow
// the reference's src/ops/trc_ops.cpp (add :17-32/:46, cont :124-134,
// cast :136-147, mul_mat :366-385, repeat_back :458-470) and
// src/core/trc_tensor.cpp (views :226-320, acc :322-361).
#include "impl.h"

#include <climits>
#include <cstring>

namespace traincpp {

Tensor* make_view(Context* ctx, Tensor* a, Op op, int n_dims, const int64_t* ne, const size_t* nb, size_t offset);

Tensor* dup(Context* ctx, const Tensor* a) {
    TRC_CHECK(a != nullptr, "dup: input is NULL");
    return tensor_dup_meta(ctx, a);
}

Tensor* view_1d(Context* ctx, Tensor* a, int64_t ne0, size_t offset) {
    const int64_t ne[4] = {ne0, 1, 1, 1};
    return make_view(ctx, a, OP_VIEW, 1, ne, a->nb, offset);
}

Tensor* view_2d(Context* ctx, Tensor* a, int64_t ne0, int64_t ne1, size_t offset) {
    const int64_t ne[4] = {ne0, ne1, 1, 1};
    return make_view(ctx, a, OP_VIEW, 2, ne, a->nb, offset);
}

Tensor* view_3d(Context* ctx, Tensor* a, int64_t ne0, int64_t ne1, int64_t ne2, size_t offset) {
    const int64_t ne[4] = {ne0, ne1, ne2, 1};
    return make_view(ctx, a, OP_VIEW, 3, ne, a->nb, offset);
}

Tensor* view_4d(Context* ctx, Tensor* a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, size_t offset) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    return make_view(ctx, a, OP_VIEW, 4, ne, a->nb, offset);
}

namespace {

Tensor* reshape(Context* ctx, Tensor* a, int n_dims, const int64_t* ne) {
    TRC_CHECK(a != nullptr, "reshape: input is NULL");
    TRC_CHECK(tensor_is_contiguous(a), "reshape: source must be contiguous");
    int64_t n = 1;
    for (int i = 0; i < n_dims; ++i) n *= ne[i];
    TRC_CHECK(n == tensor_nelements(a), "reshape: %lld elements vs %lld", (long long) n,
              (long long) tensor_nelements(a));
    return make_view(ctx, a, OP_RESHAPE, n_dims, ne, nullptr, 0);
}

}  // namespace

Tensor* reshape_1d(Context* ctx, Tensor* a, int64_t ne0) {
    const int64_t ne[4] = {ne0, 1, 1, 1};
    return reshape(ctx, a, 1, ne);
}

Tensor* reshape_2d(Context* ctx, Tensor* a, int64_t ne0, int64_t ne1) {
    const int64_t ne[4] = {ne0, ne1, 1, 1};
    return reshape(ctx, a, 2, ne);
}

Tensor* reshape_3d(Context* ctx, Tensor* a, int64_t ne0, int64_t ne1, int64_t ne2) {
    const int64_t ne[4] = {ne0, ne1, ne2, 1};
    return reshape(ctx, a, 3, ne);
}

Tensor* reshape_4d(Context* ctx, Tensor* a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    return reshape(ctx, a, 4, ne);
}

Tensor* permute(Context* ctx, Tensor* a, int axis0, int axis1, int axis2, int axis3) {
    TRC_CHECK(a != nullptr, "permute: input is NULL");
    const int axes[4] = {axis0, axis1, axis2, axis3};
    int seen = 0;
    for (int ax : axes) {
        TRC_CHECK(ax >= 0 && ax < MAX_DIMS && !(seen & (1 << ax)), "permute: invalid axes");
        seen |= 1 << ax;
    }
    int64_t ne[4];
    size_t nb[4];
    for (int i = 0; i < MAX_DIMS; ++i) {
        ne[i] = a->ne[axes[i]];
        nb[i] = a->nb[axes[i]];
    }
    Tensor* v = make_view(ctx, a, OP_PERMUTE, MAX_DIMS, ne, nb, 0);
    for (int i = 0; i < MAX_DIMS; ++i) v->op_params[i] = axes[i];
    return v;
}

Tensor* transpose(Context* ctx, Tensor* a) {
    return permute(ctx, a, 1, 0, 2, 3);
}

Tensor* cont(Context* ctx, Tensor* a) {
    TRC_CHECK(a != nullptr, "cont: input is NULL");
    if (tensor_is_contiguous(a)) return a;  // already contiguous: the source itself
    Tensor* r = new_tensor_nd(ctx, a->type, MAX_DIMS, a->ne);
    r->op = OP_CONT;
    r->src[0] = a;
    r->nsrc = 1;
    return r;
}

Tensor* cast(Context* ctx, Tensor* a, Type type) {
    TRC_CHECK(a != nullptr, "cast: input is NULL");
    if (a->type == type) return a;
    // Extension: a legacy quant source may be cast (dequantized) to F32.
    TRC_CHECK(type_is_supported(type), "cast: target type %s is not supported", type_name(type));
    TRC_CHECK(type_is_storable(a->type), "cast: source type %s is not supported", type_name(a->type));
    Tensor* r = new_tensor_nd(ctx, type, MAX_DIMS, a->ne);
    r->op = OP_CAST;
    r->src[0] = a;
    r->nsrc = 1;
    return r;
}

Tensor* mul_mat(Context* ctx, Tensor* a, Tensor* b) {
    TRC_CHECK(a != nullptr && b != nullptr, "mul_mat: input is NULL");
    const bool quant_a = type_is_quantized(a->type) && type_is_storable(a->type);
    TRC_CHECK(a->type == b->type || (quant_a && b->type == TYPE_F32),
              "mul_mat: input types %s x %s are not supported", type_name(a->type), type_name(b->type));
    TRC_CHECK(a->ne[0] == b->ne[0], "mul_mat: inner dimensions differ (a.ne[0]=%lld, b.ne[0]=%lld)",
              (long long) a->ne[0], (long long) b->ne[0]);
    TRC_CHECK(b->ne[2] % a->ne[2] == 0 && b->ne[3] % a->ne[3] == 0,
              "mul_mat: a's planes [%lld,%lld] do not divide b's [%lld,%lld]", (long long) a->ne[2],
              (long long) a->ne[3], (long long) b->ne[2], (long long) b->ne[3]);
    Tensor* r = new_tensor_4d(ctx, quant_a ? TYPE_F32 : a->type, a->ne[1], b->ne[1], b->ne[2], b->ne[3]);
    r->op = OP_MUL_MAT;
    r->src[0] = a;
    r->src[1] = b;
    r->nsrc = 2;
    return r;
}

Tensor* add(Context* ctx, Tensor* a, Tensor* b) {
    TRC_CHECK(a != nullptr && b != nullptr, "add: input is NULL");
    TRC_CHECK(a->type == b->type, "add: input types differ (%s vs %s)", type_name(a->type), type_name(b->type));
    TRC_CHECK(tensor_are_same_shape(a, b) || tensor_can_repeat(b, a), "add: b does not broadcast to a");
    Tensor* r = new_tensor_nd(ctx, a->type, MAX_DIMS, a->ne);
    r->op = OP_ADD;
    r->src[0] = a;
    r->src[1] = b;
    r->nsrc = 2;
    return r;
}

// src/ops/trc_ops.cpp:59-61 (new_binary :19-32): a's shape, b broadcast to it.
Tensor* mul(Context* ctx, Tensor* a, Tensor* b) {
    TRC_CHECK(a != nullptr && b != nullptr, "mul: input is NULL");
    TRC_CHECK(a->type == b->type, "mul: input types differ (%s vs %s)", type_name(a->type), type_name(b->type));
    TRC_CHECK(tensor_are_same_shape(a, b) || tensor_can_repeat(b, a), "mul: b does not broadcast to a");
    Tensor* r = new_tensor_nd(ctx, a->type, MAX_DIMS, a->ne);
    r->op = OP_MUL;
    r->src[0] = a;
    r->src[1] = b;
    r->nsrc = 2;
    return r;
}

// src/ops/trc_ops.cpp:214-221: a one-element tensor of a's type.
Tensor* sum(Context* ctx, Tensor* a) {
    TRC_CHECK(a != nullptr, "sum: input is NULL");
    Tensor* r = new_tensor_1d(ctx, a->type, 1);
    r->op = OP_SUM;
    r->src[0] = a;
    r->nsrc = 1;
    return r;
}

// src/ops/trc_ops.cpp:447-456: a broadcast (extent-1 dims) to target's shape.
Tensor* repeat(Context* ctx, Tensor* a, Tensor* target) {
    TRC_CHECK(a != nullptr && target != nullptr, "repeat: input is NULL");
    TRC_CHECK(tensor_can_repeat(a, target), "repeat: a does not broadcast to target's shape");
    Tensor* r = new_tensor_nd(ctx, a->type, MAX_DIMS, target->ne);
    r->op = OP_REPEAT;
    r->src[0] = a;
    r->nsrc = 1;
    return r;
}

Tensor* repeat_back(Context* ctx, Tensor* a, Tensor* b) {
    TRC_CHECK(a != nullptr && b != nullptr, "repeat_back: input is NULL");
    for (int i = 0; i < MAX_DIMS; ++i) {
        TRC_CHECK(a->ne[i] % b->ne[i] == 0, "repeat_back: a.ne[%d]=%lld is not a multiple of b.ne[%d]=%lld", i,
                  (long long) a->ne[i], i, (long long) b->ne[i]);
    }
    Tensor* r = new_tensor_nd(ctx, a->type, MAX_DIMS, b->ne);
    r->op = OP_REPEAT_BACK;
    r->src[0] = a;
    r->nsrc = 1;
    return r;
}

Tensor* acc(Context* ctx, Tensor* a, Tensor* b, size_t nb1, size_t nb2, size_t nb3, size_t offset, bool inplace) {
    TRC_CHECK(a != nullptr && b != nullptr, "acc: input is NULL");
    TRC_CHECK(a->type == b->type, "acc: input types differ");
    TRC_CHECK(tensor_is_contiguous(a), "acc: target must be contiguous");
    TRC_CHECK(tensor_is_contiguous(b), "acc: source must be contiguous");
    TRC_CHECK(type_is_supported(a->type), "acc: type %s is not supported", type_name(a->type));
    const size_t nb0 = type_size(a->type);
    size_t last = (size_t) (b->ne[0] - 1) * nb0;
    last += b->ne[1] > 1 ? (size_t) (b->ne[1] - 1) * nb1 : 0;
    last += b->ne[2] > 1 ? (size_t) (b->ne[2] - 1) * nb2 : 0;
    last += b->ne[3] > 1 ? (size_t) (b->ne[3] - 1) * nb3 : 0;
    TRC_CHECK(offset + last + nb0 <= tensor_nbytes(a), "acc: region out of range (offset=%zu last=%zu nbytes=%zu)",
              offset, last, tensor_nbytes(a));
    TRC_CHECK(nb1 <= (size_t) INT32_MAX && nb2 <= (size_t) INT32_MAX && nb3 <= (size_t) INT32_MAX &&
                  offset <= (size_t) INT32_MAX,
              "acc: strides and offset must fit int32");
    Tensor* r = inplace ? make_view(ctx, a, OP_ACC, MAX_DIMS, a->ne, a->nb, 0) : tensor_dup_meta(ctx, a);
    r->op = OP_ACC;
    r->src[0] = a;
    r->src[1] = b;
    r->nsrc = 2;
    const int32_t params[5] = {(int32_t) nb1, (int32_t) nb2, (int32_t) nb3, (int32_t) offset, inplace ? 1 : 0};
    std::memcpy(r->op_params, params, sizeof(params));
    return r;
}

}  // namespace traincpp
