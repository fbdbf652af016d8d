// Operator constructors of the HIP path (graph nodes only). Shape rules follow
// the reference's src/ops/trc_ops.cpp (cont :124-134, cast :136-147,
// mul_mat :366-385) and src/core/trc_tensor.cpp (views :226-320).
#include "impl.h"

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

}  // namespace traincpp
