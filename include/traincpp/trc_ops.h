// traincpp-compatible operator constructors used on the HIP backend's path
// (subset of include/traincpp/trc_ops.h in the reference: views, cont, cast,
// dup, mul_mat, and the add / mul / sum / repeat / acc / repeat_back nodes of a
// Linear layer's loss and autograd). They only build graph nodes; no
// computation happens here.
#pragma once

#include "trc_context.h"
#include "trc_tensor.h"

namespace traincpp {

Tensor* dup(Context* ctx, const Tensor* a);

Tensor* view_1d(Context* ctx, Tensor* a, int64_t ne0, size_t offset);
Tensor* view_2d(Context* ctx, Tensor* a, int64_t ne0, int64_t ne1, size_t offset);
Tensor* view_3d(Context* ctx, Tensor* a, int64_t ne0, int64_t ne1, int64_t ne2, size_t offset);
Tensor* view_4d(Context* ctx, Tensor* a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, size_t offset);

Tensor* reshape_1d(Context* ctx, Tensor* a, int64_t ne0);
Tensor* reshape_2d(Context* ctx, Tensor* a, int64_t ne0, int64_t ne1);
Tensor* reshape_3d(Context* ctx, Tensor* a, int64_t ne0, int64_t ne1, int64_t ne2);
Tensor* reshape_4d(Context* ctx, Tensor* a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3);

// ne[i] = a.ne[axis_i], nb[i] = a.nb[axis_i] (the reference's convention)
Tensor* permute(Context* ctx, Tensor* a, int axis0, int axis1, int axis2, int axis3);
Tensor* transpose(Context* ctx, Tensor* a);

Tensor* cont(Context* ctx, Tensor* a);
Tensor* cast(Context* ctx, Tensor* a, Type type);

// ggml mul_mat: a [k, m, a2, a3] x b [k, n, b2, b3] -> F32 [m, n, b2, b3], plane
// (i2, i3) uses a's plane (i2 % a2, i3 % a3). Extension: a may be a legacy
// quant type (Q4_0/Q4_1/Q5_0/Q5_1/Q8_0) with b F32; the result is F32.
Tensor* mul_mat(Context* ctx, Tensor* a, Tensor* b);

// a + b with b broadcast to a's shape (each b dim equal to a's or 1); result has a's shape.
Tensor* add(Context* ctx, Tensor* a, Tensor* b);

// a * b with b broadcast to a's shape; result has a's shape.
Tensor* mul(Context* ctx, Tensor* a, Tensor* b);

// Sum of every element of a, as a one-element tensor of a's type.
Tensor* sum(Context* ctx, Tensor* a);

// a broadcast to target's shape (each a dim equal to target's or 1).
Tensor* repeat(Context* ctx, Tensor* a, Tensor* target);

// Sum of a over its repeats back to b's shape (a.ne[i] % b.ne[i] == 0).
Tensor* repeat_back(Context* ctx, Tensor* a, Tensor* b);

// a with b added into the region of a that starts `offset` bytes in and has
// row/plane/batch strides nb1/nb2/nb3 (element stride = the type size). a and
// b contiguous; inplace makes the result a full view of a. op_params hold
// int32 {nb1, nb2, nb3, offset, inplace}.
Tensor* acc(Context* ctx, Tensor* a, Tensor* b, size_t nb1, size_t nb2, size_t nb3, size_t offset, bool inplace);

}  // namespace traincpp
