// Type table. Block sizes, block bytes and names are ggml's (the reference
// restates them at src/core/trc_types.cpp:22-48); GGUF files depend on them.
#include "impl.h"

namespace traincpp {

namespace {

struct TypeRow {
    Type        type;
    int64_t     blck;
    size_t      bytes;
    const char* name;
    bool        quant;
};

// Types with a defined layout; everything else reports 0 / "unknown".
constexpr TypeRow kRows[] = {
    {TYPE_F32, 1, 4, "f32", false},     {TYPE_F16, 1, 2, "f16", false},
    {TYPE_Q4_0, 32, 18, "q4_0", true},  {TYPE_Q4_1, 32, 20, "q4_1", true},
    {TYPE_Q5_0, 32, 22, "q5_0", true},  {TYPE_Q5_1, 32, 24, "q5_1", true},
    {TYPE_Q8_0, 32, 34, "q8_0", true},  {TYPE_Q8_1, 32, 36, "q8_1", true},
    {TYPE_Q2_K, 256, 84, "q2_K", true}, {TYPE_Q3_K, 256, 110, "q3_K", true},
    {TYPE_Q4_K, 256, 144, "q4_K", true}, {TYPE_Q5_K, 256, 176, "q5_K", true},
    {TYPE_Q6_K, 256, 210, "q6_K", true}, {TYPE_Q8_K, 256, 292, "q8_K", true},
    {TYPE_I8, 1, 1, "i8", false},       {TYPE_I16, 1, 2, "i16", false},
    {TYPE_I32, 1, 4, "i32", false},     {TYPE_I64, 1, 8, "i64", false},
    {TYPE_F64, 1, 8, "f64", false},     {TYPE_BF16, 1, 2, "bf16", false},
};

const TypeRow* find(Type t) {
    for (const TypeRow& r : kRows) {
        if (r.type == t) return &r;
    }
    return nullptr;
}

}  // namespace

int64_t type_blck_size(Type type) {
    const TypeRow* r = find(type);
    return r ? r->blck : 0;
}

size_t type_size(Type type) {
    const TypeRow* r = find(type);
    return r ? r->bytes : 0;
}

double type_sizef(Type type) {
    const TypeRow* r = find(type);
    return r ? (double) r->bytes / (double) r->blck : 0.0;
}

size_t type_row_size(Type type, int64_t ne) {
    const int64_t blck = type_blck_size(type);
    TRC_CHECK(blck > 0, "type_row_size: type %d has no layout", (int) type);
    TRC_CHECK(ne % blck == 0, "type_row_size: %lld elements are not whole blocks of %lld", (long long) ne,
              (long long) blck);
    return (size_t) (ne / blck) * type_size(type);
}

const char* type_name(Type type) {
    const TypeRow* r = find(type);
    return r ? r->name : "unknown";
}

bool type_is_quantized(Type type) {
    const TypeRow* r = find(type);
    return r != nullptr && r->quant;
}

bool type_is_supported(Type type) {
    switch (type) {
        case TYPE_F32: case TYPE_F16: case TYPE_BF16: case TYPE_F64:
        case TYPE_I8: case TYPE_I16: case TYPE_I32: case TYPE_I64:
            return true;
        default:
            return false;
    }
}

bool type_is_storable(Type type) {
    return type_is_supported(type) || type == TYPE_Q4_0 || type == TYPE_Q4_1 || type == TYPE_Q5_0 ||
           type == TYPE_Q5_1 || type == TYPE_Q8_0;
}

const char* op_name(Op op) {
    static const char* const names[OP_COUNT] = {
        "none", "dup", "cpy", "cont", "reshape", "view", "permute", "transpose", "cast", "concat",
        "repeat", "repeat_back", "pad", "pad_back", "acc", "add", "add1", "sub", "mul", "div",
        "sqr", "sqrt", "log", "exp", "neg", "abs", "sgn", "step", "sin", "cos",
        "clamp", "relu", "leaky_relu", "gelu", "gelu_erf", "erf", "silu", "sigmoid", "tanh", "softplus",
        "hardswish", "scale", "sum", "mean", "sum_rows", "get_rows", "get_rows_back", "set_rows", "mul_mat",
        "out_prod", "norm", "norm_back", "rms_norm", "rms_norm_back", "group_norm", "group_norm_back",
        "soft_max", "cross_entropy_loss", "cross_entropy_loss_back", "im2col", "im2col_back", "col2im",
        "conv_1d", "conv_2d", "conv_transpose_1d", "pool_2d", "pool_2d_back", "conv_transpose_2d",
        "opt_step_adamw", "opt_step_sgd", "sum_sqr_acc", "clip_scale_inplace", "weightnorm_sync",
    };
    return (op >= 0 && op < OP_COUNT) ? names[op] : "unknown";
}

}  // namespace traincpp
