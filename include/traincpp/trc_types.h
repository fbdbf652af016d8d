// traincpp-compatible type table (subset used by the HIP backend path).
//
// Interface of include/traincpp/trc_types.h in the reference (Chui-Las/train.cpp
// v0.4.0): the enum values are ggml's type ids and appear in GGUF files, so they
// must be identical; the functions keep their names, arguments and meaning.
#pragma once

#include <cstddef>
#include <cstdint>

namespace traincpp {

enum Type : int32_t {
    TYPE_F32 = 0,
    TYPE_F16 = 1,
    TYPE_Q4_0 = 2,
    TYPE_Q4_1 = 3,
    TYPE_Q5_0 = 6,
    TYPE_Q5_1 = 7,
    TYPE_Q8_0 = 8,
    TYPE_Q8_1 = 9,
    TYPE_Q2_K = 10,
    TYPE_Q3_K = 11,
    TYPE_Q4_K = 12,
    TYPE_Q5_K = 13,
    TYPE_Q6_K = 14,
    TYPE_Q8_K = 15,
    TYPE_IQ2_XXS = 16,
    TYPE_IQ2_XS = 17,
    TYPE_IQ3_XXS = 18,
    TYPE_IQ1_S = 19,
    TYPE_IQ4_NL = 20,
    TYPE_IQ3_S = 21,
    TYPE_IQ2_S = 22,
    TYPE_IQ4_XS = 23,
    TYPE_I8 = 24,
    TYPE_I16 = 25,
    TYPE_I32 = 26,
    TYPE_I64 = 27,
    TYPE_F64 = 28,
    TYPE_IQ1_M = 29,
    TYPE_BF16 = 30,
    TYPE_TQ1_0 = 34,
    TYPE_TQ2_0 = 35,
    TYPE_MXFP4 = 39,
    TYPE_NVFP4 = 40,
    TYPE_Q1_0 = 41,
    TYPE_Q2_0 = 42,
    TYPE_COUNT = 43,
};

int64_t     type_blck_size(Type type);   // elements per block; 0 if the type has no layout here
size_t      type_size(Type type);        // bytes per block; 0 if the type has no layout here
double      type_sizef(Type type);       // bytes per element
size_t      type_row_size(Type type, int64_t ne);
const char* type_name(Type type);
bool        type_is_quantized(Type type);
// Basic (element-wise) types: F32/F16/BF16/F64/I8/I16/I32/I64, as in the reference.
bool        type_is_supported(Type type);
// Extension: types a tensor may be created with. Basic types plus the five
// legacy quant formats Q4_0/Q4_1/Q5_0/Q5_1/Q8_0, which only the HIP backend
// computes with (mul_mat src0, cast to F32) and GGUF loads copy raw.
bool        type_is_storable(Type type);

}  // namespace traincpp
