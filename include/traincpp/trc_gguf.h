// traincpp-compatible GGUF reader (subset of include/traincpp/trc_gguf.h in the
// reference: parsing, metadata/tensor lookup, gguf_tensor_to_f32,
// gguf_load_tensor, gguf_new_tensor, gguf_validate). File format: GGUF v2/v3,
// little-endian; tensor data offsets contiguous and aligned (default 32).
//
// With the HIP backend the legacy quant formats are dequantized on the GPU:
// gguf_load_tensor into an F32 tensor of a HIP buffer uploads the raw blocks
// and dequantizes in place (no host F32 copy); gguf_tensor_to_f32 stages
// through the GPU when one is visible and dequantizes on the host otherwise
// (the same bits either way). The writer side is not part of this backend.
#pragma once

#include "trc_context.h"
#include "trc_tensor.h"
#include "trc_types.h"

#include <cstddef>
#include <cstdint>

namespace traincpp {

enum class GgufType : int32_t {
    U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, BOOL = 7,
    STRING = 8, ARRAY = 9, U64 = 10, I64 = 11, F64 = 12,
};

struct GgufFile;

struct GgufTensorInfo {
    const char* name = nullptr;
    Type        type = TYPE_F32;
    int64_t     ne[MAX_DIMS] = {1, 1, 1, 1};
    size_t      offset = 0;   // relative to the data section
    size_t      nbytes = 0;
};

GgufFile* gguf_open(const char* path, bool load_data = true);
void      gguf_close(GgufFile* f);

int64_t gguf_version(const GgufFile* f);
size_t  gguf_alignment(const GgufFile* f);
size_t  gguf_data_offset(const GgufFile* f);

int64_t     gguf_kv_count(const GgufFile* f);
int64_t     gguf_find_key(const GgufFile* f, const char* key);
const char* gguf_key(const GgufFile* f, int64_t index);
GgufType    gguf_kv_type(const GgufFile* f, int64_t index);
GgufType    gguf_arr_type(const GgufFile* f, int64_t index);
int64_t     gguf_arr_count(const GgufFile* f, int64_t index);
bool        gguf_has_key(const GgufFile* f, const char* key);

// Scalars: a missing key or another type logs an error and returns 0 (nullptr
// for strings). BOOL is one byte on disk.
uint8_t     gguf_get_u8(const GgufFile* f, const char* key);
int8_t      gguf_get_i8(const GgufFile* f, const char* key);
uint16_t    gguf_get_u16(const GgufFile* f, const char* key);
int16_t     gguf_get_i16(const GgufFile* f, const char* key);
uint32_t    gguf_get_u32(const GgufFile* f, const char* key);
int32_t     gguf_get_i32(const GgufFile* f, const char* key);
uint64_t    gguf_get_u64(const GgufFile* f, const char* key);
int64_t     gguf_get_i64(const GgufFile* f, const char* key);
float       gguf_get_f32(const GgufFile* f, const char* key);
bool        gguf_get_bool(const GgufFile* f, const char* key);
double      gguf_get_f64(const GgufFile* f, const char* key);
const char* gguf_get_str(const GgufFile* f, const char* key);

// Arrays: a missing key, another element type or an index out of range logs an
// error and returns nullptr.
const int32_t* gguf_get_arr_i32(const GgufFile* f, const char* key, int64_t* n);
const int64_t* gguf_get_arr_i64(const GgufFile* f, const char* key, int64_t* n);
const float*   gguf_get_arr_f32(const GgufFile* f, const char* key, int64_t* n);
const char*    gguf_get_arr_str(const GgufFile* f, const char* key, int64_t index);

int64_t               gguf_tensor_count(const GgufFile* f);
int64_t               gguf_find_tensor(const GgufFile* f, const char* name);
const GgufTensorInfo* gguf_tensor_info(const GgufFile* f, int64_t index);
int64_t               gguf_tensor_nelements(const GgufFile* f, int64_t index);
// Raw bytes of a tensor's data (nullptr if the file was opened without data).
const uint8_t*        gguf_tensor_data(const GgufFile* f, int64_t index);

bool    gguf_tensor_to_f32(const GgufFile* f, const char* name, float* out, int64_t n_elems);
bool    gguf_load_tensor(const GgufFile* f, const char* name, Tensor* dst);
Tensor* gguf_new_tensor(Context* ctx, const GgufFile* f, const char* name, Type type = TYPE_F32);
bool    gguf_validate(const char* path);

}  // namespace traincpp
