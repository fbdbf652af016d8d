// traincpp-compatible tensor. Interface of include/traincpp/trc_tensor.h in the
// reference: the struct layout and the ggml stride rules are the contract
// every backend reads (nb[0] = type size, nb[1] = nb[0] * ne[0] / block size,
// nb[i] = nb[i-1] * ne[i-1]; data_offset = byte offset inside the owning buffer).
#pragma once

#include "trc_op.h"
#include "trc_types.h"

#include <cstddef>
#include <cstdint>

namespace traincpp {

constexpr int    MAX_DIMS = 4;
constexpr int    MAX_SRC = 10;
constexpr int    MAX_NAME = 64;
constexpr size_t MAX_OP_PARAMS = 64;
constexpr size_t MEM_ALIGN = 16;

struct Context;
class Buffer;
struct Tensor;
struct Graph;

enum TensorFlags : int32_t {
    TENSOR_FLAG_NONE = 0,
    TENSOR_FLAG_INPUT = 1,
    TENSOR_FLAG_OUTPUT = 2,
    TENSOR_FLAG_PARAM = 4,
    TENSOR_FLAG_LOSS = 8,
    TENSOR_FLAG_COMPUTE = 16,
};

struct Tensor {
    Type type = TYPE_F32;
    Buffer* buffer = nullptr;               // owning buffer (set on the view root)
    int64_t ne[MAX_DIMS] = {1, 1, 1, 1};    // elements per dimension
    size_t  nb[MAX_DIMS] = {0, 0, 0, 0};    // strides in bytes
    Op op = OP_NONE;
    int32_t op_params[MAX_OP_PARAMS / sizeof(int32_t)] = {0};
    int32_t flags = 0;
    Tensor* src[MAX_SRC] = {nullptr};
    int32_t nsrc = 0;
    Tensor* view_src = nullptr;
    size_t  view_offs = 0;
    void*   data = nullptr;                 // host pointer, nullptr for device-only buffers
    size_t  data_offset = 0;                // byte offset of element 0 inside the owning buffer
    char    name[MAX_NAME] = {0};
    void*   extra = nullptr;
    Tensor* grad = nullptr;
    Tensor* grad_acc = nullptr;
    Graph*  backward_graph = nullptr;
};

int     tensor_n_dims(const Tensor* t);
int64_t tensor_nelements(const Tensor* t);
int64_t tensor_nrows(const Tensor* t);
size_t  tensor_nbytes(const Tensor* t);
size_t  tensor_element_size(const Tensor* t);
size_t  tensor_row_size(const Tensor* t);
bool    tensor_is_contiguous(const Tensor* t);
bool    tensor_are_same_shape(const Tensor* a, const Tensor* b);
bool    tensor_can_repeat(const Tensor* b, const Tensor* a);
bool    tensor_is_view(const Tensor* t);
size_t  tensor_offset_linear(const Tensor* t, int64_t i);

Tensor* new_tensor_nd(Context* ctx, Type type, int n_dims, const int64_t* ne);
Tensor* new_tensor_1d(Context* ctx, Type type, int64_t ne0);
Tensor* new_tensor_2d(Context* ctx, Type type, int64_t ne0, int64_t ne1);
Tensor* new_tensor_3d(Context* ctx, Type type, int64_t ne0, int64_t ne1, int64_t ne2);
Tensor* new_tensor_4d(Context* ctx, Type type, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3);
Tensor* tensor_dup_meta(Context* ctx, const Tensor* src);
void    tensor_set_name(Tensor* t, const char* fmt, ...);
float*       tensor_data_f32(Tensor* t);
const float* tensor_data_f32(const Tensor* t);

}  // namespace traincpp
