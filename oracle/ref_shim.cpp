// extern "C" shim over the REFERENCE library's public API, compiled together
// with the reference's own sources (under /root/reference, never copied) into
// oracle/_ref/libtrc_ref.so by oracle/Makefile. TEST INFRASTRUCTURE ONLY: it lets
// the CPU tests check the oracle restatement (oracle.cpp) against the code it
// restates, and bench.py's cpu_baseline leg time the reference's own CPU path.
// Nothing in the product loads it.
//
// Entry points go through the same public calls a traincpp user makes:
//   ref_dequant   -> gguf_open + gguf_tensor_to_f32   (src/io/trc_gguf.cpp:748,966)
//   ref_mul_mat   -> permute views + mul_mat + CPU Device::graph_compute
//                    (src/ops/trc_ops.cpp:366, src/backends/cpu/trc_cpu_ops.cpp:182)
//   ref_add       -> permute views + add + CPU Device (src/ops/trc_ops.cpp:46,
//                    src/backends/cpu/trc_cpu_ops.cpp:52)
//   ref_acc       -> acc + CPU Device (src/core/trc_tensor.cpp:322,
//                    src/backends/cpu/trc_cpu_ops.cpp:954)
//   ref_repeat_back -> permute view + repeat_back + CPU Device
//                    (src/ops/trc_ops.cpp:458, src/backends/cpu/trc_cpu_ops.cpp:932)
//   ref_mul / ref_sum / ref_repeat -> permute views + mul / sum / repeat + CPU
//                    Device (src/ops/trc_ops.cpp:59,214,447; trc_cpu_ops.cpp:52,302,913)
//   ref_headline_time -> gguf_open + gguf_tensor_to_f32 into the F32 weight's
//                    CPU buffer, then mul_mat on the CPU Device, repeated and
//                    timed (the CPU path the fused matvec replaces; bench.py's
//                    cpu_baseline leg)
//   ref_dequant_time  -> gguf_tensor_to_f32 alone, repeated and timed
//   ref_mul_mat_time  -> mul_mat on the CPU Device, repeated and timed
//   ref_fp16_*    -> core/trc_float.h:23-63
//   ref_rng_*     -> src/core/trc_rng.cpp:38-68
#include "traincpp/traincpp.h"
#include "core/trc_float.h"

#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

using namespace traincpp;

namespace {

void put(std::vector<uint8_t>& v, const void* p, size_t n) {
    const uint8_t* b = (const uint8_t*) p;
    v.insert(v.end(), b, b + n);
}

template <typename T>
void put_pod(std::vector<uint8_t>& v, T x) {
    put(v, &x, sizeof(x));
}

void pad32(std::vector<uint8_t>& v) {
    while (v.size() % 32 != 0) v.push_back(0);
}

// A one-tensor GGUF v3 file (tensor "w", 1-D, n elements of `type` blocks).
bool write_gguf_w(const char* path, int type, const void* blocks, int64_t n) {
    const size_t bsz = type_size((Type) type);
    std::vector<uint8_t> f;
    put(f, "GGUF", 4);
    put_pod<uint32_t>(f, 3);
    put_pod<uint64_t>(f, 1);  // tensors
    put_pod<uint64_t>(f, 0);  // kvs
    put_pod<uint64_t>(f, 1);
    f.push_back('w');
    put_pod<uint32_t>(f, 1);
    put_pod<int64_t>(f, n);
    put_pod<uint32_t>(f, (uint32_t) type);
    put_pod<uint64_t>(f, 0);
    pad32(f);
    put(f, blocks, bsz * (size_t) (n / 32));
    pad32(f);
    std::FILE* fp = std::fopen(path, "wb");
    if (!fp) return false;
    const bool wrote = std::fwrite(f.data(), 1, f.size(), fp) == f.size();
    std::fclose(fp);
    return wrote;
}

// Runs step() once untimed, then repeatedly for at least budget_s seconds;
// returns the mean seconds per repetition (negative if a step fails).
template <typename F>
double time_steps(F&& step, double budget_s, int* reps_out) {
    if (!step()) return -5.0;
    int reps = 0;
    double el = 0.0;
    const auto t0 = std::chrono::steady_clock::now();
    do {
        if (!step()) return -5.0;
        ++reps;
        el = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    } while (el < budget_s);
    *reps_out = reps;
    return el / reps;
}

}  // namespace

extern "C" {

float ref_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }
uint16_t ref_fp32_to_fp16(float f) { return fp32_to_fp16(f); }

uint64_t ref_rng_next_u64(uint64_t* state) {
    Rng r;
    r.state = *state;
    const uint64_t v = rng_next_u64(&r);
    *state = r.state;
    return v;
}

float ref_rng_uniform01(uint64_t* state) {
    Rng r;
    r.state = *state;
    const float v = rng_uniform01(&r);
    *state = r.state;
    return v;
}

float ref_rng_normal(uint64_t* state, float mean, float stddev) {
    Rng r;
    r.state = *state;
    const float v = rng_normal(&r, mean, stddev);
    *state = r.state;
    return v;
}

// Writes a one-tensor GGUF v3 file (tensor "w", 1-D, ne0 = 32 * n_blocks) holding
// the given raw blocks, then reads it back through the reference reader.
int ref_dequant(int type, const void* blocks, int64_t n_blocks, float* out, const char* tmp_path) {
    const size_t bsz = type_size((Type) type);
    if (bsz == 0 || n_blocks <= 0) return -1;
    std::vector<uint8_t> f;
    put(f, "GGUF", 4);
    put_pod<uint32_t>(f, 3);
    put_pod<uint64_t>(f, 1);  // tensors
    put_pod<uint64_t>(f, 0);  // kvs
    put_pod<uint64_t>(f, 1);
    f.push_back('w');
    put_pod<uint32_t>(f, 1);
    put_pod<int64_t>(f, 32 * n_blocks);
    put_pod<uint32_t>(f, (uint32_t) type);
    put_pod<uint64_t>(f, 0);
    pad32(f);
    put(f, blocks, bsz * (size_t) n_blocks);
    pad32(f);
    std::FILE* fp = std::fopen(tmp_path, "wb");
    if (!fp) return -2;
    const bool wrote = std::fwrite(f.data(), 1, f.size(), fp) == f.size();
    std::fclose(fp);
    if (!wrote) return -2;
    GgufFile* g = gguf_open(tmp_path, true);
    if (!g) return -3;
    const bool ok = gguf_tensor_to_f32(g, "w", out, 32 * n_blocks);
    gguf_close(g);
    std::remove(tmp_path);
    return ok ? 0 : -4;
}

// gguf_tensor_to_f32 of n elements of `type` blocks (a GGUF file written once
// at tmp_path and opened with its data section loaded) into out, repeated and
// timed as time_steps does.
double ref_dequant_time(int type, const void* blocks, int64_t n, float* out, double budget_s, int* reps_out,
                        const char* tmp_path) {
    if (type_size((Type) type) == 0 || n <= 0 || n % 32 != 0) return -1.0;
    if (!write_gguf_w(tmp_path, type, blocks, n)) return -2.0;
    GgufFile* g = gguf_open(tmp_path, true);
    std::remove(tmp_path);
    if (!g) return -3.0;
    const double dt = time_steps([&]() { return gguf_tensor_to_f32(g, "w", out, n); }, budget_s, reps_out);
    gguf_close(g);
    return dt;
}

// y = mul_mat(A, B) on the reference CPU Device, A = F32 [K, M], B = F32 [K, N]
// (contiguous), graph built and buffers allocated once; repeated and timed as
// time_steps does. y gets the [M, N] result.
double ref_mul_mat_time(const float* a, int64_t K, int64_t M, const float* b, int64_t N, float* y, double budget_s,
                        int* reps_out) {
    Device* dev = device_cpu();
    if (!dev) return -4.0;
    Context* ctx = context_new(1 << 20);
    Tensor* ta = new_tensor_2d(ctx, TYPE_F32, K, M);
    Tensor* tb = new_tensor_2d(ctx, TYPE_F32, K, N);
    Tensor* r = mul_mat(ctx, ta, tb);
    Graph* gr = graph_new(ctx);
    graph_build_forward_expand(ctx, gr, r);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    tensor_set(ta, a, 0, tensor_nbytes(ta));
    tensor_set(tb, b, 0, tensor_nbytes(tb));
    const double dt = time_steps([&]() { return dev->graph_compute(gr); }, budget_s, reps_out);
    if (dt > 0) tensor_get(r, y, 0, tensor_nbytes(r));
    buffer_free(buf);
    graph_free(gr);
    context_free(ctx);
    return dt;
}

// The headline workload on the reference's CPU path: W (n = K*M elements of
// `type` blocks, written once to a GGUF v3 file at tmp_path and opened with its
// data section loaded) is dequantized by gguf_tensor_to_f32 straight into the
// CPU buffer of an F32 tensor [K, M], and y = mul_mat(W, x) runs on the CPU
// Device (graph built and buffers allocated once). After one untimed pass the
// two steps repeat for at least budget_s seconds. Returns the mean seconds per
// repetition (negative on an error), y (M floats) and the repetition count.
double ref_headline_time(int type, const void* blocks, int64_t K, int64_t M, const float* x, float* y,
                         double budget_s, int* reps_out, const char* tmp_path) {
    const int64_t n = K * M;
    if (type_size((Type) type) == 0 || n <= 0 || n % 32 != 0) return -1.0;
    if (!write_gguf_w(tmp_path, type, blocks, n)) return -2.0;
    GgufFile* g = gguf_open(tmp_path, true);
    std::remove(tmp_path);
    if (!g) return -3.0;
    Device* dev = device_cpu();
    if (!dev) {
        gguf_close(g);
        return -4.0;
    }
    Context* ctx = context_new(1 << 20);
    Tensor* w = new_tensor_2d(ctx, TYPE_F32, K, M);
    Tensor* xt = new_tensor_2d(ctx, TYPE_F32, K, 1);
    Tensor* r = mul_mat(ctx, w, xt);
    Graph* gr = graph_new(ctx);
    graph_build_forward_expand(ctx, gr, r);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    tensor_set(xt, x, 0, tensor_nbytes(xt));
    double dt = -6.0;  // the F32 weight has no host-visible buffer
    if (w->data != nullptr) {
        dt = time_steps([&]() { return gguf_tensor_to_f32(g, "w", (float*) w->data, n) && dev->graph_compute(gr); },
                        budget_s, reps_out);
        if (dt > 0) tensor_get(r, y, 0, tensor_nbytes(r));
    }
    buffer_free(buf);
    graph_free(gr);
    context_free(ctx);
    gguf_close(g);
    return dt;
}

// d = mul_mat(permute(A, pa), permute(B, pb)) on the reference CPU device.
// A and B are contiguous F32 base tensors of shape a_ne / b_ne (ggml order);
// pa / pb are the permute() axes. The result is copied out contiguously
// (its shape is [A'.ne1, B'.ne1, B'.ne2, B'.ne3] for the permuted A', B').
int ref_mul_mat(const float* a, const int64_t a_ne[4], const int pa[4],
                const float* b, const int64_t b_ne[4], const int pb[4], float* out) {
    Device* dev = device_cpu();
    if (!dev) return -1;
    Context* ctx = context_new(1 << 20);
    Tensor* ta = new_tensor_4d(ctx, TYPE_F32, a_ne[0], a_ne[1], a_ne[2], a_ne[3]);
    Tensor* tb = new_tensor_4d(ctx, TYPE_F32, b_ne[0], b_ne[1], b_ne[2], b_ne[3]);
    Tensor* va = permute(ctx, ta, pa[0], pa[1], pa[2], pa[3]);
    Tensor* vb = permute(ctx, tb, pb[0], pb[1], pb[2], pb[3]);
    Tensor* r = mul_mat(ctx, va, vb);
    Graph* g = graph_new(ctx);
    graph_build_forward_expand(ctx, g, r);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    tensor_set(ta, a, 0, tensor_nbytes(ta));
    tensor_set(tb, b, 0, tensor_nbytes(tb));
    const bool ok = dev->graph_compute(g);
    tensor_get(r, out, 0, tensor_nbytes(r));
    buffer_free(buf);
    graph_free(g);
    context_free(ctx);
    return ok ? 0 : -2;
}

// a (permuted view of base a_ne) + b (permuted view of base b_ne); out gets a's
// (viewed) shape, contiguous.
int ref_add(const float* a, const int64_t a_ne[4], const int pa[4], const float* b, const int64_t b_ne[4],
            const int pb[4], float* out) {
    Device* dev = device_cpu();
    if (!dev) return -1;
    Context* ctx = context_new(1 << 20);
    Tensor* ta = new_tensor_4d(ctx, TYPE_F32, a_ne[0], a_ne[1], a_ne[2], a_ne[3]);
    Tensor* tb = new_tensor_4d(ctx, TYPE_F32, b_ne[0], b_ne[1], b_ne[2], b_ne[3]);
    Tensor* r = add(ctx, permute(ctx, ta, pa[0], pa[1], pa[2], pa[3]), permute(ctx, tb, pb[0], pb[1], pb[2], pb[3]));
    Graph* g = graph_new(ctx);
    graph_build_forward_expand(ctx, g, r);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    tensor_set(ta, a, 0, tensor_nbytes(ta));
    tensor_set(tb, b, 0, tensor_nbytes(tb));
    const bool ok = dev->graph_compute(g);
    tensor_get(r, out, 0, tensor_nbytes(r));
    buffer_free(buf);
    graph_free(g);
    context_free(ctx);
    return ok ? 0 : -2;
}

// acc(a, b, nb1, nb2, nb3, offset, inplace) with contiguous a and b; out gets the
// result (a's shape).
int ref_acc(const float* a, const int64_t a_ne[4], const float* b, const int64_t b_ne[4], size_t nb1, size_t nb2,
            size_t nb3, size_t offset, int inplace, float* out) {
    Device* dev = device_cpu();
    if (!dev) return -1;
    Context* ctx = context_new(1 << 20);
    Tensor* ta = new_tensor_4d(ctx, TYPE_F32, a_ne[0], a_ne[1], a_ne[2], a_ne[3]);
    Tensor* tb = new_tensor_4d(ctx, TYPE_F32, b_ne[0], b_ne[1], b_ne[2], b_ne[3]);
    Tensor* r = acc(ctx, ta, tb, nb1, nb2, nb3, offset, inplace != 0);
    Graph* g = graph_new(ctx);
    graph_build_forward_expand(ctx, g, r);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    tensor_set(ta, a, 0, tensor_nbytes(ta));
    tensor_set(tb, b, 0, tensor_nbytes(tb));
    const bool ok = dev->graph_compute(g);
    tensor_get(r, out, 0, tensor_nbytes(r));
    buffer_free(buf);
    graph_free(g);
    context_free(ctx);
    return ok ? 0 : -2;
}

// repeat_back(permute(a), b-shape d_ne); out contiguous with d_ne.
int ref_repeat_back(const float* a, const int64_t a_ne[4], const int pa[4], const int64_t d_ne[4], float* out) {
    Device* dev = device_cpu();
    if (!dev) return -1;
    Context* ctx = context_new(1 << 20);
    Tensor* ta = new_tensor_4d(ctx, TYPE_F32, a_ne[0], a_ne[1], a_ne[2], a_ne[3]);
    Tensor* shape = new_tensor_4d(ctx, TYPE_F32, d_ne[0], d_ne[1], d_ne[2], d_ne[3]);
    Tensor* r = repeat_back(ctx, permute(ctx, ta, pa[0], pa[1], pa[2], pa[3]), shape);
    Graph* g = graph_new(ctx);
    graph_build_forward_expand(ctx, g, r);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    tensor_set(ta, a, 0, tensor_nbytes(ta));
    const bool ok = dev->graph_compute(g);
    tensor_get(r, out, 0, tensor_nbytes(r));
    buffer_free(buf);
    graph_free(g);
    context_free(ctx);
    return ok ? 0 : -2;
}

// mul(permute(a), permute(b)); out gets a's (viewed) shape, contiguous.
int ref_mul(const float* a, const int64_t a_ne[4], const int pa[4], const float* b, const int64_t b_ne[4],
            const int pb[4], float* out) {
    Device* dev = device_cpu();
    if (!dev) return -1;
    Context* ctx = context_new(1 << 20);
    Tensor* ta = new_tensor_4d(ctx, TYPE_F32, a_ne[0], a_ne[1], a_ne[2], a_ne[3]);
    Tensor* tb = new_tensor_4d(ctx, TYPE_F32, b_ne[0], b_ne[1], b_ne[2], b_ne[3]);
    Tensor* r = mul(ctx, permute(ctx, ta, pa[0], pa[1], pa[2], pa[3]), permute(ctx, tb, pb[0], pb[1], pb[2], pb[3]));
    Graph* g = graph_new(ctx);
    graph_build_forward_expand(ctx, g, r);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    tensor_set(ta, a, 0, tensor_nbytes(ta));
    tensor_set(tb, b, 0, tensor_nbytes(tb));
    const bool ok = dev->graph_compute(g);
    tensor_get(r, out, 0, tensor_nbytes(r));
    buffer_free(buf);
    graph_free(g);
    context_free(ctx);
    return ok ? 0 : -2;
}

// sum(permute(a)) into *out.
int ref_sum(const float* a, const int64_t a_ne[4], const int pa[4], float* out) {
    Device* dev = device_cpu();
    if (!dev) return -1;
    Context* ctx = context_new(1 << 20);
    Tensor* ta = new_tensor_4d(ctx, TYPE_F32, a_ne[0], a_ne[1], a_ne[2], a_ne[3]);
    Tensor* r = sum(ctx, permute(ctx, ta, pa[0], pa[1], pa[2], pa[3]));
    Graph* g = graph_new(ctx);
    graph_build_forward_expand(ctx, g, r);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    tensor_set(ta, a, 0, tensor_nbytes(ta));
    const bool ok = dev->graph_compute(g);
    tensor_get(r, out, 0, sizeof(float));
    buffer_free(buf);
    graph_free(g);
    context_free(ctx);
    return ok ? 0 : -2;
}

// repeat(permute(a), target of shape d_ne); out contiguous with d_ne.
int ref_repeat(const float* a, const int64_t a_ne[4], const int pa[4], const int64_t d_ne[4], float* out) {
    Device* dev = device_cpu();
    if (!dev) return -1;
    Context* ctx = context_new(1 << 20);
    Tensor* ta = new_tensor_4d(ctx, TYPE_F32, a_ne[0], a_ne[1], a_ne[2], a_ne[3]);
    Tensor* target = new_tensor_4d(ctx, TYPE_F32, d_ne[0], d_ne[1], d_ne[2], d_ne[3]);
    Tensor* r = repeat(ctx, permute(ctx, ta, pa[0], pa[1], pa[2], pa[3]), target);
    Graph* g = graph_new(ctx);
    graph_build_forward_expand(ctx, g, r);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    tensor_set(ta, a, 0, tensor_nbytes(ta));
    const bool ok = dev->graph_compute(g);
    tensor_get(r, out, 0, tensor_nbytes(r));
    buffer_free(buf);
    graph_free(g);
    context_free(ctx);
    return ok ? 0 : -2;
}

// sqr(permute(a)) (sq != 0) or scale(permute(a), s) on the reference CPU device;
// out contiguous with the permuted shape.
int ref_unary(const float* a, const int64_t a_ne[4], const int pa[4], int sq, float s, float* out) {
    Device* dev = device_cpu();
    if (!dev) return -1;
    Context* ctx = context_new(1 << 20);
    Tensor* ta = new_tensor_4d(ctx, TYPE_F32, a_ne[0], a_ne[1], a_ne[2], a_ne[3]);
    Tensor* va = permute(ctx, ta, pa[0], pa[1], pa[2], pa[3]);
    Tensor* r = sq ? sqr(ctx, va) : scale(ctx, va, s);
    Graph* g = graph_new(ctx);
    graph_build_forward_expand(ctx, g, r);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    tensor_set(ta, a, 0, tensor_nbytes(ta));
    const bool ok = dev->graph_compute(g);
    tensor_get(r, out, 0, tensor_nbytes(r));
    buffer_free(buf);
    graph_free(g);
    context_free(ctx);
    return ok ? 0 : -2;
}

}  // extern "C"
