// MI355X HIP backend for traincpp: Device / BufferType / Buffer over the C ABI
// of libtrc_hip.so (include/trc_hip_abi.h).
//
// It plugs into the reference's backend interface (include/traincpp/trc_backend.h:33-88)
// the way its Vulkan backend does for a non-host device
// (src/backends/vulkan/trc_vulkan.cpp:761-948): buffers are device memory
// (base() == nullptr, tensors addressed as buffer + Tensor::data_offset),
// set_tensor/get_tensor copy synchronously, graph_compute enqueues one kernel
// per node on the null stream and waits once at the end, and any device error
// aborts with a diagnostic. This file uses only the public traincpp API and
// the C ABI, so it compiles against the reference's own headers as well.
#include "traincpp/traincpp.h"
#include "traincpp/trc_hip.h"
#include "trc_hip_abi.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

namespace traincpp {

namespace {

[[noreturn]] void hip_abort(const char* what, int code) {
    std::fflush(stdout);
    std::fprintf(stderr, "[traincpp-hip][FATAL] %s failed (status %d): %s\n", what, code, trc_hip_last_error());
    std::fflush(stderr);
    std::abort();
}

void check(int code, const char* what) {
    if (code != TRC_HIP_OK) hip_abort(what, code);
}

bool legacy_quant(Type t) {
    return t == TYPE_Q4_0 || t == TYPE_Q4_1 || t == TYPE_Q5_0 || t == TYPE_Q5_1 || t == TYPE_Q8_0;
}

size_t elem_size(Type t) {
    switch (t) {
        case TYPE_F32: case TYPE_I32: return 4;
        case TYPE_F16: case TYPE_BF16: case TYPE_I16: return 2;
        case TYPE_I8: return 1;
        case TYPE_F64: case TYPE_I64: return 8;
        default: return 0;
    }
}

bool is_f32(const Tensor* t) { return t != nullptr && t->type == TYPE_F32; }

// op_params of OP_ACC: int32 {nb1, nb2, nb3, offset, inplace} (src/core/trc_tensor.cpp:354-359).
struct AccParams {
    size_t nb1, nb2, nb3, offset;
    bool inplace;
};

AccParams acc_params(const Tensor* t) {
    int32_t p[5];
    std::memcpy(p, t->op_params, sizeof(p));
    return {(size_t) (uint32_t) p[0], (size_t) (uint32_t) p[1], (size_t) (uint32_t) p[2], (size_t) (uint32_t) p[3],
            p[4] != 0};
}

// The acc region lies inside a and no two of its elements share an address
// (the device adds every element of b concurrently).
bool acc_region_ok(const Tensor* a, const Tensor* b, const AccParams& q) {
    const size_t st[4] = {sizeof(float), q.nb1, q.nb2, q.nb3};
    size_t last = 0;
    for (int k = 0; k < 4; ++k) last += (size_t) (b->ne[k] - 1) * st[k];
    if (q.offset + last + sizeof(float) > tensor_nbytes(a)) return false;
    int idx[4] = {0, 1, 2, 3};
    for (int i = 1; i < 4; ++i)
        for (int j = i; j > 0 && st[idx[j]] < st[idx[j - 1]]; --j) std::swap(idx[j], idx[j - 1]);
    size_t span = 0;
    for (int i = 0; i < 4; ++i) {
        const int k = idx[i];
        if (b->ne[k] == 1) continue;
        const size_t covered = span == 0 ? sizeof(float) : span;
        if (st[k] < covered) return false;
        span = st[k] * (size_t) (b->ne[k] - 1) + covered;
    }
    return true;
}

const Tensor* storage_root(const Tensor* t) {
    while (t->buffer == nullptr && t->view_src != nullptr) t = t->view_src;
    return t;
}

class HipDevice;

class HipBufferType final : public BufferType {
public:
    explicit HipBufferType(HipDevice* dev, int ordinal) : dev_(dev), name_("HIP" + std::to_string(ordinal)) {}
    Device* device() const override;
    const char* name() const override { return name_.c_str(); }
    size_t alignment() const override { return 256; }
    Buffer* alloc_buffer(size_t size) override;

private:
    HipDevice* dev_;
    std::string name_;
};

class HipBuffer final : public Buffer {
public:
    HipBuffer(HipBufferType* bt, int ordinal, uint8_t* dev, size_t size)
        : bt_(bt), ordinal_(ordinal), dev_(dev), size_(size) {}
    ~HipBuffer() override {
        trc_hip_init(ordinal_, nullptr);
        trc_hip_free(dev_);
    }
    BufferType* buffer_type() const override { return bt_; }
    size_t size() const override { return size_; }
    void* base() override { return nullptr; }
    bool is_host() const override { return false; }

    void set_tensor(Tensor* t, size_t offset, const void* data, size_t size) override {
        check(trc_hip_init(ordinal_, nullptr), "select device");
        check(trc_hip_h2d(address(t) + offset, data, size, nullptr), "Buffer::set_tensor");
    }
    void get_tensor(const Tensor* t, size_t offset, void* data, size_t size) const override {
        check(trc_hip_init(ordinal_, nullptr), "select device");
        check(trc_hip_d2h(data, address(t) + offset, size, nullptr), "Buffer::get_tensor");
    }
    void clear() override {
        check(trc_hip_init(ordinal_, nullptr), "select device");
        check(trc_hip_memset(dev_, 0, size_, nullptr), "Buffer::clear");
        check(trc_hip_sync(nullptr), "Buffer::clear");
    }

    uint8_t* address(const Tensor* t) const {
        if (t->data_offset + tensor_nbytes(t) > size_) {
            std::fprintf(stderr, "[traincpp-hip][FATAL] tensor %s lies outside its buffer\n", t->name);
            std::abort();
        }
        return dev_ + t->data_offset;
    }
    int ordinal() const { return ordinal_; }

private:
    HipBufferType* bt_;
    int ordinal_;
    uint8_t* dev_;
    size_t size_;
};

HipBuffer* hip_buffer_of(const Tensor* t) {
    return dynamic_cast<HipBuffer*>(storage_root(t)->buffer);
}

trc_hip_tensor describe(const Tensor* t, const HipBuffer* b) {
    trc_hip_tensor d;
    std::memset(&d, 0, sizeof(d));
    d.data = b->address(t);
    d.type = (int32_t) t->type;
    for (int i = 0; i < 4; ++i) {
        d.ne[i] = t->ne[i];
        d.nb[i] = t->nb[i];
    }
    return d;
}

class HipDevice final : public Device {
public:
    explicit HipDevice(int ordinal) : ordinal_(ordinal), buft_(this, ordinal) {
        trc_hip_props p;
        check(trc_hip_init(ordinal, &p), "trc_hip_init");
        props_.name = "HIP" + std::to_string(ordinal);
        props_.description = std::string(p.name) + " (" + p.arch + ", " + std::to_string(p.compute_units) + " CUs)";
        props_.type = DeviceType::GPU;
        props_.memory_free = p.memory_free;
        props_.memory_total = p.memory_total;
        props_.unified_memory = p.unified_memory != 0;
    }

    const DeviceProps& props() const override { return props_; }
    BufferType* default_buffer_type() override { return &buft_; }

    bool supports_op(const Tensor* t) const override {
        const Tensor* a = t->src[0];
        const Tensor* b = t->src[1];
        switch (t->op) {
            case OP_NONE:
            case OP_VIEW:
            case OP_RESHAPE:
            case OP_PERMUTE:
            case OP_TRANSPOSE:
                return true;
            case OP_DUP:
            case OP_CPY:
            case OP_CONT:
                return a != nullptr && a->type == t->type && elem_size(t->type) != 0;
            case OP_CAST:  // dequantization of a legacy quant tensor
                return a != nullptr && legacy_quant(a->type) && t->type == TYPE_F32 && tensor_is_contiguous(a) &&
                       tensor_is_contiguous(t);
            case OP_MUL_MAT: {
                if (a == nullptr || b == nullptr || t->type != TYPE_F32 || b->type != TYPE_F32) return false;
                if (a->ne[0] != b->ne[0] || b->ne[2] % a->ne[2] != 0 || b->ne[3] % a->ne[3] != 0) return false;
                if (a->type == TYPE_F32) return true;
                // quantized src0: whole rows of blocks, activations contiguous along k
                return legacy_quant(a->type) && a->nb[0] == type_size(a->type) && b->nb[0] == sizeof(float) &&
                       t->nb[0] == sizeof(float);
            }
            case OP_ADD:  // compute_binary: b broadcasts where its extent is 1
            case OP_MUL:
                return is_f32(a) && is_f32(b) && is_f32(t) && tensor_are_same_shape(a, t) && tensor_can_repeat(b, a);
            case OP_SUM:
                return is_f32(a) && is_f32(t) && tensor_nelements(t) == 1;
            case OP_REPEAT: {
                if (!is_f32(a) || !is_f32(t)) return false;
                for (int i = 0; i < 4; ++i) {
                    if (t->ne[i] % a->ne[i] != 0) return false;
                }
                return true;
            }
            case OP_ACC: {
                if (!is_f32(a) || !is_f32(b) || !is_f32(t) || !tensor_are_same_shape(a, t)) return false;
                if (!tensor_is_contiguous(a) || !tensor_is_contiguous(t)) return false;
                return acc_region_ok(a, b, acc_params(t));
            }
            case OP_SQR:    // compute_unary(fn_sqr): one float multiply per element
            case OP_SCALE: {  // compute_scale: a * s, s in op_params
                if (!is_f32(a) || !is_f32(t)) return false;
                for (int k = 0; k < MAX_DIMS; ++k)
                    if (a->ne[k] != t->ne[k]) return false;
                return true;
            }
            case OP_REPEAT_BACK: {
                if (!is_f32(a) || !is_f32(t) || !tensor_is_contiguous(t)) return false;
                for (int i = 0; i < 4; ++i) {
                    if (a->ne[i] % t->ne[i] != 0) return false;
                }
                return true;
            }
            default:
                return false;
        }
    }

    bool graph_compute(Graph* graph) override {
        select();
        const std::vector<Tensor*>& nodes = graph->nodes;
        std::vector<char> done(nodes.size(), 0);
        for (size_t i = 0; i < nodes.size(); ++i) {
            if (done[i]) continue;
            if (fuse_gradient_product(nodes, i, done)) continue;
            compute(nodes[i]);
        }
        check(trc_hip_sync(nullptr), "graph_compute");
        return true;
    }

    bool fill_tensors(const TensorFill* fills, size_t count) override {
        select();
        for (size_t i = 0; i < count; ++i) {
            Tensor* t = fills[i].tensor;
            HipBuffer* buf = hip_buffer_of(t);
            if (buf == nullptr || t->type != TYPE_F32 || !tensor_is_contiguous(t)) {
                if (!Device::fill_tensors(&fills[i], 1)) return false;
                continue;
            }
            check(trc_hip_fill_f32((float*) buf->address(t), fills[i].value, tensor_nelements(t), nullptr),
                  "fill_tensors");
        }
        check(trc_hip_sync(nullptr), "fill_tensors");
        return true;
    }

    void select() const { check(trc_hip_init(ordinal_, nullptr), "select device"); }
    int ordinal() const { return ordinal_; }

    // Device scratch for graph computation (src0 planes dequantized for wide
    // right-hand sides): grows on demand and is kept for the next graph, released
    // with the device. GGUF staging uses buffers of its own (StagingBuffer).
    uint8_t* scratch(size_t bytes) {
        if (bytes > scratch_size_) {
            if (scratch_ != nullptr) {
                check(trc_hip_sync(nullptr), "scratch");
                trc_hip_free(scratch_);
                scratch_ = nullptr;
            }
            void* p = nullptr;
            check(trc_hip_malloc(&p, bytes), "scratch allocation");
            scratch_ = (uint8_t*) p;
            scratch_size_ = bytes;
        }
        return scratch_;
    }

private:
    [[noreturn]] void unsupported(const Tensor* t) const {
        std::fflush(stdout);
        std::fprintf(stderr,
                     "[traincpp-hip][FATAL] HIP backend cannot compute node %s (op %s, type %s); check the graph with "
                     "graph_first_unsupported() before graph_compute()\n",
                     t->name, op_name(t->op), type_name(t->type));
        std::abort();
    }

    // Byte range [first, last + 1) a tensor or view covers in its HIP buffer
    // ({0, 0} outside one): every stride counts, so transposed views are covered.
    struct Span {
        uintptr_t lo, hi;
    };
    static Span span_of(const Tensor* t) {
        HipBuffer* b = hip_buffer_of(t);
        if (b == nullptr) return {0, 0};
        const uintptr_t lo = (uintptr_t) b->address(t);
        const int64_t blck = type_blck_size(t->type);
        size_t n = type_size(t->type);
        n += (size_t) ((blck > 0 ? t->ne[0] / blck : t->ne[0]) - 1) * t->nb[0];
        for (int d = 1; d < MAX_DIMS; ++d) n += (size_t) (t->ne[d] - 1) * t->nb[d];
        return {lo, lo + n};
    }
    static bool overlap(Span a, Span b) { return a.lo < b.hi && b.lo < a.hi; }

    // The one node after position `from` that reads t (nullptr if none or more
    // than one), and its position.
    static Tensor* only_reader(const std::vector<Tensor*>& nodes, size_t from, const Tensor* t, size_t* at) {
        Tensor* found = nullptr;
        for (size_t k = from + 1; k < nodes.size(); ++k) {
            for (int s = 0; s < MAX_SRC; ++s) {
                if (nodes[k]->src[s] != t) continue;
                if (found != nullptr && found != nodes[k]) return nullptr;
                found = nodes[k];
                *at = k;
            }
        }
        return found;
    }

    // The chain autograd builds for a matrix operand's gradient
    // (src/core/trc_autograd.cpp:487-503, then grad_accumulate_inplace :58-77):
    //   m = mul_mat(x, y); v = transpose(m) (a view); c = cont(v); acc(G, c, inplace)
    // adds transpose(mul_mat(x, y)) = mul_mat(y, x) into the accumulator G, so it
    // runs as one product added into G (trc_hip_mul_mat_acc_f32): no m, no
    // transposed copy, no separate acc pass. Taken only when m, v and c have no
    // other reader and no output flag, the acc covers all of G, and no node
    // between the product and the acc touches G's bytes, so G receives the same
    // float adds at the same point of its history. TRC_HIP_NO_FUSION=1 turns it
    // off (the chain then runs node by node).
    bool fuse_gradient_product(const std::vector<Tensor*>& nodes, size_t i, std::vector<char>& done) {
        static const bool off = std::getenv("TRC_HIP_NO_FUSION") != nullptr &&
                                std::strcmp(std::getenv("TRC_HIP_NO_FUSION"), "0") != 0;
        Tensor* m = nodes[i];
        if (off || m->op != OP_MUL_MAT) return false;
        Tensor* x = m->src[0];
        Tensor* y = m->src[1];
        if (x->type != TYPE_F32 || y->type != TYPE_F32 || x->ne[2] != y->ne[2] || x->ne[3] != y->ne[3]) return false;
        size_t iv = 0, ic = 0, ia = 0;
        Tensor* v = only_reader(nodes, i, m, &iv);
        // (transpose() is permute(a, 1, 0, 2, 3) in the reference's core)
        if (v == nullptr || (v->op != OP_TRANSPOSE && v->op != OP_PERMUTE) || v->view_src != m ||
            v->view_offs != 0 || v->ne[0] != m->ne[1] ||
            v->ne[1] != m->ne[0] || v->nb[0] != m->nb[1] || v->nb[1] != m->nb[0] || v->ne[2] != m->ne[2] ||
            v->ne[3] != m->ne[3] || v->nb[2] != m->nb[2] || v->nb[3] != m->nb[3])
            return false;
        Tensor* c = only_reader(nodes, iv, v, &ic);
        if (c == nullptr || c->op != OP_CONT || c->src[0] != v || c->type != TYPE_F32 || !tensor_is_contiguous(c))
            return false;
        Tensor* a = only_reader(nodes, ic, c, &ia);
        if (a == nullptr || a->op != OP_ACC || a->src[1] != c) return false;
        Tensor* g = a->src[0];
        const AccParams q = acc_params(a);
        if (!q.inplace || q.offset != 0 || q.nb1 != c->nb[1] || q.nb2 != c->nb[2] || q.nb3 != c->nb[3] ||
            g->type != TYPE_F32 || !tensor_is_contiguous(g))
            return false;
        for (int d = 0; d < MAX_DIMS; ++d)
            if (g->ne[d] != c->ne[d]) return false;
        if ((uint64_t) g->ne[0] * (uint64_t) g->ne[1] * sizeof(float) >= (1ull << 31)) return false;  // one plane <= 2 GiB
        for (const Tensor* t : {m, v, c})
            if (t->flags & (TENSOR_FLAG_OUTPUT | TENSOR_FLAG_LOSS | TENSOR_FLAG_PARAM)) return false;
        const Span gs = span_of(g);
        for (size_t k = i + 1; k < ia; ++k) {
            if (k == iv || k == ic) continue;
            const Tensor* n = nodes[k];
            if (overlap(span_of(n), gs)) return false;
            for (int s = 0; s < MAX_SRC; ++s)
                if (n->src[s] != nullptr && overlap(span_of(n->src[s]), gs)) return false;
        }
        const trc_hip_tensor ty = describe(y, need_buffer(y));
        const trc_hip_tensor tx = describe(x, need_buffer(x));
        const trc_hip_tensor tg = describe(g, need_buffer(g));
        check(trc_hip_mul_mat_acc_f32(&ty, &tx, &tg, nullptr), "mul_mat added into a gradient accumulator");
        done[iv] = done[ic] = done[ia] = 1;
        return true;
    }

    HipBuffer* need_buffer(const Tensor* t) const {
        HipBuffer* b = hip_buffer_of(t);
        if (b == nullptr) {
            std::fprintf(stderr, "[traincpp-hip][FATAL] tensor %s is not in a HIP buffer\n", t->name);
            std::abort();
        }
        return b;
    }

    void compute(Tensor* t) {
        if (!supports_op(t)) unsupported(t);
        switch (t->op) {
            case OP_NONE: case OP_VIEW: case OP_RESHAPE: case OP_PERMUTE: case OP_TRANSPOSE:
                return;
            case OP_DUP: case OP_CPY: case OP_CONT: {
                const trc_hip_tensor s = describe(t->src[0], need_buffer(t->src[0]));
                const trc_hip_tensor d = describe(t, need_buffer(t));
                check(trc_hip_cpy(&s, &d, nullptr), op_name(t->op));
                return;
            }
            case OP_CAST: {
                const Tensor* a = t->src[0];
                check(trc_hip_dequant((int) a->type, need_buffer(a)->address(a), tensor_nelements(a) / 32,
                                      (float*) need_buffer(t)->address(t), nullptr),
                      "cast (dequantize)");
                return;
            }
            case OP_MUL_MAT:
                if (t->src[0]->type == TYPE_F32) {
                    const trc_hip_tensor a = describe(t->src[0], need_buffer(t->src[0]));
                    const trc_hip_tensor b = describe(t->src[1], need_buffer(t->src[1]));
                    const trc_hip_tensor d = describe(t, need_buffer(t));
                    check(trc_hip_mul_mat_f32(&a, &b, &d, nullptr), "mul_mat");
                } else {
                    mul_mat_quant(t);
                }
                return;
            case OP_ADD:
            case OP_MUL: {
                const trc_hip_tensor a = describe(t->src[0], need_buffer(t->src[0]));
                const trc_hip_tensor b = describe(t->src[1], need_buffer(t->src[1]));
                const trc_hip_tensor d = describe(t, need_buffer(t));
                if (t->op == OP_ADD) {
                    check(trc_hip_add_f32(&a, &b, &d, nullptr), "add");
                } else {
                    check(trc_hip_mul_f32(&a, &b, &d, nullptr), "mul");
                }
                return;
            }
            case OP_SUM: {
                const trc_hip_tensor a = describe(t->src[0], need_buffer(t->src[0]));
                const trc_hip_tensor d = describe(t, need_buffer(t));
                check(trc_hip_sum_f32(&a, &d, nullptr), "sum");
                return;
            }
            case OP_REPEAT: {
                const trc_hip_tensor a = describe(t->src[0], need_buffer(t->src[0]));
                const trc_hip_tensor d = describe(t, need_buffer(t));
                check(trc_hip_repeat_f32(&a, &d, nullptr), "repeat");
                return;
            }
            case OP_ACC: {
                const AccParams q = acc_params(t);
                const trc_hip_tensor a = describe(t->src[0], need_buffer(t->src[0]));
                const trc_hip_tensor b = describe(t->src[1], need_buffer(t->src[1]));
                const trc_hip_tensor d = describe(t, need_buffer(t));
                check(trc_hip_acc_f32(&a, &b, &d, q.nb1, q.nb2, q.nb3, q.offset, q.inplace ? 1 : 0, nullptr), "acc");
                return;
            }
            case OP_REPEAT_BACK: {
                const trc_hip_tensor a = describe(t->src[0], need_buffer(t->src[0]));
                const trc_hip_tensor d = describe(t, need_buffer(t));
                check(trc_hip_repeat_back_f32(&a, &d, nullptr), "repeat_back");
                return;
            }
            case OP_SQR: {
                const trc_hip_tensor a = describe(t->src[0], need_buffer(t->src[0]));
                const trc_hip_tensor d = describe(t, need_buffer(t));
                check(trc_hip_sqr_f32(&a, &d, nullptr), "sqr");
                return;
            }
            case OP_SCALE: {
                float sc = 0.f;
                std::memcpy(&sc, t->op_params, sizeof(float));
                const trc_hip_tensor a = describe(t->src[0], need_buffer(t->src[0]));
                const trc_hip_tensor d = describe(t, need_buffer(t));
                check(trc_hip_scale_f32(&a, &d, sc, nullptr), "scale");
                return;
            }
            default:
                unsupported(t);
        }
    }

    // mul_mat with a legacy quant src0: the fused kernel for skinny right-hand
    // sides whose columns meet its alignment (16-byte x columns, 4-byte y
    // columns), otherwise the planes of src0 are dequantized into scratch and
    // the FP32 MFMA kernel, which takes any 4-byte strides, runs on them.
    void mul_mat_quant(Tensor* t) {
        const Tensor* a = t->src[0];
        const Tensor* b = t->src[1];
        uint8_t* pa = need_buffer(a)->address(a);
        uint8_t* pb = need_buffer(b)->address(b);
        uint8_t* pd = need_buffer(t)->address(t);
        const int64_t K = a->ne[0], M = a->ne[1], N = b->ne[1];
        auto aligned = [](const uint8_t* p, const size_t* nb, const int64_t* ne, size_t al) {
            if ((uintptr_t) p % al != 0) return false;
            for (int i = 1; i < 4; ++i) {
                if (ne[i] > 1 && nb[i] % al != 0) return false;
            }
            return true;
        };
        if (N <= TRC_HIP_QMATVEC_MAX_N && aligned(pb, b->nb, b->ne, 16) && aligned(pd, t->nb, t->ne, 4)) {
            for (int64_t i3 = 0; i3 < b->ne[3]; ++i3) {
                for (int64_t i2 = 0; i2 < b->ne[2]; ++i2) {
                    const uint8_t* wa = pa + (i2 % a->ne[2]) * a->nb[2] + (i3 % a->ne[3]) * a->nb[3];
                    const float* xb = (const float*) (pb + i2 * b->nb[2] + i3 * b->nb[3]);
                    float* yd = (float*) (pd + i2 * t->nb[2] + i3 * t->nb[3]);
                    check(trc_hip_qmatvec((int) a->type, wa, K, M, a->nb[1], xb, N, b->nb[1], yd, t->nb[1], nullptr),
                          "mul_mat (fused quantized matvec)");
                }
            }
            return;
        }
        const int64_t planes = a->ne[2] * a->ne[3];
        const size_t plane_f32 = (size_t) (K * M) * sizeof(float);
        float* wf = (float*) scratch(plane_f32 * (size_t) planes);
        const size_t row_bytes = (size_t) (K / 32) * type_size(a->type);
        for (int64_t p3 = 0; p3 < a->ne[3]; ++p3) {
            for (int64_t p2 = 0; p2 < a->ne[2]; ++p2) {
                const uint8_t* src = pa + p2 * a->nb[2] + p3 * a->nb[3];
                float* dst = wf + (p2 + p3 * a->ne[2]) * K * M;
                if (a->nb[1] == row_bytes) {
                    check(trc_hip_dequant((int) a->type, src, K * M / 32, dst, nullptr), "mul_mat (dequantize src0)");
                } else {
                    for (int64_t r = 0; r < M; ++r) {
                        check(trc_hip_dequant((int) a->type, src + r * a->nb[1], K / 32, dst + r * K, nullptr),
                              "mul_mat (dequantize src0)");
                    }
                }
            }
        }
        trc_hip_tensor af;
        std::memset(&af, 0, sizeof(af));
        af.data = wf;
        af.type = TRC_HIP_TYPE_F32;
        const int64_t ne[4] = {K, M, a->ne[2], a->ne[3]};
        size_t nb = sizeof(float);
        for (int i = 0; i < 4; ++i) {
            af.ne[i] = ne[i];
            af.nb[i] = nb;
            nb *= (size_t) ne[i];
        }
        const trc_hip_tensor bd = describe(b, need_buffer(b));
        const trc_hip_tensor dd = describe(t, need_buffer(t));
        check(trc_hip_mul_mat_f32(&af, &bd, &dd, nullptr), "mul_mat (dequantized src0)");
    }

    int ordinal_;
    HipBufferType buft_;
    DeviceProps props_;
    uint8_t* scratch_ = nullptr;
    size_t scratch_size_ = 0;
};

Device* HipBufferType::device() const {
    return dev_;
}

// A new buffer reads as zeros, as the reference's backends guarantee (CpuBuffer
// memsets its allocation, src/backends/cpu/trc_cpu.cpp:26-33; the Vulkan backend
// clears device-local memory, src/backends/vulkan/trc_vulkan.cpp:1079-1084):
// graphs may read a leaf no one has set, such as the result of dup(), which only
// copies metadata (src/ops/trc_ops.cpp:11-14). Out of memory returns nullptr.
Buffer* HipBufferType::alloc_buffer(size_t size) {
    HipDevice* d = dev_;
    d->select();
    const size_t bytes = size == 0 ? 256 : size;
    void* p = nullptr;
    if (trc_hip_malloc(&p, bytes) != TRC_HIP_OK) return nullptr;
    if (trc_hip_memset(p, 0, bytes, nullptr) != TRC_HIP_OK || trc_hip_sync(nullptr) != TRC_HIP_OK) {
        trc_hip_free(p);
        return nullptr;
    }
    return new HipBuffer(this, d->ordinal(), (uint8_t*) p, bytes);
}

std::mutex g_devices_mutex;
std::vector<std::unique_ptr<HipDevice>>& devices() {
    static std::vector<std::unique_ptr<HipDevice>> v;
    return v;
}

}  // namespace

int hip_device_count() {
    int n = 0;
    if (trc_hip_device_count(&n) != TRC_HIP_OK) return 0;
    return n;
}

Device* hip_device(int ordinal) {
    std::lock_guard<std::mutex> lock(g_devices_mutex);
    const int n = hip_device_count();
    if (ordinal < 0 || ordinal >= n) return nullptr;
    auto& v = devices();
    if ((int) v.size() < n) v.resize((size_t) n);
    if (!v[(size_t) ordinal]) v[(size_t) ordinal] = std::make_unique<HipDevice>(ordinal);
    return v[(size_t) ordinal].get();
}

// ---- hooks used by the GGUF reader (core/hip_hooks.h) ----

namespace {
// Device memory for one GGUF staging call, freed when the call returns (after
// its synchronous copies), so loading a large tensor does not leave the device
// scratch that graph computation keeps grown to its size.
struct StagingBuffer {
    void* p = nullptr;
    explicit StagingBuffer(size_t bytes) { check(trc_hip_malloc(&p, bytes), "GGUF staging allocation"); }
    ~StagingBuffer() {
        if (p != nullptr) trc_hip_free(p);
    }
    StagingBuffer(const StagingBuffer&) = delete;
    StagingBuffer& operator=(const StagingBuffer&) = delete;
};
}  // namespace

bool hip_dequant_into(Tensor* dst, Type type, const void* host_blocks, int64_t n_blocks) {
    HipBuffer* buf = hip_buffer_of(dst);
    if (buf == nullptr || !legacy_quant(type) || dst->type != TYPE_F32 || !tensor_is_contiguous(dst) ||
        tensor_nelements(dst) != n_blocks * 32) {
        return false;
    }
    HipDevice* dev = static_cast<HipDevice*>(buf->buffer_type()->device());
    dev->select();
    const size_t raw = (size_t) n_blocks * type_size(type);
    StagingBuffer buf_raw(raw);
    uint8_t* staging = (uint8_t*) buf_raw.p;
    check(trc_hip_h2d(staging, host_blocks, raw, nullptr), "gguf_load_tensor (upload blocks)");
    check(trc_hip_dequant((int) type, staging, n_blocks, (float*) buf->address(dst), nullptr),
          "gguf_load_tensor (dequantize)");
    check(trc_hip_sync(nullptr), "gguf_load_tensor");
    return true;
}

bool hip_gguf_load_tensor(const char* path, const GgufFile* f, const char* name, Tensor* dst) {
    if (path == nullptr || f == nullptr || name == nullptr || dst == nullptr) return false;
    const int64_t idx = gguf_find_tensor(f, name);
    if (idx < 0) {
        std::fprintf(stderr, "[traincpp-hip][ERROR] hip_gguf_load_tensor: no tensor named %s\n", name);
        return false;
    }
    const GgufTensorInfo* info = gguf_tensor_info(f, idx);
    const int64_t n = gguf_tensor_nelements(f, idx);
    if (!legacy_quant(info->type) || dst->type != TYPE_F32 || !tensor_is_contiguous(dst) ||
        tensor_nelements(dst) != n || hip_buffer_of(dst) == nullptr) {
        return false;
    }
    const int64_t n_blocks = n / 32;
    const size_t bytes = (size_t) n_blocks * type_size(info->type);
    const size_t off = gguf_data_offset(f) + info->offset;
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) {
        std::fprintf(stderr, "[traincpp-hip][ERROR] hip_gguf_load_tensor: cannot open %s\n", path);
        return false;
    }
    struct stat st;
    if (::fstat(fd, &st) != 0 || off + bytes > (size_t) st.st_size) {
        ::close(fd);
        std::fprintf(stderr, "[traincpp-hip][ERROR] hip_gguf_load_tensor: %s is shorter than tensor %s needs\n", path,
                     name);
        return false;
    }
    const size_t page = (size_t) ::sysconf(_SC_PAGESIZE);
    const size_t lead = off % page;
    void* m = ::mmap(nullptr, lead + bytes, PROT_READ, MAP_PRIVATE, fd, (off_t) (off - lead));
    ::close(fd);
    if (m == MAP_FAILED) {
        std::fprintf(stderr, "[traincpp-hip][ERROR] hip_gguf_load_tensor: mmap of %s failed\n", path);
        return false;
    }
    ::madvise(m, lead + bytes, MADV_SEQUENTIAL);
    const bool ok = hip_dequant_into(dst, info->type, (const uint8_t*) m + lead, n_blocks);
    ::munmap(m, lead + bytes);
    return ok;
}

bool hip_dequant_host(Type type, const void* host_blocks, int64_t n_blocks, float* out) {
    Device* d = hip_device(0);
    if (d == nullptr) return false;
    HipDevice* dev = static_cast<HipDevice*>(d);
    dev->select();
    const size_t raw = (size_t) n_blocks * type_size(type);
    const size_t raw_aligned = (raw + 255) / 256 * 256;
    StagingBuffer buf(raw_aligned + (size_t) n_blocks * 32 * sizeof(float));
    uint8_t* s = (uint8_t*) buf.p;
    check(trc_hip_h2d(s, host_blocks, raw, nullptr), "gguf_tensor_to_f32 (upload blocks)");
    check(trc_hip_dequant((int) type, s, n_blocks, (float*) (s + raw_aligned), nullptr),
          "gguf_tensor_to_f32 (dequantize)");
    check(trc_hip_d2h(out, s + raw_aligned, (size_t) n_blocks * 32 * sizeof(float), nullptr),
          "gguf_tensor_to_f32 (download)");
    return true;
}

}  // namespace traincpp
