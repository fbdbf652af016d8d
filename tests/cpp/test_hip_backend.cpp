// Drop-in tests of the HIP backend through the traincpp API (libtraincpp_hip.so),
// modelled on the reference's backend conformance suite
// (tests/test_backend_conformance.cpp:43-135, 455-553, 928-934) and its GGUF
// tests (tests/test_gguf.cpp). Expected values come from the CPU oracle
// (oracle/liboracle.so), which restates the reference CPU path.
//
//   test_hip_backend            all cases (needs a HIP device)
//   test_hip_backend --cpu      only the cases that need no device
//   test_hip_backend --abort-shape   builds an invalid mul_mat (must abort)
#include "traincpp/traincpp.h"
#include "oracle.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <utility>
#include <vector>

using namespace traincpp;

namespace {

int g_failures = 0;

#define EXPECT(cond)                                                                  \
    do {                                                                              \
        if (!(cond)) {                                                                \
            std::printf("    FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond);          \
            ++g_failures;                                                             \
        }                                                                             \
    } while (0)

std::vector<float> ramp(size_t n) {  // tests/test_backend_conformance.cpp:130-135
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = (float) ((int) (i % 17) - 8) * 0.25f;
    return v;
}

std::vector<float> normal(size_t n, uint64_t seed, float stddev = 1.0f) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) {
        uint64_t s = seed + i;
        v[i] = orc_rng_normal(&s, 0.0f, stddev);
    }
    return v;
}

// max over dst rows of max|got - want| / ||want_row||_2
double row_l2_error(const std::vector<float>& got, const std::vector<float>& want, int64_t row) {
    double worst = 0;
    for (size_t r0 = 0; r0 < want.size(); r0 += (size_t) row) {
        double n2 = 0, mx = 0;
        for (int64_t i = 0; i < row; ++i) {
            n2 += (double) want[r0 + i] * want[r0 + i];
            mx = std::fmax(mx, std::fabs((double) got[r0 + i] - want[r0 + i]));
        }
        worst = std::fmax(worst, mx / std::fmax(std::sqrt(n2), 1e-30));
    }
    return worst;
}

// Host copies of the inputs of a graph, to rebuild any view's host pointer.
struct HostInputs {
    std::vector<std::pair<Tensor*, std::vector<float>>> f32;
    const float* host_of(const Tensor* view) const {
        const Tensor* root = view;
        while (root->view_src) root = root->view_src;
        for (const auto& p : f32) {
            if (p.first == root) return (const float*) ((const uint8_t*) p.second.data() + (view->data_offset - root->data_offset));
        }
        return nullptr;
    }
};

std::vector<float> oracle_mul_mat(const HostInputs& in, const Tensor* a, const Tensor* b) {
    const int64_t dne[4] = {a->ne[1], b->ne[1], b->ne[2], b->ne[3]};
    const size_t dnb[4] = {4, (size_t) (4 * dne[0]), (size_t) (4 * dne[0] * dne[1]), (size_t) (4 * dne[0] * dne[1] * dne[2])};
    std::vector<float> out((size_t) (dne[0] * dne[1] * dne[2] * dne[3]));
    const int rc = orc_mul_mat(in.host_of(a), a->ne, a->nb, in.host_of(b), b->ne, b->nb, out.data(), dne, dnb, 8);
    EXPECT(rc == 0);
    return out;
}

struct Built {
    Tensor* out = nullptr;
    HostInputs inputs;
};

using BuildFn = std::function<Built(Context*)>;

// Runs a graph on `dev` and returns its output (and the built graph's inputs).
std::vector<float> run_on(Device* dev, const BuildFn& build, Built* keep, const Tensor** first_bad = nullptr) {
    Context* ctx = context_new(1 << 20);
    Graph* g = graph_new(ctx);
    Built b = build(ctx);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    EXPECT(buf != nullptr && buf->base() == nullptr && !buf->is_host());
    for (auto& in : b.inputs.f32) tensor_set(in.first, in.second.data(), 0, in.second.size() * sizeof(float));
    graph_build_forward_expand(ctx, g, b.out);
    std::vector<float> out;
    const Tensor* bad = graph_first_unsupported(g, dev);
    if (first_bad) *first_bad = bad;
    if (bad == nullptr) {
        EXPECT(dev->graph_compute(g));
        out.resize((size_t) tensor_nelements(b.out));
        tensor_get(b.out, out.data(), 0, out.size() * sizeof(float));
    }
    if (keep) {
        // keep the mul_mat node's source views valid for the oracle: recompute here
        *keep = b;
        keep->out = nullptr;
    }
    // oracle on the same views, before the context is released
    if (keep && b.out->op == OP_MUL_MAT) {
        std::vector<float> want = oracle_mul_mat(b.inputs, b.out->src[0], b.out->src[1]);
        keep->inputs.f32.push_back({nullptr, std::move(want)});
    }
    buffer_free(buf);
    graph_free(g);
    context_free(ctx);
    return out;
}

void check_mul_mat_case(Device* dev, const char* name, const BuildFn& build) {
    Built kept;
    const std::vector<float> got = run_on(dev, build, &kept);
    const std::vector<float>& want = kept.inputs.f32.back().second;
    EXPECT(got.size() == want.size());
    if (got.size() != want.size()) return;
    int64_t bad = 0;
    double max_abs = 0;
    for (size_t i = 0; i < want.size(); ++i) {
        const double d = std::fabs((double) got[i] - want[i]);
        max_abs = std::fmax(max_abs, d);
        if (d > 1e-5 + 2e-4 * std::fabs((double) want[i])) ++bad;  // test_backend_conformance.cpp:107
    }
    EXPECT(bad == 0);
    std::printf("    [%s] %-28s max_abs=%.3g\n", bad == 0 ? " OK " : "FAIL", name, max_abs);
}

Tensor* input(Built& b, Tensor* t, std::vector<float> v) {
    b.inputs.f32.push_back({t, std::move(v)});
    return t;
}

// ---------------------------------------------------------------- device cases

void test_registry(Device* dev) {
    std::printf("registry\n");
    EXPECT(device_count() >= 1);
    EXPECT(device_by_type(DeviceType::GPU) == dev);
    EXPECT(device_cpu() == nullptr);
    EXPECT(hip_device(hip_device_count()) == nullptr);
    const DeviceProps& p = dev->props();
    EXPECT(p.type == DeviceType::GPU && p.memory_total > 0);
    std::printf("    %s: %s, %.1f GiB\n", p.name.c_str(), p.description.c_str(), p.memory_total / 1073741824.0);
    EXPECT(dev->default_buffer_type()->alignment() >= 16);
    EXPECT(dev->default_buffer_type()->alloc_buffer((size_t) 1 << 52) == nullptr);  // 4 PiB: refused, no abort
}

void test_conformance_mul_mat(Device* dev) {
    std::printf("conformance mul_mat (tests/test_backend_conformance.cpp:455-553,928-934)\n");
    check_mul_mat_case(dev, "mul_mat_basic", [](Context* ctx) {
        Built b;
        Tensor* x = input(b, new_tensor_2d(ctx, TYPE_F32, 5, 3), ramp(15));
        Tensor* y = input(b, new_tensor_2d(ctx, TYPE_F32, 5, 4), ramp(20));
        b.out = mul_mat(ctx, x, y);
        return b;
    });
    check_mul_mat_case(dev, "mul_mat_transposed_a", [](Context* ctx) {
        Built b;
        Tensor* base = input(b, new_tensor_2d(ctx, TYPE_F32, 3, 5), ramp(15));
        Tensor* y = input(b, new_tensor_2d(ctx, TYPE_F32, 5, 4), ramp(20));
        b.out = mul_mat(ctx, transpose(ctx, base), y);
        return b;
    });
    check_mul_mat_case(dev, "mul_mat_transposed_b", [](Context* ctx) {
        Built b;
        Tensor* x = input(b, new_tensor_2d(ctx, TYPE_F32, 5, 3), ramp(15));
        Tensor* base = input(b, new_tensor_2d(ctx, TYPE_F32, 4, 5), ramp(20));
        b.out = mul_mat(ctx, x, transpose(ctx, base));
        return b;
    });
    check_mul_mat_case(dev, "mul_mat_tile_boundary", [](Context* ctx) {
        Built b;
        Tensor* x = input(b, new_tensor_2d(ctx, TYPE_F32, 33, 70), ramp(33 * 70));
        Tensor* y = input(b, new_tensor_2d(ctx, TYPE_F32, 33, 66), ramp(33 * 66));
        b.out = mul_mat(ctx, x, y);
        return b;
    });
    check_mul_mat_case(dev, "mul_mat_batch", [](Context* ctx) {
        Built b;
        Tensor* x = input(b, new_tensor_4d(ctx, TYPE_F32, 5, 3, 1, 1), ramp(15));
        Tensor* y = input(b, new_tensor_4d(ctx, TYPE_F32, 5, 4, 2, 3), ramp(5 * 4 * 6));
        b.out = mul_mat(ctx, x, y);
        return b;
    });
    check_mul_mat_case(dev, "mul_mat_batch_bcast_div", [](Context* ctx) {
        Built b;
        Tensor* x = input(b, new_tensor_4d(ctx, TYPE_F32, 5, 3, 2, 1), ramp(30));
        Tensor* y = input(b, new_tensor_4d(ctx, TYPE_F32, 5, 4, 4, 1), ramp(80));
        b.out = mul_mat(ctx, x, y);
        return b;
    });
    check_mul_mat_case(dev, "mul_mat_batch_transposed", [](Context* ctx) {
        Built b;
        Tensor* xa = input(b, new_tensor_4d(ctx, TYPE_F32, 3, 5, 2, 2), ramp(60));
        Tensor* xb = input(b, new_tensor_4d(ctx, TYPE_F32, 4, 5, 2, 2), ramp(80));
        b.out = mul_mat(ctx, transpose(ctx, xa), transpose(ctx, xb));
        return b;
    });
    check_mul_mat_case(dev, "mul_mat_batch_tile_boundary", [](Context* ctx) {
        Built b;
        Tensor* x = input(b, new_tensor_4d(ctx, TYPE_F32, 33, 70, 1, 1), ramp(33 * 70));
        Tensor* y = input(b, new_tensor_4d(ctx, TYPE_F32, 33, 66, 2, 2), ramp(33 * 66 * 4));
        b.out = mul_mat(ctx, x, y);
        return b;
    });
    check_mul_mat_case(dev, "grid_mul_mat_batch_z", [](Context* ctx) {
        Built b;
        Tensor* x = input(b, new_tensor_4d(ctx, TYPE_F32, 8, 4, 1, 1), ramp(32));
        Tensor* y = input(b, new_tensor_4d(ctx, TYPE_F32, 8, 4, 65, 1), ramp(8 * 4 * 65));
        b.out = mul_mat(ctx, x, y);
        return b;
    });
    check_mul_mat_case(dev, "permuted_src1_broadcast", [](Context* ctx) {  // configuration 4 in miniature
        Built b;
        Tensor* x = input(b, new_tensor_4d(ctx, TYPE_F32, 32, 40, 2, 2), normal(32 * 40 * 4, 11));
        Tensor* base = input(b, new_tensor_4d(ctx, TYPE_F32, 32, 6, 24, 2), normal(32 * 6 * 24 * 2, 12));
        b.out = mul_mat(ctx, x, permute(ctx, base, 0, 2, 1, 3));
        return b;
    });
}

// Linear layer y = W x and the two products autograd emits for it
// (src/core/trc_autograd.cpp:487-503), with the transposed dW materialised by cont.
void test_linear_backward(Device* dev) {
    std::printf("linear layer forward + backward compositions\n");
    const int64_t K = 256, M = 192, T = 64;
    const std::vector<float> W = normal((size_t) (K * M), 1), X = normal((size_t) (K * T), 2),
                             dY = normal((size_t) (M * T), 3, 1e-2f);
    Context* ctx = context_new(1 << 20);
    Tensor* w = new_tensor_2d(ctx, TYPE_F32, K, M);
    Tensor* x = new_tensor_2d(ctx, TYPE_F32, K, T);
    Tensor* dy = new_tensor_2d(ctx, TYPE_F32, M, T);
    Tensor* y = mul_mat(ctx, w, x);
    Tensor* dx = mul_mat(ctx, transpose(ctx, w), dy);
    Tensor* dwt = mul_mat(ctx, transpose(ctx, dy), transpose(ctx, x));  // [M, K] = dW^T
    Tensor* dw = cont(ctx, transpose(ctx, dwt));                       // [K, M] like W
    Graph* g = graph_new(ctx);
    graph_build_forward_expand(ctx, g, y);
    graph_build_forward_expand(ctx, g, dx);
    graph_build_forward_expand(ctx, g, dw);
    EXPECT(graph_first_unsupported(g, dev) == nullptr);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    tensor_set(w, W.data(), 0, W.size() * 4);
    tensor_set(x, X.data(), 0, X.size() * 4);
    tensor_set(dy, dY.data(), 0, dY.size() * 4);
    EXPECT(dev->graph_compute(g));
    std::vector<float> gy((size_t) (M * T)), gdx((size_t) (K * T)), gdw((size_t) (K * M));
    tensor_get(y, gy.data(), 0, gy.size() * 4);
    tensor_get(dx, gdx.data(), 0, gdx.size() * 4);
    tensor_get(dw, gdw.data(), 0, gdw.size() * 4);
    // oracle: same views on host
    HostInputs in;
    in.f32 = {{w, W}, {x, X}, {dy, dY}};
    const std::vector<float> wy = oracle_mul_mat(in, y->src[0], y->src[1]);
    const std::vector<float> wdx = oracle_mul_mat(in, dx->src[0], dx->src[1]);
    const std::vector<float> wdwt = oracle_mul_mat(in, dwt->src[0], dwt->src[1]);
    std::vector<float> wdw((size_t) (K * M));
    for (int64_t m = 0; m < M; ++m)
        for (int64_t k = 0; k < K; ++k) wdw[(size_t) (m * K + k)] = wdwt[(size_t) (k * M + m)];
    const double ey = row_l2_error(gy, wy, M), edx = row_l2_error(gdx, wdx, K), edw = row_l2_error(gdw, wdw, K);
    EXPECT(ey <= 1e-4 && edx <= 1e-4 && edw <= 1e-4);
    std::printf("    [%s] y err %.2e, dX err %.2e, dW (cont of transposed product) err %.2e\n",
                (ey <= 1e-4 && edx <= 1e-4 && edw <= 1e-4) ? " OK " : "FAIL", ey, edx, edw);
    buffer_free(buf);
    graph_free(g);
    context_free(ctx);
}

// A Linear layer with bias whose weight is a view of a larger parameter and is
// broadcast over the activations' planes, forward and backward, with the
// backward nodes built exactly as the reference's autograd emits them for
// parameters with gradient accumulators (src/core/trc_autograd.cpp):
//   ADD   :220-227  dbias = repeat_back(G, bias)
//   MULMAT:487-503  dW = repeat_back(transpose(mul_mat(transpose(G), transpose(x))), W), dx = mul_mat(transpose(W), G)
//   VIEW  :191-195, :136-143 and :58-75  acc(P_acc, dW, W.nb1, W.nb2, W.nb3, W.view_offs, inplace)
// The element-wise nodes are checked bit for bit against the oracle applied to
// the device's own inputs to them; the products within the mul_mat bar.
void test_autograd_linear_bias(Device* dev) {
    std::printf("linear + bias autograd compositions (add / repeat_back / acc on the device)\n");
    const int64_t K = 96, M = 80, T = 24, B2 = 4, A2 = 2, P2 = 3;
    Context* ctx = context_new(1 << 20);
    Tensor* P = new_tensor_4d(ctx, TYPE_F32, K, M, P2, 1);      // parameter holding W in planes 1..2
    Tensor* Pacc = new_tensor_4d(ctx, TYPE_F32, K, M, P2, 1);   // its gradient accumulator
    Tensor* bias = new_tensor_4d(ctx, TYPE_F32, M, 1, 1, 1);
    Tensor* bacc = new_tensor_4d(ctx, TYPE_F32, M, 1, 1, 1);
    Tensor* x = new_tensor_4d(ctx, TYPE_F32, K, T, B2, 1);
    Tensor* G = new_tensor_4d(ctx, TYPE_F32, M, T, B2, 1);      // upstream gradient of y
    Tensor* W = view_4d(ctx, P, K, M, A2, 1, (size_t) P->nb[2]);
    Tensor* h = mul_mat(ctx, W, x);                             // [M, T, B2]
    Tensor* y = add(ctx, h, bias);
    Tensor* dbias = repeat_back(ctx, G, bias);
    Tensor* bacc_node = acc(ctx, bacc, dbias, dbias->nb[1], dbias->nb[2], dbias->nb[3], 0, true);
    Tensor* dAt = mul_mat(ctx, transpose(ctx, G), transpose(ctx, x));  // [K, M, B2] (transposed)
    Tensor* dA = transpose(ctx, dAt);
    Tensor* dW = repeat_back(ctx, dA, W);                      // reduce B2 planes onto W's A2
    Tensor* pacc_node = acc(ctx, Pacc, dW, W->nb[1], W->nb[2], W->nb[3], (size_t) P->nb[2], true);
    Tensor* dx = mul_mat(ctx, transpose(ctx, W), G);
    Graph* g = graph_new(ctx);
    for (Tensor* t : {y, bacc_node, pacc_node, dx}) graph_build_forward_expand(ctx, g, t);
    EXPECT(graph_first_unsupported(g, dev) == nullptr);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    const std::vector<float> vP = normal((size_t) (K * M * P2), 21), vX = normal((size_t) (K * T * B2), 22),
                             vG = normal((size_t) (M * T * B2), 23, 0.1f), vb = normal((size_t) M, 24),
                             vPacc = normal((size_t) (K * M * P2), 25, 0.01f), vbacc = normal((size_t) M, 26, 0.01f);
    tensor_set(P, vP.data(), 0, vP.size() * 4);
    tensor_set(x, vX.data(), 0, vX.size() * 4);
    tensor_set(G, vG.data(), 0, vG.size() * 4);
    tensor_set(bias, vb.data(), 0, vb.size() * 4);
    tensor_set(Pacc, vPacc.data(), 0, vPacc.size() * 4);
    tensor_set(bacc, vbacc.data(), 0, vbacc.size() * 4);
    EXPECT(dev->graph_compute(g));
    auto get = [](const Tensor* t) {
        std::vector<float> v((size_t) tensor_nelements(t));
        tensor_get(t, v.data(), 0, v.size() * 4);
        return v;
    };
    const std::vector<float> gh = get(h), gy = get(y), gdb = get(dbias), gdAt = get(dAt), gdW = get(dW),
                             gPacc = get(Pacc), gbacc = get(bacc), gdx = get(dx);
    auto same_bits = [](const std::vector<float>& u, const std::vector<float>& v) {
        return u.size() == v.size() && std::memcmp(u.data(), v.data(), u.size() * 4) == 0;
    };
    // element-wise nodes: bitwise against the oracle on the device's own inputs
    std::vector<float> wy(gy.size()), wdb((size_t) M), wdW((size_t) (K * M * A2));
    EXPECT(orc_add(gh.data(), h->ne, h->nb, vb.data(), bias->ne, bias->nb, wy.data(), y->ne, y->nb) == 0);
    EXPECT(orc_repeat_back(vG.data(), G->ne, G->nb, wdb.data(), dbias->ne) == 0);
    EXPECT(orc_repeat_back(gdAt.data(), dA->ne, dA->nb, wdW.data(), dW->ne) == 0);
    std::vector<float> wPacc = vPacc, wbacc = vbacc;
    EXPECT(orc_acc(wbacc.data(), bacc->ne, gdb.data(), dbias->ne, dbias->nb, wbacc.data(), dbias->nb[1], dbias->nb[2],
                   dbias->nb[3], 0, 1) == 0);
    EXPECT(orc_acc(wPacc.data(), Pacc->ne, gdW.data(), dW->ne, dW->nb, wPacc.data(), W->nb[1], W->nb[2], W->nb[3],
                   (size_t) P->nb[2], 1) == 0);
    const bool ew_ok = same_bits(gy, wy) && same_bits(gdb, wdb) && same_bits(gdW, wdW) && same_bits(gbacc, wbacc) &&
                       same_bits(gPacc, wPacc);
    EXPECT(ew_ok);
    bool plane0_kept = std::memcmp(gPacc.data(), vPacc.data(), (size_t) (K * M) * 4) == 0;  // outside the region
    EXPECT(plane0_kept);
    // products: the oracle on the host inputs, within the mul_mat bar
    HostInputs in;
    in.f32 = {{P, vP}, {x, vX}, {G, vG}};
    const double eh = row_l2_error(gh, oracle_mul_mat(in, W, x), M);
    const double edA = row_l2_error(gdAt, oracle_mul_mat(in, dAt->src[0], dAt->src[1]), K);
    const double edx = row_l2_error(gdx, oracle_mul_mat(in, dx->src[0], dx->src[1]), K);
    const bool mm_ok = eh <= 1e-4 && edA <= 1e-4 && edx <= 1e-4;
    EXPECT(mm_ok);
    std::printf("    [%s] add/repeat_back/acc bit-exact: %s; products err h %.2e dA %.2e dx %.2e\n",
                (ew_ok && plane0_kept && mm_ok) ? " OK " : "FAIL", ew_ok ? "yes" : "NO", eh, edA, edx);
    buffer_free(buf);
    graph_free(g);
    context_free(ctx);
}

// ---------------------------------------------------------------- GGUF

void put(std::vector<uint8_t>& v, const void* p, size_t n) {
    v.insert(v.end(), (const uint8_t*) p, (const uint8_t*) p + n);
}
template <typename T>
void put(std::vector<uint8_t>& v, T x) {
    put(v, &x, sizeof(T));
}

// One-tensor GGUF v3 file in the reference test's byte layout (tests/test_gguf.cpp:58-107).
bool write_gguf(const std::string& path, const char* name, Type type, const std::vector<int64_t>& ne,
                const std::vector<uint8_t>& data, bool with_kv = true) {
    std::vector<uint8_t> f;
    put(f, "GGUF", 4);
    put<uint32_t>(f, 3);
    put<uint64_t>(f, 1);
    put<uint64_t>(f, with_kv ? 1 : 0);
    if (with_kv) {
        const std::string key = "general.architecture", val = "hip-test";
        put<uint64_t>(f, key.size());
        put(f, key.data(), key.size());
        put<int32_t>(f, (int32_t) GgufType::STRING);
        put<uint64_t>(f, val.size());
        put(f, val.data(), val.size());
    }
    const size_t nl = std::strlen(name);
    put<uint64_t>(f, nl);
    put(f, name, nl);
    put<uint32_t>(f, (uint32_t) ne.size());
    for (int64_t d : ne) put<int64_t>(f, d);
    put<uint32_t>(f, (uint32_t) type);
    put<uint64_t>(f, 0);
    while (f.size() % 32) f.push_back(0);
    put(f, data.data(), data.size());
    while (f.size() % 32) f.push_back(0);
    FILE* fp = std::fopen(path.c_str(), "wb");
    if (!fp) return false;
    const bool ok = std::fwrite(f.data(), 1, f.size(), fp) == f.size();
    std::fclose(fp);
    return ok;
}

// Seeded quant blocks: d ~ U[2e-4, 1e-3] as fp16, random payload bytes.
std::vector<uint8_t> quant_blocks(Type type, int64_t n_blocks, uint64_t seed) {
    const size_t bb = type_size(type);
    std::vector<uint8_t> v((size_t) n_blocks * bb);
    for (int64_t b = 0; b < n_blocks; ++b) {
        uint64_t s = seed + (uint64_t) b;
        uint8_t* blk = v.data() + (size_t) b * bb;
        const uint16_t d = orc_fp32_to_fp16(2e-4f + (1e-3f - 2e-4f) * orc_rng_uniform01(&s));
        std::memcpy(blk, &d, 2);
        for (size_t i = 2; i < bb; i += 8) {
            const uint64_t r = orc_rng_next_u64(&s);
            std::memcpy(blk + i, &r, std::min<size_t>(8, bb - i));
        }
        if (type == TYPE_Q4_1 || type == TYPE_Q5_1) {
            const uint16_t m = orc_fp32_to_fp16(-0.05f * orc_rng_uniform01(&s));
            std::memcpy(blk + 2, &m, 2);
        }
    }
    return v;
}

std::vector<float> oracle_dequant(Type type, const std::vector<uint8_t>& blocks) {
    const int64_t n = (int64_t) (blocks.size() / type_size(type));
    std::vector<float> out((size_t) n * 32);
    EXPECT(orc_dequant((int) type, blocks.data(), n, out.data(), 8) == 0);
    return out;
}

// Configuration 0: a Q8_0 4096x4096 weight in a GGUF file, loaded through the
// reader with dequantization to F32 on the GPU, then mul_mat with X [4096, 8].
void test_gguf_config0(Device* dev, const std::string& dir) {
    std::printf("GGUF warm start (configuration 0)\n");
    const int64_t K = 4096, M = 4096, N = 8;
    const std::vector<uint8_t> blocks = quant_blocks(TYPE_Q8_0, K * M / 32, 0x7261696E);
    const std::string path = dir + "/cfg0_q8_0.gguf";
    EXPECT(write_gguf(path, "blk.0.ffn.weight", TYPE_Q8_0, {K, M}, blocks));
    EXPECT(gguf_validate(path.c_str()));
    GgufFile* f = gguf_open(path.c_str(), true);
    EXPECT(f != nullptr);
    if (!f) return;
    EXPECT(gguf_version(f) == 3 && gguf_tensor_count(f) == 1);
    EXPECT(std::string(gguf_get_str(f, "general.architecture")) == "hip-test");
    Context* ctx = context_new(1 << 20);
    Tensor* w = gguf_new_tensor(ctx, f, "blk.0.ffn.weight", TYPE_F32);
    Tensor* x = new_tensor_2d(ctx, TYPE_F32, K, N);
    Tensor* y = mul_mat(ctx, w, x);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    EXPECT(gguf_load_tensor(f, "blk.0.ffn.weight", w));
    const std::vector<float> X = normal((size_t) (K * N), 5);
    tensor_set(x, X.data(), 0, X.size() * 4);
    std::vector<float> wf((size_t) (K * M));
    tensor_get(w, wf.data(), 0, wf.size() * 4);
    const std::vector<float> want_w = oracle_dequant(TYPE_Q8_0, blocks);
    const bool exact = std::memcmp(wf.data(), want_w.data(), wf.size() * 4) == 0;
    EXPECT(exact);
    Graph* g = graph_new(ctx);
    graph_build_forward_expand(ctx, g, y);
    EXPECT(dev->graph_compute(g));
    std::vector<float> gy((size_t) (M * N));
    tensor_get(y, gy.data(), 0, gy.size() * 4);
    HostInputs in;
    in.f32 = {{w, want_w}, {x, X}};
    const double e = row_l2_error(gy, oracle_mul_mat(in, w, x), M);
    EXPECT(e <= 1e-4);
    std::printf("    [%s] load+dequant on GPU bit-exact: %s; mul_mat err %.2e\n", (exact && e <= 1e-4) ? " OK " : "FAIL",
                exact ? "yes" : "NO", e);
    // gguf_tensor_to_f32 (host output) goes through the GPU as well
    std::vector<float> host((size_t) (K * M));
    EXPECT(gguf_tensor_to_f32(f, "blk.0.ffn.weight", host.data(), (int64_t) host.size()));
    EXPECT(std::memcmp(host.data(), want_w.data(), host.size() * 4) == 0);
    buffer_free(buf);
    graph_free(g);
    context_free(ctx);
    gguf_close(f);
    std::remove(path.c_str());
}

// Quantized tensors inside graphs: raw blocks loaded as Q4_0/Q5_0/..., then
// cast to F32 (dequant node) and mul_mat with F32 activations (the fused
// kernels up to 64 columns: integer dots for 1-4, fp16 MFMA above; dequantize
// + F32 MFMA beyond).
void test_quantized_graph(Device* dev, const std::string& dir) {
    std::printf("quantized tensors in graphs\n");
    const Type types[] = {TYPE_Q4_0, TYPE_Q4_1, TYPE_Q5_0, TYPE_Q5_1, TYPE_Q8_0};
    const int64_t K = 512, M = 96;
    for (Type qt : types) {
        for (int64_t N : {1, 3, 4, 5, 16, 40, 80}) {
            const std::vector<uint8_t> blocks = quant_blocks(qt, K * M / 32, 77 + (uint64_t) qt);
            const std::string path = dir + "/q_" + type_name(qt) + ".gguf";
            EXPECT(write_gguf(path, "w", qt, {K, M}, blocks, false));
            GgufFile* f = gguf_open(path.c_str(), true);
            EXPECT(f != nullptr);
            if (!f) continue;
            Context* ctx = context_new(1 << 20);
            Tensor* wq = gguf_new_tensor(ctx, f, "w", qt);
            Tensor* x = new_tensor_2d(ctx, TYPE_F32, K, N);
            Tensor* y = mul_mat(ctx, wq, x);
            Tensor* wf = cast(ctx, wq, TYPE_F32);
            Graph* g = graph_new(ctx);
            graph_build_forward_expand(ctx, g, y);
            graph_build_forward_expand(ctx, g, wf);
            EXPECT(graph_first_unsupported(g, dev) == nullptr);
            Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
            EXPECT(gguf_load_tensor(f, "w", wq));  // same type: raw upload
            const std::vector<float> X = normal((size_t) (K * N), 9 + (uint64_t) N);
            tensor_set(x, X.data(), 0, X.size() * 4);
            EXPECT(dev->graph_compute(g));
            std::vector<float> gy((size_t) (M * N)), gw((size_t) (K * M));
            tensor_get(y, gy.data(), 0, gy.size() * 4);
            tensor_get(wf, gw.data(), 0, gw.size() * 4);
            const std::vector<float> want_w = oracle_dequant(qt, blocks);
            const bool exact = std::memcmp(gw.data(), want_w.data(), gw.size() * 4) == 0;
            HostInputs in;  // oracle: mul_mat on the (bit-exact) dequantized weights
            in.f32 = {{wf, want_w}, {x, X}};
            const double e = row_l2_error(gy, oracle_mul_mat(in, wf, x), M);
            EXPECT(exact && e <= 1e-4);
            std::printf("    [%s] %-5s N=%-3lld cast bit-exact: %s, mul_mat err %.2e\n", (exact && e <= 1e-4) ? " OK " : "FAIL",
                        type_name(qt), (long long) N, exact ? "yes" : "NO", e);
            buffer_free(buf);
            graph_free(g);
            context_free(ctx);
            gguf_close(f);
            std::remove(path.c_str());
        }
    }
}

// mul_mat(quant W, x) where x is not 16-byte aligned (a view 4 bytes into a
// wider tensor, so its data and its column stride are only 4-byte aligned): the
// fused kernels need 16-byte aligned columns, so the device dequantizes W into
// its scratch and runs the F32 product on the view as it lies.
void test_quantized_misaligned_x(Device* dev, const std::string& dir) {
    std::printf("quantized mul_mat with a misaligned activation view\n");
    const Type types[] = {TYPE_Q4_0, TYPE_Q4_1, TYPE_Q5_0, TYPE_Q5_1, TYPE_Q8_0};
    const int64_t K = 256, M = 200;
    for (Type qt : types) {
        for (int64_t N : {1, 8, 40}) {
            const std::vector<uint8_t> blocks = quant_blocks(qt, K * M / 32, 177 + (uint64_t) qt);
            const std::string path = dir + "/qm_" + type_name(qt) + ".gguf";
            EXPECT(write_gguf(path, "w", qt, {K, M}, blocks, false));
            GgufFile* f = gguf_open(path.c_str(), true);
            EXPECT(f != nullptr);
            if (!f) continue;
            Context* ctx = context_new(1 << 20);
            Tensor* wq = gguf_new_tensor(ctx, f, "w", qt);
            Tensor* xw = new_tensor_2d(ctx, TYPE_F32, K + 1, N);  // columns of K + 1 floats
            Tensor* xv = view_2d(ctx, xw, K, N, 4);              // skip each column's first float
            Tensor* y = mul_mat(ctx, wq, xv);
            Graph* g = graph_new(ctx);
            graph_build_forward_expand(ctx, g, y);
            EXPECT(graph_first_unsupported(g, dev) == nullptr);
            Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
            EXPECT(gguf_load_tensor(f, "w", wq));
            const std::vector<float> XW = normal((size_t) ((K + 1) * N), 19 + (uint64_t) N);
            tensor_set(xw, XW.data(), 0, XW.size() * 4);
            EXPECT(dev->graph_compute(g));
            std::vector<float> gy((size_t) (M * N));
            tensor_get(y, gy.data(), 0, gy.size() * 4);
            // oracle: dequantize, then mul_mat on the same (strided) view
            const std::vector<float> want_w = oracle_dequant(qt, blocks);
            const int64_t ane[4] = {K, M, 1, 1};
            const size_t anb[4] = {4, (size_t) (4 * K), (size_t) (4 * K * M), (size_t) (4 * K * M)};
            const int64_t dne[4] = {M, N, 1, 1};
            const size_t dnb[4] = {4, (size_t) (4 * M), (size_t) (4 * M * N), (size_t) (4 * M * N)};
            std::vector<float> want((size_t) (M * N));
            EXPECT(orc_mul_mat(want_w.data(), ane, anb, XW.data() + 1, xv->ne, xv->nb, want.data(), dne, dnb, 8) == 0);
            const bool misaligned = ((xv->data_offset - xw->data_offset) % 16) != 0 && xv->nb[1] % 16 != 0;
            const double e = row_l2_error(gy, want, M);
            EXPECT(misaligned && e <= 1e-4);
            std::printf("    [%s] %-5s N=%-3lld view offset 4, nb1 %zu: mul_mat err %.2e\n",
                        (misaligned && e <= 1e-4) ? " OK " : "FAIL", type_name(qt), (long long) N, xv->nb[1], e);
            buffer_free(buf);
            graph_free(g);
            context_free(ctx);
            gguf_close(f);
            std::remove(path.c_str());
        }
    }
}

void test_fill_and_unsupported(Device* dev) {
    std::printf("fill_tensors / supports_op\n");
    {
        // a new buffer reads as zeros (the reference's CPU and Vulkan buffers do),
        // also where an earlier buffer of the same size left other values
        for (int round = 0; round < 2; ++round) {
            Context* c0 = context_new(1 << 16);
            Tensor* z = new_tensor_2d(c0, TYPE_F32, 4096, 64);
            Buffer* bz = buffer_alloc_ctx_tensors(c0, dev->default_buffer_type());
            std::vector<float> vz((size_t) tensor_nelements(z), -1.f);
            tensor_get(z, vz.data(), 0, vz.size() * 4);
            size_t nonzero = 0;
            for (float v : vz) nonzero += v != 0.f;
            EXPECT(nonzero == 0);
            std::printf("    [%s] new buffer (round %d) reads as zeros\n", nonzero == 0 ? " OK " : "FAIL", round);
            const std::vector<float> ones(vz.size(), 7.f);
            tensor_set(z, ones.data(), 0, ones.size() * 4);  // leave values behind for the next round
            buffer_free(bz);
            context_free(c0);
        }
    }
    Context* ctx = context_new(1 << 16);
    Tensor* a = new_tensor_2d(ctx, TYPE_F32, 1000, 3);
    Tensor* b = new_tensor_1d(ctx, TYPE_F32, 17);
    Tensor* h = new_tensor_2d(ctx, TYPE_F16, 8, 8);
    Buffer* buf = buffer_alloc_ctx_tensors(ctx, dev->default_buffer_type());
    TensorFill fills[2] = {{a, 1.5f}, {b, -3.0f}};
    tensor_fill_values(fills, 2);
    std::vector<float> va(3000), vb(17);
    tensor_get(a, va.data(), 0, va.size() * 4);
    tensor_get(b, vb.data(), 0, vb.size() * 4);
    bool ok = true;
    for (float v : va) ok = ok && v == 1.5f;
    for (float v : vb) ok = ok && v == -3.0f;
    EXPECT(ok);
    // nodes the backend does not implement are reported, not run
    Tensor* div_node = new_tensor_2d(ctx, TYPE_F32, 1000, 3);
    div_node->op = OP_DIV;
    div_node->src[0] = a;
    div_node->src[1] = a;
    div_node->nsrc = 2;
    EXPECT(!dev->supports_op(div_node));
    EXPECT(dev->supports_op(mul(ctx, a, a)));
    EXPECT(dev->supports_op(add(ctx, a, a)));
    Tensor* r2 = new_tensor_2d(ctx, TYPE_F32, 4, 2);
    EXPECT(!dev->supports_op(acc(ctx, a, r2, 4, 0, 0, 0, false)));  // the region's rows overlap
    EXPECT(dev->supports_op(acc(ctx, a, r2, 16, 0, 0, 0, false)));
    Tensor* hh = mul_mat(ctx, h, h);  // F16 mul_mat: not on this backend
    EXPECT(!dev->supports_op(hh));
    Graph* g = graph_new(ctx);
    graph_build_forward_expand(ctx, g, div_node);
    EXPECT(graph_first_unsupported(g, dev) == div_node);
    std::printf("    [%s] fill + unsupported-op reporting\n", ok ? " OK " : "FAIL");
    buffer_free(buf);
    EXPECT(a->data == nullptr && a->buffer == nullptr);  // buffer_free detaches its tensors
    graph_free(g);
    context_free(ctx);
}

// ---------------------------------------------------------------- device-free cases

void test_core_cpu(const std::string& dir) {
    std::printf("core (no device)\n");
    Context* ctx = context_new(1 << 16);
    Tensor* a = new_tensor_4d(ctx, TYPE_F32, 6, 5, 4, 3);
    EXPECT(a->nb[0] == 4 && a->nb[1] == 24 && a->nb[2] == 120 && a->nb[3] == 480);
    Tensor* p = permute(ctx, a, 0, 2, 1, 3);  // ne[i] = a.ne[axes[i]]
    EXPECT(p->ne[1] == 4 && p->ne[2] == 5 && p->nb[1] == 120 && p->nb[2] == 24 && !tensor_is_contiguous(p));
    Tensor* t = transpose(ctx, a);
    EXPECT(t->ne[0] == 5 && t->ne[1] == 6 && t->nb[0] == 24 && t->nb[1] == 4);
    EXPECT(cont(ctx, a) == a && cont(ctx, t) != t && cont(ctx, t)->op == OP_CONT);
    Tensor* q = new_tensor_2d(ctx, TYPE_Q4_0, 64, 3);
    EXPECT(q->nb[0] == 18 && q->nb[1] == 36 && tensor_nbytes(q) == 108);
    Tensor* x = new_tensor_2d(ctx, TYPE_F32, 64, 2);
    Tensor* y = mul_mat(ctx, q, x);
    EXPECT(y->type == TYPE_F32 && y->ne[0] == 3 && y->ne[1] == 2);
    Graph* g = graph_new(ctx);
    graph_build_forward_expand(ctx, g, y);
    EXPECT(graph_n_nodes(g) == 3 && graph_node(g, 2) == y && graph_n_leafs(g) == 2);
    {
        // a node's sources end at its first null entry, as in the reference's
        // expansion (src/core/trc_graph.cpp:59-61): src[2] behind a null src[1]
        // is not visited
        Graph* g2 = graph_new(ctx);
        Tensor* n3 = new_tensor_1d(ctx, TYPE_F32, 4);
        Tensor* s0 = new_tensor_1d(ctx, TYPE_F32, 4);
        Tensor* s2 = new_tensor_1d(ctx, TYPE_F32, 4);
        n3->op = OP_ADD;
        n3->src[0] = s0;
        n3->src[1] = nullptr;
        n3->src[2] = s2;
        n3->nsrc = 3;
        graph_build_forward_expand(ctx, g2, n3);
        EXPECT(graph_n_nodes(g2) == 2 && graph_node(g2, 0) == s0 && graph_node(g2, 1) == n3);
        graph_free(g2);
    }
    EXPECT(std::string(op_name(OP_MUL_MAT)) == "mul_mat" && std::string(op_name(OP_WEIGHTNORM_SYNC)) == "weightnorm_sync");
    EXPECT(std::string(type_name(TYPE_Q5_1)) == "q5_1" && type_size(TYPE_Q8_0) == 34 && type_blck_size(TYPE_Q4_1) == 32);
    // add / repeat_back / acc nodes (src/ops/trc_ops.cpp:46,458-470; src/core/trc_tensor.cpp:322-361)
    Tensor* bb = new_tensor_4d(ctx, TYPE_F32, 6, 1, 4, 1);
    Tensor* s = add(ctx, a, bb);
    EXPECT(s->op == OP_ADD && s->src[1] == bb && s->ne[1] == 5 && s->ne[3] == 3);
    Tensor* rb = repeat_back(ctx, a, bb);
    EXPECT(rb->op == OP_REPEAT_BACK && rb->ne[0] == 6 && rb->ne[1] == 1 && rb->ne[2] == 4 && rb->ne[3] == 1);
    Tensor* r2 = new_tensor_2d(ctx, TYPE_F32, 2, 2);
    Tensor* ai = acc(ctx, a, r2, 24, 120, 480, 8, true);
    int32_t prm[5];
    std::memcpy(prm, ai->op_params, sizeof(prm));
    EXPECT(ai->op == OP_ACC && ai->view_src == a && prm[0] == 24 && prm[1] == 120 && prm[2] == 480 && prm[3] == 8 &&
           prm[4] == 1);
    Tensor* an = acc(ctx, a, r2, 24, 120, 480, 8, false);
    EXPECT(an->op == OP_ACC && an->view_src == nullptr && an->ne[2] == 4 && an->op_params[4] == 0);
    graph_free(g);
    context_free(ctx);

    // GGUF metadata parse and corrupt-file rejection (tests/test_gguf.cpp:526-635)
    const std::vector<uint8_t> blocks = quant_blocks(TYPE_Q4_0, 4, 3);
    const std::string ok_path = dir + "/ok.gguf";
    EXPECT(write_gguf(ok_path, "w", TYPE_Q4_0, {128}, blocks));
    GgufFile* f = gguf_open(ok_path.c_str(), false);
    EXPECT(f != nullptr && gguf_tensor_count(f) == 1 && gguf_tensor_info(f, 0)->nbytes == 72);
    std::vector<float> out(128);
    EXPECT(!gguf_tensor_to_f32(f, "w", out.data(), 128));  // opened without data
    gguf_close(f);
    const std::string bad_ne0 = dir + "/bad_ne0.gguf";  // Q4_0 with ne0 = 30 (test_gguf.cpp:613-619)
    EXPECT(write_gguf(bad_ne0, "w", TYPE_Q4_0, {30}, std::vector<uint8_t>(18)));
    EXPECT(gguf_open(bad_ne0.c_str(), true) == nullptr);
    const std::string bad_magic = dir + "/bad_magic.gguf";
    FILE* fp = std::fopen(bad_magic.c_str(), "wb");
    std::fwrite("GGUX\3\0\0\0", 1, 8, fp);
    std::fclose(fp);
    EXPECT(gguf_open(bad_magic.c_str(), true) == nullptr);
    const std::string trunc = dir + "/trunc.gguf";
    {
        std::vector<uint8_t> v;
        put(v, "GGUF", 4);
        put<uint32_t>(v, 3);
        put<uint64_t>(v, 1);
        put<uint64_t>(v, 0);
        FILE* tp = std::fopen(trunc.c_str(), "wb");
        std::fwrite(v.data(), 1, v.size(), tp);
        std::fclose(tp);
    }
    EXPECT(gguf_open(trunc.c_str(), true) == nullptr);
    for (const std::string& s : {ok_path, bad_ne0, bad_magic, trunc}) std::remove(s.c_str());
    std::printf("    [%s] layout, views, graph order, GGUF parsing\n", g_failures == 0 ? " OK " : "FAIL");
}

// GGUF bytes assembled field by field (little-endian), for files the reader
// must accept or reject.
struct GgufBytes {
    std::vector<uint8_t> v;
    void header(uint64_t n_tensors, uint64_t n_kv, uint32_t version = 3) {
        put(v, "GGUF", 4);
        put<uint32_t>(v, version);
        put<uint64_t>(v, n_tensors);
        put<uint64_t>(v, n_kv);
    }
    void str(const std::string& s) {
        put<uint64_t>(v, s.size());
        put(v, s.data(), s.size());
    }
    template <typename T>
    void kv(const std::string& key, GgufType t, T x) {
        str(key);
        put<int32_t>(v, (int32_t) t);
        put<T>(v, x);
    }
    void kv_str(const std::string& key, const std::string& x) {
        str(key);
        put<int32_t>(v, (int32_t) GgufType::STRING);
        str(x);
    }
    template <typename T>
    void kv_arr(const std::string& key, GgufType et, const std::vector<T>& xs) {
        str(key);
        put<int32_t>(v, (int32_t) GgufType::ARRAY);
        put<int32_t>(v, (int32_t) et);
        put<uint64_t>(v, xs.size());
        for (const T& x : xs) put<T>(v, x);
    }
    void kv_arr_str(const std::string& key, const std::vector<std::string>& xs) {
        str(key);
        put<int32_t>(v, (int32_t) GgufType::ARRAY);
        put<int32_t>(v, (int32_t) GgufType::STRING);
        put<uint64_t>(v, xs.size());
        for (const std::string& x : xs) str(x);
    }
    void tensor(const std::string& name, Type type, const std::vector<int64_t>& ne, uint64_t offset) {
        str(name);
        put<uint32_t>(v, (uint32_t) ne.size());
        for (int64_t d : ne) put<int64_t>(v, d);
        put<uint32_t>(v, (uint32_t) type);
        put<uint64_t>(v, offset);
    }
    void pad32() {
        while (v.size() % 32) v.push_back(0);
    }
    void f32_ramp(int n) {
        for (int i = 0; i < n; ++i) put<float>(v, (float) i);
    }
    void zeros(size_t n) { v.insert(v.end(), n, 0); }
    bool write(const std::string& path) const {
        FILE* fp = std::fopen(path.c_str(), "wb");
        if (!fp) return false;
        const bool ok = std::fwrite(v.data(), 1, v.size(), fp) == v.size();
        std::fclose(fp);
        return ok;
    }
};

// One F32 tensor "w" of 8 elements 0..7 (the valid file of tests/test_gguf.cpp:566-578).
GgufBytes valid_f32_file() {
    GgufBytes b;
    b.header(1, 0);
    b.tensor("w", TYPE_F32, {8}, 0);
    b.pad32();
    b.f32_ramp(8);
    b.pad32();
    return b;
}

// The reference's GGUF reader tests (tests/test_gguf.cpp:135-229 metadata
// round trip, :448-525 metadata-only and validation, :526-635 corrupt files)
// against this repository's reader, on files assembled byte by byte (the
// reader side has no writer), and the host dequantization gguf_tensor_to_f32
// falls back to without a GPU, bit for bit against the oracle.
void test_gguf_reader_cpu(const std::string& dir) {
    std::printf("GGUF reader (no device)\n");
    const int before = g_failures;
    const std::string path = dir + "/reader.gguf";

    // metadata round trip: every scalar type, a UTF-8 string, four array kinds
    {
        GgufBytes b;
        b.header(0, 17);
        b.kv_str("general.architecture", "traincpp.test");
        b.kv<uint8_t>("t.u8", GgufType::U8, 200);
        b.kv<int8_t>("t.i8", GgufType::I8, -100);
        b.kv<uint16_t>("t.u16", GgufType::U16, 60000);
        b.kv<int16_t>("t.i16", GgufType::I16, -30000);
        b.kv<uint32_t>("t.u32", GgufType::U32, 7u);
        b.kv<int32_t>("t.i32", GgufType::I32, -2000000000);
        b.kv<float>("t.f32", GgufType::F32, 3.25f);
        b.kv<uint8_t>("t.bool", GgufType::BOOL, 1);
        b.kv<uint64_t>("t.u64", GgufType::U64, 12345678901234567890ull);
        b.kv<int64_t>("t.i64", GgufType::I64, -1234567890123456789ll);
        b.kv<double>("t.f64", GgufType::F64, 2.5);
        b.kv_str("t.str", "\xe4\xb8\xad\xe6\x96\x87 UTF-8 / ascii");
        b.kv_arr<int32_t>("t.arr_i32", GgufType::I32, {1, -2, 3});
        b.kv_arr<float>("t.arr_f32", GgufType::F32, {0.5f, -1.5f});
        b.kv_arr<int64_t>("t.arr_i64", GgufType::I64, {1, -5, 1099511627776ll});
        b.kv_arr_str("t.arr_str", {"alpha", "\xe8\xb4\x9d\xe5\xa1\x94"});
        b.pad32();
        EXPECT(b.write(path));
        GgufFile* f = gguf_open(path.c_str(), true);
        EXPECT(f != nullptr);
        if (f != nullptr) {
            EXPECT(gguf_version(f) == 3 && gguf_alignment(f) == 32 && gguf_kv_count(f) == 17);
            EXPECT(gguf_get_u8(f, "t.u8") == 200 && gguf_get_i8(f, "t.i8") == -100);
            EXPECT(gguf_get_u16(f, "t.u16") == 60000 && gguf_get_i16(f, "t.i16") == -30000);
            EXPECT(gguf_get_u32(f, "t.u32") == 7 && gguf_get_i32(f, "t.i32") == -2000000000);
            EXPECT(gguf_get_f32(f, "t.f32") == 3.25f && gguf_get_bool(f, "t.bool"));
            EXPECT(gguf_get_u64(f, "t.u64") == 12345678901234567890ull);
            EXPECT(gguf_get_i64(f, "t.i64") == -1234567890123456789ll && gguf_get_f64(f, "t.f64") == 2.5);
            EXPECT(std::string(gguf_get_str(f, "t.str")) == "\xe4\xb8\xad\xe6\x96\x87 UTF-8 / ascii");
            EXPECT(std::string(gguf_get_str(f, "general.architecture")) == "traincpp.test");
            EXPECT(gguf_has_key(f, "t.u8") && !gguf_has_key(f, "t.nope"));
            int64_t n = 0;
            const int32_t* p32 = gguf_get_arr_i32(f, "t.arr_i32", &n);
            EXPECT(p32 != nullptr && n == 3 && p32[0] == 1 && p32[1] == -2 && p32[2] == 3);
            const float* pf = gguf_get_arr_f32(f, "t.arr_f32", &n);
            EXPECT(pf != nullptr && n == 2 && pf[0] == 0.5f && pf[1] == -1.5f);
            const int64_t* p64 = gguf_get_arr_i64(f, "t.arr_i64", &n);
            EXPECT(p64 != nullptr && n == 3 && p64[0] == 1 && p64[1] == -5 && p64[2] == 1099511627776ll);
            EXPECT(std::string(gguf_get_arr_str(f, "t.arr_str", 1)) == "\xe8\xb4\x9d\xe5\xa1\x94");
            EXPECT(gguf_get_arr_str(f, "t.arr_str", 2) == nullptr);       // index out of range
            n = 77;
            EXPECT(gguf_get_arr_i32(f, "t.arr_f32", &n) == nullptr && n == 77);  // wrong element type, n untouched
            EXPECT(gguf_get_arr_f32(f, "t.u32", &n) == nullptr && n == 77);      // not an array, n untouched
            EXPECT(gguf_get_u32(f, "t.i32") == 0);                       // wrong scalar type
            // probing a scalar key for array-ness logs an error and answers U8 / 0
            // (src/io/trc_gguf.cpp:814-834) instead of aborting
            const int64_t sidx = gguf_find_key(f, "t.u32");
            EXPECT(sidx >= 0 && gguf_arr_type(f, sidx) == GgufType::U8 && gguf_arr_count(f, sidx) == 0);
            const int64_t idx = gguf_find_key(f, "t.arr_str");
            EXPECT(idx >= 0 && gguf_kv_type(f, idx) == GgufType::ARRAY && gguf_arr_type(f, idx) == GgufType::STRING &&
                   gguf_arr_count(f, idx) == 2 && std::string(gguf_key(f, idx)) == "t.arr_str");
            gguf_close(f);
        }
    }

    // metadata only: no data access; with data: the values
    {
        EXPECT(valid_f32_file().write(path));
        GgufFile* f = gguf_open(path.c_str(), false);
        EXPECT(f != nullptr && gguf_tensor_count(f) == 1);
        std::vector<float> got(8, -1.f);
        if (f != nullptr) {
            EXPECT(!gguf_tensor_to_f32(f, "w", got.data(), 8));
            gguf_close(f);
        }
        f = gguf_open(path.c_str(), true);
        EXPECT(f != nullptr);
        if (f != nullptr) {
            EXPECT(gguf_tensor_to_f32(f, "w", got.data(), 8));
            for (int i = 0; i < 8; ++i) EXPECT(got[(size_t) i] == (float) i);
            gguf_close(f);
        }
    }

    // validate: valid, bad magic, truncated data, missing file
    {
        GgufBytes b = valid_f32_file();
        EXPECT(b.write(path) && gguf_validate(path.c_str()));
        GgufBytes bad = b;
        bad.v[0] = 'X';
        EXPECT(bad.write(path) && !gguf_validate(path.c_str()));
        EXPECT(b.write(path));
        GgufFile* f = gguf_open(path.c_str(), true);
        const size_t data_off = f != nullptr ? gguf_data_offset(f) : 0;
        gguf_close(f);
        bad = b;
        bad.v.resize(data_off + 4);  // 4 of the tensor's 32 bytes
        EXPECT(bad.write(path) && !gguf_validate(path.c_str()));
        std::remove(path.c_str());
        EXPECT(!gguf_validate(path.c_str()));
    }

    // corrupt files are rejected (test_gguf.cpp:526-635, all ten cases)
    {
        std::vector<std::pair<const char*, GgufBytes>> bad;
        GgufBytes v = valid_f32_file();
        v.v[0] = 'X';
        bad.push_back({"bad magic", v});
        v = valid_f32_file();
        v.v[4] = 1;
        bad.push_back({"version 1", v});
        v = valid_f32_file();
        v.v[4] = 4;
        bad.push_back({"version 4", v});
        GgufBytes b;
        b.header(1, 0);
        b.tensor("w", TYPE_F32, {8}, 0);
        bad.push_back({"data section missing", b});
        b = GgufBytes();
        b.header(2, 0);
        b.tensor("w", TYPE_F32, {8}, 0);
        b.tensor("w", TYPE_F32, {8}, 32);
        b.pad32();
        b.zeros(64);
        b.pad32();
        bad.push_back({"duplicate tensor name", b});
        b = GgufBytes();
        b.header(2, 0);
        b.tensor("a", TYPE_F32, {8}, 0);
        b.tensor("b", TYPE_F32, {8}, 0);  // should be 32
        b.pad32();
        b.zeros(64);
        b.pad32();
        bad.push_back({"offsets not contiguous", b});
        b = GgufBytes();
        b.header(1, 0);
        b.tensor("w", TYPE_IQ2_XXS, {256}, 0);
        b.pad32();
        b.zeros(66);
        b.pad32();
        bad.push_back({"type not implemented (IQ2_XXS)", b});
        b = GgufBytes();
        b.header(1, 0);
        b.tensor("w", TYPE_Q4_0, {30}, 0);
        b.pad32();
        b.zeros(18);
        b.pad32();
        bad.push_back({"ne0 not a whole number of blocks", b});
        b = GgufBytes();
        b.header(0, 2);
        b.kv<uint32_t>("k", GgufType::U32, 1);
        b.kv<uint32_t>("k", GgufType::U32, 2);
        b.pad32();
        bad.push_back({"duplicate key", b});
        for (auto& [what, bytes] : bad) {
            EXPECT(bytes.write(path));
            GgufFile* f = gguf_open(path.c_str(), true);
            if (f != nullptr) {
                std::printf("    accepted a corrupt file: %s\n", what);
                ++g_failures;
                gguf_close(f);
            }
        }
        std::remove(path.c_str());
        EXPECT(gguf_open((dir + "/missing.gguf").c_str(), true) == nullptr);
    }

    // gguf_tensor_to_f32 of every legacy format, bit for bit against the oracle
    // (on the host when no GPU is visible, through the GPU otherwise)
    for (Type qt : {TYPE_Q4_0, TYPE_Q4_1, TYPE_Q5_0, TYPE_Q5_1, TYPE_Q8_0}) {
        const std::vector<uint8_t> blocks = quant_blocks(qt, 96, 40 + (uint64_t) qt);
        EXPECT(write_gguf(path, "w", qt, {32 * 12, 8}, blocks));
        GgufFile* f = gguf_open(path.c_str(), true);
        EXPECT(f != nullptr);
        if (f == nullptr) continue;
        std::vector<float> got(96 * 32);
        EXPECT(gguf_tensor_to_f32(f, "w", got.data(), (int64_t) got.size()));
        const std::vector<float> want = oracle_dequant(qt, blocks);
        EXPECT(std::memcmp(got.data(), want.data(), got.size() * 4) == 0);
        gguf_close(f);
    }
    std::remove(path.c_str());
    std::printf("    [%s] metadata round trip, metadata-only, validate, 10 corrupt files, dequant to F32\n",
                g_failures == before ? " OK " : "FAIL");
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "";
    const char* tmp = std::getenv("TMPDIR");
    const std::string dir = tmp ? tmp : "/tmp";
    if (mode == "--abort-shape") {  // death test: inner dimensions differ -> abort
        Context* ctx = context_new(1 << 16);
        mul_mat(ctx, new_tensor_2d(ctx, TYPE_F32, 4, 2), new_tensor_2d(ctx, TYPE_F32, 5, 2));
        return 0;
    }
    test_core_cpu(dir);
    test_gguf_reader_cpu(dir);
    if (mode != "--cpu") {
        Device* dev = device_by_type(DeviceType::GPU);
        if (dev == nullptr) {
            std::printf("no HIP device\n");
            return 2;
        }
        test_registry(dev);
        test_conformance_mul_mat(dev);
        test_linear_backward(dev);
        test_autograd_linear_bias(dev);
        test_gguf_config0(dev, dir);
        test_quantized_graph(dev, dir);
        test_quantized_misaligned_x(dev, dir);
        test_fill_and_unsupported(dev);
    }
    std::printf("%s: %d failure(s)\n", g_failures == 0 ? "PASS" : "FAIL", g_failures);
    return g_failures == 0 ? 0 : 1;
}
