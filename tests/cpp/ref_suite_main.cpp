// Runs the reference's own golden and gradient-golden programs against the HIP
// device (tests/test_golden.cpp, tests/test_grad_golden.cpp: PyTorch goldens of
// single operators and of backward graphs), compiled unchanged from the
// reference's sources by oracle/Makefile `suite` and linked with the reference's
// core (oracle/_ref/libtrc_ref.so) and the HIP plugin. Cases whose graph holds an
// operator the device does not support are reported as skipped by the programs
// themselves (graph_first_unsupported, tests/test_golden.cpp:267,
// tests/test_grad_golden.cpp:330).
//
// This file stands in for the reference's tests/test_main.cpp: it implements the
// registry interface its tests/test_util.h declares, registers hip_device(0)
// with backend_register_device, and selects it for the programs with
// TRC_TEST_DEVICE=vulkan, their name for "the GPU device" (device_by_type(GPU),
// tests/test_util.h:18-33).
#include "test_util.h"
#include "traincpp/traincpp.h"
#include "traincpp/trc_hip.h"

#include <cstdio>
#include <cstdlib>
#include <string>
#include <utility>
#include <vector>

namespace {

std::vector<std::string> g_failures;

}  // namespace

namespace trc_test {

std::vector<TestCase>& registry() {
    static std::vector<TestCase> r;
    return r;
}

void add_failure(const std::string& msg) {
    g_failures.push_back(msg);
    std::fprintf(stderr, "    [FAIL] %s\n", msg.c_str());
}

Registrar::Registrar(const char* name, std::function<void()> fn) {
    registry().push_back({name, std::move(fn)});
}

int run_all() {
    int failed = 0, ran = 0;
    for (const TestCase& tc : registry()) {
        g_failures.clear();
        std::printf("[ RUN  ] %s\n", tc.name.c_str());
        std::fflush(stdout);
        tc.fn();
        ++ran;
        if (g_failures.empty()) {
            std::printf("[  OK  ] %s\n", tc.name.c_str());
        } else {
            std::printf("[ FAIL ] %s (%zu failed checks)\n", tc.name.c_str(), g_failures.size());
            ++failed;
        }
        std::fflush(stdout);
    }
    std::printf("%d cases run, %d failed\n", ran, failed);
    return failed == 0 ? 0 : 1;
}

}  // namespace trc_test

int main() {
    traincpp::Device* hip = traincpp::hip_device(0);
    if (hip == nullptr) {
        std::printf("SKIP: no HIP device visible\n");
        return 77;
    }
    traincpp::backend_register_device(hip);
    if (traincpp::device_by_type(traincpp::DeviceType::GPU) != hip) {
        std::printf("FAIL: device_by_type(GPU) does not return the HIP device\n");
        return 1;
    }
    setenv("TRC_TEST_DEVICE", "vulkan", 1);  // the golden programs' selector for the GPU device
    std::printf("target: %s (%s)\n", hip->props().name.c_str(), hip->props().description.c_str());
    return trc_test::run_all();
}
