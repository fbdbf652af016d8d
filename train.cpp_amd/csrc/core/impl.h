// Internal definitions of the traincpp-compatible core (not installed).
#pragma once

#include "traincpp/traincpp.h"

#include <cstdint>
#include <vector>

namespace traincpp {

// Fatal errors abort the process after printing to stderr, the reference's
// convention for invalid API use (src/core/trc_impl.cpp:8-18).
[[noreturn]] void fatal(const char* file, int line, const char* fmt, ...);
void log_error(const char* fmt, ...);

#define TRC_FAIL(...) ::traincpp::fatal(__FILE__, __LINE__, __VA_ARGS__)
#define TRC_CHECK(cond, ...)          \
    do {                              \
        if (!(cond)) TRC_FAIL(__VA_ARGS__); \
    } while (0)

struct Context {
    struct Arena {
        uint8_t* data = nullptr;
        size_t   size = 0;
        size_t   used = 0;
        bool     owned = true;
    };
    std::vector<Arena>   arenas;
    bool                 no_alloc = true;
    bool                 fixed = false;   // caller-provided memory: no growth
    std::vector<Tensor*> tensors;
    size_t               used_total = 0;
};

// The buffer that owns t's storage: t->buffer, or the view root's.
Buffer* owning_buffer(const Tensor* t);

}  // namespace traincpp
