#include "impl.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>

namespace traincpp {

void fatal(const char* file, int line, const char* fmt, ...) {
    std::fflush(stdout);
    std::fprintf(stderr, "[traincpp-hip][FATAL] %s:%d: ", file, line);
    va_list ap;
    va_start(ap, fmt);
    std::vfprintf(stderr, fmt, ap);
    va_end(ap);
    std::fputc('\n', stderr);
    std::fflush(stderr);
    std::abort();
}

void log_error(const char* fmt, ...) {
    std::fprintf(stderr, "[traincpp-hip][ERROR] ");
    va_list ap;
    va_start(ap, fmt);
    std::vfprintf(stderr, fmt, ap);
    va_end(ap);
    std::fputc('\n', stderr);
    std::fflush(stderr);
}

Buffer* owning_buffer(const Tensor* t) {
    while (t != nullptr && t->buffer == nullptr && t->view_src != nullptr) t = t->view_src;
    return t != nullptr ? t->buffer : nullptr;
}

}  // namespace traincpp
