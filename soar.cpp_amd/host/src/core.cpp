#include "soar/core.hpp"

namespace soar {

int64_t numel(const Shape& s) {
    int64_t n = 1;
    for (int64_t d : s) {
        if (d < 0) throw ShapeError("negative dimension in " + to_string(s));
        n *= d;
    }
    return n;
}

std::string to_string(const Shape& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) {
        if (i) r += ",";
        r += std::to_string(s[i]);
    }
    return r + "]";
}

namespace exec {
namespace {
thread_local void* g_stream = nullptr;
}
void* stream() noexcept { return g_stream; }
StreamScope::StreamScope(void* s) noexcept : prev_(g_stream) { g_stream = s; }
StreamScope::~StreamScope() { g_stream = prev_; }
}  // namespace exec

}  // namespace soar
