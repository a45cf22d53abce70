// The library's error state and overlap test (status.h), and the C ABI's
// bvml_dsine_last_error.  Host code only: the device translation units and
// the CPU branch share it.

#include "status.h"

#include <cstdint>
#include <string>

#include "bvml_dsine.h"

namespace bvml {

namespace {
thread_local std::string g_last_error;
}  // namespace

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

bool overlaps(const void* a, std::size_t abytes, const void* b, std::size_t bbytes) {
    const std::uintptr_t a0 = reinterpret_cast<std::uintptr_t>(a);
    const std::uintptr_t b0 = reinterpret_cast<std::uintptr_t>(b);
    return a0 < b0 + bbytes && b0 < a0 + abytes;
}

const char* last_error() { return g_last_error.c_str(); }

}  // namespace bvml

extern "C" const char* bvml_dsine_last_error(void) { return bvml::last_error(); }
