// Host-side helpers shared by the library's translation units: the calling
// thread's last error message (returned by bvml_dsine_last_error) and the
// overlap test behind BVML_DSINE_EALIAS.  Private to the library.
#pragma once

#include <cstddef>
#include <string>

namespace bvml {

// Record msg as the calling thread's last error and return code.
int fail(int code, const std::string& msg);

// Whether [a, a + abytes) and [b, b + bbytes) overlap.
bool overlaps(const void* a, std::size_t abytes, const void* b, std::size_t bbytes);

// The calling thread's last error message ("" if none).
const char* last_error();

}  // namespace bvml
