// Library-wide host state: the thread-local error message and small helpers.
#include "common.h"

namespace kcr {

namespace {
thread_local std::string g_last_error;
}

void set_last_error(const std::string& message) { g_last_error = message; }

std::string shape_string(const std::vector<int64_t>& shape) {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) {
        if (i) s += ", ";
        s += std::to_string(shape[i]);
    }
    return s + "]";
}

std::vector<int64_t> shape_of(const kcr_tensor& t) {
    return std::vector<int64_t>(t.shape, t.shape + t.ndim);
}

std::string shape_string(const kcr_tensor& t) { return shape_string(shape_of(t)); }

}  // namespace kcr

extern "C" const char* kcr_last_error(void) { return kcr::g_last_error.c_str(); }

extern "C" const char* kcr_version(void) { return "kcr_hip 0.1.0 (gfx950)"; }
