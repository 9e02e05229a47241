// Host-side helpers shared by the library's C-ABI entry points: the thread-local last error, the guard that keeps
// C++ exceptions from crossing the ABI (the role of `guard` in crates/flyhigh-capi/src/lib.rs:34-48), and string
// output into caller buffers (write_json, crates/flyhigh-capi/src/lib.rs:50-63).
#pragma once
#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <string>

namespace fhc {

void set_error(const char* msg);
void clear_error();

// records a formatted message as the last error and returns `rc`
inline int fail(int rc, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
inline int fail(int rc, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    set_error(buf);
    return rc;
}

// runs `f`, turning an escaping exception into the last error and `fallback`
template <class T, class F>
T guard(T fallback, F&& f) {
    try {
        return f();
    } catch (const std::exception& e) {
        std::string m = std::string("internal error: ") + e.what();
        set_error(m.c_str());
    } catch (...) {
        set_error("internal error");
    }
    return fallback;
}

// NUL-terminated copy into a caller buffer; bytes written (without the NUL), or -1 if `cap` is too small
inline int write_string(const std::string& s, char* buf, size_t cap) {
    if (!buf || s.size() + 1 > cap) return fail(-1, "buffer too small (%zu bytes needed)", s.size() + 1);
    memcpy(buf, s.data(), s.size());
    buf[s.size()] = 0;
    return (int)s.size();
}

}  // namespace fhc
