// errors.cpp -- thread-local error state of the C ABI and the injectable
// allocation-failure switch (host-only code).
#include "errors.hpp"

#include <atomic>
#include <cstdarg>
#include <cstdio>

namespace atlas {

static thread_local int t_err_code = ATLAS_OK;
static thread_local char t_err_msg[512] = "";

void set_error(int code, const char* fmt, ...) {
    t_err_code = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err_msg, sizeof(t_err_msg), fmt, ap);
    va_end(ap);
}

void clear_error() {
    t_err_code = ATLAS_OK;
    t_err_msg[0] = 0;
}

// skip: allocations still allowed before the failures start; fail: how many
// fail after that (0 = the switch is off).  Process-wide.
static std::atomic<long> g_alloc_skip{0}, g_alloc_fail{0};

bool alloc_should_fail() {
    if (g_alloc_fail.load(std::memory_order_relaxed) <= 0) return false;
    if (g_alloc_skip.fetch_sub(1, std::memory_order_relaxed) > 0) return false;
    g_alloc_skip.store(0, std::memory_order_relaxed);
    return g_alloc_fail.fetch_sub(1, std::memory_order_relaxed) > 0;
}

}  // namespace atlas

using namespace atlas;

ATLAS_API int atlas_last_error_code(void) { return t_err_code; }
ATLAS_API const char* atlas_last_error(void) { return t_err_msg; }
ATLAS_API void atlas_clear_error(void) { clear_error(); }

ATLAS_API int atlas_debug_fail_allocations(int skip, int count) {
    ATLAS_REQUIRE(skip >= 0 && count >= 0, "debug_fail_allocations: negative argument");
    g_alloc_fail.store(0, std::memory_order_relaxed);
    g_alloc_skip.store(skip, std::memory_order_relaxed);
    g_alloc_fail.store(count, std::memory_order_relaxed);
    return ATLAS_OK;
}
