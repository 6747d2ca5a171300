// errors.hpp -- the library's error state and allocation-failure switch,
// with no HIP dependency, so host-only sources (the checkpoint parsers) build
// with a plain C++ compiler too.
//
// Error model: every C-ABI entry point returns 0 on success or a negative
// ATLAS_E* code and records a message retrievable with atlas_last_error()
// (thread-local).  Entry points that keep the reference's `void` signature
// record the error the same way.
#pragma once

#include <cstddef>
#include <cstdint>

#include "../../include/atlas_kernels.h"   // ATLAS_OK / ATLAS_E* codes

#define ATLAS_API extern "C" __attribute__((visibility("default")))

namespace atlas {

void set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// The allocation-failure switch (atlas_debug_fail_allocations): true when the
// calling allocation site must fail as if the device were out of memory.
// Every device and pinned-host allocation the library makes asks it first.
bool alloc_should_fail();

}  // namespace atlas

#define ATLAS_REQUIRE(cond, ...)                                               \
    do {                                                                       \
        if (!(cond)) {                                                         \
            ::atlas::set_error(ATLAS_EINVAL, __VA_ARGS__);                     \
            return ATLAS_EINVAL;                                               \
        }                                                                      \
    } while (0)
