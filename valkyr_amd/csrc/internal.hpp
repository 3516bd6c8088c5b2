// Internal helpers shared by the runner and the C ABI layer.
#pragma once

#include <stdarg.h>

#include "../../include/vkhip.h"
#include "ops.hpp"

namespace vkh {

// Records a thread-local message and returns `st`.
vkh_status fail(vkh_status st, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
vkh_status hip_fail(hipError_t e, const char *what);
// Counts one allocation by the library (device or pinned memory, or a lease of
// the shared scratch buffer); read through vkh_allocation_count.
void note_allocation();

}  // namespace vkh

#define VKH_HIP(call)                                                      \
    do {                                                                   \
        hipError_t e_ = (call);                                            \
        if (e_ != hipSuccess) return ::vkh::hip_fail(e_, #call);           \
    } while (0)

#define VKH_TRY(call)                                                      \
    do {                                                                   \
        vkh_status s_ = (call);                                            \
        if (s_ != VKH_OK) return s_;                                       \
    } while (0)
