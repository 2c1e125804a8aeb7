// Host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gdn.h"

namespace gdn {

// Records a message for gdn_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Returns 0, or the pending launch error as a positive hipError_t.
int check_launch(const char* what);

inline bool valid_dtype(int d) { return d == GDN_F32 || d == GDN_BF16 || d == GDN_F16; }
inline int dtype_size(int d) { return d == GDN_F32 ? 4 : 2; }
inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// True when byte ranges [a, a+na) and [b, b+nb) overlap.
inline bool overlaps(const void* a, int64_t na, const void* b, int64_t nb) {
    const char* pa = static_cast<const char*>(a);
    const char* pb = static_cast<const char*>(b);
    return pa < pb + nb && pb < pa + na;
}

}  // namespace gdn

#define GDN_REQUIRE(cond, ...)                              \
    do {                                                    \
        if (!(cond)) return ::gdn::fail(GDN_EINVAL, __VA_ARGS__); \
    } while (0)
