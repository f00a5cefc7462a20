// wm_host.h -- host-side error macros shared by the C-ABI sources.  Internal.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/winmoe_hip.h"

// A HIP call that fails returns WM_ERR from the enclosing function, with the
// error string on stderr.
#define WM_FAIL_HIP(expr)                                                                                  \
    do {                                                                                                   \
        hipError_t e_ = (hipError_t)(expr);                                                                \
        if (e_ != hipSuccess) {                                                                            \
            fprintf(stderr, "winmoe_hip: HIP error at %s:%d: %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
            return WM_ERR;                                                                                 \
        }                                                                                                  \
    } while (0)

// A violated argument precondition returns WM_EINVAL, naming the condition.
#define WM_CHECK_ARG(cond)                                                                \
    do {                                                                                  \
        if (!(cond)) {                                                                    \
            fprintf(stderr, "winmoe_hip: invalid argument (%s) in %s\n", #cond, __func__); \
            return WM_EINVAL;                                                             \
        }                                                                                 \
    } while (0)

namespace wm {
inline int64_t round_up256(int64_t v) { return (v + 255) & ~(int64_t)255; }
}  // namespace wm
