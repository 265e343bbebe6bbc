// mx_host.h -- host-side helpers shared by the C-ABI entry points.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "mxfp4_hip.h"

namespace mxh {
// Records a printf-style message as the calling thread's last error.
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
// Maps a launch result to the C-ABI status, recording the HIP message.
int launch_status(const char* what);
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
}  // namespace mxh

#define MXH_REQUIRE(cond, ...)            \
    do {                                  \
        if (!(cond)) {                    \
            mxh::set_error(__VA_ARGS__);  \
            return MXFP4_EINVAL;          \
        }                                 \
    } while (0)
