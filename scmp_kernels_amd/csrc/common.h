// Shared helpers for the gfx950 SC matmul library (error reporting, launch checks).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/scmp_hip.h"

namespace scmp {

// Thread-local message returned by scmp_last_error().
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

#define SCMP_REQUIRE(cond, ...)          \
    do {                                 \
        if (!(cond)) {                   \
            ::scmp::set_error(__VA_ARGS__); \
            return SCMP_E_ARG;           \
        }                                \
    } while (0)

#define SCMP_LAUNCH_CHECK(what)                                                   \
    do {                                                                          \
        hipError_t e_ = hipGetLastError();                                        \
        if (e_ != hipSuccess) {                                                   \
            ::scmp::set_error("%s: launch failed: %s", what, hipGetErrorString(e_)); \
            return SCMP_E_LAUNCH;                                                 \
        }                                                                         \
    } while (0)

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Round to nearest, ties to even (IEEE default mode), as libdevice.nearbyint / torch.round.
__device__ __forceinline__ float rne(float x) { return __builtin_rintf(x); }

// std::max / std::min semantics (torch clamp; numpy maximum / minimum in the Triton
// interpreter): the first argument wins ties, so clamp(-0.0, 0, Q) stays -0.0.
__device__ __forceinline__ float fmax_first(float a, float b) { return a < b ? b : a; }
__device__ __forceinline__ float fmin_first(float a, float b) { return b < a ? b : a; }

}  // namespace scmp
