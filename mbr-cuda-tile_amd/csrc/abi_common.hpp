// Host-side helpers shared by the extern "C" entry points: thread-local error
// message, argument validation that reports an mbrt_status, and launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/mbrt.h"
#include "device.hpp"
#include "tuning.hpp"

namespace mbrt {

int set_error(int status, const char* fmt, ...);
void clear_error();

// MBRT_ARITH_BF16_INTERMEDIATES is set on the calling thread.
bool bf16_intermediates();

inline hipStream_t as_stream(mbrt_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline bool is_float_dt(int dt) { return dt == F32 || dt == F16 || dt == BF16; }
inline bool is_index_dt(int dt) { return dt == I32 || dt == I64; }
inline bool is_valid_dt(int dt) { return dt >= 0 && dt <= 4; }

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Kernel-launch epilogue: converts a launch failure into MBRT_E_HIP.
int check_launch(const char* op);

// Compute units of the current device (queried once per device), for persistent grids.
int cu_count();

// Largest grid.x we launch (2^31 - 1 allowed on AMD, but keep index math in 32 bits
// where kernels assume it).
constexpr int64_t kMaxGridX = 0x7fffffffLL;

}  // namespace mbrt

#define MBRT_REQUIRE(cond, status, ...)                         \
    do {                                                        \
        if (!(cond)) return ::mbrt::set_error((status), __VA_ARGS__); \
    } while (0)

#define MBRT_REQUIRE_FLOAT_DT(dt, name)                                                   \
    MBRT_REQUIRE(::mbrt::is_float_dt(dt), MBRT_E_UNSUPPORTED_DTYPE,                      \
                 "%s: unsupported dtype %d (expected F32/F16/BF16)", (name), (int)(dt))
