// Thread-local error state and generic entry points of the C-ABI.
#include "abi_common.hpp"

#include <atomic>

namespace mbrt {

static thread_local std::string t_error;
static thread_local uint32_t t_arith = 0;

bool bf16_intermediates() { return (t_arith & MBRT_ARITH_BF16_INTERMEDIATES) != 0; }

int set_error(int status, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    t_error.assign(buf);
    return status;
}

void clear_error() { t_error.clear(); }

int check_launch(const char* op) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return set_error(MBRT_E_HIP, "%s: kernel launch failed: %s", op, hipGetErrorString(e));
    }
    return MBRT_OK;
}

int cu_count() {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cached[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
    return n;
}

}  // namespace mbrt

extern "C" {

const char* mbrt_last_error(void) { return mbrt::t_error.c_str(); }

int mbrt_version(void) { return 1 * 10000 + 1 * 100 + 0; }

int mbrt_set_arith_flags(uint32_t flags) {
    if ((flags & ~(uint32_t)MBRT_ARITH_BF16_INTERMEDIATES) != 0)
        return mbrt::set_error(MBRT_E_INVALID_ARG, "mbrt_set_arith_flags: unknown flags 0x%x", flags);
    mbrt::t_arith = flags;
    return MBRT_OK;
}

uint32_t mbrt_get_arith_flags(void) { return mbrt::t_arith; }

int mbrt_stream_sync(mbrt_stream_t stream) {
    hipError_t e = hipStreamSynchronize(mbrt::as_stream(stream));
    if (e != hipSuccess) {
        return mbrt::set_error(MBRT_E_HIP, "mbrt_stream_sync: %s", hipGetErrorString(e));
    }
    return MBRT_OK;
}

}  // extern "C"
