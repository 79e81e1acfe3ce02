// Process-wide HIP state of the tensor layer: the stream every Tensor op is enqueued on
// and the precision switches that the model's dtype policies read.
// Mirrors cudasep::CudaContext / g_quantize_* (src/cuda_context.h:1-21).
#pragma once

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>

namespace cudasep {

// Set by the application before the model is built (src/inference_app.cpp:270).
extern bool g_quantize_fp16;
extern bool g_quantize_bf16;

// Throws std::runtime_error for a failing HIP call (the reference's CUDA_CHECK,
// src/tensor.h:30-36).
#define HIP_CHECK(call)                                                                        \
    do {                                                                                       \
        hipError_t hip_check_err_ = (call);                                                    \
        if (hip_check_err_ != hipSuccess) {                                                    \
            throw std::runtime_error(std::string("HIP error: ") + hipGetErrorString(hip_check_err_) + \
                                     " at " + __FILE__ + ":" + std::to_string(__LINE__));      \
        }                                                                                      \
    } while (0)

// Stream and device of the tensor layer.  The reference runs every op on the legacy
// default stream with synchronous copies; here every op is enqueued on stream(), which
// defaults to the null stream of the current device, and host<->device copies wait for it,
// so the program order of Tensor calls is the execution order.  set_stream() moves all
// later work to another stream.  The caching allocator hands a freed block out again at
// once, which is safe while all work runs on one stream (its order is the program order);
// so set_stream() first waits for the work queued on the previous stream, after which no
// block freed while that work was pending can be reused under it.
class HipContext {
public:
    static HipContext& instance();
    hipStream_t stream() const { return stream_; }
    void set_stream(hipStream_t s);
    void synchronize() const;

private:
    HipContext() = default;
    hipStream_t stream_ = nullptr;
};

// True when the environment variable is set to anything but "", 0, false, off
// (src/mbr_cuda_tile.cu:103-109).
bool env_flag_enabled(const char* name);

}  // namespace cudasep
