#include "hip_context.h"

#include <cstdlib>

namespace cudasep {

bool g_quantize_fp16 = false;
bool g_quantize_bf16 = false;

HipContext& HipContext::instance() {
    static HipContext ctx;
    return ctx;
}

void HipContext::synchronize() const { HIP_CHECK(hipStreamSynchronize(stream_)); }

void HipContext::set_stream(hipStream_t s) {
    if (s == stream_) return;
    // blocks freed while work on the old stream was pending may be handed out at once:
    // that work must be done before anything runs on the new stream
    HIP_CHECK(hipStreamSynchronize(stream_));
    stream_ = s;
}

bool env_flag_enabled(const char* name) {
    const char* raw = std::getenv(name);
    if (raw == nullptr) return false;
    const std::string v(raw);
    return !(v.empty() || v == "0" || v == "false" || v == "FALSE" || v == "off" || v == "OFF");
}

}  // namespace cudasep
