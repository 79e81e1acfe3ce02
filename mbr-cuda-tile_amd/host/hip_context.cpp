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

bool env_flag_enabled(const char* name) {
    const char* raw = std::getenv(name);
    if (raw == nullptr) return false;
    const std::string v(raw);
    return !(v.empty() || v == "0" || v == "false" || v == "FALSE" || v == "off" || v == "OFF");
}

}  // namespace cudasep
