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
    // Blocks freed while work on the old stream was pending may be handed out at once:
    // that work must be done before anything runs on the new stream.  A stream that is
    // being captured into a graph cannot be synchronized (the call would end the capture
    // with an error); there the new stream waits on an event recorded on the old one, which
    // orders the new stream's work after the old stream's inside the graph and brings the
    // new stream into the capture.
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    HIP_CHECK(hipStreamIsCapturing(stream_, &status));
    if (status == hipStreamCaptureStatusActive) {
        hipEvent_t ev;
        HIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
        const hipError_t rec = hipEventRecord(ev, stream_);
        const hipError_t wait = rec == hipSuccess ? hipStreamWaitEvent(s, ev, 0) : rec;
        HIP_CHECK(hipEventDestroy(ev));
        HIP_CHECK(wait);
    } else {
        HIP_CHECK(hipStreamSynchronize(stream_));
    }
    stream_ = s;
}

bool env_flag_enabled(const char* name) {
    const char* raw = std::getenv(name);
    if (raw == nullptr) return false;
    const std::string v(raw);
    return !(v.empty() || v == "0" || v == "false" || v == "FALSE" || v == "off" || v == "OFF");
}

}  // namespace cudasep
