// Status check for C-ABI calls made by the tensor layer: a failing entry point becomes a
// std::runtime_error carrying the library's message, which is how the reference reports
// argument, dtype and launch errors (src/tensor.h:30-36).
#pragma once

#include <stdexcept>
#include <string>

#include "../../include/mbrt.h"
#include "hip_context.h"

namespace cudasep {

inline void abi_check(int status, const char* what) {
    if (status != MBRT_OK) throw std::runtime_error(std::string(what) + ": " + mbrt_last_error());
}

inline mbrt_stream_t abi_stream() { return (mbrt_stream_t)HipContext::instance().stream(); }

}  // namespace cudasep
