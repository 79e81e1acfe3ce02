// Reductions (Tensor::sum / max / mean, src/tensor.cu:710-780; kernels
// src/tensor_cuda_tile.cu:264-291 and src/tensor_cuda_glue.cu:518-557).
//
// Last-dim reduce: one wave per row, lanes stride the row, then a wave butterfly (no
// 2048-column limit).  General-axis reduce dst[o, i] = reduce_r src[o, r, i]: one thread
// per (o, i), r ascending, so a thread's sum is the same sequential f32 loop as the
// reference's kernel (bit-identical), and consecutive threads read consecutive i.
#include "abi_common.hpp"

#include <algorithm>
#include <cmath>

namespace mbrt {
namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void reduce_last_kernel(const float* src, float* dst, int64_t outer,
                                                        int64_t inner, int op) {
    const int lane = threadIdx.x % 64;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + threadIdx.x / 64;
    if (row >= outer) return;
    const float* p = src + row * inner;
    float v = op == MBRT_REDUCE_SUM ? 0.0f : -INFINITY;
    for (int64_t c = lane; c < inner; c += 64) {
        const float x = p[c];
        v = op == MBRT_REDUCE_SUM ? v + x : fmaxf(v, x);
    }
    v = op == MBRT_REDUCE_SUM ? group_sum<64>(v) : group_max<64>(v);
    if (lane == 0) dst[row] = v;
}

__global__ __launch_bounds__(kThreads) void reduce_general_kernel(const float* src, float* dst, int64_t outer,
                                                           int64_t reduce, int64_t inner, int op) {
    const int64_t total = outer * inner;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < total; i += (int64_t)gridDim.x * kThreads) {
        const int64_t o = i / inner, in = i - o * inner;
        const float* p = src + o * reduce * inner + in;
        float v = op == MBRT_REDUCE_SUM ? 0.0f : -INFINITY;
        for (int64_t r = 0; r < reduce; ++r) {
            const float x = p[r * inner];
            v = op == MBRT_REDUCE_SUM ? v + x : fmaxf(v, x);
        }
        dst[i] = v;
    }
}

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_reduce_last_dim(const float* src, float* dst, int64_t outer, int64_t inner, int op_code,
                         mbrt_stream_t stream) {
    const char* op = "mbrt_reduce_last_dim";
    MBRT_REQUIRE(op_code == MBRT_REDUCE_SUM || op_code == MBRT_REDUCE_MAX, MBRT_E_INVALID_ARG, "%s: bad op", op);
    MBRT_REQUIRE(outer >= 0 && inner >= 0, MBRT_E_SHAPE, "%s: bad shape", op);
    if (outer == 0) return MBRT_OK;
    MBRT_REQUIRE(dst != nullptr && (inner == 0 || src != nullptr), MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    hipLaunchKernelGGL(reduce_last_kernel, dim3((unsigned)ceil_div(outer, kThreads / 64)), dim3(kThreads), 0,
                       as_stream(stream), src, dst, outer, inner, op_code);
    return check_launch(op);
}

int mbrt_reduce_general(const float* src, float* dst, int64_t outer, int64_t reduce, int64_t inner, int op_code,
                        mbrt_stream_t stream) {
    const char* op = "mbrt_reduce_general";
    MBRT_REQUIRE(op_code == MBRT_REDUCE_SUM || op_code == MBRT_REDUCE_MAX, MBRT_E_INVALID_ARG, "%s: bad op", op);
    MBRT_REQUIRE(outer >= 0 && reduce >= 0 && inner >= 0, MBRT_E_SHAPE, "%s: bad shape", op);
    const int64_t total = outer * inner;
    if (total == 0) return MBRT_OK;
    MBRT_REQUIRE(dst != nullptr && (reduce == 0 || src != nullptr), MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    hipLaunchKernelGGL(reduce_general_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(total, kThreads), 1 << 20)),
                       dim3(kThreads), 0, as_stream(stream), src, dst, outer, reduce, inner, op_code);
    return check_launch(op);
}

}  // extern "C"
