// Chunk overlap-add of the chunked inference driver (src/chunk_cuda_tile.cu:18-83,
// src/inference_app.cpp:72-232): each model output chunk is weighted by its fade window and
// added into the song-length output at its offset, the window itself into a weight sum;
// at the end the output is divided by the weight sum where that exceeds 1e-8.
//
// The reference adds with float atomics.  Within one call every (channel, sample) is
// written once, and calls on one stream run in order, so plain read-modify-write gives the
// same sums in a fixed order: the result is deterministic and equals an ordered f32
// accumulation bit for bit (the product src * w and the sum are rounded separately, as the
// reference's atomic add of a rounded product is).
//
// Memory-bound: per call C*n reads of src, C*n read-modify-writes of dest, n of the window
// and n read-modify-writes of the weight sum.  A thread owns one sample position (or four)
// and walks a group of channels (all channels for the normalize), so the window and the
// weight sum are not re-read per channel.  16-byte vectors when the offset, lengths and
// pointers allow, else a scalar path.
#include "abi_common.hpp"

namespace mbrt {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
// float4 through the non-temporal load / store helpers (which take ext-vector types)
template <int NT>
__device__ __forceinline__ float4 ld4(const float4* p) {
    const f32x4 v = gld<NT>(reinterpret_cast<const f32x4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
template <int NT>
__device__ __forceinline__ void st4(float4* p, float4 v) {
    gst<NT>(reinterpret_cast<f32x4*>(p), f32x4{v.x, v.y, v.z, v.w});
}

constexpr int kThreads = 256;

struct AccArgs {
    float* __restrict__ dest;       // [C, dest_len]
    float* __restrict__ wsum;       // [dest_len]
    const float* __restrict__ src;  // [C, n]
    const float* __restrict__ win;  // [n]
    int64_t n;            // chunk length (elements, or 4-element vectors on the vector path)
    int64_t dest_len;
    int64_t offset;
    int64_t channels;
};

// d + s w with the product rounded before the add (no contraction into an FMA).
__device__ __forceinline__ float acc1(float d, float s, float w) {
#pragma clang fp contract(off)
    return d + s * w;
}

// grid: x over the chunk (grid-stride), y over groups of kCG channels; a thread walks the
// channels of its group, so the window is read once per group and the weight sum once
constexpr int kCG = 1;  // measured: 1 (11.7 us) beats 4 (12.4 us) and all channels (12.8 us) at 8 x 352800

__global__ __launch_bounds__(kThreads) void accumulate_scalar_kernel(AccArgs a) {
    const int64_t c0 = (int64_t)blockIdx.y * kCG, c1 = min(c0 + kCG, a.channels);
    for (int64_t k = (int64_t)blockIdx.x * kThreads + threadIdx.x; k < a.n; k += (int64_t)gridDim.x * kThreads) {
        const float w = a.win[k];
        for (int64_t c = c0; c < c1; ++c) {
            float* d = a.dest + c * a.dest_len + a.offset + k;
            *d = acc1(*d, a.src[c * a.n + k], w);
        }
        if (blockIdx.y == 0) a.wsum[a.offset + k] = a.wsum[a.offset + k] + w;
    }
}

// n, dest_len and offset in float4 units
__global__ __launch_bounds__(kThreads) void accumulate_vec_kernel(AccArgs a) {
    const int64_t c0 = (int64_t)blockIdx.y * kCG, c1 = min(c0 + kCG, a.channels);
    for (int64_t k = (int64_t)blockIdx.x * kThreads + threadIdx.x; k < a.n; k += (int64_t)gridDim.x * kThreads) {
        const float4 w = reinterpret_cast<const float4*>(a.win)[k];
#pragma unroll
        for (int u = 0; u < kCG; ++u) {
            const int64_t c = c0 + u;
            if (c >= c1) break;
            const float4 s = reinterpret_cast<const float4*>(a.src)[c * a.n + k];
            float4* dp = reinterpret_cast<float4*>(a.dest) + c * a.dest_len + a.offset + k;
            float4 d = *dp;
            d.x = acc1(d.x, s.x, w.x);
            d.y = acc1(d.y, s.y, w.y);
            d.z = acc1(d.z, s.z, w.z);
            d.w = acc1(d.w, s.w, w.w);
            *dp = d;
        }
        if (blockIdx.y == 0) {
            float4* wp = reinterpret_cast<float4*>(a.wsum) + a.offset + k;
            float4 ws = *wp;
            ws.x = ws.x + w.x;
            ws.y = ws.y + w.y;
            ws.z = ws.z + w.z;
            ws.w = ws.w + w.w;
            *wp = ws;
        }
    }
}

// One wave per channel: a block of CPB waves takes channels [CPB y, CPB y + CPB) over the
// same 64 consecutive float4 positions of the chunk, so the window's repeated reads are
// made by waves of one CU, close together in time (float4 units as above).
template <int CPB>
__global__ __launch_bounds__(64 * CPB) void accumulate_cw_kernel(AccArgs a) {
    const int lane = threadIdx.x % 64, w = threadIdx.x / 64;
    const int64_t c = (int64_t)blockIdx.y * CPB + w;
    for (int64_t k = (int64_t)blockIdx.x * 64 + lane; k < a.n; k += (int64_t)gridDim.x * 64) {
        const float4 wv = reinterpret_cast<const float4*>(a.win)[k];
        if (c < a.channels) {
            const float4 s = ld4<MBRT_NT_CHUNK & 1>(reinterpret_cast<const float4*>(a.src) + c * a.n + k);
            float4* dp = reinterpret_cast<float4*>(a.dest) + c * a.dest_len + a.offset + k;
            float4 d = ld4<MBRT_NT_CHUNK & 1>(dp);
            d.x = acc1(d.x, s.x, wv.x);
            d.y = acc1(d.y, s.y, wv.y);
            d.z = acc1(d.z, s.z, wv.z);
            d.w = acc1(d.w, s.w, wv.w);
            st4<MBRT_NT_CHUNK & 2>(dp, d);
        }
        if (blockIdx.y == 0 && w == 0) {
            float4* wp = reinterpret_cast<float4*>(a.wsum) + a.offset + k;
            float4 ws = *wp;
            ws.x = ws.x + wv.x;
            ws.y = ws.y + wv.y;
            ws.z = ws.z + wv.z;
            ws.w = ws.w + wv.w;
            *wp = ws;
        }
    }
}

struct NormArgs {
    float* __restrict__ data;        // [C, len]
    const float* __restrict__ wsum;  // [len]
    int64_t len;          // elements, or float4 units on the vector path
    int64_t channels;
};

__device__ __forceinline__ float norm1(float v, float w) { return w > 1.0e-8f ? v / w : v; }

__global__ __launch_bounds__(kThreads) void normalize_scalar_kernel(NormArgs a) {
    for (int64_t k = (int64_t)blockIdx.x * kThreads + threadIdx.x; k < a.len; k += (int64_t)gridDim.x * kThreads) {
        const float w = a.wsum[k];
        for (int64_t c = 0; c < a.channels; ++c) a.data[c * a.len + k] = norm1(a.data[c * a.len + k], w);
    }
}

__global__ __launch_bounds__(kThreads) void normalize_vec_kernel(NormArgs a) {
    for (int64_t k = (int64_t)blockIdx.x * kThreads + threadIdx.x; k < a.len; k += (int64_t)gridDim.x * kThreads) {
        const float4 w = reinterpret_cast<const float4*>(a.wsum)[k];
#pragma unroll 4
        for (int64_t c = 0; c < a.channels; ++c) {
            float4* p = reinterpret_cast<float4*>(a.data) + c * a.len + k;
            float4 v = ld4<MBRT_NT_CHUNK & 1>(p);
            v.x = norm1(v.x, w.x);
            v.y = norm1(v.y, w.y);
            v.z = norm1(v.z, w.z);
            v.w = norm1(v.w, w.w);
            st4<MBRT_NT_CHUNK & 2>(p, v);
        }
    }
}

int64_t grid_for(int64_t work) { return std::min<int64_t>(ceil_div(work, kThreads), int64_t(1) << 14); }

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_chunk_accumulate(float* dest, float* weight_sum, const float* src, const float* window, int64_t channels,
                          int64_t chunk_len, int64_t dest_len, int64_t offset, mbrt_stream_t stream) {
    const char* op = "mbrt_chunk_accumulate";
    MBRT_REQUIRE(channels >= 0 && chunk_len >= 0 && dest_len >= 0, MBRT_E_SHAPE, "%s: negative extent", op);
    MBRT_REQUIRE(offset >= 0 && offset + chunk_len <= dest_len, MBRT_E_SHAPE,
                 "%s: chunk [%lld, %lld) outside an output of %lld samples", op, (long long)offset,
                 (long long)(offset + chunk_len), (long long)dest_len);
    if (channels == 0 || chunk_len == 0) return MBRT_OK;
    MBRT_REQUIRE(dest && weight_sum && src && window, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    AccArgs a{dest, weight_sum, src, window, chunk_len, dest_len, offset, channels};
    const bool vec = chunk_len % 4 == 0 && dest_len % 4 == 0 && offset % 4 == 0 && aligned(dest, 16) &&
                     aligned(weight_sum, 16) && aligned(src, 16) && aligned(window, 16);
    hipStream_t st = as_stream(stream);
    const unsigned gy = (unsigned)std::min<int64_t>(ceil_div(channels, kCG), 65535);
    MBRT_REQUIRE(channels <= (int64_t)kCG * 65535, MBRT_E_SHAPE, "%s: too many channels", op);
    if (vec) {
        a.n /= 4;
        a.dest_len /= 4;
        a.offset /= 4;
        if (MBRT_CHUNK_CPB > 0) {
            constexpr int CPB = MBRT_CHUNK_CPB > 0 ? MBRT_CHUNK_CPB : 1;
            const unsigned gx = (unsigned)std::min<int64_t>(ceil_div(a.n, 64), int64_t(1) << 16);
            hipLaunchKernelGGL(accumulate_cw_kernel<CPB>, dim3(gx, (unsigned)ceil_div(channels, CPB)), dim3(64 * CPB), 0,
                               st, a);
        } else {
            hipLaunchKernelGGL(accumulate_vec_kernel, dim3((unsigned)grid_for(a.n), gy), dim3(kThreads), 0, st, a);
        }
    } else {
        hipLaunchKernelGGL(accumulate_scalar_kernel, dim3((unsigned)grid_for(a.n), gy), dim3(kThreads), 0, st, a);
    }
    return check_launch(op);
}

int mbrt_chunk_normalize(float* data, const float* weight_sum, int64_t channels, int64_t length,
                         mbrt_stream_t stream) {
    const char* op = "mbrt_chunk_normalize";
    MBRT_REQUIRE(channels >= 0 && length >= 0, MBRT_E_SHAPE, "%s: negative extent", op);
    if (channels == 0 || length == 0) return MBRT_OK;
    MBRT_REQUIRE(data && weight_sum, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    NormArgs a{data, weight_sum, length, channels};
    const bool vec = length % 4 == 0 && aligned(data, 16) && aligned(weight_sum, 16);
    hipStream_t st = as_stream(stream);
    if (vec) {
        a.len /= 4;
        hipLaunchKernelGGL(normalize_vec_kernel, dim3((unsigned)grid_for(a.len)), dim3(kThreads), 0, st, a);
    } else {
        hipLaunchKernelGGL(normalize_scalar_kernel, dim3((unsigned)grid_for(a.len)), dim3(kThreads), 0, st, a);
    }
    return check_launch(op);
}

int mbrt_chunk_fade_window(float* window, int64_t chunk_size, int64_t fade_size, int first, int last) {
    MBRT_REQUIRE(chunk_size >= 0 && fade_size >= 0 && 2 * fade_size <= chunk_size, MBRT_E_SHAPE,
                 "mbrt_chunk_fade_window: fade %lld does not fit a chunk of %lld", (long long)fade_size,
                 (long long)chunk_size);
    if (chunk_size == 0) return MBRT_OK;
    MBRT_REQUIRE(window != nullptr, MBRT_E_INVALID_ARG, "mbrt_chunk_fade_window: NULL pointer");
    for (int64_t i = 0; i < chunk_size; ++i) window[i] = 1.0f;
    if (fade_size == 1) {
        if (!first) window[0] = 0.0f;
        if (!last) window[chunk_size - 1] = 0.0f;
    } else if (fade_size > 1) {
        for (int64_t i = 0; i < fade_size; ++i) {
            const float alpha = (float)i / (float)(fade_size - 1);
            if (!first) window[i] = alpha;
            if (!last) window[chunk_size - fade_size + i] = 1.0f - alpha;
        }
    }
    return MBRT_OK;
}

}  // extern "C"
