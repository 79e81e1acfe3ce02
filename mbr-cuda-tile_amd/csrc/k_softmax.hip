// Row softmax with f32 accumulation (the scale_softmax* family, src/mbr_cuda_tile.cu:5092-5285):
//   z = scale * x;  p = exp(z - max z) / sum exp(z - max z)   per row of `cols` elements.
//
// A group of G lanes owns a row and keeps it in registers, so the input is read once and
// the output written once (the reference uses one 2048-wide tile per row: 61 % of the
// lanes idle at 801 columns, 97 % at 60).  Rows of 801 / 60 elements do not start on
// 16-byte boundaries, so the group walks the 16-byte-aligned vectors that cover its row
// (measured from the buffer base, which must be 16-byte aligned): interior vectors are
// loaded and stored whole, the two edge vectors element-wise with masking.  Neighbouring
// rows share an edge vector; each group writes only its own elements, so in-place
// (out == in) is safe.
//   801 cols f32 : 202 vectors/row -> G = 64, 4 vectors per lane
//   801 cols bf16: 102 vectors/row -> G = 64, 2 vectors per lane
//   60 cols f32  : <= 16 vectors   -> G = 16, 1 vector per lane, 16 rows per block
//   60 cols bf16 : <= 9 vectors    -> G = 16, 1 vector per lane
// Rows too long for registers (> 64 lanes x 16 vectors) use a three-pass loop kernel.
#include "abi_common.hpp"

#include <algorithm>
#include <cfloat>

namespace mbrt {
namespace {

constexpr int kThreads = 256;

struct SmArgs {
    const void* in;
    void* out;
    int odt;
    int64_t rows;
    int64_t cols;
    int64_t total;  // rows * cols (elements in the buffer)
    float scale;
};

template <int IDT>
__device__ __forceinline__ void load_vec(const void* p, int64_t e, float* f) {
    if (IDT == F32) {
        float t[4];
        load4(p, F32, e, t);
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = t[i];
    } else {
        float t[8];
        load8(p, IDT, e, t);
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] = t[i];
    }
}

template <int IDT>
__device__ __forceinline__ void store_vec(void* p, int odt, int64_t e, const float* f) {
    if (IDT == F32) {
        float t[4] = {f[0], f[1], f[2], f[3]};
        store4(p, odt, e, t);
    } else {
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = f[i];
        store8(p, odt, e, t);
    }
}

template <int IDT, int G, int NV>
__global__ __launch_bounds__(kThreads) void softmax_fast_kernel(SmArgs a) {
    constexpr int VE = IDT == F32 ? 4 : 8;  // elements per 16-byte vector
    const int lane = threadIdx.x % G;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / G) + threadIdx.x / G;
    const bool valid = row < a.rows;
    const int64_t start = row * a.cols;
    const int64_t end = start + a.cols;
    const int64_t v0 = start / VE;

    float x[NV][VE];
    float m = -FLT_MAX;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t e0 = (v0 + lane + (int64_t)G * k) * VE;
        const bool any = valid && e0 < end;
        if (any && e0 >= start && e0 + VE <= end) {  // interior vector
            load_vec<IDT>(a.in, e0, x[k]);
#pragma unroll
            for (int i = 0; i < VE; ++i) {
                x[k][i] *= a.scale;
                m = fmaxf(m, x[k][i]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < VE; ++i) {
                const int64_t e = e0 + i;
                float v = -FLT_MAX;
                if (any && e >= start && e < end) {
                    v = load1(a.in, IDT, e) * a.scale;
                    m = fmaxf(m, v);
                }
                x[k][i] = v;
            }
        }
    }
    m = group_max<G>(m);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t e0 = (v0 + lane + (int64_t)G * k) * VE;
        const bool interior = valid && e0 >= start && e0 + VE <= end;
#pragma unroll
        for (int i = 0; i < VE; ++i) {
            const int64_t e = e0 + i;
            float p = fast_exp(x[k][i] - m);
            if (!interior && !(valid && e >= start && e < end)) p = 0.0f;
            x[k][i] = p;
            s += p;
        }
    }
    s = group_sum<G>(s);
    const float inv = 1.0f / s;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t e0 = (v0 + lane + (int64_t)G * k) * VE;
        const bool any = valid && e0 < end;
#pragma unroll
        for (int i = 0; i < VE; ++i) x[k][i] *= inv;
        if (any && e0 >= start && e0 + VE <= end) {
            store_vec<IDT>(a.out, a.odt, e0, x[k]);
        } else if (any) {
#pragma unroll
            for (int i = 0; i < VE; ++i) {
                const int64_t e = e0 + i;
                if (e >= start && e < end) store1(a.out, a.odt, e, x[k][i]);
            }
        }
    }
}

// Long rows: one wave per row, three passes (max, sum, write) over global memory.
__global__ __launch_bounds__(kThreads) void softmax_loop_kernel(SmArgs a, int idt) {
    const int lane = threadIdx.x % 64;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + threadIdx.x / 64;
    if (row >= a.rows) return;
    const int64_t start = row * a.cols;
    float m = -FLT_MAX;
    for (int64_t c = lane; c < a.cols; c += 64) m = fmaxf(m, load1(a.in, idt, start + c) * a.scale);
    m = group_max<64>(m);
    float s = 0.0f;
    for (int64_t c = lane; c < a.cols; c += 64) s += fast_exp(load1(a.in, idt, start + c) * a.scale - m);
    s = group_sum<64>(s);
    const float inv = 1.0f / s;
    for (int64_t c = lane; c < a.cols; c += 64)
        store1(a.out, a.odt, start + c, fast_exp(load1(a.in, idt, start + c) * a.scale - m) * inv);
}

template <int IDT>
bool launch_fast(const SmArgs& a, hipStream_t st) {
    constexpr int VE = IDT == F32 ? 4 : 8;
    // vectors a row can touch: ceil(cols / VE) + 1 (misaligned start)
    const int64_t nvec = (a.cols + VE - 1) / VE + 1;
    auto grid = [&](int G) { return dim3((unsigned)ceil_div(a.rows, kThreads / G)); };
    if (nvec <= 16) {
        hipLaunchKernelGGL((softmax_fast_kernel<IDT, 16, 1>), grid(16), dim3(kThreads), 0, st, a);
    } else if (nvec <= 32) {
        hipLaunchKernelGGL((softmax_fast_kernel<IDT, 32, 1>), grid(32), dim3(kThreads), 0, st, a);
    } else if (nvec <= 64) {
        hipLaunchKernelGGL((softmax_fast_kernel<IDT, 64, 1>), grid(64), dim3(kThreads), 0, st, a);
    } else if (nvec <= 128) {
        hipLaunchKernelGGL((softmax_fast_kernel<IDT, 64, 2>), grid(64), dim3(kThreads), 0, st, a);
    } else if (nvec <= 256) {
        hipLaunchKernelGGL((softmax_fast_kernel<IDT, 64, 4>), grid(64), dim3(kThreads), 0, st, a);
    } else if (nvec <= 512) {
        hipLaunchKernelGGL((softmax_fast_kernel<IDT, 64, 8>), grid(64), dim3(kThreads), 0, st, a);
    } else if (nvec <= 1024) {
        hipLaunchKernelGGL((softmax_fast_kernel<IDT, 64, 16>), grid(64), dim3(kThreads), 0, st, a);
    } else {
        return false;
    }
    return true;
}

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_softmax_rows(const void* in, int in_dtype, void* out, int out_dtype, int64_t rows, int64_t cols,
                      float scale, mbrt_stream_t stream) {
    const char* op = "mbrt_softmax_rows";
    MBRT_REQUIRE_FLOAT_DT(in_dtype, op);
    MBRT_REQUIRE_FLOAT_DT(out_dtype, op);
    MBRT_REQUIRE(rows >= 0 && cols >= 1, MBRT_E_SHAPE, "%s: bad shape", op);
    if (rows == 0) return MBRT_OK;
    MBRT_REQUIRE(in && out, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    MBRT_REQUIRE(in != out || in_dtype == out_dtype, MBRT_E_INVALID_ARG, "%s: in-place needs equal dtypes", op);
    SmArgs a{};
    a.in = in;
    a.out = out;
    a.odt = out_dtype;
    a.rows = rows;
    a.cols = cols;
    a.total = rows * cols;
    a.scale = scale;
    hipStream_t st = as_stream(stream);
    bool done = false;
    // the vector path walks vectors aligned to the buffer base: both bases 16B-aligned
    if (aligned(in, 16) && aligned(out, 16)) {
        if (in_dtype == F32) done = launch_fast<F32>(a, st);
        else if (in_dtype == BF16) done = launch_fast<BF16>(a, st);
        else done = launch_fast<F16>(a, st);
    }
    if (!done) {
        hipLaunchKernelGGL(softmax_loop_kernel, dim3((unsigned)ceil_div(rows, kThreads / 64)), dim3(kThreads), 0, st, a,
                           in_dtype);
    }
    return check_launch(op);
}

}  // extern "C"
