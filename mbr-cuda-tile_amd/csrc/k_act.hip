// Activation kernels: bias + activation epilogue (GELU / sigmoid / tanh), GLU over the last
// dim, and the fused sigmoid gate x head merge of the attention output.
//
// All three stream 8-element groups (16-byte accesses for 2-byte dtypes) and compute in
// f32.  GLU reads the value and gate halves of a row as two coalesced streams.  The gate
// merge reads the head-major attention output [B,H,N,D] in D-element runs (128 B at
// D = 64 bf16), applies sigmoid(logit) once per (token, head) group and writes the merged
// [B, N, H*D] rows contiguously: one pass instead of the reference's sigmoid epilogue
// pass plus a separate merge pass (src/mbr_cuda_tile.cu:5504-5534 + 4752-4789).
#include "abi_common.hpp"

#include <algorithm>

namespace mbrt {
namespace {

constexpr int kThreads = 256;
constexpr int kU = 2;  // 8-element groups per thread

// ---- bias + activation ------------------------------------------------------------

struct BiasActArgs {
    const void* x;
    const void* bias;  // may be NULL
    void* out;
    int xdt, bdt, odt;
    int64_t n;          // rows * cols
    int64_t groups;     // n / 8 (vector path)
    FastDiv cols_div;   // cols (vector path with bias needs cols % 8 == 0)
    int64_t cols;
};

template <int ACT>
__device__ __forceinline__ float act_fn(float v) {
    if (ACT == MBRT_ACT_GELU_REF) return gelu_ref(v);
    if (ACT == MBRT_ACT_GELU_STD) return gelu_std(v);
    if (ACT == MBRT_ACT_SIGMOID) return sigmoidf(v);
    if (ACT == MBRT_ACT_TANH) return tanhf(v);
    return v;
}

template <int ACT, bool HAS_BIAS>
__global__ __launch_bounds__(kThreads) void bias_act_vec_kernel(BiasActArgs a) {
    const int64_t base = (int64_t)blockIdx.x * (kThreads * kU) + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const int64_t g = base + u * kThreads;
        if (g < a.groups) {
            const int64_t e = g << 3;
            float v[8];
            load8(a.x, a.xdt, e, v);
            if (HAS_BIAS) {
                const uint32_t col = (uint32_t)e - fdiv((uint32_t)e, a.cols_div) * a.cols_div.d;
                float b[8];
                load8(a.bias, a.bdt, col, b);
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] += b[i];
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = act_fn<ACT>(v[i]);
            store8(a.out, a.odt, e, v);
        }
    }
    if (blockIdx.x == 0) {  // tail when n % 8 != 0 (only possible without bias)
        const int64_t e = (a.groups << 3) + threadIdx.x;
        if (e < a.n) store1(a.out, a.odt, e, act_fn<ACT>(load1(a.x, a.xdt, e)));
    }
}

template <int ACT>
__global__ __launch_bounds__(kThreads) void bias_act_scalar_kernel(BiasActArgs a) {
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < a.n; i += (int64_t)gridDim.x * kThreads) {
        float v = load1(a.x, a.xdt, i);
        if (a.bias != nullptr) v += load1(a.bias, a.bdt, i % a.cols);
        store1(a.out, a.odt, i, act_fn<ACT>(v));
    }
}

template <int ACT>
void launch_bias_act(const BiasActArgs& a, bool vec, hipStream_t st) {
    if (vec) {
        const dim3 grid((unsigned)std::max<int64_t>(1, ceil_div(a.groups, (int64_t)kThreads * kU)));
        if (a.bias != nullptr) hipLaunchKernelGGL((bias_act_vec_kernel<ACT, true>), grid, dim3(kThreads), 0, st, a);
        else hipLaunchKernelGGL((bias_act_vec_kernel<ACT, false>), grid, dim3(kThreads), 0, st, a);
    } else {
        const dim3 grid((unsigned)std::min<int64_t>(ceil_div(a.n, kThreads), 1 << 20));
        hipLaunchKernelGGL(bias_act_scalar_kernel<ACT>, grid, dim3(kThreads), 0, st, a);
    }
}

// ---- GLU ------------------------------------------------------------------------------

struct GluArgs {
    const void* x;
    void* out;
    int xdt, odt;
    int64_t rows, half;
    int64_t groups;   // rows * half / 8
    FastDiv gpr;      // groups per row = half / 8
};

__global__ __launch_bounds__(kThreads) void glu_vec_kernel(GluArgs a) {
    const int64_t base = (int64_t)blockIdx.x * (kThreads * kU) + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const int64_t g = base + u * kThreads;
        if (g < a.groups) {
            uint32_t row, c;
            fdivmod((uint32_t)g, a.gpr, row, c);
            const int64_t in0 = (int64_t)row * (2 * a.half) + (int64_t)c * 8;
            float v[8], gt[8];
            load8(a.x, a.xdt, in0, v);
            load8(a.x, a.xdt, in0 + a.half, gt);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = v[i] * sigmoidf(gt[i]);
            store8(a.out, a.odt, g << 3, v);
        }
    }
}

__global__ __launch_bounds__(kThreads) void glu_scalar_kernel(GluArgs a) {
    const int64_t n = a.rows * a.half;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < n; i += (int64_t)gridDim.x * kThreads) {
        const int64_t row = i / a.half, d = i - row * a.half;
        const int64_t in0 = row * 2 * a.half + d;
        store1(a.out, a.odt, i, load1(a.x, a.xdt, in0) * sigmoidf(load1(a.x, a.xdt, in0 + a.half)));
    }
}

// ---- sigmoid gate x head merge ------------------------------------------------------

struct GateArgs {
    const void* attn;
    const void* gate;
    void* out;
    int adt, gdt, odt;
    int logit;
    int layout;
    int64_t B, H, N, D;
    int64_t groups;    // B*N*H*D / 8
    FastDiv gpt;       // groups per token = H*D/8
    FastDiv gph;       // groups per head = D/8
    FastDiv n_div;     // N
};

__device__ __forceinline__ float gate_value(const GateArgs& a, int64_t gi) {
    float g = load1(a.gate, a.gdt, gi);
    return a.logit ? sigmoidf(g) : g;
}

__global__ __launch_bounds__(kThreads) void gate_merge_vec_kernel(GateArgs a) {
    const int64_t base = (int64_t)blockIdx.x * (kThreads * kU) + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const int64_t g = base + u * kThreads;
        if (g < a.groups) {
            uint32_t token, rem, h, c;
            fdivmod((uint32_t)g, a.gpt, token, rem);
            fdivmod(rem, a.gph, h, c);
            int64_t src;
            if (a.layout == MBRT_LAYOUT_BHND) {
                uint32_t b, n;
                fdivmod(token, a.n_div, b, n);
                src = (((int64_t)b * a.H + h) * a.N + n) * a.D + (int64_t)c * 8;
            } else {
                src = g << 3;
            }
            float v[8];
            load8(a.attn, a.adt, src, v);
            const float gv = gate_value(a, (int64_t)token * a.H + h);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] *= gv;
            store8(a.out, a.odt, g << 3, v);
        }
    }
}

__global__ __launch_bounds__(kThreads) void gate_merge_scalar_kernel(GateArgs a) {
    const int64_t n_total = a.B * a.N * a.H * a.D;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < n_total; i += (int64_t)gridDim.x * kThreads) {
        const int64_t hd = a.H * a.D;
        const int64_t token = i / hd, rem = i - token * hd;
        const int64_t h = rem / a.D, d = rem - h * a.D;
        int64_t src;
        if (a.layout == MBRT_LAYOUT_BHND) {
            const int64_t b = token / a.N, n = token - b * a.N;
            src = ((b * a.H + h) * a.N + n) * a.D + d;
        } else {
            src = i;
        }
        store1(a.out, a.odt, i, load1(a.attn, a.adt, src) * gate_value(a, token * a.H + h));
    }
}

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_bias_act(const void* x, int x_dtype, const void* bias, int bias_dtype, void* out, int out_dtype,
                  int64_t rows, int64_t cols, int act, mbrt_stream_t stream) {
    const char* op = "mbrt_bias_act";
    MBRT_REQUIRE_FLOAT_DT(x_dtype, op);
    MBRT_REQUIRE_FLOAT_DT(out_dtype, op);
    MBRT_REQUIRE(bias == nullptr || bias_dtype == F32 || bias_dtype == BF16, MBRT_E_UNSUPPORTED_DTYPE,
                 "%s: bias dtype %d (expected F32/BF16)", op, bias_dtype);
    MBRT_REQUIRE(act >= 0 && act <= 4, MBRT_E_INVALID_ARG, "%s: bad activation %d", op, act);
    MBRT_REQUIRE(rows >= 0 && cols >= 1, MBRT_E_SHAPE, "%s: bad shape", op);
    BiasActArgs a{};
    a.x = x;
    a.bias = bias;
    a.out = out;
    a.xdt = x_dtype;
    a.bdt = bias_dtype;
    a.odt = out_dtype;
    a.n = rows * cols;
    a.cols = cols;
    if (a.n == 0) return MBRT_OK;
    MBRT_REQUIRE(x && out, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    // In place with a wider output than input would overwrite unread input.
    MBRT_REQUIRE(x != out || dt_size(x_dtype) == dt_size(out_dtype), MBRT_E_INVALID_ARG,
                 "%s: in-place needs equal element sizes", op);
    bool vec = aligned(x, 16) && aligned(out, 16) && (bias == nullptr || (aligned(bias, 16) && cols % 8 == 0)) &&
               (bias == nullptr || a.n < (1ll << 32));
    a.groups = a.n >> 3;
    if (bias != nullptr && vec) a.cols_div = make_fastdiv((uint32_t)cols);
    hipStream_t st = as_stream(stream);
    switch (act) {
        case MBRT_ACT_GELU_REF: launch_bias_act<MBRT_ACT_GELU_REF>(a, vec, st); break;
        case MBRT_ACT_GELU_STD: launch_bias_act<MBRT_ACT_GELU_STD>(a, vec, st); break;
        case MBRT_ACT_SIGMOID: launch_bias_act<MBRT_ACT_SIGMOID>(a, vec, st); break;
        case MBRT_ACT_TANH: launch_bias_act<MBRT_ACT_TANH>(a, vec, st); break;
        default: launch_bias_act<MBRT_ACT_NONE>(a, vec, st); break;
    }
    return check_launch(op);
}

int mbrt_glu_last_dim(const void* x, int x_dtype, void* out, int out_dtype, int64_t rows, int64_t half_dim,
                      mbrt_stream_t stream) {
    const char* op = "mbrt_glu_last_dim";
    MBRT_REQUIRE_FLOAT_DT(x_dtype, op);
    MBRT_REQUIRE_FLOAT_DT(out_dtype, op);
    MBRT_REQUIRE(rows >= 0 && half_dim >= 1, MBRT_E_SHAPE, "%s: bad shape", op);
    if (rows == 0) return MBRT_OK;
    MBRT_REQUIRE(x && out, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    GluArgs a{};
    a.x = x;
    a.out = out;
    a.xdt = x_dtype;
    a.odt = out_dtype;
    a.rows = rows;
    a.half = half_dim;
    hipStream_t st = as_stream(stream);
    const bool vec = half_dim % 8 == 0 && aligned(x, 16) && aligned(out, 16) && rows * half_dim / 8 < (1ll << 32);
    if (vec) {
        a.groups = rows * half_dim / 8;
        a.gpr = make_fastdiv((uint32_t)(half_dim / 8));
        hipLaunchKernelGGL(glu_vec_kernel, dim3((unsigned)ceil_div(a.groups, (int64_t)kThreads * kU)), dim3(kThreads),
                           0, st, a);
    } else {
        hipLaunchKernelGGL(glu_scalar_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(rows * half_dim, kThreads), 1 << 20)),
                           dim3(kThreads), 0, st, a);
    }
    return check_launch(op);
}

int mbrt_sigmoid_gate_merge(const void* attn, int attn_dtype, const void* gate, int gate_dtype, int gate_is_logit,
                            void* merged, int out_dtype, int64_t B, int64_t H, int64_t N, int64_t D, int layout,
                            mbrt_stream_t stream) {
    const char* op = "mbrt_sigmoid_gate_merge";
    MBRT_REQUIRE_FLOAT_DT(attn_dtype, op);
    MBRT_REQUIRE_FLOAT_DT(gate_dtype, op);
    MBRT_REQUIRE_FLOAT_DT(out_dtype, op);
    MBRT_REQUIRE(layout == MBRT_LAYOUT_BHND || layout == MBRT_LAYOUT_BNHD, MBRT_E_INVALID_ARG, "%s: bad layout", op);
    MBRT_REQUIRE(B >= 0 && H >= 1 && N >= 0 && D >= 1, MBRT_E_SHAPE, "%s: bad shape", op);
    const int64_t total = B * N * H * D;
    if (total == 0) return MBRT_OK;
    MBRT_REQUIRE(attn && gate && merged, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    GateArgs a{};
    a.attn = attn;
    a.gate = gate;
    a.out = merged;
    a.adt = attn_dtype;
    a.gdt = gate_dtype;
    a.odt = out_dtype;
    a.logit = gate_is_logit ? 1 : 0;
    a.layout = layout;
    a.B = B;
    a.H = H;
    a.N = N;
    a.D = D;
    hipStream_t st = as_stream(stream);
    const bool vec = D % 8 == 0 && aligned(attn, 16) && aligned(merged, 16) && total / 8 < (1ll << 32) &&
                     B * N < (1ll << 31);
    if (vec) {
        a.groups = total / 8;
        a.gpt = make_fastdiv((uint32_t)(H * D / 8));
        a.gph = make_fastdiv((uint32_t)(D / 8));
        a.n_div = make_fastdiv((uint32_t)N);
        hipLaunchKernelGGL(gate_merge_vec_kernel, dim3((unsigned)ceil_div(a.groups, (int64_t)kThreads * kU)),
                           dim3(kThreads), 0, st, a);
    } else {
        hipLaunchKernelGGL(gate_merge_scalar_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(total, kThreads), 1 << 20)),
                           dim3(kThreads), 0, st, a);
    }
    return check_launch(op);
}

}  // extern "C"
