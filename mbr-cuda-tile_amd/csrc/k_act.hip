// Activation kernels: bias + activation epilogue (GELU / sigmoid / tanh), GLU over the last
// dim, and the fused sigmoid gate x head merge of the attention output.
//
// The vector kernels are templated on their dtypes.  Each thread owns kU groups of VE
// elements (16 bytes of the widest operand), issues all of its loads first (group index
// clamped into the tensor, so no load is predicated), then computes in f32 and stores
// with a predicate.  GLU reads the value and gate halves of a row as two coalesced
// streams.  The gate merge reads the head-major attention output [B,H,N,D] in D-element
// runs (128 B at D = 64 bf16), applies sigmoid(logit) once per (token, head) group and
// writes the merged [B, N, H*D] rows contiguously: one pass instead of the reference's
// sigmoid epilogue pass plus a separate merge pass (src/mbr_cuda_tile.cu:5504-5534 +
// 4752-4789).  Unaligned operands take runtime-dtype element kernels.
// With MBRT_ARITH_BF16_INTERMEDIATES set, GLU (bf16 -> bf16) rounds the gate sigmoid to bf16
// and the gate merge (bf16 attention) rounds the gate and the product to bf16, as the
// reference's kernels do in full-bf16 mode (src/mbr_cuda_tile.cu:5918-5940, 4718-4750).
#include "abi_common.hpp"

#include <algorithm>

namespace mbrt {
namespace {

constexpr int kThreads = 256;
constexpr int kU = MBRT_ACT_U;      // 16-byte groups per thread: bias + activation
constexpr int kUGlu = MBRT_GLU_U;   // GLU
constexpr int kUGate = MBRT_GATE_U; // sigmoid gate x head merge
constexpr int kNoBias = -1;  // bias dtype tag: no bias

__device__ __forceinline__ int64_t clamp_group(int64_t g, int64_t groups) { return g < groups ? g : groups - 1; }
__device__ __forceinline__ int64_t ceil_div_dev(int64_t a, int64_t b) { return (a + b - 1) / b; }

// GELU rounded to bf16/f16 uses the A&S 7.1.26 complement; f32 output uses erfcf.
// ACT >= 0 fixes the activation at compile time (the element loop is then straight-line
// code); ACT < 0 takes it from `act` at run time.
template <bool LOWP, int ACT = -1>
__device__ __forceinline__ float act_fn(float v, int act) {
    if constexpr (ACT == MBRT_ACT_GELU_REF) return LOWP ? gelu_ref_lowp(v) : gelu_ref(v);
    if constexpr (ACT == MBRT_ACT_GELU_STD) return LOWP ? gelu_std_lowp(v) : gelu_std(v);
    switch (act) {
        case MBRT_ACT_GELU_REF: return LOWP ? gelu_ref_lowp(v) : gelu_ref(v);
        case MBRT_ACT_GELU_STD: return LOWP ? gelu_std_lowp(v) : gelu_std(v);
        case MBRT_ACT_SIGMOID: return sigmoidf(v);
        case MBRT_ACT_TANH: return tanhf(v);
        default: return v;
    }
}

// ---- bias + activation ------------------------------------------------------------

struct BiasActArgs {
    const void* x;
    const void* bias;  // may be NULL
    void* out;
    int xdt, bdt, odt;
    int act;
    int64_t n;         // rows * cols
    int64_t cols;
    FastDiv cols_div;  // cols (vector path with bias needs cols % VE == 0 and n < 2^32)
};

template <int XDT, int ODT, int BDT, int ACT>
__global__ __launch_bounds__(kThreads) void bias_act_vec_kernel(BiasActArgs a) {
    constexpr int VE = (XDT == F32 || ODT == F32 || BDT == F32) ? 4 : 8;
    constexpr bool LOWP = ODT != F32;
    const int64_t groups = a.n / VE;
    const int64_t base = (int64_t)blockIdx.x * (kThreads * kU) + threadIdx.x;
    if (groups > 0) {
        Vec<XDT, VE> xv[kU];
        Vec<(BDT == kNoBias ? F32 : BDT), VE> bv[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t e = clamp_group(base + u * kThreads, groups) * VE;
            xv[u].template load<MBRT_NT_ACT>(a.x, e);
            if constexpr (BDT != kNoBias) {
                const uint32_t col = (uint32_t)e - fdiv((uint32_t)e, a.cols_div) * a.cols_div.d;
                bv[u].load(a.bias, col);
            }
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t g = base + u * kThreads;
            if (g < groups) {
                float v[VE];
                xv[u].to_f32(v);
                if constexpr (BDT != kNoBias) {
                    float b[VE];
                    bv[u].to_f32(b);
#pragma unroll
                    for (int i = 0; i < VE; ++i) v[i] += b[i];
                }
#pragma unroll
                for (int i = 0; i < VE; ++i) v[i] = act_fn<LOWP, ACT>(v[i], a.act);
                Vec<ODT, VE> o;
                o.from_f32(v);
                o.template store<MBRT_NT_ACT>(a.out, g * VE);
            }
        }
    }
    if (blockIdx.x == 0) {  // tail when n % VE != 0 (only possible without bias)
        const int64_t e = groups * VE + threadIdx.x;
        if (e < a.n) st1<ODT>(a.out, e, act_fn<LOWP, ACT>(ld1<XDT>(a.x, e), a.act));
    }
}

__global__ __launch_bounds__(kThreads) void bias_act_elem_kernel(BiasActArgs a) {
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < a.n; i += (int64_t)gridDim.x * kThreads) {
        float v = load1(a.x, a.xdt, i);
        if (a.bias != nullptr) v += load1(a.bias, a.bdt, i % a.cols);
        store1(a.out, a.odt, i, a.odt == F32 ? act_fn<false>(v, a.act) : act_fn<true>(v, a.act));
    }
}

// ---- GLU ------------------------------------------------------------------------------

struct GluArgs {
    const void* x;
    void* out;
    int xdt, odt;
    int64_t rows, half;
    int64_t groups;   // rows * half / VE
    FastDiv gpr;      // groups per row = half / VE
    int fb;           // bf16 intermediates (element kernel; the vector kernel takes FB)
};

template <int XDT, int ODT, bool FB>
__global__ __launch_bounds__(kThreads) void glu_vec_kernel(GluArgs a) {
    constexpr int VE = (XDT == F32 || ODT == F32) ? 4 : 8;
    const int64_t base = (int64_t)blockIdx.x * (kThreads * kUGlu) + threadIdx.x;
    Vec<XDT, VE> xv[kUGlu], gv[kUGlu];
#pragma unroll
    for (int u = 0; u < kUGlu; ++u) {
        uint32_t row, c;
        fdivmod((uint32_t)clamp_group(base + u * kThreads, a.groups), a.gpr, row, c);
        const int64_t in0 = (int64_t)row * (2 * a.half) + (int64_t)c * VE;
        xv[u].template load<MBRT_NT_GLU>(a.x, in0);
        gv[u].template load<MBRT_NT_GLU>(a.x, in0 + a.half);
    }
#pragma unroll
    for (int u = 0; u < kUGlu; ++u) {
        const int64_t g = base + u * kThreads;
        if (g < a.groups) {
            float v[VE], gt[VE];
            xv[u].to_f32(v);
            gv[u].to_f32(gt);
#pragma unroll
            for (int i = 0; i < VE; ++i) v[i] = v[i] * (FB ? bf16r(sigmoidf(gt[i])) : sigmoidf(gt[i]));
            Vec<ODT, VE> o;
            o.from_f32(v);
            o.template store<MBRT_NT_GLU>(a.out, g * VE);
        }
    }
}

__global__ __launch_bounds__(kThreads) void glu_elem_kernel(GluArgs a) {
    const int64_t n = a.rows * a.half;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < n; i += (int64_t)gridDim.x * kThreads) {
        const int64_t row = i / a.half, d = i - row * a.half;
        const int64_t in0 = row * 2 * a.half + d;
        const float g = sigmoidf(load1(a.x, a.xdt, in0 + a.half));
        store1(a.out, a.odt, i, load1(a.x, a.xdt, in0) * (a.fb ? bf16r(g) : g));
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
    int64_t groups;    // B*N*H*D / VE
    FastDiv gpt;       // groups per token = H*D/VE
    FastDiv gph;       // groups per head = D/VE
    FastDiv n_div;     // N
    FastDiv sb_div;    // MBRT_GATE_TPW * groups per token
    int tpw_ok;        // B * N is a multiple of MBRT_GATE_TPW
    int fb;            // bf16 intermediates (element kernel; the vector kernel takes FB)
};

template <int ADT, int GDT, int ODT, bool FB>
__global__ __launch_bounds__(kThreads) void gate_merge_vec_kernel(GateArgs a) {
    constexpr int VE = (ADT == F32 || ODT == F32) ? 4 : 8;
    // chunks of kThreads * kUGate groups; a grid smaller than the chunk count walks them
    const int64_t chunks = ceil_div_dev(a.groups, (int64_t)kThreads * kUGate);
    for (int64_t chunk = blockIdx.x; chunk < chunks; chunk += gridDim.x) {
    const int64_t base = chunk * (kThreads * kUGate) + threadIdx.x;
    Vec<ADT, VE> av[kUGate];
    float gl[kUGate];
    int64_t dst[kUGate];
#pragma unroll
    for (int u = 0; u < kUGate; ++u) {
        const uint32_t g = (uint32_t)clamp_group(base + u * kThreads, a.groups);
        uint32_t token, rem, h, c;
        int64_t src;
        if (MBRT_GATE_TPW > 1 && a.tpw_ok && a.layout == MBRT_LAYOUT_BHND) {
            // super-blocks of TPW tokens x all heads; within one, c fastest, then the token,
            // then the head: a head's TPW rows are read as one run of TPW * D elements, and
            // each token row is written in runs of (heads covered) * D
            uint32_t sb, r, r2, ti, b, n;
            fdivmod(g, a.sb_div, sb, r);
            fdivmod(r, a.gph, r2, c);
            h = r2 / MBRT_GATE_TPW;
            ti = r2 - h * MBRT_GATE_TPW;
            token = sb * MBRT_GATE_TPW + ti;
            fdivmod(token, a.n_div, b, n);
            src = (((int64_t)b * a.H + h) * a.N + n) * a.D + (int64_t)c * VE;
            dst[u] = (((int64_t)token * a.H + h) * a.gph.d + c) * VE;
        } else {
            fdivmod(g, a.gpt, token, rem);
            fdivmod(rem, a.gph, h, c);
            if (a.layout == MBRT_LAYOUT_BHND) {
                uint32_t b, n;
                fdivmod(token, a.n_div, b, n);
                src = (((int64_t)b * a.H + h) * a.N + n) * a.D + (int64_t)c * VE;
            } else {
                src = (int64_t)g * VE;
            }
            dst[u] = (int64_t)g * VE;
        }
        av[u].template load<MBRT_NT_GATE>(a.attn, src);
        gl[u] = ld1<GDT>(a.gate, (int64_t)token * a.H + h);
    }
#pragma unroll
    for (int u = 0; u < kUGate; ++u) {
        const int64_t g = base + u * kThreads;
        if (g < a.groups) {
            float v[VE];
            av[u].to_f32(v);
            float gv = a.logit ? sigmoidf(gl[u]) : gl[u];
            if constexpr (FB) gv = bf16r(gv);
#pragma unroll
            for (int i = 0; i < VE; ++i) v[i] = FB ? bf16r(v[i] * gv) : v[i] * gv;
            Vec<ODT, VE> o;
            o.from_f32(v);
            o.template store<MBRT_NT_GATE>(a.out, dst[u]);
        }
    }
    }
}

__global__ __launch_bounds__(kThreads) void gate_merge_elem_kernel(GateArgs a) {
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
        const float gl = load1(a.gate, a.gdt, token * a.H + h);
        const float g = a.logit ? sigmoidf(gl) : gl;
        const float y = a.fb ? bf16r(load1(a.attn, a.adt, src) * bf16r(g)) : load1(a.attn, a.adt, src) * g;
        store1(a.out, a.odt, i, y);
    }
}

inline dim3 elem_grid(int64_t n) { return dim3((unsigned)std::min<int64_t>(std::max<int64_t>(1, ceil_div(n, kThreads)), 1 << 20)); }
inline dim3 vec_grid(int64_t groups, int u = kU) {
    return dim3((unsigned)std::max<int64_t>(1, ceil_div(groups, (int64_t)kThreads * u)));
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
    a.act = act;
    a.n = rows * cols;
    a.cols = cols;
    if (a.n == 0) return MBRT_OK;
    MBRT_REQUIRE(x && out, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    // In place with a wider output than input would overwrite unread input.
    MBRT_REQUIRE(x != out || dt_size(x_dtype) == dt_size(out_dtype), MBRT_E_INVALID_ARG,
                 "%s: in-place needs equal element sizes", op);
    hipStream_t st = as_stream(stream);
    const int ve = (x_dtype == F32 || out_dtype == F32 || (bias != nullptr && bias_dtype == F32)) ? 4 : 8;
    const bool vec = aligned(x, 16) && aligned(out, 16) &&
                     (bias == nullptr || (aligned(bias, 16) && cols % ve == 0 && a.n < (1ll << 32)));
    if (vec) {
        if (bias != nullptr) a.cols_div = make_fastdiv((uint32_t)cols);
        const dim3 grid = vec_grid(a.n / ve);
        // the two GELU forms (the model's activations) get kernels of their own
        auto launch = [&](auto act_tag) {
            constexpr int A = decltype(act_tag)::value;
            with_dt(x_dtype, [&](auto xt) {
                with_dt(out_dtype, [&](auto ot) {
                    constexpr int X = decltype(xt)::value, O = decltype(ot)::value;
                    if (bias == nullptr)
                        hipLaunchKernelGGL((bias_act_vec_kernel<X, O, kNoBias, A>), grid, dim3(kThreads), 0, st, a);
                    else if (bias_dtype == F32)
                        hipLaunchKernelGGL((bias_act_vec_kernel<X, O, F32, A>), grid, dim3(kThreads), 0, st, a);
                    else
                        hipLaunchKernelGGL((bias_act_vec_kernel<X, O, BF16, A>), grid, dim3(kThreads), 0, st, a);
                });
            });
        };
        if (act == MBRT_ACT_GELU_REF) launch(std::integral_constant<int, MBRT_ACT_GELU_REF>{});
        else if (act == MBRT_ACT_GELU_STD) launch(std::integral_constant<int, MBRT_ACT_GELU_STD>{});
        else launch(std::integral_constant<int, -1>{});
    } else {
        hipLaunchKernelGGL(bias_act_elem_kernel, elem_grid(a.n), dim3(kThreads), 0, st, a);
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
    a.fb = bf16_intermediates() && x_dtype == BF16 && out_dtype == BF16;
    hipStream_t st = as_stream(stream);
    const int ve = (x_dtype == F32 || out_dtype == F32) ? 4 : 8;
    const bool vec = half_dim % ve == 0 && aligned(x, 16) && aligned(out, 16) && rows * half_dim / ve < (1ll << 32);
    if (vec) {
        a.groups = rows * half_dim / ve;
        a.gpr = make_fastdiv((uint32_t)(half_dim / ve));
        with_dt(x_dtype, [&](auto xt) {
            with_dt(out_dtype, [&](auto ot) {
                constexpr int X = decltype(xt)::value, O = decltype(ot)::value;
                if constexpr (X == BF16 && O == BF16) {
                    if (a.fb) {
                        hipLaunchKernelGGL((glu_vec_kernel<X, O, true>), vec_grid(a.groups, kUGlu), dim3(kThreads), 0, st, a);
                        return;
                    }
                }
                hipLaunchKernelGGL((glu_vec_kernel<X, O, false>), vec_grid(a.groups, kUGlu), dim3(kThreads), 0, st, a);
            });
        });
    } else {
        hipLaunchKernelGGL(glu_elem_kernel, elem_grid(rows * half_dim), dim3(kThreads), 0, st, a);
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
    // bf16 intermediates: the reference's gate merge kernels take the flag for bf16 attention
    a.fb = bf16_intermediates() && attn_dtype == BF16;
    hipStream_t st = as_stream(stream);
    const int ve = (attn_dtype == F32 || out_dtype == F32) ? 4 : 8;
    const bool vec = D % ve == 0 && aligned(attn, 16) && aligned(merged, 16) && total / ve < (1ll << 32) &&
                     B * N < (1ll << 31);
    if (vec) {
        a.groups = total / ve;
        a.gpt = make_fastdiv((uint32_t)(H * D / ve));
        a.gph = make_fastdiv((uint32_t)(D / ve));
        a.n_div = make_fastdiv((uint32_t)N);
        a.sb_div = make_fastdiv((uint32_t)(MBRT_GATE_TPW * H * D / ve));
        a.tpw_ok = (B * N) % MBRT_GATE_TPW == 0 ? 1 : 0;
        with_dt(attn_dtype, [&](auto at) {
            with_dt(gate_dtype, [&](auto gt) {
                with_dt(out_dtype, [&](auto ot) {
                    constexpr int A = decltype(at)::value, G = decltype(gt)::value, O = decltype(ot)::value;
                    dim3 grid = vec_grid(a.groups, kUGate);
                    if (MBRT_GATE_BPC > 0) grid.x = (unsigned)std::min<int64_t>(grid.x, (int64_t)cu_count() * MBRT_GATE_BPC);
                    if constexpr (A == BF16) {
                        if (a.fb) {
                            hipLaunchKernelGGL((gate_merge_vec_kernel<A, G, O, true>), grid, dim3(kThreads), 0, st, a);
                            return;
                        }
                    }
                    hipLaunchKernelGGL((gate_merge_vec_kernel<A, G, O, false>), grid, dim3(kThreads), 0, st, a);
                });
            });
        });
    } else {
        hipLaunchKernelGGL(gate_merge_elem_kernel, elem_grid(total), dim3(kThreads), 0, st, a);
    }
    return check_launch(op);
}

}  // extern "C"
