// Flat element-wise kernels of the tensor library (src/tensor_cuda_tile.cu:51-339 and the
// broadcast binary of src/tensor_cuda_glue.cu:57-114).
//
// The vector kernels are templated on the dtypes: every thread owns kU groups of VE
// elements (16 bytes of its widest operand), issues all of its loads first (group indices
// clamped into the array, so no load is predicated), then converts, computes and stores
// with a predicate.  The n % VE tail is handled element-wise by block 0 in the same launch.
// Operands that are not 16-byte aligned use runtime-dtype element kernels.  The broadcast
// binary replaces per-element 64-bit div/mod over 8 dims with 32-bit multiply-shift
// division over the (merged) output dims.
#include "abi_common.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace mbrt {
namespace {

constexpr int kThreads = 256;
constexpr int kU = MBRT_EW_U;  // 16-byte groups per thread

// ---- fill / arange ------------------------------------------------------------------

template <int E>
__global__ __launch_bounds__(kThreads) void fill_kernel(void* dst, int64_t n, uint64_t bits, int vec) {
    typedef typename std::conditional<E == 8, uint64_t, typename std::conditional<E == 4, uint32_t, uint16_t>::type>::type T;
    const T v = (T)bits;
    T* d = static_cast<T*>(dst);
    if (vec) {
        constexpr int PER = 16 / E;
        const int64_t groups = n / PER;
        const int64_t base = (int64_t)blockIdx.x * (kThreads * kU) + threadIdx.x;
        T pat[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) pat[i] = v;
        u32x4 w;
        __builtin_memcpy(&w, pat, 16);
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            int64_t g = base + u * kThreads;
            if (g < groups) reinterpret_cast<u32x4*>(d)[g] = w;
        }
        if (blockIdx.x == 0) {
            int64_t e = groups * PER + threadIdx.x;
            if (e < n) d[e] = v;
        }
    } else {
        int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
        for (; i < n; i += (int64_t)gridDim.x * kThreads) d[i] = v;
    }
}

__global__ __launch_bounds__(kThreads) void arange_kernel(void* dst, int dt, int64_t n, int64_t start) {
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < n; i += (int64_t)gridDim.x * kThreads) {
        int64_t v = start + i;
        if (dt == I64) reinterpret_cast<int64_t*>(dst)[i] = v;
        else if (dt == I32) reinterpret_cast<int32_t*>(dst)[i] = (int32_t)v;
        else store1(dst, dt, i, (float)v);
    }
}

// ---- typed vector kernels ---------------------------------------------------------------

#define MBRT_FLAT_PROLOGUE(VE_)                                                   \
    constexpr int VE = (VE_);                                                     \
    const int64_t groups = n / VE;                                                \
    const int64_t base = (int64_t)blockIdx.x * (kThreads * kU) + threadIdx.x;

__device__ __forceinline__ int64_t clamp_group(int64_t g, int64_t groups) { return g < groups ? g : groups - 1; }

template <int SDT, int DDT>
__global__ __launch_bounds__(kThreads) void convert_vec_kernel(const void* src, void* dst, int64_t n) {
    MBRT_FLAT_PROLOGUE((SDT == F32 || DDT == F32) ? 4 : 8)
    if (groups > 0) {
        Vec<SDT, VE> v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) v[u].template load<MBRT_NT_EW>(src, clamp_group(base + u * kThreads, groups) * VE);
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t g = base + u * kThreads;
            if (g < groups) {
                float f[VE];
                v[u].to_f32(f);
                Vec<DDT, VE> o;
                o.from_f32(f);
                o.template store<MBRT_NT_EW>(dst, g * VE);
            }
        }
    }
    if (blockIdx.x == 0) {
        const int64_t e = groups * VE + threadIdx.x;
        if (e < n) st1<DDT>(dst, e, ld1<SDT>(src, e));
    }
}

__device__ __forceinline__ float scalar_fn(float x, int op, float a, float b) {
    if (op == MBRT_SCALAR_ADD) return x + a;
    if (op == MBRT_SCALAR_MUL) return x * a;
    return fminf(fmaxf(x, a), b);
}

__device__ __forceinline__ float unary_fn(float x, int op, float value) {
    if (op == MBRT_UNARY_NEG) return -x;
    return x > value ? 1.0f : 0.0f;
}

// In-place scalar ops (op code runs after the loads) and out-of-place unary ops.
template <int DT, bool UNARY>
__global__ __launch_bounds__(kThreads) void map_vec_kernel(const void* src, void* dst, int64_t n, int op, float a,
                                                     float b) {
    MBRT_FLAT_PROLOGUE(ve_for<DT>())
    if (groups > 0) {
        Vec<DT, VE> v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) v[u].template load<MBRT_NT_EW>(src, clamp_group(base + u * kThreads, groups) * VE);
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t g = base + u * kThreads;
            if (g < groups) {
                float f[VE];
                v[u].to_f32(f);
#pragma unroll
                for (int i = 0; i < VE; ++i) f[i] = UNARY ? unary_fn(f[i], op, a) : scalar_fn(f[i], op, a, b);
                v[u].from_f32(f);
                v[u].template store<MBRT_NT_EW>(dst, g * VE);
            }
        }
    }
    if (blockIdx.x == 0) {
        const int64_t e = groups * VE + threadIdx.x;
        if (e < n) {
            const float x = ld1<DT>(src, e);
            st1<DT>(dst, e, UNARY ? unary_fn(x, op, a) : scalar_fn(x, op, a, b));
        }
    }
}

// ---- runtime-dtype element kernels (unaligned operands, integer conversions) ---------

__global__ __launch_bounds__(kThreads) void convert_elem_kernel(const void* src, int sdt, void* dst, int ddt,
                                                         int64_t n) {
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < n; i += (int64_t)gridDim.x * kThreads) {
        if (sdt == I64 || sdt == I32) {
            const int64_t v = sdt == I64 ? reinterpret_cast<const int64_t*>(src)[i]
                                         : (int64_t)reinterpret_cast<const int32_t*>(src)[i];
            if (ddt == I64) reinterpret_cast<int64_t*>(dst)[i] = v;
            else if (ddt == I32) reinterpret_cast<int32_t*>(dst)[i] = (int32_t)v;
            else store1(dst, ddt, i, (float)v);
        } else {
            const float f = load1(src, sdt, i);
            // float -> int truncates toward zero, as a C cast
            if (ddt == I64) reinterpret_cast<int64_t*>(dst)[i] = (int64_t)f;
            else if (ddt == I32) reinterpret_cast<int32_t*>(dst)[i] = (int32_t)f;
            else store1(dst, ddt, i, f);
        }
    }
}

__global__ __launch_bounds__(kThreads) void map_elem_kernel(const void* src, void* dst, int dt, int64_t n, int op,
                                                     float a, float b, int unary) {
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < n; i += (int64_t)gridDim.x * kThreads) {
        const float x = load1(src, dt, i);
        store1(dst, dt, i, unary ? unary_fn(x, op, a) : scalar_fn(x, op, a, b));
    }
}

inline dim3 elem_grid(int64_t n) { return dim3((unsigned)std::min<int64_t>(std::max<int64_t>(1, ceil_div(n, kThreads)), 1 << 20)); }
inline dim3 vec_grid(int64_t n, int ve) { return dim3((unsigned)std::max<int64_t>(1, ceil_div(n / ve, (int64_t)kThreads * kU))); }

// ---- binary -------------------------------------------------------------------------

template <int OP>
__device__ __forceinline__ float binop(float x, float y) {
    if (OP == MBRT_ADD) return x + y;
    if (OP == MBRT_SUB) return x - y;
    if (OP == MBRT_MUL) return x * y;
    return x / y;
}

template <int OP, int DT>
__global__ __launch_bounds__(kThreads) void binary_vec_kernel(const void* a, const void* b, void* out, int64_t n) {
    MBRT_FLAT_PROLOGUE(ve_for<DT>())
    if (groups > 0) {
        Vec<DT, VE> va[kU], vb[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t g = clamp_group(base + u * kThreads, groups) * VE;
            va[u].template load<MBRT_NT_EW>(a, g);
            vb[u].template load<MBRT_NT_EW>(b, g);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t g = base + u * kThreads;
            if (g < groups) {
                float x[VE], y[VE];
                va[u].to_f32(x);
                vb[u].to_f32(y);
#pragma unroll
                for (int i = 0; i < VE; ++i) x[i] = binop<OP>(x[i], y[i]);
                va[u].from_f32(x);
                va[u].template store<MBRT_NT_EW>(out, g * VE);
            }
        }
    }
    if (blockIdx.x == 0) {
        const int64_t e = groups * VE + threadIdx.x;
        if (e < n) st1<DT>(out, e, binop<OP>(ld1<DT>(a, e), ld1<DT>(b, e)));
    }
}

template <int OP>
__global__ __launch_bounds__(kThreads) void binary_elem_kernel(const void* a, const void* b, void* out, int dt,
                                                        int64_t n) {
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < n; i += (int64_t)gridDim.x * kThreads) store1(out, dt, i, binop<OP>(load1(a, dt, i), load1(b, dt, i)));
}

struct BcastArgs {
    const void* a;
    const void* b;
    void* out;
    int dt;
    uint32_t total;
    int nd;
    FastDiv shape[MBRT_MAX_DIMS];  // innermost first
    int64_t sa[MBRT_MAX_DIMS];
    int64_t sb[MBRT_MAX_DIMS];
};

template <int OP>
__global__ __launch_bounds__(kThreads) void bcast_kernel(BcastArgs p) {
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= p.total) return;
    uint32_t rem = i;
    int64_t oa = 0, ob = 0;
#pragma unroll
    for (int d = 0; d < MBRT_MAX_DIMS; ++d) {
        if (d < p.nd) {
            uint32_t q, r;
            fdivmod(rem, p.shape[d], q, r);
            oa += (int64_t)r * p.sa[d];
            ob += (int64_t)r * p.sb[d];
            rem = q;
        }
    }
    store1(p.out, p.dt, i, binop<OP>(load1(p.a, p.dt, oa), load1(p.b, p.dt, ob)));
}

struct BcastArgs64 {
    const void* a;
    const void* b;
    void* out;
    int dt;
    int64_t total;
    int nd;
    int64_t shape[MBRT_MAX_DIMS];  // innermost first
    int64_t sa[MBRT_MAX_DIMS];
    int64_t sb[MBRT_MAX_DIMS];
};

template <int OP>
__global__ __launch_bounds__(kThreads) void bcast_kernel64(BcastArgs64 p) {
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < p.total; i += (int64_t)gridDim.x * kThreads) {
        int64_t rem = i, oa = 0, ob = 0;
        for (int d = 0; d < p.nd; ++d) {
            int64_t q = rem / p.shape[d];
            int64_t r = rem - q * p.shape[d];
            oa += r * p.sa[d];
            ob += r * p.sb[d];
            rem = q;
        }
        store1(p.out, p.dt, i, binop<OP>(load1(p.a, p.dt, oa), load1(p.b, p.dt, ob)));
    }
}

template <class F>
int dispatch_op(int op, F f) {
    switch (op) {
        case MBRT_ADD: f(std::integral_constant<int, MBRT_ADD>()); break;
        case MBRT_SUB: f(std::integral_constant<int, MBRT_SUB>()); break;
        case MBRT_MUL: f(std::integral_constant<int, MBRT_MUL>()); break;
        default: f(std::integral_constant<int, MBRT_DIV>()); break;
    }
    return MBRT_OK;
}

// 2-byte vector path needs 16B alignment, f32 needs 16B as well (two 16B accesses).
inline bool vec_ok(const void* p) { return aligned(p, 16); }

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_fill(void* dst, int dtype, int64_t n, double value, mbrt_stream_t stream) {
    const char* op = "mbrt_fill";
    MBRT_REQUIRE(is_valid_dt(dtype), MBRT_E_UNSUPPORTED_DTYPE, "%s: bad dtype %d", op, dtype);
    MBRT_REQUIRE(n >= 0, MBRT_E_SHAPE, "%s: negative size", op);
    if (n == 0) return MBRT_OK;
    MBRT_REQUIRE(dst != nullptr, MBRT_E_INVALID_ARG, "%s: NULL dst", op);
    uint64_t bits = 0;
    switch (dtype) {
        case F32: { float f = (float)value; uint32_t b; std::memcpy(&b, &f, 4); bits = b; break; }
        case F16: { _Float16 h = (_Float16)(float)value; uint16_t b; std::memcpy(&b, &h, 2); bits = b; break; }
        case BF16: { __bf16 h = (__bf16)(float)value; uint16_t b; std::memcpy(&b, &h, 2); bits = b; break; }
        case I64: { int64_t v = (int64_t)value; std::memcpy(&bits, &v, 8); break; }
        default: { int32_t v = (int32_t)value; uint32_t b; std::memcpy(&b, &v, 4); bits = b; break; }
    }
    const int esz = dt_size(dtype);
    const int vec = aligned(dst, 16) ? 1 : 0;
    int64_t grid = vec ? std::max<int64_t>(1, ceil_div(n / (16 / esz), (int64_t)kThreads * kU))
                       : std::min<int64_t>(ceil_div(n, kThreads), 1 << 20);
    hipStream_t st = as_stream(stream);
    if (esz == 2) hipLaunchKernelGGL(fill_kernel<2>, dim3((unsigned)grid), dim3(kThreads), 0, st, dst, n, bits, vec);
    else if (esz == 4) hipLaunchKernelGGL(fill_kernel<4>, dim3((unsigned)grid), dim3(kThreads), 0, st, dst, n, bits, vec);
    else hipLaunchKernelGGL(fill_kernel<8>, dim3((unsigned)grid), dim3(kThreads), 0, st, dst, n, bits, vec);
    return check_launch(op);
}

int mbrt_arange(void* dst, int dtype, int64_t n, int64_t start, mbrt_stream_t stream) {
    const char* op = "mbrt_arange";
    MBRT_REQUIRE(is_valid_dt(dtype), MBRT_E_UNSUPPORTED_DTYPE, "%s: bad dtype %d", op, dtype);
    MBRT_REQUIRE(dtype != BF16, MBRT_E_UNSUPPORTED_DTYPE, "%s: unsupported BF16 dtype", op);
    MBRT_REQUIRE(n >= 0, MBRT_E_SHAPE, "%s: negative size", op);
    if (n == 0) return MBRT_OK;
    int64_t grid = std::min<int64_t>(ceil_div(n, kThreads), 1 << 20);
    hipLaunchKernelGGL(arange_kernel, dim3((unsigned)grid), dim3(kThreads), 0, as_stream(stream), dst, dtype, n, start);
    return check_launch(op);
}

int mbrt_convert(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, mbrt_stream_t stream) {
    const char* op = "mbrt_convert";
    MBRT_REQUIRE(is_valid_dt(src_dtype) && is_valid_dt(dst_dtype), MBRT_E_UNSUPPORTED_DTYPE,
                 "%s: bad dtype pair %d -> %d", op, src_dtype, dst_dtype);
    MBRT_REQUIRE(n >= 0, MBRT_E_SHAPE, "%s: negative size", op);
    if (n == 0) return MBRT_OK;
    hipStream_t st = as_stream(stream);
    if (is_float_dt(src_dtype) && is_float_dt(dst_dtype) && vec_ok(src) && vec_ok(dst)) {
        const int ve = (src_dtype == F32 || dst_dtype == F32) ? 4 : 8;
        with_dt(src_dtype, [&](auto sd) {
            with_dt(dst_dtype, [&](auto dd) {
                constexpr int S = decltype(sd)::value, D = decltype(dd)::value;
                hipLaunchKernelGGL((convert_vec_kernel<S, D>), vec_grid(n, ve), dim3(kThreads), 0, st, src, dst, n);
            });
        });
    } else {
        hipLaunchKernelGGL(convert_elem_kernel, elem_grid(n), dim3(kThreads), 0, st, src, src_dtype, dst, dst_dtype, n);
    }
    return check_launch(op);
}

int mbrt_scalar_op(void* data, int dtype, int64_t n, int op_code, float a, float b, mbrt_stream_t stream) {
    const char* op = "mbrt_scalar_op";
    MBRT_REQUIRE(dtype == F32 || dtype == F16, MBRT_E_UNSUPPORTED_DTYPE, "%s: unsupported dtype %d", op, dtype);
    MBRT_REQUIRE(op_code >= 0 && op_code <= 2, MBRT_E_INVALID_ARG, "%s: bad op %d", op, op_code);
    MBRT_REQUIRE(n >= 0, MBRT_E_SHAPE, "%s: negative size", op);
    if (n == 0) return MBRT_OK;
    hipStream_t st = as_stream(stream);
    if (vec_ok(data)) {
        if (dtype == F32) hipLaunchKernelGGL((map_vec_kernel<F32, false>), vec_grid(n, 4), dim3(kThreads), 0, st, data, data, n, op_code, a, b);
        else hipLaunchKernelGGL((map_vec_kernel<F16, false>), vec_grid(n, 8), dim3(kThreads), 0, st, data, data, n, op_code, a, b);
    } else {
        hipLaunchKernelGGL(map_elem_kernel, elem_grid(n), dim3(kThreads), 0, st, data, data, dtype, n, op_code, a, b, 0);
    }
    return check_launch(op);
}

int mbrt_unary(const void* src, void* dst, int dtype, int64_t n, int op_code, float value, mbrt_stream_t stream) {
    const char* op = "mbrt_unary";
    MBRT_REQUIRE(dtype == F32 || dtype == F16, MBRT_E_UNSUPPORTED_DTYPE, "%s: unsupported dtype %d", op, dtype);
    MBRT_REQUIRE(op_code == 0 || op_code == 1, MBRT_E_INVALID_ARG, "%s: bad op %d", op, op_code);
    MBRT_REQUIRE(n >= 0, MBRT_E_SHAPE, "%s: negative size", op);
    if (n == 0) return MBRT_OK;
    hipStream_t st = as_stream(stream);
    if (vec_ok(src) && vec_ok(dst)) {
        if (dtype == F32) hipLaunchKernelGGL((map_vec_kernel<F32, true>), vec_grid(n, 4), dim3(kThreads), 0, st, src, dst, n, op_code, value, 0.0f);
        else hipLaunchKernelGGL((map_vec_kernel<F16, true>), vec_grid(n, 8), dim3(kThreads), 0, st, src, dst, n, op_code, value, 0.0f);
    } else {
        hipLaunchKernelGGL(map_elem_kernel, elem_grid(n), dim3(kThreads), 0, st, src, dst, dtype, n, op_code, value, 0.0f, 1);
    }
    return check_launch(op);
}

int mbrt_binary(const void* a, const void* b, void* out, int dtype, int64_t n, int op_code, mbrt_stream_t stream) {
    const char* op = "mbrt_binary";
    MBRT_REQUIRE_FLOAT_DT(dtype, op);
    MBRT_REQUIRE(op_code >= 0 && op_code <= 3, MBRT_E_INVALID_ARG, "%s: bad op %d", op, op_code);
    MBRT_REQUIRE(n >= 0, MBRT_E_SHAPE, "%s: negative size", op);
    if (n == 0) return MBRT_OK;
    MBRT_REQUIRE(a && b && out, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    hipStream_t st = as_stream(stream);
    const bool vec = vec_ok(a) && vec_ok(b) && vec_ok(out);
    dispatch_op(op_code, [&](auto opc) {
        constexpr int OP = decltype(opc)::value;
        if (vec) {
            with_dt(dtype, [&](auto dtc) {
                constexpr int DT = decltype(dtc)::value;
                hipLaunchKernelGGL((binary_vec_kernel<OP, DT>), vec_grid(n, ve_for<DT>()), dim3(kThreads), 0, st, a, b,
                                   out, n);
            });
        } else {
            hipLaunchKernelGGL(binary_elem_kernel<OP>, elem_grid(n), dim3(kThreads), 0, st, a, b, out, dtype, n);
        }
    });
    return check_launch(op);
}

int mbrt_binary_broadcast(const void* a, const void* b, void* out, int dtype, const mbrt_broadcast_meta* meta,
                          int op_code, mbrt_stream_t stream) {
    const char* op = "mbrt_binary_broadcast";
    MBRT_REQUIRE(meta != nullptr, MBRT_E_INVALID_ARG, "%s: meta is NULL", op);
    MBRT_REQUIRE_FLOAT_DT(dtype, op);
    MBRT_REQUIRE(op_code >= 0 && op_code <= 3, MBRT_E_INVALID_ARG, "%s: bad op %d", op, op_code);
    MBRT_REQUIRE(meta->ndim >= 1 && meta->ndim <= MBRT_MAX_DIMS, MBRT_E_INVALID_ARG, "%s: ndim %d", op, meta->ndim);
    // merge adjacent dims that are contiguous in the output and in both operands
    int64_t shape[MBRT_MAX_DIMS], sa[MBRT_MAX_DIMS], sb[MBRT_MAX_DIMS];
    int nd = 0;
    int64_t total = 1;
    for (int d = 0; d < meta->ndim; ++d) {
        const int64_t n = meta->out_shape[d];
        MBRT_REQUIRE(n >= 0, MBRT_E_SHAPE, "%s: negative extent", op);
        total *= n;
        if (n == 1) continue;
        if (nd > 0 && sa[nd - 1] == meta->a_strides[d] * n && sb[nd - 1] == meta->b_strides[d] * n) {
            shape[nd - 1] *= n;
            sa[nd - 1] = meta->a_strides[d];
            sb[nd - 1] = meta->b_strides[d];
        } else {
            shape[nd] = n;
            sa[nd] = meta->a_strides[d];
            sb[nd] = meta->b_strides[d];
            ++nd;
        }
    }
    if (total == 0) return MBRT_OK;
    if (nd == 0) {
        nd = 1;
        shape[0] = 1;
        sa[0] = sb[0] = 0;
    }
    hipStream_t st = as_stream(stream);
    bool small = total < (1ll << 31);  // block * 256 + thread cannot wrap in 32 bits
    for (int d = 0; d < nd; ++d) small = small && shape[d] < (1ll << 31);
    dispatch_op(op_code, [&](auto opc) {
        constexpr int OP = decltype(opc)::value;
        if (small) {
            BcastArgs p;
            p.a = a;
            p.b = b;
            p.out = out;
            p.dt = dtype;
            p.total = (uint32_t)total;
            p.nd = nd;
            for (int d = 0; d < nd; ++d) {
                p.shape[d] = make_fastdiv((uint32_t)shape[nd - 1 - d]);
                p.sa[d] = sa[nd - 1 - d];
                p.sb[d] = sb[nd - 1 - d];
            }
            hipLaunchKernelGGL(bcast_kernel<OP>, dim3((unsigned)ceil_div(total, kThreads)), dim3(kThreads), 0, st, p);
        } else {
            BcastArgs64 p;
            p.a = a;
            p.b = b;
            p.out = out;
            p.dt = dtype;
            p.total = total;
            p.nd = nd;
            for (int d = 0; d < nd; ++d) {
                p.shape[d] = shape[nd - 1 - d];
                p.sa[d] = sa[nd - 1 - d];
                p.sb[d] = sb[nd - 1 - d];
            }
            int64_t grid = std::min<int64_t>(ceil_div(total, kThreads), 1 << 20);
            hipLaunchKernelGGL(bcast_kernel64<OP>, dim3((unsigned)grid), dim3(kThreads), 0, st, p);
        }
    });
    return check_launch(op);
}

}  // extern "C"
