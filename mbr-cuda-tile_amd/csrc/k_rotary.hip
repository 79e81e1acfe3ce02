// Rotary position embedding (src/mbr_cuda_tile.cu:3897-4458, 7454-7530).
// Interleaved pairs: for pair i of a head vector at position n,
//   (x0, x1) -> (x0 c - x1 s, x0 s + x1 c),  c = cos[n, i], s = sin[n, i].
//
// In-place kernel: one thread rotates an 8-element (4-pair) group of q and the same group
// of k, with one 16-byte load and store each (bf16) and the 4 matching cos/sin values
// read from the [n_pos, D/2] tables, which stay L2-resident (801 x 32 x 4 B = 100 KB each)
// while being broadcast over batch*heads.  The position of a row is row % n_pos for
// [B*H, N, D] and (row / H) % n_pos for [B, N, H, D].
#include "abi_common.hpp"

#include <algorithm>

namespace mbrt {
namespace {

constexpr int kThreads = 256;

struct RotArgs {
    void* q;
    void* k;
    int dt, tdt;
    const void* cosp;
    const void* sinp;
    int64_t rows, n_pos, heads;
    int D;
    int layout;
    uint32_t groups;   // rows * D / 8
    FastDiv gpr;       // groups per row (D / 8)
    FastDiv npos_div;
    FastDiv heads_div;
};

__device__ __forceinline__ void rotate8(float (&x)[8], const float (&c)[4], const float (&s)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float x0 = x[2 * i], x1 = x[2 * i + 1];
        x[2 * i] = x0 * c[i] - x1 * s[i];
        x[2 * i + 1] = x0 * s[i] + x1 * c[i];
    }
}

__global__ __launch_bounds__(kThreads) void rotary_vec_kernel(RotArgs a) {
    const uint32_t g = blockIdx.x * kThreads + threadIdx.x;
    if (g >= a.groups) return;
    uint32_t row, c;
    fdivmod(g, a.gpr, row, c);
    uint32_t pos_row = row;
    if (a.layout == MBRT_LAYOUT_BNHD) pos_row = fdiv(row, a.heads_div);
    const uint32_t n = pos_row - fdiv(pos_row, a.npos_div) * a.npos_div.d;
    const int64_t t = (int64_t)n * (a.D / 2) + (int64_t)c * 4;
    float cs[4], sn[4];
    load4(a.cosp, a.tdt, t, cs);
    load4(a.sinp, a.tdt, t, sn);
    const int64_t e = (int64_t)g * 8;
    float x[8];
    load8(a.q, a.dt, e, x);
    if (a.k != nullptr) {
        float y[8];
        load8(a.k, a.dt, e, y);
        rotate8(x, cs, sn);
        rotate8(y, cs, sn);
        store8(a.q, a.dt, e, x);
        store8(a.k, a.dt, e, y);
    } else {
        rotate8(x, cs, sn);
        store8(a.q, a.dt, e, x);
    }
}

__global__ __launch_bounds__(kThreads) void rotary_scalar_kernel(RotArgs a) {
    const int half = a.D / 2;
    const int64_t pairs = a.rows * half;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < pairs; i += (int64_t)gridDim.x * kThreads) {
        const int64_t row = i / half, p = i - row * half;
        int64_t pos_row = a.layout == MBRT_LAYOUT_BNHD ? row / a.heads : row;
        const int64_t n = pos_row % a.n_pos;
        const float c = load1(a.cosp, a.tdt, n * half + p), s = load1(a.sinp, a.tdt, n * half + p);
        const int64_t e = row * a.D + 2 * p;
        for (int t = 0; t < 2; ++t) {
            void* buf = t == 0 ? a.q : a.k;
            if (buf == nullptr) continue;
            const float x0 = load1(buf, a.dt, e), x1 = load1(buf, a.dt, e + 1);
            store1(buf, a.dt, e, x0 * c - x1 * s);
            store1(buf, a.dt, e + 1, x0 * s + x1 * c);
        }
    }
}

// ---- split fused qkv + rotary --------------------------------------------------------

struct SplitArgs {
    const void* qkv;
    void* q;
    void* k;
    void* v;
    int idt, tdt, odt;
    const void* cosp;
    const void* sinp;
    int64_t B, N, H, D, outN;
};

// One thread per 8-element group of the [B, H, outN, D] outputs (q, k and v together).
__global__ __launch_bounds__(kThreads) void split_qkv_vec_kernel(SplitArgs a, uint32_t groups, FastDiv gpr,
                                                          FastDiv outn_div, FastDiv h_div) {
    const uint32_t g = blockIdx.x * kThreads + threadIdx.x;
    if (g >= groups) return;
    uint32_t orow, c, bh, n, b, h;
    fdivmod(g, gpr, orow, c);        // orow = (b*H + h)*outN + n
    fdivmod(orow, outn_div, bh, n);
    fdivmod(bh, h_div, b, h);
    const int64_t e = (int64_t)g * 8;
    float xq[8], xk[8], xv[8];
    if ((int64_t)n < a.N) {
        const int64_t src = ((int64_t)b * a.N + n) * (3 * a.H * a.D) + (int64_t)h * a.D + (int64_t)c * 8;
        load8(a.qkv, a.idt, src, xq);
        load8(a.qkv, a.idt, src + a.H * a.D, xk);
        load8(a.qkv, a.idt, src + 2 * a.H * a.D, xv);
        float cs[4], sn[4];
        const int64_t t = (int64_t)n * (a.D / 2) + (int64_t)c * 4;
        load4(a.cosp, a.tdt, t, cs);
        load4(a.sinp, a.tdt, t, sn);
        rotate8(xq, cs, sn);
        rotate8(xk, cs, sn);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) xq[i] = xk[i] = xv[i] = 0.0f;
    }
    store8(a.q, a.odt, e, xq);
    store8(a.k, a.odt, e, xk);
    store8(a.v, a.odt, e, xv);
}

__global__ __launch_bounds__(kThreads) void split_qkv_scalar_kernel(SplitArgs a) {
    const int half = (int)(a.D / 2);
    const int64_t pairs = a.B * a.H * a.outN * half;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < pairs; i += (int64_t)gridDim.x * kThreads) {
        const int64_t orow = i / half, p = i - orow * half;
        const int64_t n = orow % a.outN, bh = orow / a.outN;
        const int64_t h = bh % a.H, b = bh / a.H;
        const int64_t e = orow * a.D + 2 * p;
        if (n < a.N) {
            const int64_t src = (b * a.N + n) * (3 * a.H * a.D) + h * a.D + 2 * p;
            const float c = load1(a.cosp, a.tdt, n * half + p), s = load1(a.sinp, a.tdt, n * half + p);
            for (int part = 0; part < 3; ++part) {
                void* dst = part == 0 ? a.q : part == 1 ? a.k : a.v;
                const float x0 = load1(a.qkv, a.idt, src + part * a.H * a.D);
                const float x1 = load1(a.qkv, a.idt, src + part * a.H * a.D + 1);
                if (part < 2) {
                    store1(dst, a.odt, e, x0 * c - x1 * s);
                    store1(dst, a.odt, e + 1, x0 * s + x1 * c);
                } else {
                    store1(dst, a.odt, e, x0);
                    store1(dst, a.odt, e + 1, x1);
                }
            }
        } else {
            for (int part = 0; part < 3; ++part) {
                void* dst = part == 0 ? a.q : part == 1 ? a.k : a.v;
                store1(dst, a.odt, e, 0.0f);
                store1(dst, a.odt, e + 1, 0.0f);
            }
        }
    }
}

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_rotary_inplace(void* q, void* k, int dtype, const void* cos_table, const void* sin_table, int trig_dtype,
                        int64_t rows, int64_t n_pos, int64_t heads, int64_t dim_head, int layout,
                        mbrt_stream_t stream) {
    const char* op = "mbrt_rotary_inplace";
    MBRT_REQUIRE_FLOAT_DT(dtype, op);
    MBRT_REQUIRE(trig_dtype == F32 || trig_dtype == BF16, MBRT_E_UNSUPPORTED_DTYPE, "%s: trig dtype %d", op,
                 trig_dtype);
    MBRT_REQUIRE(layout == MBRT_LAYOUT_BHND || layout == MBRT_LAYOUT_BNHD, MBRT_E_INVALID_ARG, "%s: bad layout", op);
    MBRT_REQUIRE(dim_head >= 2 && dim_head % 2 == 0, MBRT_E_SHAPE, "%s: dim_head must be even", op);
    MBRT_REQUIRE(rows >= 0 && n_pos >= 1 && heads >= 1, MBRT_E_SHAPE, "%s: bad shape", op);
    if (rows == 0) return MBRT_OK;
    MBRT_REQUIRE(q && cos_table && sin_table, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    RotArgs a{};
    a.q = q;
    a.k = k;
    a.dt = dtype;
    a.tdt = trig_dtype;
    a.cosp = cos_table;
    a.sinp = sin_table;
    a.rows = rows;
    a.n_pos = n_pos;
    a.heads = heads;
    a.D = (int)dim_head;
    a.layout = layout;
    hipStream_t st = as_stream(stream);
    const int64_t groups = rows * dim_head / 8;
    const bool tab_al = trig_dtype == F32 ? (aligned(cos_table, 16) && aligned(sin_table, 16))
                                          : (aligned(cos_table, 8) && aligned(sin_table, 8));
    const bool vec = dim_head % 8 == 0 && aligned(q, 16) && (k == nullptr || aligned(k, 16)) && tab_al &&
                     groups < (1ll << 32) && rows < (1ll << 31);
    if (vec) {
        a.groups = (uint32_t)groups;
        a.gpr = make_fastdiv((uint32_t)(dim_head / 8));
        a.npos_div = make_fastdiv((uint32_t)n_pos);
        a.heads_div = make_fastdiv((uint32_t)heads);
        hipLaunchKernelGGL(rotary_vec_kernel, dim3((unsigned)ceil_div(groups, kThreads)), dim3(kThreads), 0, st, a);
    } else {
        const int64_t pairs = rows * dim_head / 2;
        hipLaunchKernelGGL(rotary_scalar_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(pairs, kThreads), 1 << 20)),
                           dim3(kThreads), 0, st, a);
    }
    return check_launch(op);
}

int mbrt_split_qkv_heads_rotary(const void* qkv, int qkv_dtype, const void* cos_table, const void* sin_table,
                                int trig_dtype, void* q, void* k, void* v, int out_dtype, int64_t B, int64_t N,
                                int64_t H, int64_t D, int64_t out_N, mbrt_stream_t stream) {
    const char* op = "mbrt_split_qkv_heads_rotary";
    MBRT_REQUIRE_FLOAT_DT(qkv_dtype, op);
    MBRT_REQUIRE_FLOAT_DT(out_dtype, op);
    MBRT_REQUIRE(trig_dtype == F32 || trig_dtype == BF16, MBRT_E_UNSUPPORTED_DTYPE, "%s: trig dtype %d", op,
                 trig_dtype);
    MBRT_REQUIRE(D >= 2 && D % 2 == 0, MBRT_E_SHAPE, "%s: dim_head must be even", op);
    MBRT_REQUIRE(B >= 0 && N >= 0 && H >= 1 && out_N >= N, MBRT_E_SHAPE, "%s: bad shape", op);
    const int64_t total = B * H * out_N * D;
    if (total == 0) return MBRT_OK;
    MBRT_REQUIRE(qkv && q && k && v && cos_table && sin_table, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    SplitArgs a{};
    a.qkv = qkv;
    a.q = q;
    a.k = k;
    a.v = v;
    a.idt = qkv_dtype;
    a.tdt = trig_dtype;
    a.odt = out_dtype;
    a.cosp = cos_table;
    a.sinp = sin_table;
    a.B = B;
    a.N = N;
    a.H = H;
    a.D = D;
    a.outN = out_N;
    hipStream_t st = as_stream(stream);
    const int64_t groups = total / 8;
    const bool tab_al = trig_dtype == F32 ? (aligned(cos_table, 16) && aligned(sin_table, 16))
                                          : (aligned(cos_table, 8) && aligned(sin_table, 8));
    const bool vec = D % 8 == 0 && aligned(qkv, 16) && aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && tab_al &&
                     groups < (1ll << 32);
    if (vec) {
        hipLaunchKernelGGL(split_qkv_vec_kernel, dim3((unsigned)ceil_div(groups, kThreads)), dim3(kThreads), 0, st, a,
                           (uint32_t)groups, make_fastdiv((uint32_t)(D / 8)), make_fastdiv((uint32_t)out_N),
                           make_fastdiv((uint32_t)H));
    } else {
        const int64_t pairs = total / 2;
        hipLaunchKernelGGL(split_qkv_scalar_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(pairs, kThreads), 1 << 20)),
                           dim3(kThreads), 0, st, a);
    }
    return check_launch(op);
}

}  // extern "C"
