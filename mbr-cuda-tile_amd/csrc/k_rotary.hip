// Rotary position embedding (src/mbr_cuda_tile.cu:3897-4458, 7454-7530).
// Interleaved pairs: for pair i of a head vector at position n,
//   (x0, x1) -> (x0 c - x1 s, x0 s + x1 c),  c = cos[n, i], s = sin[n, i].
//
// In-place kernel: one thread rotates a VE-element group of q (VE = 8 for bf16/f16: one
// 16-byte access; 4 for f32) and the same group of k, with the VE/2 matching cos/sin
// values read from the [n_pos, D/2] tables, which stay L2-resident (801 x 32 x 4 B = 100 KB each)
// while being broadcast over batch*heads.  The position of a row is row % n_pos for
// [B*H, N, D] and (row / H) % n_pos for [B, N, H, D].
// With MBRT_ARITH_BF16_INTERMEDIATES set and bf16 data, cos and sin are rounded to bf16
// before the rotation, as the reference's bf16 rotary kernels do in full-bf16 mode
// (src/mbr_cuda_tile.cu:4033-4060 and their in-place variants); with bf16 operands the
// products are exact in f32 and the rotated pair is rounded once, on its store.
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
    uint32_t groups;   // rows * D / VE
    FastDiv gpr;       // groups per row (D / VE)
    FastDiv npos_div;
    FastDiv heads_div;
    int fb;  // bf16 intermediates (scalar kernel; the vector kernel takes FB)
};

// One thread = one VE-element group (VE/2 pairs) of q and the same group of k.  All four
// loads (q, k, cos, sin) are issued before the rotation.
template <int DT, int TDT, bool HAS_K, bool FB>
__global__ __launch_bounds__(kThreads) void rotary_vec_kernel(RotArgs a) {
    constexpr int VE = ve_for<DT>();
    const uint32_t g = blockIdx.x * kThreads + threadIdx.x;
    if (g >= a.groups) return;
    uint32_t row, c;
    fdivmod(g, a.gpr, row, c);
    uint32_t pos_row = row;
    if (a.layout == MBRT_LAYOUT_BNHD) pos_row = fdiv(row, a.heads_div);
    const uint32_t n = pos_row - fdiv(pos_row, a.npos_div) * a.npos_div.d;
    const int64_t t = (int64_t)n * (a.D / 2) + (int64_t)c * (VE / 2);
    const int64_t e = (int64_t)g * VE;
    Vec<DT, VE> q, k;
    Vec<TDT, VE / 2> cv, sv;
    q.template load<MBRT_NT_ROT>(a.q, e);
    if (HAS_K) k.template load<MBRT_NT_ROT>(a.k, e);
    cv.load(a.cosp, t);
    sv.load(a.sinp, t);
    float cs[VE / 2], sn[VE / 2], x[VE];
    cv.to_f32(cs);
    sv.to_f32(sn);
    if constexpr (FB) {
#pragma unroll
        for (int i = 0; i < VE / 2; ++i) {
            cs[i] = bf16r(cs[i]);
            sn[i] = bf16r(sn[i]);
        }
    }
    q.to_f32(x);
    rotate<VE>(x, cs, sn);
    q.from_f32(x);
    q.template store<MBRT_NT_ROT>(a.q, e);
    if (HAS_K) {
        k.to_f32(x);
        rotate<VE>(x, cs, sn);
        k.from_f32(x);
        k.template store<MBRT_NT_ROT>(a.k, e);
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
        float c = load1(a.cosp, a.tdt, n * half + p), s = load1(a.sinp, a.tdt, n * half + p);
        if (a.fb) {
            c = bf16r(c);
            s = bf16r(s);
        }
        const int64_t e = row * a.D + 2 * p;
        for (int t = 0; t < 2; ++t) {
            void* buf = t == 0 ? a.q : a.k;
            if (buf == nullptr) continue;
            const float x0 = load1(buf, a.dt, e), x1 = load1(buf, a.dt, e + 1);
            float y0, y1;
            rotate_pair(x0, x1, c, s, y0, y1);
            store1(buf, a.dt, e, y0);
            store1(buf, a.dt, e + 1, y1);
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
    int fb;  // bf16 intermediates (scalar kernel; the vector kernel takes FB)
};

// One thread per VE-element group of the [B, H, outN, D] outputs (q, k and v together);
// the three qkv loads and the table loads are issued before any use.
template <int IDT, int ODT, int TDT, bool FB>
__global__ __launch_bounds__(kThreads) void split_qkv_vec_kernel(SplitArgs a, uint32_t groups, FastDiv gpr,
                                                          FastDiv outn_div, FastDiv h_div) {
    constexpr int VE = (IDT == F32 || ODT == F32) ? 4 : 8;
    const uint32_t g = blockIdx.x * kThreads + threadIdx.x;
    if (g >= groups) return;
    uint32_t orow, c, bh, n, b, h;
    fdivmod(g, gpr, orow, c);        // orow = (b*H + h)*outN + n
    fdivmod(orow, outn_div, bh, n);
    fdivmod(bh, h_div, b, h);
    const int64_t e = (int64_t)g * VE;
    const bool pad = (int64_t)n >= a.N;
    const int64_t nn = pad ? a.N - 1 : n;  // padded rows load a valid row and store zeros
    const int64_t src = ((int64_t)b * a.N + nn) * (3 * a.H * a.D) + (int64_t)h * a.D + (int64_t)c * VE;
    const int64_t t = nn * (a.D / 2) + (int64_t)c * (VE / 2);
    Vec<IDT, VE> vq, vk, vv;
    Vec<TDT, VE / 2> cv, sv;
    vq.template load<MBRT_NT_ROT>(a.qkv, src);
    vk.template load<MBRT_NT_ROT>(a.qkv, src + a.H * a.D);
    vv.template load<MBRT_NT_ROT>(a.qkv, src + 2 * a.H * a.D);
    cv.load(a.cosp, t);
    sv.load(a.sinp, t);
    float xq[VE], xk[VE], xv[VE], cs[VE / 2], sn[VE / 2];
    vq.to_f32(xq);
    vk.to_f32(xk);
    vv.to_f32(xv);
    cv.to_f32(cs);
    sv.to_f32(sn);
    if constexpr (FB) {
#pragma unroll
        for (int i = 0; i < VE / 2; ++i) {
            cs[i] = bf16r(cs[i]);
            sn[i] = bf16r(sn[i]);
        }
    }
    rotate<VE>(xq, cs, sn);
    rotate<VE>(xk, cs, sn);
    if (pad) {
#pragma unroll
        for (int i = 0; i < VE; ++i) xq[i] = xk[i] = xv[i] = 0.0f;
    }
    Vec<ODT, VE> o;
    o.from_f32(xq);
    o.template store<MBRT_NT_ROT>(a.q, e);
    o.from_f32(xk);
    o.template store<MBRT_NT_ROT>(a.k, e);
    o.from_f32(xv);
    o.template store<MBRT_NT_ROT>(a.v, e);
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
            float c = load1(a.cosp, a.tdt, n * half + p), s = load1(a.sinp, a.tdt, n * half + p);
            if (a.fb) {
                c = bf16r(c);
                s = bf16r(s);
            }
            for (int part = 0; part < 3; ++part) {
                void* dst = part == 0 ? a.q : part == 1 ? a.k : a.v;
                const float x0 = load1(a.qkv, a.idt, src + part * a.H * a.D);
                const float x1 = load1(a.qkv, a.idt, src + part * a.H * a.D + 1);
                if (part < 2) {
                    float y0, y1;
                    rotate_pair(x0, x1, c, s, y0, y1);
                    store1(dst, a.odt, e, y0);
                    store1(dst, a.odt, e + 1, y1);
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
    // bf16 intermediates: bf16 data; the rounding only changes f32 tables
    a.fb = bf16_intermediates() && dtype == BF16;
    hipStream_t st = as_stream(stream);
    const int ve = dtype == F32 ? 4 : 8;
    const int64_t groups = rows * dim_head / ve;
    const uintptr_t tab_bytes = (uintptr_t)(ve / 2) * dt_size(trig_dtype);  // table bytes per group
    const bool tab_al = aligned(cos_table, tab_bytes) && aligned(sin_table, tab_bytes);
    // the vector kernel indexes groups as block * 256 + thread in 32 bits: below 2^31 groups
    // that sum cannot wrap onto a group another thread rotates (in place) as well
    const bool vec = dim_head % ve == 0 && aligned(q, 16) && (k == nullptr || aligned(k, 16)) && tab_al &&
                     groups < (1ll << 31) && rows < (1ll << 31);
    if (vec) {
        a.groups = (uint32_t)groups;
        a.gpr = make_fastdiv((uint32_t)(dim_head / ve));
        a.npos_div = make_fastdiv((uint32_t)n_pos);
        a.heads_div = make_fastdiv((uint32_t)heads);
        const dim3 grid((unsigned)ceil_div(groups, kThreads));
        with_dt(dtype, [&](auto dt_) {
            constexpr int DTv = decltype(dt_)::value;
            if constexpr (DTv == BF16) {
                if (a.fb && trig_dtype == F32) {
                    if (k != nullptr) hipLaunchKernelGGL((rotary_vec_kernel<DTv, F32, true, true>), grid, dim3(kThreads), 0, st, a);
                    else hipLaunchKernelGGL((rotary_vec_kernel<DTv, F32, false, true>), grid, dim3(kThreads), 0, st, a);
                    return;
                }
            }
            if (k != nullptr) {
                if (trig_dtype == F32) hipLaunchKernelGGL((rotary_vec_kernel<DTv, F32, true, false>), grid, dim3(kThreads), 0, st, a);
                else hipLaunchKernelGGL((rotary_vec_kernel<DTv, BF16, true, false>), grid, dim3(kThreads), 0, st, a);
            } else {
                if (trig_dtype == F32) hipLaunchKernelGGL((rotary_vec_kernel<DTv, F32, false, false>), grid, dim3(kThreads), 0, st, a);
                else hipLaunchKernelGGL((rotary_vec_kernel<DTv, BF16, false, false>), grid, dim3(kThreads), 0, st, a);
            }
        });
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
    // bf16 intermediates: bf16 qkv to bf16 heads; the rounding only changes f32 tables
    a.fb = bf16_intermediates() && qkv_dtype == BF16 && out_dtype == BF16;
    hipStream_t st = as_stream(stream);
    const int ve = (qkv_dtype == F32 || out_dtype == F32) ? 4 : 8;
    const int64_t groups = total / ve;
    const uintptr_t tab_bytes = (uintptr_t)(ve / 2) * dt_size(trig_dtype);
    const bool tab_al = aligned(cos_table, tab_bytes) && aligned(sin_table, tab_bytes);
    const bool vec = D % ve == 0 && N >= 1 && aligned(qkv, 16) && aligned(q, 16) && aligned(k, 16) && aligned(v, 16) &&
                     tab_al && groups < (1ll << 31);
    if (vec) {
        const dim3 grid((unsigned)ceil_div(groups, kThreads));
        const FastDiv gpr = make_fastdiv((uint32_t)(D / ve)), od = make_fastdiv((uint32_t)out_N),
                      hd = make_fastdiv((uint32_t)H);
        with_dt(qkv_dtype, [&](auto it) {
            with_dt(out_dtype, [&](auto ot) {
                constexpr int IDTv = decltype(it)::value, ODTv = decltype(ot)::value;
                if constexpr (IDTv == BF16 && ODTv == BF16) {
                    if (a.fb && trig_dtype == F32) {
                        hipLaunchKernelGGL((split_qkv_vec_kernel<IDTv, ODTv, F32, true>), grid, dim3(kThreads), 0, st,
                                           a, (uint32_t)groups, gpr, od, hd);
                        return;
                    }
                }
                if (trig_dtype == F32)
                    hipLaunchKernelGGL((split_qkv_vec_kernel<IDTv, ODTv, F32, false>), grid, dim3(kThreads), 0, st, a,
                                       (uint32_t)groups, gpr, od, hd);
                else
                    hipLaunchKernelGGL((split_qkv_vec_kernel<IDTv, ODTv, BF16, false>), grid, dim3(kThreads), 0, st, a,
                                       (uint32_t)groups, gpr, od, hd);
            });
        });
    } else {
        const int64_t pairs = total / 2;
        hipLaunchKernelGGL(split_qkv_scalar_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(pairs, kThreads), 1 << 20)),
                           dim3(kThreads), 0, st, a);
    }
    return check_launch(op);
}

}  // extern "C"
