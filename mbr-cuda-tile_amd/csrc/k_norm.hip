// RMSNorm and fused residual-add + RMSNorm (mbr_tile::rms_norm / try_residual_add_rms_norm,
// src/mbr_cuda_tile.cu:4791-4965, 6297-6417).
//
//   out[r, d] = x[r, d] * (1 / sqrt(sum_d x[r, d]^2 + eps)) * gamma[d] * scale
//
// Register-resident fast path: a group of G lanes (16/32/64) owns one row, split into
// 16-byte chunks of VE elements (VE = 4 for f32 rows, 8 for bf16/f16 rows); lane l holds
// chunks l, l+G, l+2G, ..., so each load instruction of the group reads G consecutive
// 16-byte chunks.  Every byte of x (and of the residual) is read from HBM once, the sum
// of squares is a G-lane butterfly, the sum (residual variant) and the output are written
// once.  The reference launches one 1024-wide tile per row (62.5 % masked at D = 384) and,
// at D != 256, runs the residual add as a separate pass.
//   D = 384 f32 : 96 chunks -> G = 16 lanes x 6 chunks, 4 rows per wave
//   D = 384 bf16: 48 chunks -> G = 16 lanes x 3 chunks
// Fallback (unaligned pointers, D not a whole number of chunks, D > 4096): one wave per
// row with a scalar two-pass loop.
// With MBRT_ARITH_BF16_INTERMEDIATES set and a BF16 output, both paths round their
// intermediates to bf16 as the reference's bf16-output kernels do in full-bf16 mode.
#include "abi_common.hpp"

#include <algorithm>

namespace mbrt {
namespace {

constexpr int kThreads = 256;


struct RmsArgs {
    const void* x;
    const void* res;  // NULL: plain RMSNorm
    const void* gamma;
    void* sum_out;    // NULL: do not store the residual sum
    void* out;
    int xdt, gdt, sdt, odt;
    int64_t rows;
    int dim;
    int nchunk;  // dim / VE
    float scale;
    float eps;
    int fb;      // bf16 intermediates (loop kernel; the fast kernel takes it as FB)
};

// One block = 256 / G rows.  gamma * scale is staged once per block in LDS as f32.  The
// row loads are unconditional (row and chunk indices clamped into the tensor), so all of a
// lane's x (and residual) chunks are in flight together; stores are predicated.
// FB: bf16 intermediates (src/mbr_cuda_tile.cu:4815-4843, 4870-4905): the row values (the
// residual sum where there is one), the sum of squares, 1/sqrt and gamma are each rounded
// to bf16, and the output is ((v * inv) * gamma) * scale.
template <int XDT, int ODT, bool RES, int G, int NC, bool FB>
__global__ __launch_bounds__(kThreads) void rms_fast_kernel(RmsArgs a) {
    constexpr int VE = (XDT == F32 || ODT == F32) ? 4 : 8;
    extern __shared__ float gs[];
    const int lane = threadIdx.x % G;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / G) + threadIdx.x / G;
    const bool valid = row < a.rows;
    const int64_t base = (valid ? row : a.rows - 1) * a.dim;
    const int lastc = a.nchunk - 1;
    Vec<XDT, VE> xv[NC], rv[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        const int c = min(lane + G * k, lastc);
        xv[k].template load<MBRT_NT_RMS>(a.x, base + c * VE);
        if (RES) rv[k].template load<MBRT_NT_RMS>(a.res, base + c * VE);
    }
    for (int d = threadIdx.x; d < a.dim; d += kThreads)
        gs[d] = FB ? bf16r(load1(a.gamma, a.gdt, d)) : load1(a.gamma, a.gdt, d) * a.scale;
    float v[NC][VE];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        xv[k].to_f32(v[k]);
        if (RES) {
            float r[VE];
            rv[k].to_f32(r);
#pragma unroll
            for (int i = 0; i < VE; ++i) v[k][i] = v[k][i] + r[i];
            if (XDT != F32) {  // the sum is stored in the input dtype and normalised from there
                Vec<XDT, VE> t;
                t.from_f32(v[k]);
                t.to_f32(v[k]);
            }
        }
        const bool in = lane + G * k <= lastc;
#pragma unroll
        for (int i = 0; i < VE; ++i) {
            const float u = FB ? bf16r(v[k][i]) : v[k][i];
            ss = fmaf(u, in ? u : 0.0f, ss);
        }
    }
    const int full = a.nchunk / G;
    if (RES && a.sum_out != nullptr && valid) {
#pragma unroll
        for (int k = 0; k < NC; ++k) {
            if (k < full || lane + G * k <= lastc) {
                Vec<XDT, VE> t;
                t.from_f32(v[k]);
                t.template store<MBRT_NT_RMS>(a.sum_out, base + (lane + G * k) * VE);
            }
        }
    }
    ss = group_sum<G>(ss);
    const float inv = FB ? bf16r(rsqrtf(bf16r(ss) + a.eps)) : rsqrtf(ss + a.eps);
    __syncthreads();
    if (!valid) return;
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        if (k < full || lane + G * k <= lastc) {
            const int c = lane + G * k;
#pragma unroll
            for (int i = 0; i < VE; ++i) {
                if constexpr (FB) v[k][i] = bf16r(bf16r(v[k][i]) * inv * gs[c * VE + i] * a.scale);
                else v[k][i] = v[k][i] * inv * gs[c * VE + i];
            }
            Vec<ODT, VE> o;
            o.from_f32(v[k]);
            o.template store<MBRT_NT_RMS>(a.out, base + c * VE);
        }
    }
}

// Fallback: one wave per row, scalar accesses, two passes over the row.
__global__ __launch_bounds__(kThreads) void rms_loop_kernel(RmsArgs a) {
    const int lane = threadIdx.x % 64;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + threadIdx.x / 64;
    if (row >= a.rows) return;  // whole wave exits together
    const int64_t base = row * a.dim;
    float ss = 0.0f;
    for (int d = lane; d < a.dim; d += 64) {
        float v = load1(a.x, a.xdt, base + d);
        if (a.res != nullptr) {
            v = round_through(v + load1(a.res, a.xdt, base + d), a.sdt);
            if (a.sum_out != nullptr) store1(a.sum_out, a.sdt, base + d, v);
        }
        if (a.fb) v = bf16r(v);
        ss = fmaf(v, v, ss);
    }
    ss = group_sum<64>(ss);
    const float inv = a.fb ? bf16r(rsqrtf(bf16r(ss) + a.eps)) : rsqrtf(ss + a.eps) * a.scale;
    for (int d = lane; d < a.dim; d += 64) {
        float v;
        if (a.res == nullptr) {
            v = load1(a.x, a.xdt, base + d);
        } else if (a.sum_out != nullptr) {
            // re-read the stored sum: sum_out may alias x (in-place residual)
            v = load1(a.sum_out, a.sdt, base + d);
        } else {
            v = round_through(load1(a.x, a.xdt, base + d) + load1(a.res, a.xdt, base + d), a.sdt);
        }
        if (a.fb) store1(a.out, a.odt, base + d, bf16r(bf16r(v) * inv * bf16r(load1(a.gamma, a.gdt, d)) * a.scale));
        else store1(a.out, a.odt, base + d, v * inv * load1(a.gamma, a.gdt, d));
    }
}

template <int XDT, int ODT, bool RES, int G, int NC, bool FB>
void launch_fast(const RmsArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((rms_fast_kernel<XDT, ODT, RES, G, NC, FB>), dim3((unsigned)ceil_div(a.rows, kThreads / G)),
                       dim3(kThreads), a.dim * sizeof(float), st, a);
}

// Group width / chunks per lane for `nchunk` chunks; false when the row is too long.
template <int XDT, int ODT, bool RES, bool FB>
bool launch_chunks(const RmsArgs& a, hipStream_t st) {
    constexpr int G = MBRT_RMS_G;
    const int n = a.nchunk;
    if (n <= 2 * G) launch_fast<XDT, ODT, RES, G, 2, FB>(a, st);
    else if (n <= 4 * G) launch_fast<XDT, ODT, RES, G, 4, FB>(a, st);
    else if (n <= 6 * G) launch_fast<XDT, ODT, RES, G, 6, FB>(a, st);
    else if (n <= 128) launch_fast<XDT, ODT, RES, G, 128 / G, FB>(a, st);
    else if (n <= 512) launch_fast<XDT, ODT, RES, 64, 8, FB>(a, st);
    else if (n <= 1024) launch_fast<XDT, ODT, RES, 64, 16, FB>(a, st);
    else return false;
    return true;
}

int launch_rms(RmsArgs a, hipStream_t st, const char* op) {
    if (a.rows == 0) return MBRT_OK;
    a.fb = bf16_intermediates() && a.odt == BF16;
    const int ve = (a.xdt == F32 || a.odt == F32) ? 4 : 8;
    const bool res = a.res != nullptr;
    const bool al = aligned(a.x, 16) && aligned(a.out, 16) && (!res || aligned(a.res, 16)) &&
                    (a.sum_out == nullptr || aligned(a.sum_out, 16));
    // the fused path stores the residual sum in the input dtype
    const bool sum_ok = !res || a.sdt == a.xdt;
    bool done = false;
    if (al && sum_ok && a.dim % ve == 0 && (a.dim * dt_size(a.xdt)) % 16 == 0 && a.dim <= 4096) {
        a.nchunk = a.dim / ve;
        with_dt(a.xdt, [&](auto xt) {
            with_dt(a.odt, [&](auto ot) {
                constexpr int X = decltype(xt)::value, O = decltype(ot)::value;
                if constexpr (O == BF16) {
                    if (a.fb) {
                        done = res ? launch_chunks<X, O, true, true>(a, st) : launch_chunks<X, O, false, true>(a, st);
                        return;
                    }
                }
                done = res ? launch_chunks<X, O, true, false>(a, st) : launch_chunks<X, O, false, false>(a, st);
            });
        });
    }
    if (!done) {
        const dim3 grid((unsigned)ceil_div(a.rows, kThreads / 64));
        hipLaunchKernelGGL(rms_loop_kernel, grid, dim3(kThreads), 0, st, a);
    }
    return check_launch(op);
}

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_rms_norm(const void* x, int x_dtype, const void* gamma, int gamma_dtype, void* out, int out_dtype,
                  int64_t rows, int64_t dim, float scale, float eps, mbrt_stream_t stream) {
    const char* op = "mbrt_rms_norm";
    MBRT_REQUIRE_FLOAT_DT(x_dtype, op);
    MBRT_REQUIRE_FLOAT_DT(out_dtype, op);
    MBRT_REQUIRE(gamma_dtype == F32 || gamma_dtype == BF16, MBRT_E_UNSUPPORTED_DTYPE,
                 "%s: gamma dtype %d (expected F32/BF16)", op, gamma_dtype);
    MBRT_REQUIRE(rows >= 0 && dim >= 1 && dim < (1 << 30), MBRT_E_SHAPE, "%s: bad shape rows=%lld dim=%lld", op,
                 (long long)rows, (long long)dim);
    MBRT_REQUIRE(rows == 0 || (x && gamma && out), MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    RmsArgs a{};
    a.x = x;
    a.res = nullptr;
    a.gamma = gamma;
    a.sum_out = nullptr;
    a.out = out;
    a.xdt = x_dtype;
    a.gdt = gamma_dtype;
    a.sdt = F32;
    a.odt = out_dtype;
    a.rows = rows;
    a.dim = (int)dim;
    a.scale = scale;
    a.eps = eps;
    return launch_rms(a, as_stream(stream), op);
}

int mbrt_residual_add_rms_norm(const void* residual, const void* update, int in_dtype, const void* gamma,
                               int gamma_dtype, void* sum_out, int sum_dtype, void* normed, int normed_dtype,
                               int64_t rows, int64_t dim, float scale, float eps, mbrt_stream_t stream) {
    const char* op = "mbrt_residual_add_rms_norm";
    MBRT_REQUIRE_FLOAT_DT(in_dtype, op);
    MBRT_REQUIRE_FLOAT_DT(sum_dtype, op);
    MBRT_REQUIRE_FLOAT_DT(normed_dtype, op);
    MBRT_REQUIRE(gamma_dtype == F32 || gamma_dtype == BF16, MBRT_E_UNSUPPORTED_DTYPE,
                 "%s: gamma dtype %d (expected F32/BF16)", op, gamma_dtype);
    MBRT_REQUIRE(rows >= 0 && dim >= 1 && dim < (1 << 30), MBRT_E_SHAPE, "%s: bad shape", op);
    MBRT_REQUIRE(rows == 0 || (residual && update && gamma && normed), MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    MBRT_REQUIRE(sum_out != update || sum_out == nullptr, MBRT_E_INVALID_ARG, "%s: sum_out may not alias update", op);
    RmsArgs a{};
    a.x = residual;
    a.res = update;
    a.gamma = gamma;
    a.sum_out = sum_out;
    a.out = normed;
    a.xdt = in_dtype;
    a.gdt = gamma_dtype;
    a.sdt = sum_dtype;
    a.odt = normed_dtype;
    a.rows = rows;
    a.dim = (int)dim;
    a.scale = scale;
    a.eps = eps;
    return launch_rms(a, as_stream(stream), op);
}

}  // extern "C"
