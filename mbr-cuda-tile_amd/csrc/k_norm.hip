// RMSNorm and fused residual-add + RMSNorm (mbr_tile::rms_norm / try_residual_add_rms_norm,
// src/mbr_cuda_tile.cu:4791-4965, 6297-6417).
//
//   out[r, d] = x[r, d] * (1 / sqrt(sum_d x[r, d]^2 + eps)) * gamma[d] * scale
//
// Register-resident fast path: a group of G lanes (16/32/64) owns one row and holds it as
// ceil(D / 8 / G) 8-element vectors per lane, so every byte of x is read from HBM once,
// the sum of squares is a G-lane butterfly, and the output is written once.  The
// reference launches one 1024-wide tile per row (62.5 % masked at D = 384) and, at
// D != 256, runs the residual add as a separate pass.  At D = 384: 48 vectors per row,
// G = 16 lanes x 3 vectors, 4 rows per wave, 16 rows per 256-thread block.
// The fallback (unaligned pointers, D % 8 != 0 or D > 4096) is one wave per row with
// a scalar two-pass loop.
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
    int nvec;  // dim / 8
    float scale;
    float eps;
};

template <int G, int NVMAX>
__global__ __launch_bounds__(kThreads) void rms_fast_kernel(RmsArgs a) {
    constexpr int kRowsPerBlock = kThreads / G;
    const int lane = threadIdx.x % G;
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / G;
    const bool valid = row < a.rows;
    const int64_t base = row * a.dim;

    float v[NVMAX][8];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NVMAX; ++k) {
        const int c = lane + G * k;
        if (valid && c < a.nvec) {
            load8(a.x, a.xdt, base + c * 8, v[k]);
            if (a.res != nullptr) {
                float r[8];
                load8(a.res, a.xdt, base + c * 8, r);
#pragma unroll
                for (int i = 0; i < 8; ++i) v[k][i] = round_through(v[k][i] + r[i], a.sdt);
                if (a.sum_out != nullptr) store8(a.sum_out, a.sdt, base + c * 8, v[k]);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = fmaf(v[k][i], v[k][i], ss);
        }
    }
    ss = group_sum<G>(ss);
    const float inv = rsqrtf(ss + a.eps) * a.scale;
#pragma unroll
    for (int k = 0; k < NVMAX; ++k) {
        const int c = lane + G * k;
        if (valid && c < a.nvec) {
            float g[8];
            load8(a.gamma, a.gdt, c * 8, g);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[k][i] = v[k][i] * inv * g[i];
            store8(a.out, a.odt, base + c * 8, v[k]);
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
        ss = fmaf(v, v, ss);
    }
    ss = group_sum<64>(ss);
    const float inv = rsqrtf(ss + a.eps) * a.scale;
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
        store1(a.out, a.odt, base + d, v * inv * load1(a.gamma, a.gdt, d));
    }
}

int launch_rms(RmsArgs a, hipStream_t st, const char* op) {
    if (a.rows == 0) return MBRT_OK;
    bool vec = (a.dim % 8) == 0 && a.dim <= 4096 && aligned(a.x, 16) && aligned(a.gamma, 16) &&
               aligned(a.out, 16) && (a.res == nullptr || aligned(a.res, 16)) &&
               (a.sum_out == nullptr || aligned(a.sum_out, 16));
    if (vec) {
        a.nvec = a.dim / 8;
        int G;
        int nv;
        if (a.nvec <= 16 * 4) G = 16;
        else if (a.nvec <= 32 * 4) G = 32;
        else G = 64;
        nv = (a.nvec + G - 1) / G;
        const int rows_per_block = kThreads / G;
        const dim3 grid((unsigned)ceil_div(a.rows, rows_per_block));
        if (G == 16) hipLaunchKernelGGL((rms_fast_kernel<16, 4>), grid, dim3(kThreads), 0, st, a);
        else if (G == 32) hipLaunchKernelGGL((rms_fast_kernel<32, 4>), grid, dim3(kThreads), 0, st, a);
        else if (nv <= 4) hipLaunchKernelGGL((rms_fast_kernel<64, 4>), grid, dim3(kThreads), 0, st, a);
        else hipLaunchKernelGGL((rms_fast_kernel<64, 8>), grid, dim3(kThreads), 0, st, a);
    } else {
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
