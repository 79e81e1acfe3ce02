// Fused attention O = softmax(scale * Q K^T) V on MFMA, for bf16 q, k, v [BH, N, 64]:
// the time attention (N = 801) and frequency attention (N = 60) of the band-split
// transformer (src/mbr_cuda_tile.cu:6530-6709, src/mbr_time_attention_cutile.cu:108-196).
// The [BH, N, N] score matrix never reaches HBM: each workgroup streams K/V tiles through
// LDS and keeps an online softmax (running max m, running sum l) per query.
//
// Workgroup = 4 waves = 64 queries of one (b, h); wave w owns queries q0 .. q0+15.
// Per 64-key tile, with v_mfma_f32_16x16x32_bf16 (lane l: A[l%16][8(l/16)+j],
// B[8(l/16)+j][l%16], C[4(l/16)+i][l%16]):
//   S^T = K Q^T     8 MFMAs: A = K rows from LDS, B = the wave's Q fragment (registers).
//                   Lane l then holds S^T[key 16kb + 4(l/16) + i][query l%16].
//   online softmax  per query l%16: max/sum over the lane's 16 keys, then over the four
//                   lane groups (xor 16, xor 32); the accumulator is rescaled in place.
//   O^T += V^T P^T  16 MFMAs: B = P^T straight from the S^T registers, as a bf16 pair
//                   P_hi + P_lo; A = V^T from a transposed LDS copy of the V tile.  The contraction runs over
//                   keys in the order the S^T layout holds them (slot j of lane group g is
//                   key 4g+j for j < 4, 16+4g+(j-4) after), used for both operands.
//   Lane l accumulates O^T[d 16db + 4(l/16) + i][query l%16]: the softmax statistics and
//   the accumulator share one lane mapping, so rescaling needs no lane exchange.
// Keys past N are masked to -inf; query rows past N are computed from a clamped row and
// not stored.  f32 accumulation throughout; carrying P as a bf16 pair keeps the result at
// f32 accuracy (the reference rounds its probabilities to bf16 once).
#include "abi_common.hpp"

#include <algorithm>
#include <cmath>

namespace mbrt {
namespace {

constexpr int kHeadDim = 64;
constexpr int kKeys = 64;      // keys per tile
constexpr int kQWave = 16;     // queries per wave
constexpr int kWaves = 4;
constexpr int kQBlock = kQWave * kWaves;
constexpr int kPad = 8;        // LDS row padding (bf16 elements)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct AttnArgs {
    const __bf16* q;
    const __bf16* k;
    const __bf16* v;
    void* out;
    int nq, nk;
    uint32_t qtiles;
    float scale_log2e;
};

__device__ __forceinline__ float xor_max(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float xor_sum(float x) {
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}

template <int ODT>
__global__ __launch_bounds__(kWaves * 64) void attention_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) __bf16 ks[kKeys][kHeadDim + kPad];   // K tile [key][d]
    __shared__ __attribute__((aligned(16))) __bf16 vts[kHeadDim][kKeys + kPad];  // V tile transposed [d][key]
    const int tid = threadIdx.x;
    const int lane = tid % 64, g = lane / 16, c = lane % 16;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    // one linear grid, query tiles of one (b, h) adjacent so that they share its K/V in L2
    const int64_t bh = blockIdx.x / a.qtiles;
    const int q0 = (blockIdx.x % a.qtiles) * kQBlock + w * kQWave;
    const __bf16* kbase = a.k + bh * a.nk * kHeadDim;
    const __bf16* vbase = a.v + bh * a.nk * kHeadDim;

    // Q fragment: lane holds Q[q0 + c][32s + 8g .. +7] for s = 0, 1
    const __bf16* qrow = a.q + (bh * a.nq + min(q0 + c, a.nq - 1)) * kHeadDim;
    bf16x8 qf[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) qf[s] = *reinterpret_cast<const bf16x8*>(qrow + 32 * s + 8 * g);

    f32x4 o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;

    // K/V tiles: 64 keys x 64 d = 512 16-byte vectors each, 2 per thread.  The next tile
    // is fetched into registers while the current one is computed from LDS.
    // Lane l of wave w stages key l, d chunks 8 (w + 4u): the transposed V writes of one
    // instruction then fill one LDS row with 64 consecutive keys.
    bf16x8 kv[2], vv[2];
    auto fetch = [&](int kt) {
        const int64_t row = min(kt + lane, a.nk - 1);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int dc = 8 * (w + 4 * u);
            kv[u] = *reinterpret_cast<const bf16x8*>(kbase + row * kHeadDim + dc);
            vv[u] = *reinterpret_cast<const bf16x8*>(vbase + row * kHeadDim + dc);
        }
    };
    fetch(0);
    for (int kt = 0; kt < a.nk; kt += kKeys) {
        __syncthreads();  // the previous tile is no longer read
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int dc = 8 * (w + 4 * u);
            *reinterpret_cast<bf16x8*>(&ks[lane][dc]) = kv[u];
#pragma unroll
            for (int j = 0; j < 8; ++j) vts[dc + j][lane] = vv[u][j];
        }
        __syncthreads();
        if (kt + kKeys < a.nk) fetch(kt + kKeys);

        // S^T = K Q^T for the 4 key blocks of the tile
        f32x4 st[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            st[kb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const bf16x8 ka = *reinterpret_cast<const bf16x8*>(&ks[16 * kb + c][32 * s + 8 * g]);
                st[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qf[s], st[kb], 0, 0, 0);
            }
        }
        // online softmax over this tile, per query c, on raw scores: the scale is folded
        // into the exponent, exp2(scale log2e (s - max)); keys past N only in the last tile
        if (kt + kKeys > a.nk) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (kt + 16 * kb + 4 * g + i >= a.nk) st[kb][i] = -INFINITY;
        }
        float mx = m;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
            mx = fmaxf(mx, fmaxf(fmaxf(st[kb][0], st[kb][1]), fmaxf(st[kb][2], st[kb][3])));
        mx = xor_max(mx);
        const float mxs = mx * a.scale_log2e;
        float psum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = __builtin_amdgcn_exp2f(fmaf(st[kb][i], a.scale_log2e, -mxs));
                st[kb][i] = p;
                psum += p;
            }
        }
        psum = xor_sum(psum);
        if (mx != m) {  // the accumulator keeps its scale until some running max moves
            const float alpha = __builtin_amdgcn_exp2f((m - mx) * a.scale_log2e);
            l *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db) o[db] *= alpha;
        }
        l += psum;
        m = mx;

        // O^T += V^T P^T over the two 32-key chunks
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            // P = P_hi + P_lo, both bf16: the pair carries 16 mantissa bits of P, so the
            // second product loses nothing measurable to the bf16 operand format
            bf16x8 ph, pl;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p0 = st[2 * cc][i], p1 = st[2 * cc + 1][i];
                ph[i] = (__bf16)p0;
                ph[4 + i] = (__bf16)p1;
                pl[i] = (__bf16)(p0 - (float)ph[i]);
                pl[4 + i] = (__bf16)(p1 - (float)ph[4 + i]);
            }
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const __bf16* vr = &vts[16 * db + c][32 * cc + 4 * g];
                const bf16x4 lo = *reinterpret_cast<const bf16x4*>(vr);
                const bf16x4 hi = *reinterpret_cast<const bf16x4*>(vr + 16);
                const bf16x8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, ph, o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pl, o[db], 0, 0, 0);
            }
        }
    }

    const int q = q0 + c;
    if (q >= a.nq) return;
    const float inv = 1.0f / l;
    const int64_t obase = (bh * a.nq + q) * kHeadDim;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        const int d = 16 * db + 4 * g;
        if constexpr (ODT == F32) {
            *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + obase + d) = o[db] * inv;
        } else {
            u32x2 pk;
            pk.x = pack_bf16x2(o[db][0] * inv, o[db][1] * inv);
            pk.y = pack_bf16x2(o[db][2] * inv, o[db][3] * inv);
            *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(a.out) + obase + d) = pk;
        }
    }
}

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_attention(const void* q, const void* k, const void* v, int dtype, void* out, int out_dtype, int64_t BH,
                   int64_t n_q, int64_t n_k, int64_t head_dim, float scale, mbrt_stream_t stream) {
    const char* op = "mbrt_attention";
    MBRT_REQUIRE(dtype == BF16, MBRT_E_UNSUPPORTED_DTYPE, "%s: q/k/v must be BF16", op);
    MBRT_REQUIRE(out_dtype == BF16 || out_dtype == F32, MBRT_E_UNSUPPORTED_DTYPE, "%s: out must be BF16/F32", op);
    MBRT_REQUIRE(head_dim == kHeadDim, MBRT_E_SHAPE, "%s: head_dim %lld (only 64 is built)", op, (long long)head_dim);
    MBRT_REQUIRE(BH >= 0 && n_q >= 0 && n_k >= 0, MBRT_E_SHAPE, "%s: bad shape", op);
    if (BH == 0 || n_q == 0) return MBRT_OK;
    MBRT_REQUIRE(n_k >= 1, MBRT_E_SHAPE, "%s: attention over zero keys", op);
    MBRT_REQUIRE(n_q < (1 << 30) && n_k < (1 << 30), MBRT_E_SHAPE, "%s: shape too large", op);
    MBRT_REQUIRE(q && k && v && out, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    MBRT_REQUIRE(scale >= 0.0f && std::isfinite(scale), MBRT_E_INVALID_ARG, "%s: scale must be finite and >= 0", op);
    MBRT_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(out, 16), MBRT_E_ALIGN,
                 "%s: q, k, v and out must be 16-byte aligned", op);
    MBRT_REQUIRE(BH * ceil_div(n_q, kQBlock) < (int64_t(1) << 31), MBRT_E_SHAPE, "%s: too many tiles", op);
    AttnArgs a{};
    a.q = static_cast<const __bf16*>(q);
    a.k = static_cast<const __bf16*>(k);
    a.v = static_cast<const __bf16*>(v);
    a.out = out;
    a.nq = (int)n_q;
    a.nk = (int)n_k;
    a.scale_log2e = (scale == 0.0f ? 1.0f / std::sqrt((float)head_dim) : scale) * 1.44269504088896340736f;
    a.qtiles = (uint32_t)ceil_div(n_q, kQBlock);
    const dim3 grid((unsigned)(BH * a.qtiles));
    if (out_dtype == BF16) hipLaunchKernelGGL(attention_kernel<BF16>, grid, dim3(kWaves * 64), 0, as_stream(stream), a);
    else hipLaunchKernelGGL(attention_kernel<F32>, grid, dim3(kWaves * 64), 0, as_stream(stream), a);
    return check_launch(op);
}

}  // extern "C"
