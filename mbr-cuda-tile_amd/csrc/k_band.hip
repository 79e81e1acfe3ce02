// Mel band split / merge around the band-split transformer
// (mbr_tile::gather_freqs_fold_complex and apply_mask_and_scatter,
//  src/mbr_cuda_tile.cu:4554-4601, 5586-5803, 6215-6241, 7951-8081; zero_dc 5805-5838).
//
// Layouts (complex values are interleaved (re, im) f32 pairs, 8 bytes):
//   stft  [B, F, T]      freq-major: F = bins * channels, freq = bin * channels + ch
//   bands [B, T, J]      time-major: J band-bins, idx[j] = freq of band-bin j
//   out   [B*S*C, bins, T]
// Both directions are transposes between a freq-major and a time-major complex matrix,
// so both stage 64-frame tiles through LDS: every global access is a run of consecutive
// complex values along T (stft/out) or along J (bands), never a stride-T gather.
//
// Gather: a block owns (b, 64 frames, 64 band-bins).  It reads, for each band-bin j, the
// 64 frames of stft row idx[j] (512 contiguous bytes), then writes, for each frame, the 64
// band-bins (512 contiguous bytes of the output row).
//
// Merge: a block owns (b, stem, 32 freqs, 64 frames).  The band-bins that feed those
// freqs are the CSR entries [off[f0], off[f0+32]) (<= 64 when no freq has more than 2
// bands; larger lists are processed in chunks of 64).  Their mask rows are staged in LDS,
// then each thread forms sum_e stft * mask_e over its freq's entries in ascending e and
// divides by max(count, 1e-8).  Each output is written once: no float atomics and no
// zero-fill pass, and the summation order is fixed.
#include "abi_common.hpp"

#include <algorithm>

namespace mbrt {
namespace {

constexpr int kThreads = 256;
constexpr int kTT = 64;   // frames per tile
constexpr int kTJ = 64;   // band-bins per gather tile
constexpr int kTF = 32;   // freqs per merge tile
constexpr int kME = 64;   // CSR entries staged per merge chunk

__device__ __forceinline__ int64_t load_index(const void* p, int i64, int64_t i) {
    return i64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
}

template <bool I64>
__device__ __forceinline__ int ld_idx(const void* p, int64_t i) {
    if constexpr (I64) return (int)reinterpret_cast<const int64_t*>(p)[i];
    else return reinterpret_cast<const int32_t*>(p)[i];
}

struct GatherArgs {
    const float* stft;
    const void* idx;
    int idx64;
    void* out;
    int odt;
    int64_t F, T, J;
    uint32_t tiles_j, tiles_t, tiles;  // tile grid: band-bin tiles fastest, then frames, then batch
};

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x / 64); }

template <int ODT>
__device__ __forceinline__ void store_complex(void* out, int64_t o, f32x2 v) {
    constexpr int NT = MBRT_NT_BAND;
    if constexpr (ODT == F32) gst<NT>(reinterpret_cast<f32x2*>(out) + o, v);
    else if constexpr (ODT == BF16) gst<NT>(reinterpret_cast<uint32_t*>(out) + o, pack_bf16x2(v.x, v.y));
    else gst<NT>(reinterpret_cast<uint32_t*>(out) + o, pack_f16x2(v.x, v.y));
}

template <int MDT>
__device__ __forceinline__ f32x2 load_complex(const void* p, int64_t i) {
    constexpr int NT = MBRT_NT_BAND;
    if constexpr (MDT == F32) return gld<NT>(reinterpret_cast<const f32x2*>(p) + i);
    const uint32_t w = gld<NT>(reinterpret_cast<const uint32_t*>(p) + i);
    if constexpr (MDT == BF16) return f32x2{bf16_lo(w), bf16_hi(w)};
    else return unpack_f16x2(w);
}

// Block (j-tile, t-tile, b).  Wave w reads tile rows jj = w, w+4, ..., w+60: the 64 frames
// of stft row idx[j0+jj] (512 contiguous bytes).  The row index is loaded once per lane and
// broadcast with readlane; indices are clamped into the tensors so the 16 loads of a lane
// are unconditional and in flight together.
template <int ODT, bool I64>
__global__ __launch_bounds__(kThreads) void band_gather_kernel(GatherArgs a) {
    __shared__ f32x2 tile[kTJ][kTT + 1];
    // one linear grid; neighbouring band-bin tiles (which read the same stft rows where
    // bands overlap) run on one XCD
    const uint32_t tid = xcd_runs<MBRT_BAND_XCD>(blockIdx.x, a.tiles);
    const uint32_t tj = tid % a.tiles_j, rest = tid / a.tiles_j;
    const int64_t j0 = (int64_t)tj * kTJ;
    const int64_t t0 = (int64_t)(rest % a.tiles_t) * kTT;
    const int64_t b = rest / a.tiles_t;
    const int lane = threadIdx.x % 64;
    const int w = wave_id();
    const int64_t tq = min(t0 + lane, a.T - 1);
    const f32x2* stft = reinterpret_cast<const f32x2*>(a.stft) + b * a.F * a.T + tq;
    constexpr int kR = kTJ / (kThreads / 64);  // 16 rows per wave
    f32x2 v[kR];
    if constexpr (MBRT_BAND_SLOAD) {
        // the row indices of a wave are uniform: scalar loads through the constant cache
        int64_t f[kR];
#pragma unroll
        for (int r = 0; r < kR; ++r) f[r] = ld_idx<I64>(a.idx, min(j0 + w + 4 * r, a.J - 1));
#pragma unroll
        for (int r = 0; r < kR; ++r) v[r] = gld<MBRT_NT_BAND>(stft + f[r] * a.T);
    } else {
        const int f_lane = ld_idx<I64>(a.idx, min(j0 + lane, a.J - 1));
#pragma unroll
        for (int r = 0; r < kR; ++r) {
            const int64_t f = __builtin_amdgcn_readlane(f_lane, w + 4 * r);
            v[r] = gld<MBRT_NT_BAND>(stft + f * a.T);
        }
    }
#pragma unroll
    for (int r = 0; r < kR; ++r) tile[w + 4 * r][lane] = v[r];
    __syncthreads();
    // write: out[b, t0+tt, j0 : j0+64] for tt = w, w+4, ...
    const int64_t j = j0 + lane;
    if (j >= a.J) return;
#pragma unroll
    for (int r = 0; r < kR; ++r) {
        const int tt = w + 4 * r;
        if (t0 + tt < a.T) store_complex<ODT>(a.out, (b * a.T + t0 + tt) * a.J + j, tile[lane][tt]);
    }
}

struct MergeArgs {
    const float* stft;
    const void* mask[2];
    const void* off;
    const void* ind;
    const void* cnt;
    void* out;
    int cdt;
    int S;
    int F, T, J;
    FastDiv C;  // audio channels: freq = bin * C + ch
    uint32_t tiles_f, tiles_t, tiles;  // tile grid: freq tiles fastest, then frames, then b*S+s
};

// Block (t-tile, f-tile, b*S+s).  Wave w owns freqs f0+w, f0+w+4, ... (8 of them) and lane
// t of the tile.  Lane l of every wave holds off[f0+l] (l <= 32) and 1/count[f0+l]; the
// ranges and scales of a wave's freqs are broadcast from there with readlane.  The CSR
// entries of the tile's freqs are staged 64 at a time: lane e loads mask[b, t, ind[c0+e]]
// for 16 frames, the tile is transposed through LDS, and each thread sums its freqs'
// entries in ascending order.  All loads use clamped indices and are unconditional.
template <int MDT, int ODT, bool I64>
__global__ __launch_bounds__(kThreads) void band_merge_kernel(MergeArgs a) {
    __shared__ f32x2 ms[kME][kTT + 1];
    // one linear grid; neighbouring freq tiles (whose CSR runs split cache lines of the
    // mask rows) run on one XCD
    const uint32_t tile = xcd_runs<MBRT_BAND_XCD>(blockIdx.x, a.tiles);
    const uint32_t tf = tile % a.tiles_f, rest = tile / a.tiles_f;
    const int f0 = (int)tf * kTF;
    const int t0 = (int)(rest % a.tiles_t) * kTT;
    const int bs = (int)(rest / a.tiles_t);  // b * S + s
    const int b = a.S == 2 ? bs >> 1 : bs;
    const void* mask = a.mask[bs - b * a.S];
    const int lane = threadIdx.x % 64;
    const int w = wave_id();
    constexpr int kPer = kTF / (kThreads / 64);  // freqs per wave (8)
    constexpr int kR = kTT / (kThreads / 64);    // staged frames per wave (16)
    const int nf = min(kTF, a.F - f0);           // freqs in this tile
    const int t = t0 + lane;
    const int tq = min(t, a.T - 1);

    // CSR offsets of the tile's freqs: uniform scalar loads, or lane l holds off[f0 + l]
    int off_s[kPer + 1];
    int off_lane = 0;
    int e_begin, e_end;
    if constexpr (MBRT_BAND_SLOAD) {
        e_begin = ld_idx<I64>(a.off, f0);
        e_end = ld_idx<I64>(a.off, f0 + nf);
    } else {
        off_lane = ld_idx<I64>(a.off, f0 + min(lane, nf));
        e_begin = __builtin_amdgcn_readlane(off_lane, 0);
        e_end = __builtin_amdgcn_readlane(off_lane, nf);
    }
    float c = load1(a.cnt, a.cdt, f0 + min(lane, nf - 1));
    const float inv_lane = 1.0f / (c > 1.0e-8f ? c : 1.0e-8f);
    if constexpr (MBRT_BAND_SLOAD) {
#pragma unroll
        for (int r = 0; r < kPer; ++r) off_s[r] = ld_idx<I64>(a.off, f0 + min(w + 4 * r, nf));
        off_s[kPer] = 0;
    }

    const f32x2* srow = reinterpret_cast<const f32x2*>(a.stft) + ((int64_t)b * a.F + f0) * a.T + tq;
    f32x2 sv[kPer], acc[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        sv[r] = gld<MBRT_NT_BAND>(srow + (int64_t)min(w + 4 * r, nf - 1) * a.T);
        acc[r] = f32x2{0.0f, 0.0f};
    }
    const int64_t mbase = (int64_t)b * a.T;
    for (int c0 = e_begin; c0 < e_end; c0 += kME) {
        const int c1 = min(c0 + kME, e_end);
        const int j = min(max(ld_idx<I64>(a.ind, min(c0 + lane, c1 - 1)), 0), a.J - 1);
        f32x2 mv[kR];
#pragma unroll
        for (int r = 0; r < kR; ++r)
            mv[r] = load_complex<MDT>(mask, (mbase + min(t0 + w + 4 * r, a.T - 1)) * a.J + j);
#pragma unroll
        for (int r = 0; r < kR; ++r) ms[lane][w + 4 * r] = mv[r];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kPer; ++r) {
            const int fl = w + 4 * r;  // local freq (wave-uniform); entries [off[f], off[f+1])
            int lo, hi;
            if constexpr (MBRT_BAND_SLOAD) {
                lo = max(off_s[r], c0);
                hi = fl < nf ? min(ld_idx<I64>(a.off, f0 + fl + 1), c1) : lo;
            } else {
                lo = max(__builtin_amdgcn_readlane(off_lane, fl), c0);
                hi = fl < nf ? min(__builtin_amdgcn_readlane(off_lane, fl + 1), c1) : lo;
            }
            for (int e = lo; e < hi; ++e) {
                const f32x2 m = ms[e - c0][lane];
                acc[r].x += sv[r].x * m.x - sv[r].y * m.y;
                acc[r].y += sv[r].x * m.y + sv[r].y * m.x;
            }
        }
        __syncthreads();
    }
    // readlane reads lanes regardless of EXEC: broadcast the scales while all lanes are active
    float inv[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r)
        inv[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, inv_lane), w + 4 * r));
    if (t >= a.T) return;
    const int64_t bins = a.F / a.C.d;
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int fl = w + 4 * r;
        if (fl < nf) {
            uint32_t bin, ch;
            fdivmod((uint32_t)(f0 + fl), a.C, bin, ch);
            const int64_t o = (((int64_t)bs * a.C.d + ch) * bins + bin) * a.T + t;
            store_complex<ODT>(a.out, o, f32x2{acc[r].x * inv[r], acc[r].y * inv[r]});
        }
    }
}

__global__ __launch_bounds__(kThreads) void zero_dc_kernel(void* spec, int dt, int64_t outer, int64_t bins, int64_t T) {
    const int64_t per = T * 2;
    const int64_t n = outer * per;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i < n; i += (int64_t)gridDim.x * kThreads) {
        const int64_t o = i / per, r = i - o * per;
        const int64_t e = o * bins * per + r;
        if (dt == F32) reinterpret_cast<float*>(spec)[e] = 0.0f;
        else reinterpret_cast<uint16_t*>(spec)[e] = 0;
    }
}

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_band_gather(const float* stft, const void* freq_indices, int index_dtype, void* out, int out_dtype, int64_t B,
                     int64_t total_freq, int64_t frames, int64_t n_band_freqs, mbrt_stream_t stream) {
    const char* op = "mbrt_band_gather";
    MBRT_REQUIRE(is_index_dt(index_dtype), MBRT_E_UNSUPPORTED_DTYPE, "%s: indices must be I32/I64", op);
    MBRT_REQUIRE_FLOAT_DT(out_dtype, op);
    MBRT_REQUIRE(B >= 0 && total_freq >= 1 && frames >= 0 && n_band_freqs >= 0, MBRT_E_SHAPE, "%s: bad shape", op);
    if (B == 0 || frames == 0 || n_band_freqs == 0) return MBRT_OK;
    MBRT_REQUIRE(stft && freq_indices && out, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    MBRT_REQUIRE(aligned(stft, 8) && aligned(out, out_dtype == F32 ? 8 : 4), MBRT_E_ALIGN,
                 "%s: complex buffers must be aligned to one complex value", op);
    GatherArgs a{stft, freq_indices, index_dtype == I64, out, out_dtype, total_freq, frames, n_band_freqs, 0, 0, 0};
    const int64_t tiles = ceil_div(n_band_freqs, kTJ) * ceil_div(frames, kTT) * B;
    MBRT_REQUIRE(tiles < (int64_t(1) << 31), MBRT_E_SHAPE, "%s: too many tiles", op);
    a.tiles_j = (uint32_t)ceil_div(n_band_freqs, kTJ);
    a.tiles_t = (uint32_t)ceil_div(frames, kTT);
    a.tiles = (uint32_t)tiles;
    const dim3 grid(a.tiles);
    with_dt(out_dtype, [&](auto ot) {
        constexpr int O = decltype(ot)::value;
        if (index_dtype == I64) hipLaunchKernelGGL((band_gather_kernel<O, true>), grid, dim3(kThreads), 0, as_stream(stream), a);
        else hipLaunchKernelGGL((band_gather_kernel<O, false>), grid, dim3(kThreads), 0, as_stream(stream), a);
    });
    return check_launch(op);
}

int mbrt_band_mask_merge(const float* stft, const void* const* masks, int mask_dtype, int num_stems,
                         const void* csr_offsets, const void* csr_indices, int index_dtype, const void* counts,
                         int counts_dtype, void* out, int out_dtype, int64_t B, int64_t total_freq, int64_t frames,
                         int64_t n_band_freqs, int64_t channels, mbrt_stream_t stream) {
    const char* op = "mbrt_band_mask_merge";
    MBRT_REQUIRE(num_stems == 1 || num_stems == 2, MBRT_E_INVALID_ARG, "%s: expected one or two stems", op);
    MBRT_REQUIRE(is_index_dt(index_dtype), MBRT_E_UNSUPPORTED_DTYPE, "%s: CSR must be I32/I64", op);
    MBRT_REQUIRE_FLOAT_DT(mask_dtype, op);
    MBRT_REQUIRE(counts_dtype == F32 || counts_dtype == BF16, MBRT_E_UNSUPPORTED_DTYPE, "%s: counts must be F32/BF16", op);
    MBRT_REQUIRE_FLOAT_DT(out_dtype, op);
    MBRT_REQUIRE(channels >= 1 && total_freq >= 1 && total_freq % channels == 0, MBRT_E_SHAPE,
                 "%s: invalid audio channel count", op);
    MBRT_REQUIRE(B >= 0 && frames >= 0 && n_band_freqs >= 0, MBRT_E_SHAPE, "%s: bad shape", op);
    if (B == 0 || frames == 0) return MBRT_OK;
    MBRT_REQUIRE(stft && masks && csr_offsets && counts && out && (n_band_freqs == 0 || csr_indices),
                 MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    for (int s = 0; s < num_stems; ++s) MBRT_REQUIRE(masks[s] != nullptr, MBRT_E_INVALID_ARG, "%s: NULL mask", op);
    MBRT_REQUIRE(total_freq < (1 << 30) && frames < (1 << 30) && n_band_freqs < (1 << 30) && B * frames < (1 << 30),
                 MBRT_E_SHAPE, "%s: dimension exceeds 2^30", op);
    MergeArgs a{};
    a.stft = stft;
    a.mask[0] = masks[0];
    a.mask[1] = num_stems == 2 ? masks[1] : masks[0];
    a.off = csr_offsets;
    a.ind = csr_indices;
    a.cnt = counts;
    a.out = out;
    a.cdt = counts_dtype;
    a.S = num_stems;
    a.F = (int)total_freq;
    a.T = (int)frames;
    a.J = (int)std::max<int64_t>(n_band_freqs, 1);
    a.C = make_fastdiv((uint32_t)channels);
    const int64_t tiles = ceil_div(total_freq, kTF) * ceil_div(frames, kTT) * B * num_stems;
    MBRT_REQUIRE(tiles < (int64_t(1) << 31), MBRT_E_SHAPE, "%s: too many tiles", op);
    a.tiles_f = (uint32_t)ceil_div(total_freq, kTF);
    a.tiles_t = (uint32_t)ceil_div(frames, kTT);
    a.tiles = (uint32_t)tiles;
    const dim3 grid(a.tiles);
    with_dt(mask_dtype, [&](auto mt) {
        with_dt(out_dtype, [&](auto ot) {
            constexpr int M = decltype(mt)::value, O = decltype(ot)::value;
            if (index_dtype == I64)
                hipLaunchKernelGGL((band_merge_kernel<M, O, true>), grid, dim3(kThreads), 0, as_stream(stream), a);
            else
                hipLaunchKernelGGL((band_merge_kernel<M, O, false>), grid, dim3(kThreads), 0, as_stream(stream), a);
        });
    });
    return check_launch(op);
}

int mbrt_zero_dc(void* spec, int dtype, int64_t outer, int64_t freq_bins, int64_t frames, mbrt_stream_t stream) {
    const char* op = "mbrt_zero_dc";
    MBRT_REQUIRE_FLOAT_DT(dtype, op);
    MBRT_REQUIRE(outer >= 0 && freq_bins >= 1 && frames >= 0, MBRT_E_SHAPE, "%s: bad shape", op);
    const int64_t n = outer * frames * 2;
    if (n == 0) return MBRT_OK;
    MBRT_REQUIRE(spec != nullptr, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    hipLaunchKernelGGL(zero_dc_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(n, kThreads), 1 << 20)), dim3(kThreads),
                       0, as_stream(stream), spec, dtype, outer, freq_bins, frames);
    return check_launch(op);
}

}  // extern "C"
