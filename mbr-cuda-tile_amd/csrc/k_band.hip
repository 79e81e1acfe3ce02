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
// Gather: a tile is (b, 64 frames, 64 band-bins).  For each band-bin j it reads the 64
// frames of stft row idx[j] (512 contiguous bytes), then writes, for each frame, the 64
// band-bins (512 contiguous bytes of the output row).  Persistent blocks walk the tiles
// with three LDS buffers, so the rows of the next two tiles are in flight (direct-to-LDS
// loads) while the current tile is stored; a one-tile-per-block kernel covers tensors
// whose element offsets exceed 32 bits.  Indices outside [0, F) read the nearest row.
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
constexpr int kTF = MBRT_BAND_MTF;   // freqs per merge tile
constexpr int kME = MBRT_BAND_MME;   // CSR entries staged per merge chunk
constexpr int kMW = MBRT_BAND_MNW;   // waves per merge block
static_assert(kTF <= 64 && kTF % kMW == 0 && kME % 64 == 0 && kTT % kMW == 0, "merge tile shape");

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

// One tile per block (tensors whose element offsets exceed 32 bits).  Block (j-tile, t-tile,
// b).  Wave w reads tile rows jj = w, w+4, ..., w+60: the 64 frames of stft row idx[j0+jj]
// (512 contiguous bytes).  The row index is loaded once per lane and broadcast with
// readlane; indices are clamped into the tensors so the 16 loads of a lane are
// unconditional and in flight together.
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
    // indices outside [0, F) read the nearest valid row
    const int64_t fl = load_index(a.idx, I64, min(j0 + lane, a.J - 1));
    const int f_lane = (int)min(max(fl, (int64_t)0), a.F - 1);
#pragma unroll
    for (int r = 0; r < kR; ++r) {
        const int64_t f = __builtin_amdgcn_readlane(f_lane, w + 4 * r);
        v[r] = gld<MBRT_NT_BAND>(stft + f * a.T);
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

// ---- pipelined gather ----------------------------------------------------------------
// Persistent blocks walk the tiles (band-bin tiles fastest, then frames, then batch) with a
// stride of the grid size.  Three LDS buffers hold tiles i, i+1 and i+2: while tile i is
// read out of LDS and stored, the stft rows of tiles i+1 and i+2 are in flight straight
// into LDS (global_load_lds_dword: one wave instruction = 256 contiguous bytes = 32 frames
// of one row), so no wave waits for a load it issued less than two tiles ago.
//
// Counting: per tile a wave issues a variable number of stores, then exactly kLPT direct
// loads (row indices and frames are clamped, never skipped).  vmcnt retires in issue
// order, so "at most kLPT outstanding" means every op before the newest tile's loads has
// completed, in particular the loads of the tile about to be read.
//
// Line-aligned stores (MBRT_BAND_GALIGN).  An output row (one frame, J band-bins) starts
// at (b T + t) J complex values, so with J = 3958 most 64-value runs start inside a
// 128-byte line and share their first and last lines with the neighbouring tiles; those
// split lines cost about 8 % (measured with a padded row pitch).  So tile k owns, in frame
// row t, the band-bins [64 k - ph(t), 64 k + 64 - ph(t)), ph(t) the row's offset into its
// line (in complex values, < 16): every run of an f32 output is whole lines (a 2-byte
// output's runs start on 64-byte boundaries).  Its LDS buffer holds the 16 band-bins
// before 64 k as well (80 rows), and the tile grid has one more band-bin tile.
constexpr int kGTJ = 64;  // band-bins per tile: one per lane when storing
constexpr int kGShift = MBRT_BAND_GALIGN ? 16 : 0;  // extra rows before a tile's first band-bin
constexpr int kGRows = kGTJ + kGShift;              // LDS rows per tile

struct GatherPipeArgs {
    const float* stft;
    const void* idx;
    void* out;
    int32_t F, T, J;
    int32_t bft2;                 // F * T * 2: floats per batch of stft (B * F * T * 2 < 2^31)
    FastDiv tiles_j, tiles_t;     // tile grid: band-bin tiles fastest, then frames, then batch
    uint32_t tiles;
    uint32_t oph;                 // (output address / bytes per complex value) % 16
};

// Barrier for data that arrived by direct-to-LDS loads: the caller has waited (vmcnt) for
// this wave's own loads; the barrier then makes every wave's data visible.  Unlike
// __syncthreads() it carries no memory fence, which would wait for every outstanding
// load, including those of the tiles still in flight.  The empty asm statements keep the
// compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// 16 ds_read_b64: v[q + 4 m] from LDS byte address a[q] + 128 m (q, m < 4), completed
// before the statement ends; one asm block for the reason given at lds_read_b64_n.
__device__ __forceinline__ void lds_read_b64_4x4(const uint32_t (&a)[4], f32x2 (&v)[16]) {
#define MBRT_DSR4(i, q, m) "ds_read_b64 %" #i ", %" #q " offset:" #m "\n\t"
    asm volatile(MBRT_DSR4(0, 16, 0) MBRT_DSR4(1, 17, 0) MBRT_DSR4(2, 18, 0) MBRT_DSR4(3, 19, 0)
                 MBRT_DSR4(4, 16, 128) MBRT_DSR4(5, 17, 128) MBRT_DSR4(6, 18, 128) MBRT_DSR4(7, 19, 128)
                 MBRT_DSR4(8, 16, 256) MBRT_DSR4(9, 17, 256) MBRT_DSR4(10, 18, 256) MBRT_DSR4(11, 19, 256)
                 MBRT_DSR4(12, 16, 384) MBRT_DSR4(13, 17, 384) MBRT_DSR4(14, 18, 384) MBRT_DSR4(15, 19, 384)
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
                   "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]), "=&v"(v[12]), "=&v"(v[13]),
                   "=&v"(v[14]), "=&v"(v[15])
                 : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3])
                 : "memory");
#undef MBRT_DSR4
}

// Freq of a row from its raw index (int32, or the low/high words of an int64), clamped
// into [0, F): an index outside the tensor reads the nearest valid row.
__device__ __forceinline__ int32_t clamp_freq(int32_t lo, int32_t hi, int32_t F) {
    const int32_t f = hi == (lo >> 31) ? lo : (hi < 0 ? -1 : F);
    return min(max(f, 0), F - 1);
}

template <int ODT, bool I64, int NW, int TT>
__global__ __launch_bounds__(64 * NW) void band_gather_pipe_kernel(GatherPipeArgs a) {
    constexpr int kRowF = 2 * TT + 2;    // floats per LDS row: TT complex values + 8 B of padding
    constexpr int kRPW = kGRows / NW;    // rows a wave loads per tile
    constexpr int kIPR = TT / 32;        // direct loads per row
    constexpr int kLPT = kRPW * kIPR;    // direct loads per wave per tile
    constexpr int kFPW = TT / NW;        // frames a wave stores per tile
    static_assert(TT % 32 == 0 && kGRows % NW == 0 && TT % NW == 0 && kLPT < 64, "tile shape");
    // the frames a wave stores, w + NW r, have at most 4 line offsets (period 4 in r)
    static_assert(kGShift == 0 || (NW == 4 && kFPW == 16), "aligned stores: 4 waves, 64-frame tiles");
    // three separate LDS objects: the compiler can tell the loads in flight into one buffer
    // from the reads of another
    __shared__ float buf0[kGRows * kRowF];
    __shared__ float buf1[kGRows * kRowF];
    __shared__ float buf2[kGRows * kRowF];
    const int lane = threadIdx.x % 64;
    const int w = wave_id();
    const int64_t n = a.tiles, G = gridDim.x;

    struct Tile {
        int32_t j0, t0, b;
    };
    // This block's tiles: blockIdx.x, + G, ..., dealt to the XCDs in runs of consecutive
    // tiles.  (Giving each XCD its own range of band-bin columns, or walking the frame
    // tiles of one column on one CU, cut the stft over-fetch but ran 15-20 % slower.)
    const int64_t count = blockIdx.x < n ? (n - 1 - blockIdx.x) / G + 1 : 0;
    auto tile = [&](int k) {
        uint32_t tj, rest, tt, b;
        fdivmod(xcd_runs<MBRT_BAND_XCD>((uint32_t)(blockIdx.x + (int64_t)k * G), a.tiles), a.tiles_j, rest, tj);
        fdivmod(rest, a.tiles_t, b, tt);
        return Tile{(int32_t)tj * kGTJ, (int32_t)tt * TT, (int32_t)b};
    };
    // raw indices of this wave's rows of a tile, by scalar loads (rows past J repeat row
    // J - 1); they are clamped where used, so the loads of a tile are all in flight at once
    int32_t flo[kRPW], fhi[kRPW];
    auto fetch_rows = [&](const Tile& t) {
        const int32_t jb = t.j0 - kGShift + w * kRPW;
#pragma unroll
        for (int q = 0; q < kRPW; ++q) {
            const int32_t j = min(max(jb + q, 0), a.J - 1);
            if constexpr (I64) {
                flo[q] = scalar_load_i32(a.idx, 2 * (int64_t)j);
                fhi[q] = scalar_load_i32(a.idx, 2 * (int64_t)j + 1);
            } else {
                flo[q] = scalar_load_i32(a.idx, j);
            }
        }
    };
    // lane l loads float (l & 1) of frame t0 + 32 h + l / 2 (clamped to the last frame)
    auto issue = [&](const Tile& t, float* buf) {
        int lo[kIPR];
#pragma unroll
        for (int h = 0; h < kIPR; ++h) lo[h] = min(t.t0 + 32 * h + lane / 2, a.T - 1) * 2 + (lane & 1);
        // first LDS row of this wave, re-derived every step (kept out of registers across
        // the loop: the rows of three buffers would not fit the scalar register file)
        int32_t rb = w * kRPW;
        asm volatile("" : "+s"(rb));
#pragma unroll
        for (int q = 0; q < kRPW; ++q) {
            const int32_t f = clamp_freq(flo[q], I64 ? fhi[q] : (flo[q] >> 31), a.F);
            const int32_t row = t.b * a.bft2 + f * a.T * 2;
#pragma unroll
            for (int h = 0; h < kIPR; ++h)
                __builtin_amdgcn_global_load_lds((global_void*)(a.stft + row + lo[h]),
                                                 (lds_void*)&buf[(rb + q) * kRowF + 64 * h], 4, 0, 0);
        }
    };
    // lane = band-bin j0 + lane, frames w + NW r: one 8-byte LDS read and one store each
    // (element offsets fit 32 bits: B * T * J * 2 < 2^31 is checked on the host)
    auto store = [&](const Tile& t, const float* buf) {
        f32x2 v[kFPW];
        if constexpr (kGShift == 0) {
            lds_read_b64_n<kFPW, 0, 8 * NW>(lds_addr(buf) + (uint32_t)(lane * kRowF + 2 * w) * 4, v);
            const int32_t j = t.j0 + lane;
            if (j >= a.J) return;
            int32_t o = (t.b * a.T + t.t0 + w) * a.J + j;
            const int32_t step_o = NW * a.J;
            if (t.t0 + TT <= a.T) {
#pragma unroll
                for (int r = 0; r < kFPW; ++r, o += step_o) store_complex<ODT>(a.out, o, v[r]);
            } else {
                const int nv = (a.T - t.t0 - w + NW - 1) / NW;  // frames of this wave inside T
#pragma unroll
                for (int r = 0; r < kFPW; ++r, o += step_o)
                    if (r < nv) store_complex<ODT>(a.out, o, v[r]);
            }
        } else {
            // frame w + 4 (q + 4 m) of the tile: its row's line offset ph_q depends on q only
            // (4 J (q + 4 m) = 4 J q mod 16); lane l writes band-bin j0 - ph_q + l, which
            // is LDS row l + 16 - ph_q
            int32_t jq[4], oq[4];
            uint32_t aq[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int32_t row0 = (t.b * a.T + t.t0 + w + 4 * q) * a.J;  // first value of the frame row
                const int32_t ph = (int32_t)(((uint32_t)(row0 + t.j0) + a.oph) & 15u);
                jq[q] = t.j0 - ph + lane;
                oq[q] = row0 + jq[q];
                aq[q] = lds_addr(buf) + (uint32_t)((lane + kGShift - ph) * kRowF + 2 * (w + 4 * q)) * 4;
            }
            lds_read_b64_4x4(aq, v);
            const int32_t step_o = 16 * a.J;  // 16 frames
            const int nv = t.t0 + TT <= a.T ? kFPW : (a.T - t.t0 - w + NW - 1) / NW;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (jq[q] >= 0 && jq[q] < a.J) {
#pragma unroll
                    for (int m = 0; m < 4; ++m)
                        if (q + 4 * m < nv) store_complex<ODT>(a.out, oq[q] + m * step_o, v[q + 4 * m]);
                }
            }
        }
    };
    // Tile k of this block is p0 + k G and lives in buffer k % 3.  A steady step k reads
    // tile k and issues the loads of tile k + 2 into the buffer that held tile k - 1; its
    // issue order is the stores of tile k, then exactly kLPT loads, so at the next step
    // only the newest kLPT ops may still be outstanding.  Every load of the steady loop is
    // unconditional, which also lets the compiler's own wait before the LDS reads be the
    // same vmcnt(kLPT).
    if (count == 0) return;
    const int m = (int)count;  // tiles of this block
    auto steady = [&](int k, const float* cur, float* nxt2) {
        wait_vmcnt<kLPT>();
        // every wave's loads into `cur` have landed, and no wave still reads `nxt2`
        lds_barrier();
        store(tile(k), cur);
        issue(tile(k + 2), nxt2);
        if (k + 3 < m) fetch_rows(tile(k + 3));
    };
    fetch_rows(tile(0));
    issue(tile(0), buf0);
    if (m >= 2) {
        fetch_rows(tile(1));
        issue(tile(1), buf1);
    }
    int k = 0;
    if (m >= 3) {
        fetch_rows(tile(2));
        for (;;) {
            steady(k, buf0, buf2);
            if (++k + 2 >= m) break;
            steady(k, buf1, buf0);
            if (++k + 2 >= m) break;
            steady(k, buf2, buf1);
            if (++k + 2 >= m) break;
        }
    }
    // the last one or two tiles (k and k + 1), whose loads are already issued
    auto buf_of = [&](int i) -> const float* { return i % 3 == 0 ? buf0 : i % 3 == 1 ? buf1 : buf2; };
    if (k + 1 < m) {
        wait_vmcnt<kLPT>();
        lds_barrier();
        store(tile(k), buf_of(k));
        ++k;
    }
    wait_vmcnt<0>();
    lds_barrier();
    store(tile(k), buf_of(k));
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
// FB (bf16 masks, bf16-intermediates mode; src/mbr_cuda_tile.cu:5650-5797): a BF16 output
// sums the freq's masks with a bf16 rounding after every add, then divides
// stft * sum by the count and rounds; an F32 output adds, in ascending entry order, each
// entry's stft * mask / count rounded to bf16.
template <int MDT, int ODT, bool I64, bool FB>
__global__ __launch_bounds__(64 * kMW) void band_merge_kernel(MergeArgs a) {
    __shared__ f32x2 ms[kME][kTT + 1];
    // one linear grid; neighbouring freq tiles (whose CSR runs split cache lines of the
    // mask rows) run on one XCD
    const uint32_t tile = xcd_runs<MBRT_BAND_XCD>(blockIdx.x, a.tiles);
    uint32_t tf, tt, rest;
    if constexpr (MBRT_BAND_MERGE_PAIRS) {
        // pairs of frame tiles: tiles (f, 2p) and (f, 2p + 1) are consecutive, then f + 1, so
        // that a run of 8 tiles on one XCD holds 4 freq tiles x 2 frame tiles (an odd last
        // frame tile follows the pairs, freq tiles in order)
        const uint32_t per = a.tiles_f * a.tiles_t;
        rest = tile / per;
        const uint32_t sidx = tile - rest * per;
        const uint32_t paired = (a.tiles_t / 2) * 2 * a.tiles_f;
        if (sidx < paired) {
            const uint32_t p = sidx / (2 * a.tiles_f), r = sidx - p * 2 * a.tiles_f;
            tf = r / 2;
            tt = 2 * p + (r & 1);
        } else {
            tt = a.tiles_t - 1;
            tf = sidx - paired;
        }
    } else if constexpr (MBRT_BAND_MERGE_TFAST) {
        tt = tile % a.tiles_t;
        rest = tile / a.tiles_t;
        tf = rest % a.tiles_f;
        rest = rest / a.tiles_f;
    } else {
        tf = tile % a.tiles_f;
        rest = tile / a.tiles_f;
        tt = rest % a.tiles_t;
        rest = rest / a.tiles_t;
    }
    const int f0 = (int)tf * kTF;
    const int t0 = (int)tt * kTT;
    const int bs = (int)rest;  // b * S + s
    const int b = a.S == 2 ? bs >> 1 : bs;
    const void* mask = a.mask[bs - b * a.S];
    const int lane = threadIdx.x % 64;
    const int w = wave_id();
    constexpr int kPer = kTF / kMW;   // freqs per wave
    constexpr int kR = kTT / kMW;     // staged frames per wave
    constexpr int kEL = kME / 64;     // staged entries per lane
    const int nf = min(kTF, a.F - f0);           // freqs in this tile
    const int t = t0 + lane;
    const int tq = min(t, a.T - 1);

    // CSR offsets of the tile's freqs: lane l holds off[f0 + l] (l < nf; lane nf and up
    // off[f0 + nf]), broadcast by readlane; off_end = off[f0 + nf]
    const int off_lane = ld_idx<I64>(a.off, f0 + min(lane, nf));
    const int off_end = kTF < 64 ? __builtin_amdgcn_readlane(off_lane, kTF < 64 ? nf : 0) : ld_idx<I64>(a.off, f0 + nf);
    // with no band-bins (J = 0) no entry is read, whatever the offsets hold
    const int e_begin = __builtin_amdgcn_readlane(off_lane, 0);
    const int e_end = a.J > 0 ? off_end : e_begin;
    float c = load1(a.cnt, a.cdt, f0 + min(lane, nf - 1));
    const float den_lane = c > 1.0e-8f ? c : 1.0e-8f;
    const float inv_lane = 1.0f / den_lane;
    // readlane reads lanes regardless of EXEC: broadcast while all lanes are active
    float den[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r)
        den[r] = FB ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, den_lane), w + kMW * r))
                    : 1.0f;

    const f32x2* srow = reinterpret_cast<const f32x2*>(a.stft) + ((int64_t)b * a.F + f0) * a.T + tq;
    f32x2 sv[kPer], acc[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        sv[r] = gld<MBRT_NT_BAND>(srow + (int64_t)min(w + kMW * r, nf - 1) * a.T);
        acc[r] = f32x2{0.0f, 0.0f};
    }
    const int64_t mbase = (int64_t)b * a.T;
    for (int c0 = e_begin; c0 < e_end; c0 += kME) {
        const int c1 = min(c0 + kME, e_end);
        // entry and band-bin clamped into ind[0, J) and [0, J): offsets past J read in bounds
        int j[kEL];
#pragma unroll
        for (int h = 0; h < kEL; ++h) {
            const int ei = min(max(min(c0 + 64 * h + lane, c1 - 1), 0), a.J - 1);
            j[h] = min(max(ld_idx<I64>(a.ind, ei), 0), a.J - 1);
        }
        f32x2 mv[kEL][kR];
#pragma unroll
        for (int h = 0; h < kEL; ++h)
#pragma unroll
            for (int r = 0; r < kR; ++r)
                mv[h][r] = load_complex<MDT>(mask, (mbase + min(t0 + w + kMW * r, a.T - 1)) * a.J + j[h]);
#pragma unroll
        for (int h = 0; h < kEL; ++h)
#pragma unroll
            for (int r = 0; r < kR; ++r) ms[64 * h + lane][w + kMW * r] = mv[h][r];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kPer; ++r) {
            const int fl = w + kMW * r;  // local freq (wave-uniform); entries [off[f], off[f+1])
            const int lo = max(__builtin_amdgcn_readlane(off_lane, fl), c0);
            const int nxt = fl + 1 < 64 ? __builtin_amdgcn_readlane(off_lane, min(fl + 1, 63)) : off_end;
            const int hi = fl < nf ? min(nxt, c1) : lo;
            for (int e = lo; e < hi; ++e) {
                const f32x2 m = ms[e - c0][lane];
                if constexpr (!FB) {
                    acc[r].x += sv[r].x * m.x - sv[r].y * m.y;
                    acc[r].y += sv[r].x * m.y + sv[r].y * m.x;
                } else if constexpr (ODT == BF16) {
                    acc[r].x = bf16r(acc[r].x + m.x);
                    acc[r].y = bf16r(acc[r].y + m.y);
                } else {
                    acc[r].x += bf16r((sv[r].x * m.x - sv[r].y * m.y) / den[r]);
                    acc[r].y += bf16r((sv[r].x * m.y + sv[r].y * m.x) / den[r]);
                }
            }
        }
        __syncthreads();
    }
    // readlane reads lanes regardless of EXEC: broadcast the scales while all lanes are active
    float inv[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r)
        inv[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, inv_lane), w + kMW * r));
    if (t >= a.T) return;
    const int64_t bins = a.F / a.C.d;
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int fl = w + kMW * r;
        if (fl < nf) {
            uint32_t bin, ch;
            fdivmod((uint32_t)(f0 + fl), a.C, bin, ch);
            const int64_t o = (((int64_t)bs * a.C.d + ch) * bins + bin) * a.T + t;
            if constexpr (!FB) {
                store_complex<ODT>(a.out, o, f32x2{acc[r].x * inv[r], acc[r].y * inv[r]});
            } else if constexpr (ODT == BF16) {  // rounded on the store
                const f32x2 s = sv[r], m = acc[r];
                store_complex<ODT>(a.out, o, f32x2{(s.x * m.x - s.y * m.y) / den[r], (s.x * m.y + s.y * m.x) / den[r]});
            } else {
                store_complex<ODT>(a.out, o, acc[r]);
            }
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
    if (MBRT_BAND_GATHER_PIPE && B * total_freq * frames * 2 < (int64_t(1) << 31) &&
        B * frames * n_band_freqs * 2 < (int64_t(1) << 31)) {
        constexpr int TT = MBRT_BAND_GTT, NW = MBRT_BAND_GNW;
        GatherPipeArgs g{};
        g.stft = stft;
        g.idx = freq_indices;
        g.out = out;
        g.F = (int32_t)total_freq;
        g.T = (int32_t)frames;
        g.J = (int32_t)n_band_freqs;
        g.bft2 = (int32_t)(total_freq * frames * 2);
        // aligned stores shift a tile's band-bins down by up to 15: one more tile covers the end
        const int64_t tj = ceil_div(n_band_freqs + (kGShift ? 15 : 0), kGTJ), tt = ceil_div(frames, TT);
        const int64_t tiles = tj * tt * B;
        g.oph = (uint32_t)((reinterpret_cast<uintptr_t>(out) / (out_dtype == F32 ? 8 : 4)) % 16);
        g.tiles_j = make_fastdiv((uint32_t)tj);
        g.tiles_t = make_fastdiv((uint32_t)tt);
        g.tiles = (uint32_t)tiles;
        // persistent grid: a multiple of the 8 XCDs, so that block b stays on XCD b % 8
        int64_t grid = std::min<int64_t>(tiles, (int64_t)cu_count() * MBRT_BAND_GBPC);
        if (grid >= kXcds) grid -= grid % kXcds;
        with_dt(out_dtype, [&](auto ot) {
            constexpr int O = decltype(ot)::value;
            if (index_dtype == I64)
                hipLaunchKernelGGL((band_gather_pipe_kernel<O, true, NW, TT>), dim3((unsigned)grid), dim3(64 * NW), 0,
                                   as_stream(stream), g);
            else
                hipLaunchKernelGGL((band_gather_pipe_kernel<O, false, NW, TT>), dim3((unsigned)grid), dim3(64 * NW), 0,
                                   as_stream(stream), g);
        });
        return check_launch(op);
    }
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
    // with no band-bins csr_indices may be NULL: the kernel then reads no index and no mask
    // (a.J = 0), and every output is 0 / max(count, 1e-8) = 0
    a.ind = n_band_freqs > 0 ? csr_indices : csr_offsets;
    a.cnt = counts;
    a.out = out;
    a.cdt = counts_dtype;
    a.S = num_stems;
    a.F = (int)total_freq;
    a.T = (int)frames;
    a.J = (int)n_band_freqs;
    a.C = make_fastdiv((uint32_t)channels);
    const int64_t tiles = ceil_div(total_freq, kTF) * ceil_div(frames, kTT) * B * num_stems;
    MBRT_REQUIRE(tiles < (int64_t(1) << 31), MBRT_E_SHAPE, "%s: too many tiles", op);
    a.tiles_f = (uint32_t)ceil_div(total_freq, kTF);
    a.tiles_t = (uint32_t)ceil_div(frames, kTT);
    a.tiles = (uint32_t)tiles;
    const dim3 grid(a.tiles);
    // bf16 intermediates: bf16 masks into a BF16 or F32 output, as in the reference
    const bool fb = bf16_intermediates() && mask_dtype == BF16 && (out_dtype == BF16 || out_dtype == F32);
    with_dt(mask_dtype, [&](auto mt) {
        with_dt(out_dtype, [&](auto ot) {
            constexpr int M = decltype(mt)::value, O = decltype(ot)::value;
            if constexpr (M == BF16 && O != F16) {
                if (fb) {
                    if (index_dtype == I64)
                        hipLaunchKernelGGL((band_merge_kernel<M, O, true, true>), grid, dim3(64 * kMW), 0, as_stream(stream), a);
                    else
                        hipLaunchKernelGGL((band_merge_kernel<M, O, false, true>), grid, dim3(64 * kMW), 0, as_stream(stream), a);
                    return;
                }
            }
            if (index_dtype == I64)
                hipLaunchKernelGGL((band_merge_kernel<M, O, true, false>), grid, dim3(64 * kMW), 0, as_stream(stream), a);
            else
                hipLaunchKernelGGL((band_merge_kernel<M, O, false, false>), grid, dim3(64 * kMW), 0, as_stream(stream), a);
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
