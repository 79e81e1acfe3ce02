// Fused attention O = softmax(scale * Q K^T) V on MFMA, for bf16 q, k, v [BH, N, 64]:
// the time attention (N = 801) and frequency attention (N = 60) of the band-split
// transformer (src/mbr_cuda_tile.cu:6530-6709, src/mbr_time_attention_cutile.cu:108-196).
// The [BH, N, N] score matrix never reaches HBM: each workgroup streams K/V tiles through
// LDS and keeps an online softmax (running max m, running sum l) per query.  The tiles go
// from HBM straight into LDS (global_load_lds_dwordx4), double buffered: the next tile
// loads while the current one is computed, one barrier per tile.
//
// Workgroup = 4 waves of one (b, h); wave w owns 16 or 32 queries (QS sub-blocks of 16).
// Per 64-key tile, with v_mfma_f32_16x16x32_bf16 (lane l: A[l%16][8(l/16)+j],
// B[8(l/16)+j][l%16], C[4(l/16)+i][l%16]):
//   S^T = K Q^T     8 MFMAs: A = K rows from LDS, B = the wave's Q fragment (registers).
//                   Lane l then holds S^T[key 16kb + 4(l/16) + i][query l%16].
//   online softmax  per query l%16: each lane keeps a partial row sum over its own keys
//                   (the four lane groups are added after the last tile).  The exponent
//                   reference moves only when a score outgrows it by 2^8; only then is
//                   the max taken over the four lane groups (xor 16, xor 32) and the
//                   accumulator rescaled in place.
//   O^T += V^T P^T  16 MFMAs: B = P^T straight from the S^T registers, as a bf16 pair
//                   P_hi + P_lo; A = V^T read from the row-major V tile with the gfx950
//                   LDS transpose read (ds_read_b64_tr_b16).
//   (MFMA counts per 16-query sub-block.)  The contraction runs over
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
constexpr float kLazy = 8.0f;  // log2 units the running max may outgrow the exponent reference
// Word 3 of a raw buffer resource on gfx9-family parts (32-bit data format, no swizzle,
// no stride): loads of byte offset o < num_records read base + o.
constexpr int kBufferDword3 = 0x00020000;
#ifndef MBRT_ATTN_WPE
#define MBRT_ATTN_WPE 4  // waves per SIMD the register budget is sized for (4: at most 128 VGPRs)
#endif
#ifndef MBRT_ATTN_PRIO_PAIR
#define MBRT_ATTN_PRIO_PAIR 1  // the bf16-pair mode raises wave priority around its MFMA blocks
#endif
#ifndef MBRT_ATTN_QS2_MIN
#define MBRT_ATTN_QS2_MIN 1  // 32 queries per wave when n_q exceeds this many 64-query blocks
#endif

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;  // an LDS-resident bf16x4

// K/V tiles in LDS: [64 keys][64 d] bf16 without padding, a key row = eight 16-byte chunks.
// Logical chunk j of key r sits at chunk j ^ (r & 7), so that the 16-byte fragment reads
// of 8 consecutive keys (same logical chunk) fall on 8 different bank groups.
__device__ __forceinline__ int tile_at(int r, int chunk, int within) {
    return r * kHeadDim + 8 * (chunk ^ (r & 7)) + within;
}

// Element (bh, n, d) of q sits at q + b q_bs + h q_hs + n q_rs + d, with b = bh / H and
// h = bh % H; k and v likewise with the kv strides.  Contiguous [BH, N, 64] is H = 1.
struct AttnArgs {
    const __bf16* q;
    const __bf16* k;
    const __bf16* v;
    void* out;
    int nq, nk;
    uint32_t qtiles;
    float scale_log2e;
    FastDiv heads;
    int64_t q_bs, q_hs, kv_bs, kv_hs;
    int q_rs, kv_rs;
    const void* cosp;   // q rotary tables [n_q, 32] of dtype tdt, or NULL: q used as given
    const void* sinp;
    int tdt;
    const void* gate;   // gate [B, n_q, H] of dtype gdt, or NULL: out [BH, n_q, 64]
    int gdt;
    int glogit;         // the gate holds logits: sigmoid(gate) multiplies
    uint32_t nbh;       // B * H (the persistent form walks heads blockIdx.x, + gridDim.x, ...)
};

// Barrier for data that arrived by direct-to-LDS loads: the caller has waited (vmcnt) for
// this wave's own loads, and the barrier makes every wave's visible.  Unlike
// __syncthreads() it carries no memory fence, which would also wait for the previous
// head's output stores.  The empty asm statements keep LDS accesses on their side.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// max of the 16 scores a lane holds for one 16-query sub-block (the file is built without
// NaN semantics, so the maxima need no quieting and fold into v_max3)
__device__ __forceinline__ float max16(const f32x4 (&s)[4]) {
    float m = s[0][0];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) m = fmaxf(m, s[kb][i]);
    return m;
}
__device__ __forceinline__ float xor_max(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    return fmaxf(x, __shfl_xor(x, 32));
}
// The eight V^T transpose reads of one 32-key chunk (four 16-column blocks db, rows r and
// r + 16 each) at LDS byte addresses ad[db] + OFF and ad[db] + OFF + 2048, issued together
// and completed before the statement ends: the compiler, short of registers, would
// otherwise interleave them with the MFMAs and wait for each pair on its own.
template <int OFF>
__device__ __forceinline__ void lds_read_vt(const uint32_t (&ad)[4], bf16x8 (&va)[4]) {
    u32x2 r[8];
    asm volatile(
        "ds_read_b64_tr_b16 %0, %8 offset:%[lo]\n\t"
        "ds_read_b64_tr_b16 %1, %8 offset:%[hi]\n\t"
        "ds_read_b64_tr_b16 %2, %9 offset:%[lo]\n\t"
        "ds_read_b64_tr_b16 %3, %9 offset:%[hi]\n\t"
        "ds_read_b64_tr_b16 %4, %10 offset:%[lo]\n\t"
        "ds_read_b64_tr_b16 %5, %10 offset:%[hi]\n\t"
        "ds_read_b64_tr_b16 %6, %11 offset:%[lo]\n\t"
        "ds_read_b64_tr_b16 %7, %11 offset:%[hi]\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
        : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), [lo] "n"(OFF), [hi] "n"(OFF + 2048)
        : "memory");
#pragma unroll
    for (int db = 0; db < 4; ++db)
        va[db] = __builtin_bit_cast(bf16x8, u32x4{r[2 * db].x, r[2 * db].y, r[2 * db + 1].x, r[2 * db + 1].y});
}

// 16-byte fragments of a swizzled [64][64] bf16 LDS tile, read in one asm block and completed
// before the statement ends: the persistent form reads its K and Q tiles this way, so that
// the compiler, which cannot tell one LDS buffer from another, does not wait for the next
// head's loads in flight (vmcnt 0) before these reads.  f[i] is read at byte address
// ad[i % NA] + 2048 (i / NA).
template <int N, int NA>
__device__ __forceinline__ void lds_read_frags(const uint32_t (&ad)[NA], bf16x8 (&f)[N]) {
    static_assert((N == 8 && NA == 2) || (N == 2 && NA == 2), "K: 4 key blocks x 2 halves; Q: 2 halves");
    u32x4 r[N];
    if constexpr (N == 8) {
        asm volatile(
            "ds_read_b128 %0, %8\n\t"
            "ds_read_b128 %1, %9\n\t"
            "ds_read_b128 %2, %8 offset:2048\n\t"
            "ds_read_b128 %3, %9 offset:2048\n\t"
            "ds_read_b128 %4, %8 offset:4096\n\t"
            "ds_read_b128 %5, %9 offset:4096\n\t"
            "ds_read_b128 %6, %8 offset:6144\n\t"
            "ds_read_b128 %7, %9 offset:6144\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
            : "v"(ad[0]), "v"(ad[1])
            : "memory");
    } else {
        asm volatile(
            "ds_read_b128 %0, %2\n\t"
            "ds_read_b128 %1, %3\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(r[0]), "=&v"(r[1])
            : "v"(ad[0]), "v"(ad[1])
            : "memory");
    }
#pragma unroll
    for (int i = 0; i < N; ++i) f[i] = __builtin_bit_cast(bf16x8, r[i]);
}

// LDS writes and reads of the persistent form's output staging, as asm so that the
// compiler, which cannot tell this wave's staging rows from the next head's tiles loading
// into other buffers, does not wait for those loads (vmcnt 0) before them.  The writes
// end with their own lgkmcnt(0); the two reads of lds_read_b128_x2 complete before it
// returns.
__device__ __forceinline__ void lds_write_b64(uint32_t ad, u32x2 v) {
    asm volatile("ds_write_b64 %0, %1" ::"v"(ad), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_write_b128(uint32_t ad, u32x4 v) {
    asm volatile("ds_write_b128 %0, %1" ::"v"(ad), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void lds_read_b128_x2(uint32_t a0, uint32_t a1, u32x4& r0, u32x4& r1) {
    asm volatile(
        "ds_read_b128 %0, %2\n\t"
        "ds_read_b128 %1, %3\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r0), "=&v"(r1)
        : "v"(a0), "v"(a1)
        : "memory");
}

__device__ __forceinline__ float xor_sum(float x) {
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}

// QS = 16-query sub-blocks per wave (1 or 2): every K and V^T fragment read from LDS
// feeds QS MFMAs, so longer sequences use QS = 2 (128 queries per workgroup).
// PM = precision of P in the second product: MBRT_ATTN_P_PAIR (P as a bf16 hi + lo pair,
// f32 accuracy, lazy max), MBRT_ATTN_P_BF16 (the reference's arithmetic,
// src/mbr_time_attention_cutile.cu:160-180: the running max moves every 64-key tile, P is
// rounded once to bf16 for one P V product, and the row sum adds the unrounded P) or
// MBRT_ATTN_P_BF16_FAST (P rounded once to bf16 under the lazy max, and the row sum formed
// by the MFMA from the same rounded P, as a 17th block of V columns that are all 1: no
// rescale on most tiles and no VALU row sum).
// HEADS: the persistent form for heads of at most 64 queries and 64 keys (the frequency
// attention): a workgroup walks heads blockIdx.x, + gridDim.x, ..., and while it computes
// one head the next head's K, V and Q tiles are already loading into the other LDS buffers,
// so that the loads, the arithmetic and the output stores of consecutive heads overlap.  A
// workgroup per head instead (the general form) runs load, arithmetic and store of its head
// in turn, in step with every other workgroup on the CU.
template <int ODT, int QS, int PM, bool HEADS>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(HEADS ? 3 : MBRT_ATTN_WPE))) void attention_kernel(AttnArgs a) {
    // two K and two V tiles: the next pair is loaded (straight into LDS) while the current
    // one is read; the persistent form also loads Q into LDS
    __shared__ __attribute__((aligned(16))) __bf16 k0[kKeys * kHeadDim];
    __shared__ __attribute__((aligned(16))) __bf16 v0[kKeys * kHeadDim];
    __shared__ __attribute__((aligned(16))) __bf16 k1[kKeys * kHeadDim];
    __shared__ __attribute__((aligned(16))) __bf16 v1[kKeys * kHeadDim];
    constexpr int kQTile = HEADS ? kQBlock * kHeadDim : 8;
    __shared__ __attribute__((aligned(16))) __bf16 qt0[kQTile];
    __shared__ __attribute__((aligned(16))) __bf16 qt1[kQTile];
    static_assert(!HEADS || QS == 1, "the persistent form holds 16 queries per wave");
    constexpr int kQB = kQWave * QS * kWaves;  // queries per workgroup
    const int tid = threadIdx.x;
    const int lane = tid % 64, g = lane / 16, c = lane % 16;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    // one linear grid of (b, h, query tile), the query tiles of one (b, h) adjacent; each
    // XCD walks one contiguous range of it, so that the query tiles of a (b, h) run on one
    // XCD, close in time, and read its K/V once into that XCD's L2.  The persistent form
    // starts at head blockIdx.x and has a single query tile.
    const uint32_t tile = HEADS ? blockIdx.x : xcd_tile(blockIdx.x, gridDim.x);
    uint32_t bh = tile / a.qtiles;
    const int q0 = (tile % a.qtiles) * kQB + w * kQWave * QS;
    uint32_t b, h;
    fdivmod(bh, a.heads, b, h);
    const __bf16* kbase = a.k + b * a.kv_bs + h * a.kv_hs;
    const __bf16* vbase = a.v + b * a.kv_bs + h * a.kv_hs;

    // Q fragments: for sub-block x, lane holds Q[q0 + 16x + c][32s + 8g .. +7], s = 0, 1
    // (the persistent form reads them from its LDS Q tile, head by head)
    bf16x8 qf[QS][2];
    if constexpr (!HEADS) {
#pragma unroll
    for (int x = 0; x < QS; ++x) {
        const __bf16* qrow = a.q + b * a.q_bs + h * a.q_hs + (int64_t)min(q0 + 16 * x + c, a.nq - 1) * a.q_rs;
#pragma unroll
        for (int s = 0; s < 2; ++s) qf[x][s] = gld<MBRT_ATTN_NT & 1>(reinterpret_cast<const bf16x8*>(qrow + 32 * s + 8 * g));
    }
    }
    if (!HEADS && a.cosp != nullptr) {
        // in-kernel rotary of q: the lane's 8 values are the pairs 16s + 4g .. +3 of its query
        // row, rotated by the shared rotate() in f32 and rounded to bf16 as the rotary kernel
        // does (src/mbr_time_attention_cutile.cu:80-106, 489-490)
#pragma unroll
        for (int x = 0; x < QS; ++x) {
            const int64_t t = (int64_t)min(q0 + 16 * x + c, a.nq - 1) * (kHeadDim / 2);
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                float cs[4], sn[4];
                if (a.tdt == F32) {
                    Vec<F32, 4> cv, sv;
                    cv.load(a.cosp, t + 16 * s + 4 * g);
                    sv.load(a.sinp, t + 16 * s + 4 * g);
                    cv.to_f32(cs);
                    sv.to_f32(sn);
                } else {
                    Vec<BF16, 4> cv, sv;
                    cv.load(a.cosp, t + 16 * s + 4 * g);
                    sv.load(a.sinp, t + 16 * s + 4 * g);
                    cv.to_f32(cs);
                    sv.to_f32(sn);
                }
                Vec<BF16, 8> qv;
                const u32x4 qw = __builtin_bit_cast(u32x4, qf[x][s]);
                qv.w[0] = qw.x; qv.w[1] = qw.y; qv.w[2] = qw.z; qv.w[3] = qw.w;
                float xv[8];
                qv.to_f32(xv);
                rotate<8>(xv, cs, sn);
                qv.from_f32(xv);
                qf[x][s] = __builtin_bit_cast(bf16x8, u32x4{qv.w[0], qv.w[1], qv.w[2], qv.w[3]});
            }
        }
    }

    constexpr bool kLazyMax = PM != MBRT_ATTN_P_BF16;
    constexpr bool kSumMfma = PM == MBRT_ATTN_P_BF16_FAST;
    // The pair mode issues 24 MFMAs per 16 queries and tile; a wave inside one of its MFMA
    // blocks runs at priority 1, so that its MFMAs issue ahead of the softmax VALU work of
    // the other waves on the SIMD (measured: pair mode about 2 % faster; the single-P modes
    // ran 3-4 % slower with it and keep priority 0).
    constexpr bool kPrio = PM == MBRT_ATTN_P_PAIR && MBRT_ATTN_PRIO_PAIR;
    f32x4 o[QS][4];
    f32x4 osum[QS];  // kSumMfma: lane (g, c) holds the row sum of query c, four times
    float m[QS], l[QS];
    auto reset_state = [&]() {
#pragma unroll
        for (int x = 0; x < QS; ++x) {
#pragma unroll
            for (int db = 0; db < 4; ++db) o[x][db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            osum[x] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            m[x] = -INFINITY;
            l[x] = 0.0f;
        }
    };
    reset_state();
    // A operand of the row-sum MFMA: a 16 x 32 block of bf16 ones
    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});

    // Tile loads go from HBM straight into LDS (global_load_lds_dwordx4: lane i of a wave
    // instruction writes the 16 bytes at base + 16 i).  Wave w loads keys 16w .. 16w + 15 of
    // a tile, 8 per instruction: lane i -> key 16w + 8u + i/8, stored chunk i % 8, which
    // holds logical chunk (i % 8) ^ (i / 8).  Keys past N load a clamped row (masked later).
    // Element offsets within one (b, h) fit 32 bits (n_k * 64 < 2^31 is checked on the host).
    // A whole tile (no key past N) loads through buffer resources of this head's K and V
    // rows: the tile's first row is a scalar offset (kt rows in bytes) and each lane's two
    // chunks fixed 32-bit offsets from it, so a tile's addresses cost no vector
    // instructions.  The rows of one head span < 2^32 bytes (checked on the host), so the
    // offsets and their sums stay below the descriptors' 2^32 - 1 records.
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)0, -1, kBufferDword3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, -1, kBufferDword3);
    uint32_t loff[2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
        loff[u] = 2u * ((uint32_t)(16 * w + 8 * u + (lane >> 3)) * (uint32_t)a.kv_rs + 8u * ((lane & 7) ^ (lane >> 3)));
    auto load_tile = [&](int kt, int buf) {
        __bf16* kd = buf ? k1 : k0;
        __bf16* vd = buf ? v1 : v0;
        if (kt + kKeys <= a.nk) {
            const int soff = (int)(2u * (uint32_t)kt * (uint32_t)a.kv_rs);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int r0 = 16 * w + 8 * u;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)&kd[r0 * kHeadDim], 16, loff[u], soff, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)&vd[r0 * kHeadDim], 16, loff[u], soff, 0, 0);
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int r0 = 16 * w + 8 * u, key = r0 + (lane >> 3);
            const uint32_t off = (uint32_t)min(kt + key, a.nk - 1) * a.kv_rs + 8 * ((lane & 7) ^ (lane >> 3));
            __builtin_amdgcn_global_load_lds((global_void*)(kbase + off), (lds_void*)&kd[r0 * kHeadDim], 16, 0, 0);
            __builtin_amdgcn_global_load_lds((global_void*)(vbase + off), (lds_void*)&vd[r0 * kHeadDim], 16, 0, 0);
        }
    };
    // The persistent form's loads of one head (a single key tile and the query tile) into
    // kd/vd/qd: wave w loads keys and queries 16w .. 16w + 15 as above, rows past n_k or
    // n_q clamped.
    auto load_head = [&](uint32_t hh, __bf16* kd, __bf16* vd, __bf16* qd) {
        uint32_t hb, hh2;
        fdivmod(hh, a.heads, hb, hh2);
        const __bf16* kb = a.k + hb * a.kv_bs + hh2 * a.kv_hs;
        const __bf16* vb = a.v + hb * a.kv_bs + hh2 * a.kv_hs;
        const __bf16* qb = a.q + hb * a.q_bs + hh2 * a.q_hs;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int r0 = 16 * w + 8 * u, row = r0 + (lane >> 3);
            const uint32_t chunk = 8 * ((lane & 7) ^ (lane >> 3));
            const uint32_t koff = (uint32_t)min(row, a.nk - 1) * a.kv_rs + chunk;
            const uint32_t qoff = (uint32_t)min(row, a.nq - 1) * a.q_rs + chunk;
            __builtin_amdgcn_global_load_lds((global_void*)(kb + koff), (lds_void*)&kd[r0 * kHeadDim], 16, 0, (MBRT_ATTN_HEADS_NT & 2) ? kCpolNt : 0);
            __builtin_amdgcn_global_load_lds((global_void*)(vb + koff), (lds_void*)&vd[r0 * kHeadDim], 16, 0, (MBRT_ATTN_HEADS_NT & 2) ? kCpolNt : 0);
            __builtin_amdgcn_global_load_lds((global_void*)(qb + qoff), (lds_void*)&qd[r0 * kHeadDim], 16, 0, (MBRT_ATTN_HEADS_NT & 2) ? kCpolNt : 0);
        }
    };
    if constexpr (HEADS) load_head(bh, k0, v0, qt0);
    else load_tile(0, 0);
    // The arithmetic of one key tile held in ks/vs (below); the caller has made the tile
    // visible to every wave.
    auto tile_compute = [&](int kt, const __bf16* ks, const __bf16* vs) {
        // S^T = K Q^T for the 4 key blocks of the tile and every query sub-block
        if constexpr (kPrio) __builtin_amdgcn_s_setprio(1);
        f32x4 st[QS][4];
        // the persistent form reads the tile's K fragments in one asm block (see
        // lds_read_frags): kfr[2 kb + s] = K[16 kb + c][32 s + 8 g .. +7]
        bf16x8 kfr[HEADS ? 8 : 1];
        if constexpr (HEADS) {
            const uint32_t kad[2] = {lds_addr(ks) + 2 * (uint32_t)tile_at(c, g, 0),
                                     lds_addr(ks) + 2 * (uint32_t)tile_at(c, 4 + g, 0)};
            lds_read_frags<8, 2>(kad, kfr);
        }
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int x = 0; x < QS; ++x) st[x][kb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                bf16x8 ka;
                if constexpr (HEADS) ka = kfr[2 * kb + s];
                else ka = *reinterpret_cast<const bf16x8*>(&ks[tile_at(16 * kb + c, 4 * s + g, 0)]);
#pragma unroll
                for (int x = 0; x < QS; ++x)
                    st[x][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qf[x][s], st[x][kb], 0, 0, 0);
            }
        }
        if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
        // online softmax per query, on raw scores: the scale is folded into the exponent,
        // exp2(scale log2e (s - max)); keys past N occur only in the last tile
        if (kt + kKeys > a.nk) {
#pragma unroll
            for (int x = 0; x < QS; ++x)
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (kt + 16 * kb + 4 * g + i >= a.nk) st[x][kb][i] = -INFINITY;
        }
        if constexpr (!kLazyMax) {
            // the reference's running max: m[x] = max(m[x], max of the tile's scaled scores)
            // every tile, the accumulator and row sum rescaled by exp2(m_old - m_new)
#pragma unroll
            for (int x = 0; x < QS; ++x) {
                const float mx = max16(st[x]);
                const float mn = fmaxf(m[x], xor_max(mx) * a.scale_log2e);
                const float alpha = __builtin_amdgcn_exp2f(m[x] - mn);
                l[x] *= alpha;
#pragma unroll
                for (int db = 0; db < 4; ++db) o[x][db] *= alpha;
                m[x] = mn;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float p = __builtin_amdgcn_exp2f(fmaf(st[x][kb][i], a.scale_log2e, -m[x]));
                        st[x][kb][i] = p;
                        l[x] += p;
                    }
                }
            }
        } else {
#pragma unroll
        for (int x = 0; x < QS; ++x) {
            // m[x] is the exponent reference in log2 units, the same in the four lanes of a
            // query.  It moves only when a score exceeds it by more than kLazy (scaled):
            // P <= 2^kLazy otherwise, harmless in f32 and in the bf16 pair, and the
            // accumulator is rescaled about once per query.  The lane's own 16 scores decide
            // whether to look; the max over the query's four lanes is formed only then.
            float mx = max16(st[x]);
            // wave-uniform branch, taken on the (rare) tiles where some score of the wave
            // outgrows its reference; queries that do not grow keep alpha = 1
            if (__builtin_amdgcn_ballot_w64(mx * a.scale_log2e > m[x] + kLazy) != 0) {
                mx = xor_max(mx) * a.scale_log2e;
                const float mn = mx > m[x] + kLazy ? mx : m[x];
                const float alpha = __builtin_amdgcn_exp2f(m[x] - mn);
                l[x] *= alpha;
                osum[x] *= alpha;
#pragma unroll
                for (int db = 0; db < 4; ++db) o[x][db] *= alpha;
                m[x] = mn;
            }
            // l[x] is the lane's partial row sum over its own keys; the four lanes of a
            // query are added once, after the last tile (the MFMA forms it when kSumMfma)
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(st[x][kb][i], a.scale_log2e, -m[x]));
                    st[x][kb][i] = p;
                    if constexpr (!kSumMfma) l[x] += p;
                }
            }
        }

        }  // PM
        // O^T += V^T P^T over the two 32-key chunks.  P = P_hi + P_lo, both bf16: hi is P
        // truncated to bf16 (exact), lo = P - hi (exact in f32) rounded to bf16, so the
        // pair carries 16 mantissa bits and the product keeps f32 accuracy.
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            bf16x8 ph[QS], pl[QS];
#pragma unroll
            for (int x = 0; x < QS; ++x) {
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int i = 0; i < 4; i += 2) {
                        const float p0 = st[x][2 * cc + h][i], p1 = st[x][2 * cc + h][i + 1];
                        if constexpr (PM != MBRT_ATTN_P_PAIR) {
                            hw[2 * h + i / 2] = pack_bf16x2(p0, p1);  // one RNE rounding
                        } else {
                            const uint32_t b0 = __float_as_uint(p0) & 0xffff0000u;
                            const uint32_t b1 = __float_as_uint(p1) & 0xffff0000u;
                            hw[2 * h + i / 2] = __builtin_amdgcn_perm(b1, b0, 0x07060302u);
                            lw[2 * h + i / 2] = pack_bf16x2(p0 - __uint_as_float(b0), p1 - __uint_as_float(b1));
                        }
                    }
                }
                ph[x] = __builtin_bit_cast(bf16x8, u32x4{hw[0], hw[1], hw[2], hw[3]});
                if constexpr (PM == MBRT_ATTN_P_PAIR) pl[x] = __builtin_bit_cast(bf16x8, u32x4{lw[0], lw[1], lw[2], lw[3]});
                if constexpr (kSumMfma) osum[x] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, ph[x], osum[x], 0, 0, 0);
            }
            // V^T operand by LDS transpose reads: in each 16-lane group, lane i receives
            // element i%4 of the 8-byte chunks of lanes 4r + i/4 (r = 0..3), so lane
            // (g, c) supplies V[32cc + 4g + c/4 (+16)][16db + 4(c%4) ..] and receives
            // V[32cc + 4g + r (+16)][16db + c] for r = 0..3: slots j and 4 + j.  The
            // eight reads of a chunk are issued together, ahead of its MFMAs (rows 32cc
            // and 16 further are 4096 and 2048 bytes on; the chunk swizzle depends on
            // the row mod 8 only).
            uint32_t vad[4];
#pragma unroll
            for (int db = 0; db < 4; ++db)
                vad[db] = lds_addr(vs) + 2 * (uint32_t)tile_at(4 * g + (c >> 2), 2 * db + ((c & 3) >> 1), 4 * (c & 1));
            bf16x8 vat[4];
            if (cc == 0) lds_read_vt<0>(vad, vat);
            else lds_read_vt<4096>(vad, vat);
            if constexpr (kPrio) __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const bf16x8 va = vat[db];
#pragma unroll
                for (int x = 0; x < QS; ++x) {
                    o[x][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, ph[x], o[x][db], 0, 0, 0);
                    if constexpr (PM == MBRT_ATTN_P_PAIR)
                        o[x][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pl[x], o[x][db], 0, 0, 0);
                }
            }
            if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
        }
    };
    // One key tile: ks/vs hold it, kn/vn receive the next one.  The two buffer pairs are
    // separate LDS objects and the loop below is unrolled by two, so the compiler sees that
    // the loads in flight into kn/vn never alias the reads of ks/vs and waits for them only
    // at the next tile's barrier.
    auto tile_step = [&](int kt, const __bf16* ks, const __bf16* vs, int nbuf) {
        // this wave's loads of the tile have landed (vmcnt 0); after the barrier every
        // wave's have, and no wave still reads the other buffer, which is refilled next
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
        if (kt + kKeys < a.nk) load_tile(kt + kKeys, nbuf);
        // a wave whose queries all lie past N (in the last query tile of a head) loads its
        // share of every K/V tile and joins every barrier, but has nothing to compute
        if (q0 >= a.nq) return;
        tile_compute(kt, ks, vs);
    };

    // the output of the head (b, h) = bh
    auto store_out = [&]() {
#pragma unroll
    for (int x = 0; x < QS; ++x) {
        const float lsum = kSumMfma ? osum[x][0] : xor_sum(l[x]);
        const int q = q0 + 16 * x + c;
        if (q >= a.nq) continue;
        const float inv = 1.0f / lsum;
        if (a.gate != nullptr) {
            // gate and head merge: merged[b, q, h*64 + d] = O * g(b, q, h), O first rounded to
            // the output dtype, so that the result equals the attention output passed through
            // mbrt_sigmoid_gate_merge
            const int64_t tok = ((int64_t)b * a.nq + q) * a.heads.d + h;
            const float gl = load1(a.gate, a.gdt, tok);
            const float gv = a.glogit ? sigmoidf(gl) : gl;
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const int64_t e = tok * kHeadDim + 16 * db + 4 * g;
                if constexpr (ODT == F32) {
                    gst<MBRT_ATTN_NT & 2>(reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + e), (o[x][db] * inv) * gv);
                } else {
                    const uint32_t r0 = pack_bf16x2(o[x][db][0] * inv, o[x][db][1] * inv);
                    const uint32_t r1 = pack_bf16x2(o[x][db][2] * inv, o[x][db][3] * inv);
                    u32x2 pk;
                    pk.x = pack_bf16x2(bf16_lo(r0) * gv, bf16_hi(r0) * gv);
                    pk.y = pack_bf16x2(bf16_lo(r1) * gv, bf16_hi(r1) * gv);
                    gst<MBRT_ATTN_NT & 2>(reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(a.out) + e), pk);
                }
            }
            continue;
        }
        const int64_t obase = ((int64_t)bh * a.nq + q) * kHeadDim;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const int d = 16 * db + 4 * g;
            if constexpr (ODT == F32) {
                gst<MBRT_ATTN_NT & 2>(reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + obase + d), o[x][db] * inv);
            } else {
                u32x2 pk;
                pk.x = pack_bf16x2(o[x][db][0] * inv, o[x][db][1] * inv);
                pk.y = pack_bf16x2(o[x][db][2] * inv, o[x][db][3] * inv);
                gst<MBRT_ATTN_NT & 2>(reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(a.out) + obase + d), pk);
            }
        }
    }
    };

    if constexpr (!HEADS) {
        for (int kt = 0; kt < a.nk; kt += 2 * kKeys) {
            tile_step(kt, k0, v0, 1);
            if (kt + kKeys < a.nk) tile_step(kt + kKeys, k1, v1, 0);
        }
        store_out();
    } else {
        // Head `cur` sits in ks/vs/qs; the next head of this workgroup loads into kn/vn/qn.
        // Vector-memory operations retire in issue order, so when the previous head left
        // exactly its kStores output stores behind the loads of `cur`, waiting until at most
        // kStores are outstanding completes those loads and leaves the stores in flight.
        // A wave without queries (q0 >= n_q) stores nothing and waits for all.
        // The output leaves through this wave's 16 rows of the head's Q tile (2 KB, free once
        // the Q fragments are in registers, private to the wave): O is written there in
        // query rows, each 16-byte chunk at chunk ^ (row % 8), and read back as whole rows,
        // so every store instruction writes 8 full query rows (1 KB of a bf16 output, 512 B
        // per half of an f32 one) instead of 32 bytes in each of 16 rows.  Rows past n_q
        // were computed from the clamped query row n_q - 1 and hold its output bit for bit;
        // they are stored again over row n_q - 1, so every store instruction has all lanes
        // active and the store count per head is fixed.
        constexpr int kStores = ODT == F32 ? 4 : 2;  // output stores per wave and head
        auto store_staged = [&](const __bf16* qs) {
            const float lsum = kSumMfma ? osum[0][0] : xor_sum(l[0]);
            const float inv = 1.0f / lsum;
            const uint32_t base = lds_addr(qs) + 16u * 128u * (uint32_t)w;
            const int r0 = lane >> 3, r1 = 8 + (lane >> 3), ck = lane & 7;
            const uint32_t rd0 = base + 128u * r0 + 16u * (uint32_t)(ck ^ (r0 & 7));
            const uint32_t rd1 = base + 128u * r1 + 16u * (uint32_t)(ck ^ (r1 & 7));
            const int64_t row0 = (int64_t)bh * a.nq + min(q0 + r0, a.nq - 1);
            const int64_t row1 = (int64_t)bh * a.nq + min(q0 + r1, a.nq - 1);
            if constexpr (ODT == F32) {
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                    for (int k2 = 0; k2 < 2; ++k2) {
                        const f32x4 v = o[0][2 * hh + k2] * inv;
                        lds_write_b128(base + 128u * c + 16u * (uint32_t)((4 * k2 + g) ^ (c & 7)),
                                       __builtin_bit_cast(u32x4, v));
                    }
                    lds_wait();
                    u32x4 v0, v1;
                    lds_read_b128_x2(rd0, rd1, v0, v1);
                    float* out = reinterpret_cast<float*>(a.out);
                    gst<(MBRT_ATTN_HEADS_NT & 1) ? 2 : 0>(reinterpret_cast<u32x4*>(out + row0 * kHeadDim + 32 * hh + 4 * ck), v0);
                    gst<(MBRT_ATTN_HEADS_NT & 1) ? 2 : 0>(reinterpret_cast<u32x4*>(out + row1 * kHeadDim + 32 * hh + 4 * ck), v1);
                }
            } else {
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    u32x2 pk;
                    pk.x = pack_bf16x2(o[0][db][0] * inv, o[0][db][1] * inv);
                    pk.y = pack_bf16x2(o[0][db][2] * inv, o[0][db][3] * inv);
                    lds_write_b64(base + 128u * c + 16u * (uint32_t)((2 * db + (g >> 1)) ^ (c & 7)) + 8u * (g & 1), pk);
                }
                lds_wait();
                u32x4 v0, v1;
                lds_read_b128_x2(rd0, rd1, v0, v1);
                uint16_t* out = reinterpret_cast<uint16_t*>(a.out);
                gst<(MBRT_ATTN_HEADS_NT & 1) ? 2 : 0>(reinterpret_cast<u32x4*>(out + row0 * kHeadDim + 8 * ck), v0);
                gst<(MBRT_ATTN_HEADS_NT & 1) ? 2 : 0>(reinterpret_cast<u32x4*>(out + row1 * kHeadDim + 8 * ck), v1);
            }
        };
        bool first = true;
        auto head_step = [&](uint32_t cur, const __bf16* ks, const __bf16* vs, const __bf16* qs, __bf16* kn,
                             __bf16* vn, __bf16* qn) {
            if (first || q0 >= a.nq) wait_vmcnt<0>();
            else wait_vmcnt<kStores>();
            first = false;
            // every wave's loads of `cur` have landed, and no wave still reads kn/vn/qn
            lds_barrier();
            if (cur + gridDim.x < a.nbh) load_head(cur + gridDim.x, kn, vn, qn);
            if (q0 >= a.nq) return;
            bh = cur;
            fdivmod(bh, a.heads, b, h);
            // Q fragments of this wave's 16 queries from the swizzled LDS tile
            const uint32_t qad[2] = {lds_addr(qs) + 2 * (uint32_t)tile_at(16 * w + c, g, 0),
                                     lds_addr(qs) + 2 * (uint32_t)tile_at(16 * w + c, 4 + g, 0)};
            lds_read_frags<2, 2>(qad, qf[0]);
            reset_state();
            tile_compute(0, ks, vs);
            store_staged(qs);
        };
        for (uint32_t cur = bh;;) {
            head_step(cur, k0, v0, qt0, k1, v1, qt1);
            if ((cur += gridDim.x) >= a.nbh) break;
            head_step(cur, k1, v1, qt1, k0, v0, qt0);
            if ((cur += gridDim.x) >= a.nbh) break;
        }
    }
}

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_attention_ex(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t n_q,
                      int64_t n_k, int64_t head_dim, int64_t q_batch_stride, int64_t q_head_stride,
                      int64_t q_row_stride, int64_t kv_batch_stride, int64_t kv_head_stride, int64_t kv_row_stride,
                      const void* rot_cos, const void* rot_sin, int trig_dtype, const void* gate, int gate_dtype,
                      int gate_is_logit, void* out, int out_dtype, float scale, int p_precision,
                      mbrt_stream_t stream) {
    const char* op = "mbrt_attention";
    MBRT_REQUIRE(p_precision == MBRT_ATTN_P_PAIR || p_precision == MBRT_ATTN_P_BF16 ||
                     p_precision == MBRT_ATTN_P_BF16_FAST,
                 MBRT_E_INVALID_ARG, "%s: unknown P precision %d", op, p_precision);
    MBRT_REQUIRE(dtype == BF16, MBRT_E_UNSUPPORTED_DTYPE, "%s: q/k/v must be BF16", op);
    MBRT_REQUIRE(out_dtype == BF16 || out_dtype == F32, MBRT_E_UNSUPPORTED_DTYPE, "%s: out must be BF16/F32", op);
    MBRT_REQUIRE(head_dim == kHeadDim, MBRT_E_SHAPE, "%s: head_dim %lld (only 64 is built)", op, (long long)head_dim);
    MBRT_REQUIRE(B >= 0 && H >= 1 && n_q >= 0 && n_k >= 0, MBRT_E_SHAPE, "%s: bad shape", op);
    if (B == 0 || n_q == 0) return MBRT_OK;
    MBRT_REQUIRE(n_k >= 1, MBRT_E_SHAPE, "%s: attention over zero keys", op);
    MBRT_REQUIRE(n_q < (1 << 24) && n_k < (1 << 24) && H < (1 << 24), MBRT_E_SHAPE, "%s: dimension beyond 2^24", op);
    MBRT_REQUIRE(q && k && v && out, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    MBRT_REQUIRE(scale >= 0.0f && std::isfinite(scale), MBRT_E_INVALID_ARG, "%s: scale must be finite and >= 0", op);
    MBRT_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(out, 16), MBRT_E_ALIGN,
                 "%s: q, k, v and out must be 16-byte aligned", op);
    // rows are read in 16-byte pieces: every stride a multiple of 8 elements, rows of 64
    const int64_t st[6] = {q_batch_stride, q_head_stride, q_row_stride, kv_batch_stride, kv_head_stride, kv_row_stride};
    for (int i = 0; i < 6; ++i)
        MBRT_REQUIRE(st[i] >= 0 && st[i] % 8 == 0, MBRT_E_ALIGN, "%s: strides must be non-negative multiples of 8", op);
    MBRT_REQUIRE(q_row_stride >= kHeadDim && kv_row_stride >= kHeadDim, MBRT_E_SHAPE, "%s: row stride below head_dim",
                 op);
    // key offsets within one (b, h) are 32-bit
    MBRT_REQUIRE((n_k - 1) * kv_row_stride + kHeadDim < (int64_t(1) << 31), MBRT_E_SHAPE,
                 "%s: k/v rows of one head span 2^31 elements", op);
    MBRT_REQUIRE((rot_cos == nullptr) == (rot_sin == nullptr), MBRT_E_INVALID_ARG, "%s: give both cos and sin", op);
    if (rot_cos) {
        MBRT_REQUIRE(trig_dtype == F32 || trig_dtype == BF16, MBRT_E_UNSUPPORTED_DTYPE, "%s: cos/sin must be F32/BF16",
                     op);
        MBRT_REQUIRE(aligned(rot_cos, trig_dtype == F32 ? 16 : 8) && aligned(rot_sin, trig_dtype == F32 ? 16 : 8),
                     MBRT_E_ALIGN, "%s: cos/sin tables must be aligned to 4 elements", op);
    }
    if (gate) {
        MBRT_REQUIRE(gate_dtype == F32 || gate_dtype == BF16 || gate_dtype == F16, MBRT_E_UNSUPPORTED_DTYPE,
                     "%s: gate must be F32/BF16/F16", op);
    }
    const int64_t BH = B * H;
    AttnArgs a{};
    a.q = static_cast<const __bf16*>(q);
    a.k = static_cast<const __bf16*>(k);
    a.v = static_cast<const __bf16*>(v);
    a.out = out;
    a.nq = (int)n_q;
    a.nk = (int)n_k;
    a.scale_log2e = (scale == 0.0f ? 1.0f / std::sqrt((float)head_dim) : scale) * 1.44269504088896340736f;
    a.heads = make_fastdiv((uint32_t)H);
    a.q_bs = q_batch_stride;
    a.q_hs = q_head_stride;
    a.kv_bs = kv_batch_stride;
    a.kv_hs = kv_head_stride;
    MBRT_REQUIRE(q_row_stride < (int64_t(1) << 31) && kv_row_stride < (int64_t(1) << 31), MBRT_E_SHAPE,
                 "%s: row stride beyond 2^31", op);
    a.q_rs = (int)q_row_stride;
    a.kv_rs = (int)kv_row_stride;
    a.cosp = rot_cos;
    a.sinp = rot_sin;
    a.tdt = trig_dtype;
    a.gate = gate;
    a.gdt = gate_dtype;
    a.glogit = gate_is_logit ? 1 : 0;
    // two query sub-blocks per wave once a (b, h) has more than one workgroup of queries
    const int qs = n_q > kQBlock * MBRT_ATTN_QS2_MIN ? 2 : 1;
    a.qtiles = (uint32_t)ceil_div(n_q, (int64_t)kQBlock * qs);
    MBRT_REQUIRE(BH * a.qtiles < (int64_t(1) << 31), MBRT_E_SHAPE, "%s: too many tiles", op);
    a.nbh = (uint32_t)BH;
    // heads of at most one query tile and one key tile, without the rotary or gate fusions:
    // persistent workgroups that walk the heads (MBRT_ATTN_HEADS_WPC per CU)
    const bool heads = MBRT_ATTN_HEADS_WPC > 0 && n_q <= kQBlock && n_k <= kKeys && rot_cos == nullptr &&
                       gate == nullptr;
    const dim3 grid(heads ? (unsigned)std::min<int64_t>(BH, (int64_t)cu_count() * std::max(MBRT_ATTN_HEADS_WPC, 1))
                          : (unsigned)(BH * a.qtiles));
    hipStream_t stm = as_stream(stream);
    auto launch = [&](auto pm) {
        constexpr int PM = decltype(pm)::value;
        if (heads) {
            if (out_dtype == BF16) hipLaunchKernelGGL((attention_kernel<BF16, 1, PM, true>), grid, dim3(kWaves * 64), 0, stm, a);
            else hipLaunchKernelGGL((attention_kernel<F32, 1, PM, true>), grid, dim3(kWaves * 64), 0, stm, a);
        } else if (qs == 2) {
            if (out_dtype == BF16) hipLaunchKernelGGL((attention_kernel<BF16, 2, PM, false>), grid, dim3(kWaves * 64), 0, stm, a);
            else hipLaunchKernelGGL((attention_kernel<F32, 2, PM, false>), grid, dim3(kWaves * 64), 0, stm, a);
        } else {
            if (out_dtype == BF16) hipLaunchKernelGGL((attention_kernel<BF16, 1, PM, false>), grid, dim3(kWaves * 64), 0, stm, a);
            else hipLaunchKernelGGL((attention_kernel<F32, 1, PM, false>), grid, dim3(kWaves * 64), 0, stm, a);
        }
    };
    if (p_precision == MBRT_ATTN_P_BF16) launch(std::integral_constant<int, MBRT_ATTN_P_BF16>{});
    else if (p_precision == MBRT_ATTN_P_BF16_FAST) launch(std::integral_constant<int, MBRT_ATTN_P_BF16_FAST>{});
    else launch(std::integral_constant<int, MBRT_ATTN_P_PAIR>{});
    return check_launch(op);
}

int mbrt_attention_strided(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t n_q,
                           int64_t n_k, int64_t head_dim, int64_t q_batch_stride, int64_t q_head_stride,
                           int64_t q_row_stride, int64_t kv_batch_stride, int64_t kv_head_stride,
                           int64_t kv_row_stride, const void* rot_cos, const void* rot_sin, int trig_dtype,
                           const void* gate, int gate_dtype, int gate_is_logit, void* out, int out_dtype,
                           float scale, mbrt_stream_t stream) {
    return mbrt_attention_ex(q, k, v, dtype, B, H, n_q, n_k, head_dim, q_batch_stride, q_head_stride, q_row_stride,
                             kv_batch_stride, kv_head_stride, kv_row_stride, rot_cos, rot_sin, trig_dtype, gate,
                             gate_dtype, gate_is_logit, out, out_dtype, scale, MBRT_ATTN_P_PAIR, stream);
}

int mbrt_attention(const void* q, const void* k, const void* v, int dtype, void* out, int out_dtype, int64_t BH,
                   int64_t n_q, int64_t n_k, int64_t head_dim, float scale, mbrt_stream_t stream) {
    return mbrt_attention_strided(q, k, v, dtype, BH, 1, n_q, n_k, head_dim, n_q * head_dim, 0, head_dim,
                                  n_k * head_dim, 0, head_dim, nullptr, nullptr, F32, nullptr, F32, 0, out, out_dtype,
                                  scale, stream);
}

}  // extern "C"
