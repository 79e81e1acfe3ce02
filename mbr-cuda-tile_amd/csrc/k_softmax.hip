// Row softmax with f32 accumulation (the scale_softmax* family, src/mbr_cuda_tile.cu:5092-5285):
//   z = scale * x;  p = exp(z - max z) / sum exp(z - max z)   per row of `cols` elements.
//
// A group of G lanes owns one row and keeps it in registers: lane l holds elements
// l, l+G, l+2G, ...  Every load and store instruction of the group then touches G
// consecutive elements (256 B per wave instruction for f32 rows at G = 64), rows need
// no alignment (801-element rows start at arbitrary offsets), and only the last slot
// of a row is predicated.  The row is read once and written once.  exp is evaluated as
// exp2 of the pre-scaled input (z * log2 e), one v_exp_f32 per element.
//   801 cols : G = 64, 13 elements per lane, 4 rows per 256-thread block
//   60 cols  : G = 16, 4 elements per lane, 16 rows per block
// Rows of at most 1024 elements are staged when the spans align: a block owns 256 / G
// consecutive rows, one contiguous span of the tensor, which it reads and writes with
// 16-byte vector accesses through LDS, so a 60-element bf16 row (120 bytes) or an
// 801-element one (1602 bytes) costs no 2-byte accesses.
// Rows longer than 64 x 32 elements use a three-pass loop kernel.
#include "abi_common.hpp"

#include <type_traits>

#include <algorithm>
#include <cfloat>

namespace mbrt {
namespace {

constexpr int kThreads = 256;
constexpr float kLog2e = 1.44269504088896340736f;

struct SmArgs {
    const void* in;
    void* out;
    int odt;
    int64_t rows;
    int cols;
    float scale_log2e;
    float scale;  // bf16-intermediates mode: the scale is applied (and rounded) on its own
};

// Bf16-intermediates mode (scale_softmax_bf16_to_bf16_kernel in full-bf16 mode,
// src/mbr_cuda_tile.cu:5224-5252): z = bf16(x * scale), the row max, e = bf16(exp(z - max)),
// the sum bf16(sum e) and p = bf16(e / sum) are each rounded to bf16.  The FB kernels are
// instantiated for bf16 -> bf16 rows only.
__device__ __forceinline__ float fb_exp(float z, float m) { return bf16r(__builtin_amdgcn_exp2f((z - m) * kLog2e)); }

// Loads are unconditional (the row index and the element index are clamped into the
// tensor), so all NM loads of a lane are issued before the first use; only stores are
// predicated, and only the last slot of a row ever needs a per-lane predicate.
template <int IDT, int G, int NM, bool FB>
__global__ __launch_bounds__(kThreads) void softmax_rows_kernel(SmArgs a) {
    const int lane = threadIdx.x % G;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / G) + threadIdx.x / G;
    const bool valid = row < a.rows;
    const int64_t base = (valid ? row : a.rows - 1) * a.cols;
    const int last = a.cols - 1;
    float z[NM];
#pragma unroll
    for (int k = 0; k < NM; ++k) z[k] = ld1<IDT, MBRT_NT_SMR>(a.in, base + min(lane + G * k, last));
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < NM; ++k) {
        z[k] = lane + G * k <= last ? (FB ? bf16r(z[k] * a.scale) : z[k] * a.scale_log2e) : -INFINITY;
        m = fmaxf(m, z[k]);
    }
    m = group_max<G>(m);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NM; ++k) {
        z[k] = FB ? fb_exp(z[k], m) : __builtin_amdgcn_exp2f(z[k] - m);  // masked slots: exp2(-inf) = 0
        s += z[k];
    }
    s = group_sum<G>(s);
    const float inv = 1.0f / s;
    const float den = bf16r(s);
    const int full = a.cols / G;  // slots [0, full) hold a valid element in every lane
    auto store_all = [&](auto odt_tag) {
        constexpr int ODT = decltype(odt_tag)::value;
        if (!valid) return;
#pragma unroll
        for (int k = 0; k < NM; ++k) {
            if (k < full || lane + G * k <= last)
                st1<ODT, MBRT_NT_SMR>(a.out, base + lane + G * k, FB ? bf16r(z[k] / den) : z[k] * inv);
        }
    };
    with_dt(a.odt, store_all);
}

// Staged short rows.  Block b owns rows [b*RB, b*RB + RB), RB = RPG * 256 / G (each group
// of G lanes takes RPG rows in turn), i.e. the span of RB*cols elements starting at element
// b*RB*cols.  The launcher only picks this kernel when
// that span is a whole number of 16-byte vectors for the input and the output dtype, both
// pointers are 16-byte aligned and rows*cols fills whole vectors, so every vector lies in
// one block's span.  Phase 1 loads the span into LDS (straight from HBM, or through
// registers where it changes dtype), phase 2 is the same register-resident group softmax
// as above but fed from LDS, writing the probabilities back over their inputs, phase 3
// stores the span.  In-place calls are safe: the whole span is in LDS before its first
// store.
template <int IDT, int ODT, int G, int NM, int RPG, bool FB>
__global__ __launch_bounds__(kThreads) void softmax_staged_kernel(SmArgs a) {
    constexpr int RB = RPG * kThreads / G;
    // rows of more than 128 elements (groups of 32 or 64 lanes) have their own cache policy
    constexpr int NT = G >= 32 ? MBRT_NT_SML : MBRT_NT_SMS;
    constexpr int VI = 16 / DtSize<IDT>::value, VO = 16 / DtSize<ODT>::value;
    constexpr int CAP = RB * G * NM;  // elements of LDS (RB rows of at most G*NM elements)
    constexpr int KI = (CAP / VI + kThreads - 1) / kThreads, KO = (CAP / VO + kThreads - 1) / kThreads;
    // bf16 -> bf16 and f16 -> f16 spans stay in their 2-byte format in LDS: 16-byte vectors
    // move in and out unchanged (no 32-byte-per-lane f32 staging, which conflicts on the
    // LDS banks), and the probabilities are rounded where they are written back, exactly
    // where the f32 staging would round them on the way out
    constexpr bool K16 = IDT == ODT && IDT != F32 && MBRT_SM_STAGE16;
    using Elem = typename std::conditional<K16, uint16_t, float>::type;
    __shared__ __attribute__((aligned(16))) Elem buf[CAP];
    const int tid = threadIdx.x;
    // f32 spans of 64-lane rows (4 rows of 801: 12,816 B, 16 mod 128) share a cache line
    // with the next span.  Each XCD walks one contiguous range of spans, so that both
    // halves go through one L2.  Measured 0.5 % faster, though the counted HBM traffic did
    // not drop; the other shapes ran 2-4 % slower in this order and keep the launch order.
    constexpr bool kXcdRuns = IDT == F32 && ODT == F32 && G == 64;
    const uint32_t span = kXcdRuns ? xcd_tile(blockIdx.x, gridDim.x) : blockIdx.x;
    const int64_t row0 = (int64_t)span * RB;
    const int nrows = (int)min((int64_t)RB, a.rows - row0);
    const int nel = nrows * a.cols;
    const int64_t ebase = row0 * a.cols;
    const int nvi = nel / VI;
    // When LDS holds the span's raw bytes (f32 -> f32, and 2-byte spans kept 2-byte), the
    // span goes straight from HBM into LDS: lane i of wave w's k-th load writes vector
    // 256 k + 64 w + i at its place in buf (global_load_lds_dwordx4, non-temporal when the
    // kernel's loads are).  Time f32 428.0-428.4 -> 425.1-425.3 us against the same loads
    // through registers.
    constexpr bool kDma = MBRT_SM_DMA != 0 && (K16 || (IDT == F32 && ODT == F32));
    if constexpr (kDma) {
        const char* src = reinterpret_cast<const char*>(a.in) + ebase * DtSize<IDT>::value;
        const int w = tid / 64;
#pragma unroll
        for (int k = 0; k < KI; ++k) {
            const int v = tid + kThreads * k;
            if (v < nvi)
                __builtin_amdgcn_global_load_lds((global_void*)(src + (int64_t)v * 16),
                                                 (lds_void*)&buf[(kThreads * k + 64 * w) * VI], 16, 0,
                                                 (NT & 1) != 0 ? kCpolNt : 0);
        }
    } else {
        // through registers: the loads are all issued first (vector indices clamped into
        // the span), then converted and written to LDS
        Vec<IDT, VI> iv[KI];
#pragma unroll
        for (int k = 0; k < KI; ++k)
            iv[k].template load<NT>(a.in, ebase + (int64_t)min(tid + kThreads * k, nvi - 1) * VI);
#pragma unroll
        for (int k = 0; k < KI; ++k) {
            const int v = tid + kThreads * k;
            if (v < nvi) {
                if constexpr (K16) {
                    *reinterpret_cast<u32x4*>(&buf[v * VI]) = u32x4{iv[k].w[0], iv[k].w[1], iv[k].w[2], iv[k].w[3]};
                } else {
                    float f[VI];
                    iv[k].to_f32(f);
#pragma unroll
                    for (int i = 0; i < VI; ++i) buf[v * VI + i] = f[i];
                }
            }
        }
    }
    // Direct-to-LDS data is only in LDS once this wave's loads have completed (vmcnt), and
    // the workgroup-scope fence of __syncthreads() is not required to wait for them: wait
    // explicitly, then the barrier makes every wave's part of the span visible.
    if constexpr (kDma) wait_vmcnt<0>();
    __syncthreads();
    auto get = [&](int e) -> float {
        if constexpr (!K16) return buf[e];
        else if constexpr (IDT == BF16) return __uint_as_float((uint32_t)buf[e] << 16);
        else return (float)__builtin_bit_cast(_Float16, buf[e]);
    };
    auto put = [&](int e, float v) {
        if constexpr (!K16) buf[e] = v;
        else if constexpr (IDT == BF16) buf[e] = f32_to_bf16_bits(v);
        else buf[e] = f32_to_f16_bits(v);
    };
    const int lane = tid % G;
    const int last = a.cols - 1;
    // Rows of 33..64 elements (8 groups of 8 lanes per wave, 64 slots per row): each wave
    // instruction reads 8 rows, `cols` elements apart.  Group g walks its row's slots from
    // rot = g (8 - cols) mod 64 on, slot (lane + 8 k + rot) mod 64, so that the 8 blocks of
    // an instruction start at element 8 g + 8 k (mod 64) of the span's 32-bank window:
    // every group reads its own 4 (2-byte) or 8 (f32) banks, with no bank conflict.  Slots
    // at or past `cols` are masked; their reads stay inside the span's LDS buffer.
    constexpr bool kRot = G == 8 && NM == 8;
    const int rot = kRot ? (((tid / G) % (64 / G)) * (8 - a.cols)) & 63 : 0;
    auto slot = [&](int k) { return kRot ? (lane + G * k + rot) & 63 : lane + G * k; };
#pragma unroll
    for (int rr = 0; rr < RPG; ++rr) {
        const int r = tid / G + rr * (kThreads / G);
        const int rbase = min(r, nrows - 1) * a.cols;
        float z[NM];
        float m = -INFINITY;
#pragma unroll
        for (int k = 0; k < NM; ++k) {
            const int e = slot(k);
            const float x = get(rbase + (kRot ? e : min(e, last)));
            z[k] = e <= last ? (FB ? bf16r(x * a.scale) : x * a.scale_log2e) : -INFINITY;
            m = fmaxf(m, z[k]);
        }
        m = group_max<G>(m);
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < NM; ++k) {
            z[k] = FB ? fb_exp(z[k], m) : __builtin_amdgcn_exp2f(z[k] - m);
            s += z[k];
        }
        s = group_sum<G>(s);
        const float inv = 1.0f / s;
        const float den = bf16r(s);
        if (r < nrows) {
#pragma unroll
            for (int k = 0; k < NM; ++k)
                if (slot(k) <= last) put(rbase + slot(k), FB ? bf16r(z[k] / den) : z[k] * inv);
        }
    }
    __syncthreads();
    const int nvo = nel / VO;
#pragma unroll
    for (int k = 0; k < KO; ++k) {
        const int v = tid + kThreads * k;
        if (v < nvo) {
            Vec<ODT, VO> o;
            if constexpr (K16) {
                const u32x4 t = *reinterpret_cast<const u32x4*>(&buf[v * VO]);
                o.w[0] = t.x; o.w[1] = t.y; o.w[2] = t.z; o.w[3] = t.w;
            } else {
                float f[VO];
#pragma unroll
                for (int i = 0; i < VO; ++i) f[i] = buf[v * VO + i];
                o.from_f32(f);
            }
            o.template store<NT>(a.out, ebase + (int64_t)v * VO);
        }
    }
}

// Rows of 33..64 two-byte elements, `cols` a multiple of 4, the same dtype in and out:
// a pair of rows is cols/4 16-byte vectors (at most 16) and starts 16-byte aligned, so one
// 16-lane group moves it straight between HBM and registers, lane i holding vector i
// (elements 8i..8i+7 of the pair).  Each 4-element half of a lane's vector then lies in
// one row; a lane reduces its halves, and the group reduces a max and a sum per row with
// the 16-lane DPP steps, each half contributing to its own row.  No LDS, no barrier.
// Lanes past the pair's last vector load that vector again (every load is issued before
// the first use) and store nothing; groups past the last pair re-read it and store
// nothing.  In-place calls are safe: a vector is written only by the lane that read it,
// after every load of its wave.
template <int DT, int U>
__global__ __launch_bounds__(kThreads) void softmax_pair_kernel(SmArgs a) {
    constexpr int kGroups = kThreads / 16;
    const int i = threadIdx.x & 15;
    const int nv = a.cols >> 2;  // vectors per pair
    const int64_t pairs = a.rows >> 1;
    const int vi = min(i, nv - 1);
    const bool lane_ok = i < nv;
    const bool rowA = 8 * i < a.cols, rowB = 8 * i + 4 < a.cols;  // half in the pair's first row
    // chunks of kGroups * U pairs; a grid smaller than the chunk count walks them
    const int64_t chunks = (pairs + kGroups * U - 1) / (kGroups * U);
    for (int64_t chunk = blockIdx.x; chunk < chunks; chunk += gridDim.x) {
    const int64_t p0 = chunk * (kGroups * U) + (threadIdx.x >> 4);
    Vec<DT, 8> x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t p = min(p0 + u * kGroups, pairs - 1);
        x[u].template load<MBRT_NT_SMP>(a.in, (p * nv + vi) * 8);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        float z[8];
        x[u].to_f32(z);
        float hA = -INFINITY, hB = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            z[j] *= a.scale_log2e;
            z[j + 4] *= a.scale_log2e;
            hA = fmaxf(hA, z[j]);
            hB = fmaxf(hB, z[j + 4]);
        }
        float m0 = fmaxf(rowA ? hA : -INFINITY, rowB ? hB : -INFINITY);
        float m1 = lane_ok ? fmaxf(rowA ? -INFINITY : hA, rowB ? -INFINITY : hB) : -INFINITY;
        m0 = group_max<16>(m0);
        m1 = group_max<16>(m1);
        const float mA = rowA ? m0 : m1, mB = rowB ? m0 : m1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            z[j] = __builtin_amdgcn_exp2f(z[j] - mA);
            z[j + 4] = __builtin_amdgcn_exp2f(z[j + 4] - mB);
        }
        const float sA = (z[0] + z[1]) + (z[2] + z[3]), sB = (z[4] + z[5]) + (z[6] + z[7]);
        float s0 = (rowA ? sA : 0.0f) + (rowB ? sB : 0.0f);
        float s1 = lane_ok ? (rowA ? 0.0f : sA) + (rowB ? 0.0f : sB) : 0.0f;
        s0 = group_sum<16>(s0);
        s1 = group_sum<16>(s1);
        const float inv0 = MBRT_SM_PAIR_RCP ? __builtin_amdgcn_rcpf(s0) : 1.0f / s0;
        const float inv1 = MBRT_SM_PAIR_RCP ? __builtin_amdgcn_rcpf(s1) : 1.0f / s1;
        const float iA = rowA ? inv0 : inv1, iB = rowB ? inv0 : inv1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            z[j] *= iA;
            z[j + 4] *= iB;
        }
        x[u].from_f32(z);
        const int64_t p = p0 + u * kGroups;
        if (p < pairs && lane_ok) x[u].template store<MBRT_NT_SMP>(a.out, (p * nv + i) * 8);
    }
    }
}

// Long rows: one wave per row, three passes (max, sum, write) over global memory.
__global__ __launch_bounds__(kThreads) void softmax_loop_kernel(SmArgs a, int idt, int fb) {
    const int lane = threadIdx.x % 64;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + threadIdx.x / 64;
    if (row >= a.rows) return;
    const int64_t start = row * a.cols;
    if (fb) {
        float m = -INFINITY;
        for (int64_t c = lane; c < a.cols; c += 64) m = fmaxf(m, bf16r(load1(a.in, idt, start + c) * a.scale));
        m = group_max<64>(m);
        float s = 0.0f;
        for (int64_t c = lane; c < a.cols; c += 64) s += fb_exp(bf16r(load1(a.in, idt, start + c) * a.scale), m);
        const float den = bf16r(group_sum<64>(s));
        for (int64_t c = lane; c < a.cols; c += 64)
            store1(a.out, a.odt, start + c, bf16r(fb_exp(bf16r(load1(a.in, idt, start + c) * a.scale), m) / den));
        return;
    }
    float m = -INFINITY;
    for (int64_t c = lane; c < a.cols; c += 64) m = fmaxf(m, load1(a.in, idt, start + c) * a.scale_log2e);
    m = group_max<64>(m);
    float s = 0.0f;
    for (int64_t c = lane; c < a.cols; c += 64)
        s += __builtin_amdgcn_exp2f(load1(a.in, idt, start + c) * a.scale_log2e - m);
    s = group_sum<64>(s);
    const float inv = 1.0f / s;
    for (int64_t c = lane; c < a.cols; c += 64)
        store1(a.out, a.odt, start + c,
               __builtin_amdgcn_exp2f(load1(a.in, idt, start + c) * a.scale_log2e - m) * inv);
}

template <int IDT, int G, int NM, int RPG = 1>
void launch_staged(const SmArgs& a, bool fb, hipStream_t st) {
    const dim3 grid((unsigned)ceil_div(a.rows, RPG * kThreads / G));
    if constexpr (IDT == BF16) {
        if (fb) {
            hipLaunchKernelGGL((softmax_staged_kernel<BF16, BF16, G, NM, RPG, true>), grid, dim3(kThreads), 0, st, a);
            return;
        }
    }
    with_dt(a.odt, [&](auto ot) {
        hipLaunchKernelGGL((softmax_staged_kernel<IDT, decltype(ot)::value, G, NM, RPG, false>), grid, dim3(kThreads),
                           0, st, a);
    });
}

// Staged path: rows of at most 1024 elements, when every block span is made of whole
// 16-byte vectors of both dtypes (see softmax_staged_kernel).  Short rows use narrow
// groups (many rows per block); rows of 129..1024 use 64 lanes per row (4 rows per block)
// or, when 4 rows do not fill whole vectors (bf16 rows of odd length), 32 lanes (8 rows).
template <int IDT>
bool launch_short(const SmArgs& a, int in_esize, int out_esize, bool fb, hipStream_t st) {
    const int c = a.cols;
    if (c > 1024 || !aligned(a.in, 16) || !aligned(a.out, 16)) return false;
    auto fits = [&](int rb) {
        for (int es : {in_esize, out_esize})
            if (((int64_t)rb * c * es) % 16 != 0 || (a.rows * c * es) % 16 != 0) return false;
        return true;
    };
    // rows of 33..64: a block of 32 rows moves 32*c*in_esize bytes in; below
    // MBRT_SM_SHORT_BYTES of input its fixed cost dominates, so each group takes
    // MBRT_SM_SHORT_RPG rows
    const bool two = 32 * c * in_esize < MBRT_SM_SHORT_BYTES;
    if constexpr (IDT != F32) {
        if (MBRT_SM_PAIR_U > 0 && !fb && out_esize == 2 && a.odt == IDT && c > 32 && c <= 64 && c % 4 == 0 &&
            a.rows % 2 == 0) {
            constexpr int U = MBRT_SM_PAIR_U > 0 ? MBRT_SM_PAIR_U : 1;
            dim3 grid((unsigned)ceil_div(a.rows / 2, (int64_t)(kThreads / 16) * U));
            if (MBRT_SM_PAIR_BPC > 0) grid.x = (unsigned)std::min<int64_t>(grid.x, (int64_t)cu_count() * MBRT_SM_PAIR_BPC);
            hipLaunchKernelGGL((softmax_pair_kernel<IDT, U>), grid, dim3(kThreads), 0, st, a);
            return true;
        }
    }
    if (c <= 16 && fits(64)) launch_staged<IDT, 4, 4>(a, fb, st);
    else if (c <= 32 && fits(32)) launch_staged<IDT, 8, 4>(a, fb, st);
    else if (c <= 64 && two && fits(32 * MBRT_SM_SHORT_RPG)) launch_staged<IDT, 8, 8, MBRT_SM_SHORT_RPG>(a, fb, st);
    else if (c <= 64 && fits(32)) launch_staged<IDT, 8, 8>(a, fb, st);
    else if (c <= 128 && fits(16)) launch_staged<IDT, 16, 8>(a, fb, st);
    else if (c <= 128 || !MBRT_SM_STAGE_LONG) return false;
    else if (MBRT_SM_LONG_G == 64 && fits(4 * MBRT_SM_LONG_RPG)) {
        constexpr int R = MBRT_SM_LONG_RPG;
        if (c <= 256) launch_staged<IDT, 64, 4, R>(a, fb, st);
        else if (c <= 512) launch_staged<IDT, 64, 8, R>(a, fb, st);
        else if (c <= 832) launch_staged<IDT, 64, 13, R>(a, fb, st);
        else launch_staged<IDT, 64, 16, R>(a, fb, st);
    } else if (fits(8 * MBRT_SM_LONG_RPG)) {
        constexpr int R = MBRT_SM_LONG_RPG;
        if (c <= 256) launch_staged<IDT, 32, 8, R>(a, fb, st);
        else if (c <= 512) launch_staged<IDT, 32, 16, R>(a, fb, st);
        else if (c <= 832) launch_staged<IDT, 32, 26, R>(a, fb, st);
        else launch_staged<IDT, 32, 32, R>(a, fb, st);
    } else {
        return false;
    }
    return true;
}

template <int IDT, int G, int NM>
void launch_rows(const SmArgs& a, bool fb, hipStream_t st) {
    const dim3 grid((unsigned)ceil_div(a.rows, kThreads / G));
    if constexpr (IDT == BF16) {
        if (fb) {
            hipLaunchKernelGGL((softmax_rows_kernel<IDT, G, NM, true>), grid, dim3(kThreads), 0, st, a);
            return;
        }
    }
    hipLaunchKernelGGL((softmax_rows_kernel<IDT, G, NM, false>), grid, dim3(kThreads), 0, st, a);
}

// Picks the group width and slots per lane for a row length; false when too long.
template <int IDT>
bool launch_fast(const SmArgs& a, bool fb, hipStream_t st) {
    const int c = a.cols;
    if (c <= 8) launch_rows<IDT, 8, 1>(a, fb, st);
    else if (c <= 16) launch_rows<IDT, 16, 1>(a, fb, st);
    else if (c <= 32) launch_rows<IDT, 16, 2>(a, fb, st);
    else if (c <= 64) launch_rows<IDT, 16, 4>(a, fb, st);
    else if (c <= 128) launch_rows<IDT, 32, 4>(a, fb, st);
    else if (c <= 256) launch_rows<IDT, 64, 4>(a, fb, st);
    else if (c <= 512) launch_rows<IDT, 64, 8>(a, fb, st);
    else if (c <= 832) launch_rows<IDT, 64, 13>(a, fb, st);
    else if (c <= 1024) launch_rows<IDT, 64, 16>(a, fb, st);
    else if (c <= 1344) launch_rows<IDT, 64, 21>(a, fb, st);
    else if (c <= 2048) launch_rows<IDT, 64, 32>(a, fb, st);
    else return false;
    return true;
}

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_softmax_rows(const void* in, int in_dtype, void* out, int out_dtype, int64_t rows, int64_t cols,
                      float scale, mbrt_stream_t stream) {
    const char* op = "mbrt_softmax_rows";
    MBRT_REQUIRE_FLOAT_DT(in_dtype, op);
    MBRT_REQUIRE_FLOAT_DT(out_dtype, op);
    MBRT_REQUIRE(rows >= 0 && cols >= 1 && cols < (1 << 30), MBRT_E_SHAPE, "%s: bad shape", op);
    if (rows == 0) return MBRT_OK;
    MBRT_REQUIRE(in && out, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    MBRT_REQUIRE(in != out || in_dtype == out_dtype, MBRT_E_INVALID_ARG, "%s: in-place needs equal dtypes", op);
    SmArgs a{};
    a.in = in;
    a.out = out;
    a.odt = out_dtype;
    a.rows = rows;
    a.cols = (int)cols;
    a.scale_log2e = scale * kLog2e;
    a.scale = scale;
    // bf16 intermediates: bf16 -> bf16 rows, as in the reference
    const bool fb = bf16_intermediates() && in_dtype == BF16 && out_dtype == BF16;
    hipStream_t st = as_stream(stream);
    const int ies = dt_size(in_dtype), oes = dt_size(out_dtype);
    bool done;
    if (in_dtype == F32) done = launch_short<F32>(a, ies, oes, false, st) || launch_fast<F32>(a, false, st);
    else if (in_dtype == BF16) done = launch_short<BF16>(a, ies, oes, fb, st) || launch_fast<BF16>(a, fb, st);
    else done = launch_short<F16>(a, ies, oes, false, st) || launch_fast<F16>(a, false, st);
    if (!done) {
        hipLaunchKernelGGL(softmax_loop_kernel, dim3((unsigned)ceil_div(rows, kThreads / 64)), dim3(kThreads), 0, st, a,
                           in_dtype, fb ? 1 : 0);
    }
    return check_launch(op);
}

}  // extern "C"
