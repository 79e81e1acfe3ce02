// STFT and iSTFT for n_fft = win_length = 2048 (src/stft_cuda_tile.cu:530-717): the
// spectrogram producer in front of the band gather and the waveform consumer after the
// mask merge, in the layouts those ops use ([B, 1025, T, 2] f32 spectra).
//
// The 2048-point real transform is a 1024-point complex FFT of z[m] = x[2m] + i x[2m+1]
// with the standard real-input split X[f] = (Z[f] + Z*[1024-f])/2 - i W^f (Z[f] -
// Z*[1024-f])/2 (W = exp(-2 pi i / 2048)), and the inverse split for the iSTFT.
// One wave transforms one frame; lane l holds z[l + 64a], a = 0..15, in registers.  The
// 1024-point FFT runs as three Stockham passes, radix 16 (in registers), 16 and 4, with
// two exchanges through the frame's LDS slot (index p stored at p + p/16, which keeps
// both the strided and the contiguous access patterns free of bank conflicts).  The STFT
// takes the last pass's butterflies in mirror pairs so the real split needs no exchange.
//
// Workgroup = kTF waves = kTF consecutive frames of one signal.  The frames' spectra stay
// in LDS so that the [B, F, T] layout is written (STFT) or read (iSTFT) as runs of kTF
// consecutive frames per bin, instead of one 8-byte element per 8*T bytes.
//
// STFT   one kernel: the workgroup's sample span ((kTF - 1) hop + 2048 samples, reflect
//        padded at the signal ends) and the window are staged once into the frame slots
//        with coalesced loads (for hops up to 1910; larger hops read frame by frame), each
//        wave takes its windowed frame from there, then FFT, real split, optional
//        1/sqrt(2048), transposed store.
// iSTFT  two kernels: (1) per block of kTF frames of one signal: transposed spectrum load
//        (f32 or bf16, times sqrt(2048) when normalized), inverse split, inverse FFT,
//        window and 1/2048 into the frame's LDS slot, then the block's frames overlap-added
//        in LDS (frame order) into a partial signal in a caller workspace; (2) per output
//        sample: the partials of the blocks covering it (block order), divided by the
//        window sum of squares where that exceeds 1e-8; centre trim and the `length` trim /
//        zero fill are part of the same pass.  No atomics: the result is deterministic.
#include "abi_common.hpp"

#include <atomic>

#include <cmath>

namespace mbrt {
namespace {

constexpr int kN = 2048;        // n_fft = win_length
constexpr int kBins = kN / 2 + 1;
#ifndef MBRT_STFT_TF
#define MBRT_STFT_TF 8
#endif
// Frames per workgroup; one wave per frame.  A workgroup holds kTF frame slots and the
// twiddle table in LDS (78 KB at kTF = 8: two workgroups, 16 waves, per CU).
constexpr int kTF = MBRT_STFT_TF;
#ifndef MBRT_STFT_XCD
#define MBRT_STFT_XCD 32
#endif
#ifndef MBRT_ISTFT_XCD
#define MBRT_ISTFT_XCD 8
#endif
// Frame blocks are dealt to the XCDs in runs of this many consecutive blocks, so the blocks
// that share the cache lines of a bin row ([B, 1025, T] holds kTF frames of a bin in
// 8 kTF bytes) meet in one L2, and so do the STFT's overlapping sample spans.  Measured on
// the chunk (8 signals, 801 blocks): STFT 31.2-31.5 us with runs of 8, 30.6-30.8 with 16,
// 29.7-30.1 with 32 (kept), 34.2 with 64; the iSTFT block kernel moved by under 1 % and
// keeps 8.
constexpr uint32_t kXcdRun = MBRT_STFT_XCD;
constexpr uint32_t kXcdRunInv = MBRT_ISTFT_XCD;
// LDS slot of one frame, in complex elements: holds padded indices up to pad(1024) = 1088;
// 1092 complex = 2184 words = 8 (mod 64) words, so the transposed pass (kTF lanes of one
// bin reading kTF slots) spreads over all banks.
constexpr int kSlot = 1092;
constexpr int kTwHalf = 1024;  // LDS twiddles W^i, i < 1024 (W^(i + 1024) = -W^i)
// W^i sits at i + i/32 in LDS: the strided index sets of the passes (8qk over k, 2q(l + 64s)
// over l) then fall on distinct banks.
constexpr int kTwSlots = kTwHalf + kTwHalf / 32;
__device__ __forceinline__ int tw_pos(int i) { return i + (i >> 5); }
static_assert(kTF == 4 || kTF == 8 || kTF == 16, "frames per workgroup");

__device__ __forceinline__ int pad16(int p) { return p + (p >> 4); }

// ---- twiddles W^i = exp(-2 pi i i / 2048), built at compile time -----------------------
// cos/sin on [0, pi/4] by their Taylor series in double, extended to the circle by the
// octant symmetries, then rounded once to f32.
struct TwiddleTable {
    float v[2 * kN];  // (re, im) pairs
};

constexpr void taylor_cos_sin(double x, double& c, double& s) {
    double tc = 1.0, ts = x;
    const double x2 = x * x;
    c = 0.0;
    s = 0.0;
    for (int k = 0; k < 16; ++k) {
        c += tc;
        s += ts;
        tc *= -x2 / (double)((2 * k + 1) * (2 * k + 2));
        ts *= -x2 / (double)((2 * k + 2) * (2 * k + 3));
    }
}

constexpr TwiddleTable make_twiddles() {
    TwiddleTable t{};
    constexpr double kPi = 3.14159265358979323846;
    for (int i = 0; i < kN; ++i) {
        const int quarter = i / 512, j = i % 512;
        double c = 0.0, s = 0.0;
        if (j <= 256) {
            taylor_cos_sin(kPi * j / 1024.0, c, s);
        } else {
            double c2 = 0.0, s2 = 0.0;
            taylor_cos_sin(kPi * (512 - j) / 1024.0, c2, s2);
            c = s2;
            s = c2;
        }
        double cc = c, ss = s;  // cos, sin of quarter * pi/2 + theta
        if (quarter == 1) { cc = -s; ss = c; }
        if (quarter == 2) { cc = -c; ss = -s; }
        if (quarter == 3) { cc = s; ss = -c; }
        t.v[2 * i] = (float)cc;
        t.v[2 * i + 1] = (float)(-ss);
    }
    return t;
}

__constant__ const TwiddleTable kTwiddles = make_twiddles();

struct cf {
    float x, y;
};
__device__ __forceinline__ cf cadd(cf a, cf b) { return {a.x + b.x, a.y + b.y}; }
__device__ __forceinline__ cf csub(cf a, cf b) { return {a.x - b.x, a.y - b.y}; }
__device__ __forceinline__ cf cmul(cf a, cf b) { return {a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x}; }
// times -i (forward) or +i (inverse)
template <bool INV>
__device__ __forceinline__ cf rot(cf a) {
    return INV ? cf{-a.y, a.x} : cf{a.y, -a.x};
}
// W^i (forward) or its conjugate (inverse), 0 <= i < 2048, from the LDS half table:
// W^(i + 1024) = -W^i flips both signs.
template <bool INV>
__device__ __forceinline__ cf twiddle(const float2* tw, int i) {
    const float2 t = tw[tw_pos(i & (kTwHalf - 1))];
    const uint32_t s = (uint32_t)(i >> 10) << 31;
    return {__uint_as_float(__float_as_uint(t.x) ^ s),
            __uint_as_float(__float_as_uint(t.y) ^ s ^ (INV ? 0x80000000u : 0u))};
}

// Copies W^i, i < 1024, into the workgroup's LDS table (all threads take part).
template <int NT>
__device__ __forceinline__ void load_twiddles(float2* tw) {
    static_assert(kTwHalf % NT == 0, "threads per workgroup divide the table");
    constexpr int kPer = kTwHalf / NT;
    const float2* src = reinterpret_cast<const float2*>(kTwiddles.v);
    float2 t[kPer];  // every load in flight before the first LDS write
#pragma unroll
    for (int k = 0; k < kPer; ++k) t[k] = src[threadIdx.x + k * NT];
#pragma unroll
    for (int k = 0; k < kPer; ++k) tw[tw_pos(threadIdx.x + k * NT)] = t[k];
}

template <bool INV>
__device__ __forceinline__ void dft4(cf& a0, cf& a1, cf& a2, cf& a3) {
    const cf t0 = cadd(a0, a2), t1 = csub(a0, a2), t2 = cadd(a1, a3), t3 = rot<INV>(csub(a1, a3));
    a0 = cadd(t0, t2);
    a2 = csub(t0, t2);
    a1 = cadd(t1, t3);
    a3 = csub(t1, t3);
}

// a * W16^E (conjugated for the inverse)
template <bool INV, int E>
__device__ __forceinline__ cf mul_w16(cf a) {
    constexpr float C1 = 0.92387953251128675613f, S1 = 0.38268343236508977173f, H = 0.70710678118654752440f;
    if constexpr (E == 4) return rot<INV>(a);
    constexpr float re = E == 1 ? C1 : E == 2 ? H : E == 3 ? S1 : E == 6 ? -H : -C1;  // E = 9
    constexpr float im = E == 1 ? -S1 : E == 2 ? -H : E == 3 ? -C1 : E == 6 ? -H : S1;
    return cmul(a, cf{re, INV ? -im : im});
}

// 16-point DFT in place: v[r] <- sum_q v[q] W16^(q r)  (radix 4 x 4)
template <bool INV>
__device__ __forceinline__ void dft16(cf (&v)[16]) {
#pragma unroll
    for (int q0 = 0; q0 < 4; ++q0) dft4<INV>(v[q0], v[q0 + 4], v[q0 + 8], v[q0 + 12]);
    // v[q0 + 4 r0] now holds A[q0][r0]; twiddle by W16^(q0 r0)
    v[5] = mul_w16<INV, 1>(v[5]);
    v[9] = mul_w16<INV, 2>(v[9]);
    v[13] = mul_w16<INV, 3>(v[13]);
    v[6] = mul_w16<INV, 2>(v[6]);
    v[10] = mul_w16<INV, 4>(v[10]);
    v[14] = mul_w16<INV, 6>(v[14]);
    v[7] = mul_w16<INV, 3>(v[7]);
    v[11] = mul_w16<INV, 6>(v[11]);
    v[15] = mul_w16<INV, 9>(v[15]);
    // DFT over q0 for each r0: inputs v[4 r0 + q0], outputs V[r0 + 4 r1]
    cf o[16];
#pragma unroll
    for (int r0 = 0; r0 < 4; ++r0) {
        cf a0 = v[4 * r0], a1 = v[4 * r0 + 1], a2 = v[4 * r0 + 2], a3 = v[4 * r0 + 3];
        dft4<INV>(a0, a1, a2, a3);
        o[r0] = a0;
        o[r0 + 4] = a1;
        o[r0 + 8] = a2;
        o[r0 + 12] = a3;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = o[r];
}

// Orders this wave's LDS accesses: lanes of one wave exchange data through the slot.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ cf lds_ld(const float2* s, int i) {
    const float2 t = s[i];
    return {t.x, t.y};
}
__device__ __forceinline__ void lds_st(float2* s, int i, cf v) { s[i] = make_float2(v.x, v.y); }

// Passes 1 and 2 of the 1024-point FFT of one frame by one wave.  In: lane l holds z[l + 64a]
// in v[a].  Out: the slot holds y2 (pass-2 output) at padded indices.  Previous slot
// contents are overwritten.
template <bool INV>
__device__ __forceinline__ void fft_pass12(cf (&v)[16], float2* slot, const float2* tw, int lane) {
    // pass 1: radix 16 over z[j + 64q]; y[16j + r]
    dft16<INV>(v);
    wave_lds_sync();
#pragma unroll
    for (int r = 0; r < 16; ++r) lds_st(slot, 17 * lane + r, v[r]);
    wave_lds_sync();
    // pass 2: radix 16, span 16: inputs y[j + 64q] * W256^(qk), k = j % 16;
    // outputs y2[(j - k) 16 + k + 16 r].  W^(8qk) = W^(8 q0 k) W^(32 q1 k) for q = q0 + 4 q1:
    // six table reads and nine products instead of fifteen reads.
    const int k = lane & 15, rb = pad16(lane);
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] = lds_ld(slot, rb + 68 * q);
    const cf t1 = twiddle<INV>(tw, 8 * k), t2 = twiddle<INV>(tw, 16 * k), t3 = twiddle<INV>(tw, 24 * k);
    const cf u1 = twiddle<INV>(tw, 32 * k), u2 = twiddle<INV>(tw, 64 * k), u3 = twiddle<INV>(tw, 96 * k);
    const cf tq0[4] = {cf{1.f, 0.f}, t1, t2, t3}, tq1[4] = {cf{1.f, 0.f}, u1, u2, u3};
#pragma unroll
    for (int q = 1; q < 16; ++q) {
        const int q0 = q & 3, q1 = q >> 2;
        const cf w = q0 == 0 ? tq1[q1] : (q1 == 0 ? tq0[q0] : cmul(tq0[q0], tq1[q1]));
        v[q] = cmul(v[q], w);
    }
    dft16<INV>(v);
    wave_lds_sync();
    const int wb = 272 * (lane >> 4) + k;
#pragma unroll
    for (int r = 0; r < 16; ++r) lds_st(slot, wb + 17 * r, v[r]);
    wave_lds_sync();
}

// Radix-4 butterfly jj of pass 3 (span 256): inputs y2[jj + 256q] * W1024^(q jj) from the slot,
// outputs Z[jj + 256 r] in z[r].
template <bool INV>
__device__ __forceinline__ void pass3_butterfly(const float2* slot, const float2* tw, int jj, cf (&z)[4]) {
    const int base = jj + (jj >> 4);  // pad16(jj + 256 q) = base + 272 q
#pragma unroll
    for (int q = 0; q < 4; ++q) z[q] = lds_ld(slot, base + 272 * q);
    z[1] = cmul(z[1], twiddle<INV>(tw, 2 * jj));
    z[2] = cmul(z[2], twiddle<INV>(tw, 4 * jj));
    z[3] = cmul(z[3], twiddle<INV>(tw, 6 * jj));
    dft4<INV>(z[0], z[1], z[2], z[3]);
}

// 1024-point FFT of one frame by one wave.  In: lane l holds z[l + 64a] in v[a].  Out: lane
// l holds Z[l + 64a] in v[a].
template <bool INV>
__device__ __forceinline__ void fft1024(cf (&v)[16], float2* slot, const float2* tw, int lane) {
    fft_pass12<INV>(v, slot, tw, lane);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        cf z[4];
        pass3_butterfly<INV>(slot, tw, lane + 64 * s, z);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[s + 4 * r] = z[r];
    }
}

// Real-input split of one mirror pair: from Z[f] and Z[1024 - f] (W^f = wf) writes X[f] and
// X[1024 - f] into the slot.  f = 0 (with zg = Z[0]) yields X[0] and X[1024].
__device__ __forceinline__ void r2c_pair(float2* slot, int f, cf zf, cf zg, cf wf) {
    const cf A{zf.x + zg.x, zf.y - zg.y}, Bv{zf.x - zg.x, zf.y + zg.y};
    const cf P = cmul(wf, Bv);
    lds_st(slot, pad16(f), cf{0.5f * (A.x + P.y), 0.5f * (A.y - P.x)});
    lds_st(slot, pad16(kN / 2 - f), cf{0.5f * (A.x - P.y), -0.5f * (A.y + P.x)});
}

// ---- STFT -------------------------------------------------------------------------------
struct StftArgs {
    const float* x;    // [B, L]
    const float* w;    // [2048]
    float2* out;       // [B, 1025, T] complex
    int L;
    uint32_t T;        // frames per signal
    FastDiv ntb;       // workgroups per signal: block index -> (signal, block in signal)
    int hop;
    int offset;        // 1024 when centred (reflect padding), else 0
    int wvec;          // window is 8-byte aligned: read it as float2
    int xvec;          // signal is 16-byte aligned: stage it with float4 loads
    int staged;        // the workgroup's sample span and the window fit its frame slots
    float norm;
};

// Windowed frame of sample pairs: v[q] = (x[n] w[n], x[n+1] w[n+1]), n = 2 (lane + 64 q).
__device__ __forceinline__ void load_frame(const StftArgs& a, uint32_t b, uint32_t t, int lane, cf (&v)[16]) {
    const float* xb = a.x + (int64_t)b * a.L;
    const int start = (int)t * a.hop - a.offset;
    float2 w[16];
    if (a.wvec) {
#pragma unroll
        for (int q = 0; q < 16; ++q) w[q] = reinterpret_cast<const float2*>(a.w)[lane + 64 * q];
    } else {
#pragma unroll
        for (int q = 0; q < 16; ++q) w[q] = make_float2(a.w[2 * (lane + 64 * q)], a.w[2 * (lane + 64 * q) + 1]);
    }
    if (start >= 0 && start + kN <= a.L) {
        const float* xs = xb + start;
        if ((reinterpret_cast<uintptr_t>(xs) & 7) == 0) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const float2 p = reinterpret_cast<const float2*>(xs)[lane + 64 * q];
                v[q] = cf{p.x * w[q].x, p.y * w[q].y};
            }
        } else {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int n = 2 * (lane + 64 * q);
                v[q] = cf{xs[n] * w[q].x, xs[n + 1] * w[q].y};
            }
        }
    } else {
        // reflect once about the ends, then clamp (the reference's pad_reflect rule)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int n = 2 * (lane + 64 * q);
            float e[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                int c = start + n + h;
                if (c < 0) c = -c;
                if (c >= a.L) c = 2 * (a.L - 1) - c;
                c = c < 0 ? 0 : (c > a.L - 1 ? a.L - 1 : c);
                e[h] = xb[c];
            }
            v[q] = cf{e[0] * w[q].x, e[1] * w[q].y};
        }
    }
}

// Stages the workgroup's window (2048 floats) and sample span ((nf - 1) hop + 2048 floats
// from sample s of signal b) into LDS: the span with aligned float4 loads when it lies
// inside the signal, else sample by sample through the reflect-then-clamp rule.  Returns
// the span's offset in the staging area.
template <int NT>
__device__ __forceinline__ int stage_span(const StftArgs& a, float* stage, uint32_t b, int s, int span) {
    // Loads are issued in groups of 4 per thread before their LDS writes, so that each
    // thread has several in flight.
    const int tid = threadIdx.x;
    if (a.wvec) {
        static_assert((kN / 2) % NT == 0, "threads per workgroup divide the window");
        constexpr int kPer = kN / 2 / NT;
        float2 wv[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) wv[k] = reinterpret_cast<const float2*>(a.w)[tid + k * NT];
#pragma unroll
        for (int k = 0; k < kPer; ++k) reinterpret_cast<float2*>(stage)[tid + k * NT] = wv[k];
    } else {
        constexpr int kPer = kN / NT;
        float wv[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) wv[k] = a.w[tid + k * NT];
#pragma unroll
        for (int k = 0; k < kPer; ++k) stage[tid + k * NT] = wv[k];
    }
    float* xst = stage + kN;
    if (a.xvec && s >= 0 && s + span <= a.L) {
        const int64_t base = (int64_t)b * a.L + s, end = base + span;
        const int64_t a4 = base & ~int64_t(3);  // >= 0; float4 loads from a4 are 16-byte aligned
        const int xoff = (int)(base - a4), n4 = (xoff + span + 3) >> 2;
        for (int i0 = tid; i0 < n4; i0 += 4 * NT) {
            float4 v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int i = i0 + k * NT;
                const int64_t e = a4 + 4 * (int64_t)i;
                if (i >= n4) {
                    v[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                } else if (e + 4 <= end) {
                    v[k] = *reinterpret_cast<const float4*>(a.x + e);
                } else {  // the last partial vector: nothing at or past the span's end is read
                    v[k].x = e < end ? a.x[e] : 0.0f;
                    v[k].y = e + 1 < end ? a.x[e + 1] : 0.0f;
                    v[k].z = e + 2 < end ? a.x[e + 2] : 0.0f;
                    v[k].w = 0.0f;
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (i0 + k * NT < n4) reinterpret_cast<float4*>(xst)[i0 + k * NT] = v[k];
        }
        return xoff;
    }
    const float* xb = a.x + (int64_t)b * a.L;
    for (int j0 = tid; j0 < span; j0 += 4 * NT) {
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // reflect once about the ends, then clamp (the reference's pad_reflect rule)
            int c = s + j0 + k * NT;
            if (c < 0) c = -c;
            if (c >= a.L) c = 2 * (a.L - 1) - c;
            c = c < 0 ? 0 : (c > a.L - 1 ? a.L - 1 : c);
            v[k] = j0 + k * NT < span ? xb[c] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (j0 + k * NT < span) xst[j0 + k * NT] = v[k];
    }
    return 0;
}

// The staged prologue when the workgroup's span lies inside its signal and the window and
// signal are aligned (the common case): the window, the twiddles and the span (KS float4
// per thread, indices clamped to the span's last whole vector) are all loaded before the
// first LDS write, so the workgroup pays one memory round trip instead of one per load
// group.  The span's last partial vector (1..3 samples) is read by thread 0.  Returns the
// span's offset in the staging area, as stage_span.
template <int NT, int KS>
__device__ __forceinline__ int stage_all(const StftArgs& a, float* stage, float2* tw, uint32_t b, int s, int span) {
    const int tid = threadIdx.x;
    const int64_t base = (int64_t)b * a.L + s, end = base + span;
    const int64_t a4 = base & ~int64_t(3);
    const int xoff = (int)(base - a4), n4 = (xoff + span + 3) >> 2;
    const int nfull = (int)((end - a4) >> 2);  // vectors wholly inside the span (>= 1)
    constexpr int kW = kN / 2 / NT, kT = kTwHalf / NT;
    float2 wv[kW], tv[kT];
    float4 xv[KS];
    const float2* tsrc = reinterpret_cast<const float2*>(kTwiddles.v);
#pragma unroll
    for (int k = 0; k < kW; ++k) wv[k] = reinterpret_cast<const float2*>(a.w)[tid + k * NT];
#pragma unroll
    for (int k = 0; k < kT; ++k) tv[k] = tsrc[tid + k * NT];
    const float4* x4 = reinterpret_cast<const float4*>(a.x + a4);
#pragma unroll
    for (int k = 0; k < KS; ++k) xv[k] = x4[min(tid + k * NT, nfull - 1)];
    float tail[3] = {0.0f, 0.0f, 0.0f};
    if (tid == 0 && n4 > nfull) {
#pragma unroll
        for (int e = 0; e < 3; ++e) {
            const int64_t q = a4 + 4 * (int64_t)nfull + e;
            tail[e] = q < end ? a.x[q] : 0.0f;
        }
    }
#pragma unroll
    for (int k = 0; k < kW; ++k) reinterpret_cast<float2*>(stage)[tid + k * NT] = wv[k];
#pragma unroll
    for (int k = 0; k < kT; ++k) tw[tw_pos(tid + k * NT)] = tv[k];
    float* xst = stage + kN;
    // unconditional writes (threads past the span rewrite its last whole vector with the
    // same bytes): a predicated write would let the compiler sink each load into its branch
    // and wait for it there, one round trip per load
#pragma unroll
    for (int k = 0; k < KS; ++k) reinterpret_cast<float4*>(xst)[min(tid + k * NT, nfull - 1)] = xv[k];
    if (tid == 0 && n4 > nfull) {
#pragma unroll
        for (int e = 0; e < 3; ++e) xst[4 * nfull + e] = tail[e];
    }
    return xoff;
}

template <int TF>
__global__ __launch_bounds__(64 * TF) void stft_kernel(StftArgs a) {
    constexpr int NT = 64 * TF;
    __shared__ __attribute__((aligned(16))) float2 lds[TF * kSlot + kTwSlots];
    float2* tw = lds + TF * kSlot;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    // workgroup = frames t0 .. t0 + nf - 1 of signal b
    uint32_t b, tb;
    fdivmod(xcd_runs<kXcdRun>(blockIdx.x, gridDim.x), a.ntb, b, tb);
    const uint32_t t0 = tb * TF;
    const int nf = (int)min((uint32_t)TF, a.T - t0);
    const bool live = wave < nf;
    cf v[16];
    if (a.staged) {
        // the frames of a workgroup overlap (hop < 2048): their span and the window are read
        // from HBM once, coalesced, into the frame slots, and each wave takes its frame there
        const int s = (int)t0 * a.hop - a.offset;
        float* stage = reinterpret_cast<float*>(lds);
        const int span = (nf - 1) * a.hop + kN;
        int xoff;
        if (a.wvec && a.xvec && s >= 0 && s + span <= a.L && span + 3 <= 4 * 4 * NT) {
            xoff = stage_all<NT, 4>(a, stage, tw, b, s, span);
        } else {
            xoff = stage_span<NT>(a, stage, b, s, span);
            load_twiddles<NT>(tw);
        }
        __syncthreads();
        if (live) {
            const float* xs = stage + kN + xoff + wave * a.hop;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int n = 2 * (lane + 64 * q);
                const float2 w = reinterpret_cast<const float2*>(stage)[lane + 64 * q];
                v[q] = cf{xs[n] * w.x, xs[n + 1] * w.y};
            }
        }
        __syncthreads();  // the staging area becomes the frame slots
    } else {
        if (live) load_frame(a, b, t0 + wave, lane, v);
        load_twiddles<NT>(tw);
        __syncthreads();
    }
    if (live) {
        float2* slot = lds + wave * kSlot;
        fft_pass12<false>(v, slot, tw, lane);
        // pass 3 over butterflies chosen in mirror pairs (jj, 256 - jj), so that every lane
        // holds both Z[f] and Z[1024 - f] of its outputs: lanes 1..63 take l, 256 - l,
        // 128 + l, 128 - l; lane 0 takes 0, 128 (each its own mirror), 64, 192.
        const int jA = lane, jB = lane ? 256 - lane : 128;
        const int jC = lane ? 128 + lane : 64, jD = lane ? 128 - lane : 192;
        cf zA[4], zB[4], zC[4], zD[4];
        pass3_butterfly<false>(slot, tw, jA, zA);
        pass3_butterfly<false>(slot, tw, jB, zB);
        pass3_butterfly<false>(slot, tw, jC, zC);
        pass3_butterfly<false>(slot, tw, jD, zD);
        wave_lds_sync();
        // real split: Z[1024 - (jA + 256 r)] is zB[3 - r] (lane 0: zA[(4 - r) % 4]); Z[1024 -
        // (jC + 256 r)] is zD[3 - r]; lane 0 also splits butterfly 128 against itself.
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const cf za = lane ? zB[3 - r] : zA[(4 - r) & 3];
            r2c_pair(slot, jA + 256 * r, zA[r], za, twiddle<false>(tw, jA + 256 * r));
            r2c_pair(slot, jC + 256 * r, zC[r], zD[3 - r], twiddle<false>(tw, jC + 256 * r));
        }
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < 2; ++r)
                r2c_pair(slot, 128 + 256 * r, zB[r], zB[3 - r], twiddle<false>(tw, 128 + 256 * r));
        }
    }
    __syncthreads();
    // transposed store: thread -> (frame t0 + tl, bins fr, fr + 64, ...)
    const int tl = threadIdx.x % TF, fr = threadIdx.x / TF;
    if (tl >= nf) return;
    float2* dst = a.out + ((int64_t)b * kBins * a.T + t0 + tl);
    const float2* src = lds + tl * kSlot;
    const int64_t step = (int64_t)(NT / TF) * a.T;
    dst += (int64_t)fr * a.T;
#pragma unroll 4
    for (int f = fr; f < kBins; f += NT / TF, dst += step) {
        const float2 X = src[pad16(f)];
        gst<MBRT_NT_STFT & 2>(reinterpret_cast<f32x2*>(dst), f32x2{X.x * a.norm, X.y * a.norm});
    }
}

// ---- iSTFT ------------------------------------------------------------------------------
// Block kernel: one workgroup = kTF consecutive frames of one signal.  Their spectra are
// loaded transposed, each wave inverts one frame and leaves it, windowed and scaled, in its
// LDS slot; the workgroup then overlap-adds its frames in LDS (frame order) and writes the
// block's partial signal, (nf - 1) hop + 2048 samples from sample t0 hop.  The final
// kernel adds, per output sample, the partials of the blocks that cover it (block order)
// and divides by the window sum.
struct IstftBlockArgs {
    const void* spec;   // [B, 1025, T] complex, f32 or bf16
    const float* w;
    float* part;        // [B, nTB, span] block partials
    uint32_t T;
    FastDiv ntb;        // blocks per signal
    FastDiv hop;
    uint32_t span;      // (kTF - 1) hop + 2048: stride of a block's partial
    uint32_t blocks;    // B * nTB
    int wvec;           // window is 8-byte aligned
    float spec_scale;
};

template <int SDT>
__device__ __forceinline__ float2 load_bin(const void* spec, int64_t i) {
    if constexpr (SDT == F32) {
        const f32x2 v = gld<MBRT_NT_STFT & 1>(static_cast<const f32x2*>(spec) + i);
        return make_float2(v.x, v.y);
    } else {
        const uint32_t u = gld<MBRT_NT_STFT & 1>(static_cast<const uint32_t*>(spec) + i);
        return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
    }
}

template <int TF, int SDT>
__global__ __launch_bounds__(64 * TF) void istft_block_kernel(IstftBlockArgs a) {
    constexpr int NT = 64 * TF;
    __shared__ __attribute__((aligned(16))) float2 lds[TF * kSlot + kTwSlots];
    float2* tw = lds + TF * kSlot;
    const uint32_t blk = xcd_runs<kXcdRunInv>(blockIdx.x, gridDim.x);
    uint32_t b, tb;
    fdivmod(blk, a.ntb, b, tb);
    const uint32_t t0 = tb * TF;
    const uint32_t nf = min((uint32_t)TF, a.T - t0);
    // the twiddle loads go out with the spectrum's, one memory round trip for both
    constexpr int kT = kTwHalf / NT;
    float2 tv[kT];
#pragma unroll
    for (int k = 0; k < kT; ++k) tv[k] = reinterpret_cast<const float2*>(kTwiddles.v)[threadIdx.x + k * NT];
    {
        // transposed spectrum load: thread -> (frame tl, bins fr + 64 k, k = 0..15, and bin
        // 1024 for fr = 0); all 16 (17) loads are in flight before the first LDS write
        static_assert(NT / TF == 64, "64 bin rows per pass");
        const int tl = threadIdx.x % TF, fr = threadIdx.x / TF;
        if ((uint32_t)tl < nf) {
            const int64_t idx = (int64_t)b * kBins * a.T + t0 + tl + (int64_t)fr * a.T;
            const int64_t step = (int64_t)64 * a.T;
            float2 X[17];
#pragma unroll
            for (int k = 0; k < 16; ++k) X[k] = load_bin<SDT>(a.spec, idx + k * step);
            if (fr == 0) X[16] = load_bin<SDT>(a.spec, idx + 16 * step);
            float2* slot = lds + tl * kSlot;
#pragma unroll
            for (int k = 0; k < 16; ++k)
                slot[pad16(fr + 64 * k)] = make_float2(X[k].x * a.spec_scale, X[k].y * a.spec_scale);
            if (fr == 0) slot[pad16(kN / 2)] = make_float2(X[16].x * a.spec_scale, X[16].y * a.spec_scale);
        }
    }
#pragma unroll
    for (int k = 0; k < kT; ++k) tw[tw_pos(threadIdx.x + k * NT)] = tv[k];
    __syncthreads();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if ((uint32_t)wave < nf) {
        float2* slot = lds + wave * kSlot;
        // inverse real split, in place: (X[k], X[1024 - k]) -> (Z[k], Z[1024 - k]) scaled by 2;
        // Z[0] from the real parts of X[0] and X[1024] (their imaginary parts drop out).
        cf x0{0.f, 0.f}, xn{0.f, 0.f};
        if (lane == 0) {
            x0 = lds_ld(slot, 0);
            xn = lds_ld(slot, pad16(kN / 2));
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int k = 1 + lane + 64 * q, gg = kN / 2 - k;
            const cf xk = lds_ld(slot, pad16(k)), xg = lds_ld(slot, pad16(gg));
            const cf A{xk.x + xg.x, xk.y - xg.y}, Bv{xk.x - xg.x, xk.y + xg.y};
            const cf Q = cmul(Bv, twiddle<true>(tw, k));
            lds_st(slot, pad16(k), cf{A.x - Q.y, A.y + Q.x});
            lds_st(slot, pad16(gg), cf{A.x + Q.y, Q.x - A.y});
        }
        if (lane == 0) lds_st(slot, 0, cf{x0.x + xn.x, x0.x - xn.x});
        wave_lds_sync();
        cf v[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) v[q] = lds_ld(slot, pad16(lane) + 68 * q);
        fft1024<true>(v, slot, tw, lane);
        // lane l holds 2048 * (x[2m], x[2m + 1]), m = l + 64a: the windowed frame goes back into
        // the slot as 2048 consecutive floats
        wave_lds_sync();
        constexpr float kInvN = 1.0f / (float)kN;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int m = lane + 64 * q;
            float2 w;
            if (a.wvec) w = reinterpret_cast<const float2*>(a.w)[m];
            else w = make_float2(a.w[2 * m], a.w[2 * m + 1]);
            slot[m] = make_float2(v[q].x * w.x * kInvN, v[q].y * w.y * kInvN);
        }
    }
    __syncthreads();
    // overlap-add of the block's frames in frame order: partial[u], u = s - t0 hop
    const uint32_t hop = a.hop.d;
    const uint32_t span = (nf - 1) * hop + kN;
    float* part = a.part + (int64_t)blk * a.span;
    for (uint32_t u = threadIdx.x; u < span; u += NT) {
        const uint32_t jhi = min(nf - 1, fdiv(u, a.hop));
        const uint32_t jlo = u >= (uint32_t)kN ? fdiv(u - kN, a.hop) + 1 : 0;
        float acc = 0.0f;
        for (uint32_t j = jlo; j <= jhi; ++j) acc += reinterpret_cast<const float*>(lds + j * kSlot)[u - j * hop];
        gst<MBRT_NT_ISTFT & 2>(part + u, acc);
    }
}

struct IstftFinalArgs {
    const float* part;    // [B, nTB, span]
    const float* w;
    float* out;           // [B, out_len]
    uint32_t batch;
    uint32_t out_len;
    FastDiv hop;
    FastDiv bhop;         // kTF * hop: block stride in samples
    uint32_t span;
    uint32_t ntb;
    uint32_t T;
    uint32_t valid;       // samples of the (trimmed) signal; out_len - valid zeros follow
    uint32_t offset;      // 1024 when centred
};

// One thread per output sample position, for every signal of the batch: the window sum
// (the same for all signals) is formed once.
__global__ __launch_bounds__(256) void istft_final_kernel(IstftFinalArgs a) {
    const uint32_t hop = a.hop.d, bhop = a.bhop.d;
    for (uint32_t so = blockIdx.x * 256 + threadIdx.x; so < a.out_len; so += gridDim.x * 256) {
        if (so >= a.valid) {
            for (uint32_t b = 0; b < a.batch; ++b) gst<(MBRT_NT_ISTFT & 4) ? 2 : 0>(a.out + (int64_t)b * a.out_len + so, 0.0f);
            continue;
        }
        const uint32_t s = so + a.offset;
        // window sum of squares in frame order (f32), as the reference's window_sum; the
        // loads go 8 at a time, all in flight before their terms are added
        const uint32_t thi = min(a.T - 1, fdiv(s, a.hop));
        const uint32_t tlo = s >= (uint32_t)kN ? fdiv(s - kN, a.hop) + 1 : 0;
        float ws = 0.0f;
        for (uint32_t t = tlo; t <= thi; t += 8) {
            float wv[8];
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) wv[k] = a.w[t + k <= thi ? s - (t + k) * hop : 0];
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) {
#pragma clang fp contract(off)
                if (t + k <= thi) ws = ws + wv[k] * wv[k];
            }
        }
        // blocks covering s, in block order; a block's partial is shorter when it is the last
        // one of its signal
        const uint32_t bhi = min(a.ntb - 1, fdiv(s, a.bhop));
        const uint32_t blo = s >= a.span ? fdiv(s - a.span, a.bhop) + 1 : 0;
        if (bhi <= blo + 1) {
            // at most two blocks (every hop >= 256): the same two offsets for every signal,
            // whose loads go 4 signals at a time
            bool v[2];
            int64_t off[2];
#pragma unroll
            for (uint32_t i = 0; i < 2; ++i) {
                const uint32_t tb = blo + i, u = s - tb * bhop;
                v[i] = tb <= bhi && u < (min((uint32_t)kTF, a.T - tb * kTF) - 1) * hop + kN;
                off[i] = v[i] ? (int64_t)tb * a.span + u : 0;
            }
            for (uint32_t b0 = 0; b0 < a.batch; b0 += 4) {
                float p[4][2];
#pragma unroll
                for (uint32_t k = 0; k < 4; ++k) {
                    const float* pb = a.part + (int64_t)min(b0 + k, a.batch - 1) * a.ntb * a.span;
                    p[k][0] = gld<MBRT_NT_ISTFT & 1>(pb + off[0]);
                    p[k][1] = gld<MBRT_NT_ISTFT & 1>(pb + off[1]);
                }
#pragma unroll
                for (uint32_t k = 0; k < 4; ++k) {
                    if (b0 + k >= a.batch) break;
                    float acc = 0.0f;
                    if (v[0]) acc += p[k][0];
                    if (v[1]) acc += p[k][1];
                    gst<(MBRT_NT_ISTFT & 4) ? 2 : 0>(a.out + (int64_t)(b0 + k) * a.out_len + so, ws > 1.0e-8f ? acc / ws : acc);
                }
            }
            continue;
        }
#pragma unroll 4
        for (uint32_t b = 0; b < a.batch; ++b) {
            const float* pb = a.part + (int64_t)b * a.ntb * a.span;
            float acc = 0.0f;
            for (uint32_t tb = blo; tb <= bhi; ++tb) {
                const uint32_t u = s - tb * bhop;
                const uint32_t nf = min((uint32_t)kTF, a.T - tb * kTF);
                if (u < (nf - 1) * hop + kN) acc += gld<MBRT_NT_ISTFT & 1>(pb + (int64_t)tb * a.span + u);
            }
            gst<(MBRT_NT_ISTFT & 4) ? 2 : 0>(a.out + (int64_t)b * a.out_len + so, ws > 1.0e-8f ? acc / ws : acc);
        }
    }
}

__global__ __launch_bounds__(256) void hann_kernel(float* out, int64_t size) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= size) return;
    const float phase = (float)i * (6.28318530717958647692f / (float)size);
    out[i] = 0.5f * (1.0f - cosf(phase));
}

int check_fixed_size(const char* op, int64_t n_fft, int64_t win_length, int64_t window_numel) {
    MBRT_REQUIRE(n_fft == kN && win_length == kN && window_numel == kN, MBRT_E_SHAPE,
                 "%s: only n_fft=2048, win_length=2048 with a 2048-sample window is supported "
                 "(got n_fft=%lld, win_length=%lld, window %lld)", op, (long long)n_fft,
                 (long long)win_length, (long long)window_numel);
    return MBRT_OK;
}

constexpr int64_t kMaxHop = int64_t(1) << 20;  // keeps block spans and sample indices in 32 bits

int64_t grid_for(int64_t work, int64_t per_block) {
    return std::min<int64_t>(ceil_div(work, per_block), int64_t(1) << 20);
}

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int64_t mbrt_stft_num_frames(int64_t length, int64_t hop, int center) {
    if (length < 0 || hop < 1) return -1;
    const int64_t padded = length + (center ? kN : 0);
    if (padded < kN) return 0;
    return (padded - kN) / hop + 1;
}

int mbrt_hann_window(float* out, int64_t size, mbrt_stream_t stream) {
    const char* op = "mbrt_hann_window";
    MBRT_REQUIRE(size >= 0 && size < (int64_t(1) << 31), MBRT_E_SHAPE, "%s: bad size %lld", op, (long long)size);
    if (size == 0) return MBRT_OK;
    MBRT_REQUIRE(out != nullptr, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    if (size == 1) return mbrt_fill(out, F32, 1, 1.0, stream);
    hipLaunchKernelGGL(hann_kernel, dim3((unsigned)ceil_div(size, 256)), dim3(256), 0, as_stream(stream), out, size);
    return check_launch(op);
}

int mbrt_stft(const float* signal, const float* window, float* out, int64_t batch, int64_t length, int64_t n_fft,
              int64_t hop, int64_t win_length, int64_t window_numel, int center, int normalized,
              mbrt_stream_t stream) {
    const char* op = "mbrt_stft";
    int s = check_fixed_size(op, n_fft, win_length, window_numel);
    if (s != MBRT_OK) return s;
    MBRT_REQUIRE(batch >= 0 && length >= 1 && hop >= 1 && hop < (1 << 30), MBRT_E_SHAPE,
                 "%s: bad shape (batch %lld, length %lld, hop %lld)", op, (long long)batch, (long long)length,
                 (long long)hop);
    const int64_t T = mbrt_stft_num_frames(length, hop, center);
    MBRT_REQUIRE(T >= 1, MBRT_E_SHAPE, "%s: signal of %lld samples is shorter than n_fft=2048", op,
                 (long long)length);
    MBRT_REQUIRE(length <= (1 << 30) && batch * T < (int64_t(1) << 31), MBRT_E_SHAPE, "%s: too many samples or frames",
                 op);
    if (batch == 0) return MBRT_OK;
    MBRT_REQUIRE(signal && window && out, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    MBRT_REQUIRE(aligned(out, 8), MBRT_E_ALIGN, "%s: out must be 8-byte aligned", op);
    StftArgs a{};
    a.x = signal;
    a.w = window;
    a.out = reinterpret_cast<float2*>(out);
    a.L = (int)length;
    a.T = (uint32_t)T;
    const int64_t ntb = ceil_div(T, kTF);
    a.ntb = make_fastdiv((uint32_t)ntb);
    a.hop = (int)hop;
    a.offset = center ? kN / 2 : 0;
    a.norm = normalized ? 1.0f / std::sqrt((float)kN) : 1.0f;
    a.wvec = aligned(window, 8) ? 1 : 0;
    a.xvec = aligned(signal, 16) ? 1 : 0;
    // window + span (+ up to 6 floats of float4 alignment) within the kTF frame slots
    a.staged = kN + (kTF - 1) * hop + kN + 6 <= 2 * kTF * kSlot ? 1 : 0;
    const int64_t blocks = batch * ntb;
    MBRT_REQUIRE(blocks < kMaxGridX, MBRT_E_SHAPE, "%s: too many frames", op);
    hipLaunchKernelGGL((stft_kernel<kTF>), dim3((unsigned)blocks), dim3(64 * kTF), 0, as_stream(stream), a);
    return check_launch(op);
}

int64_t mbrt_istft_output_length(int64_t frames, int64_t hop, int center, int64_t length) {
    if (frames < 1 || hop < 1) return -1;
    if (length > 0) return length;
    const int64_t full = kN + (frames - 1) * hop;
    return center ? full - kN : full;
}

int64_t mbrt_istft_workspace_bytes(int64_t batch, int64_t frames, int64_t hop) {
    if (batch < 0 || frames < 0 || hop < 1 || hop > kMaxHop) return -1;
    return batch * ceil_div(frames, kTF) * ((kTF - 1) * hop + kN) * (int64_t)sizeof(float);
}

}  // extern "C"

namespace {

// Scratch of the allocation-free iSTFT (mbrt_istft_noalloc): the block partials of one
// call.  A file-scope device array of MBRT_ISTFT_SCRATCH_BYTES, allocated on every GPU
// that loads the library's code object and held until the process ends; all calls on one
// GPU share it, so calls that overlap there race.  Nothing in it needs clearing: the block
// pass writes every partial sample the final pass reads.  In host code `scratch` names a
// host-side stand-in, not device memory: its device address on the current GPU is taken
// once per device with hipGetSymbolAddress, and only that pointer reaches the kernels.
__device__ __align__(256) float scratch[MBRT_ISTFT_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];

int scratch_ptr(const char* op, void** ptr) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    MBRT_REQUIRE(e == hipSuccess, MBRT_E_HIP, "%s: hipGetDevice: %s", op, hipGetErrorString(e));
    MBRT_REQUIRE(dev >= 0 && dev < kMaxDevices, MBRT_E_HIP, "%s: device %d beyond %d", op, dev, kMaxDevices);
    void* p = g_scratch[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        MBRT_REQUIRE(e == hipSuccess && p != nullptr, MBRT_E_HIP, "%s: hipGetSymbolAddress: %s", op,
                     hipGetErrorString(e));
        g_scratch[dev].store(p, std::memory_order_release);
    }
    *ptr = p;
    return MBRT_OK;
}

// The two iSTFT passes over a workspace of block partials; `workspace` is NULL for the
// allocation-free entry point, which then uses this GPU's scratch array.
int istft_impl(const char* op, const void* spec, int spec_dtype, const float* window, float* out, int64_t batch,
               int64_t freq_bins, int64_t frames, int64_t n_fft, int64_t hop, int64_t win_length,
               int64_t window_numel, int center, int normalized, int64_t length, void* workspace,
               int64_t workspace_bytes, mbrt_stream_t stream) {
    const bool scratch = workspace == nullptr;
    int s = check_fixed_size(op, n_fft, win_length, window_numel);
    if (s != MBRT_OK) return s;
    MBRT_REQUIRE(freq_bins == kBins, MBRT_E_SHAPE, "%s: %lld frequency bins (expected 1025)", op,
                 (long long)freq_bins);
    MBRT_REQUIRE(spec_dtype == F32 || spec_dtype == BF16, MBRT_E_UNSUPPORTED_DTYPE,
                 "%s: spectrum must be F32 or BF16", op);
    MBRT_REQUIRE(batch >= 0 && frames >= 1 && frames < (1 << 30) && hop >= 1 && hop <= kMaxHop, MBRT_E_SHAPE,
                 "%s: bad shape (batch %lld, frames %lld, hop %lld)", op, (long long)batch, (long long)frames,
                 (long long)hop);
    const int64_t out_len = mbrt_istft_output_length(frames, hop, center, length);
    if (batch == 0 || out_len == 0) return MBRT_OK;
    MBRT_REQUIRE(spec && window && out, MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    const int64_t need = mbrt_istft_workspace_bytes(batch, frames, hop);
    if (scratch) {
        MBRT_REQUIRE(need <= MBRT_ISTFT_SCRATCH_BYTES, MBRT_E_SHAPE,
                     "%s: needs %lld bytes of scratch, more than the %lld the library holds per GPU (use mbrt_istft "
                     "with a workspace)",
                     op, (long long)need, (long long)MBRT_ISTFT_SCRATCH_BYTES);
        s = scratch_ptr(op, &workspace);
        if (s != MBRT_OK) return s;
        workspace_bytes = MBRT_ISTFT_SCRATCH_BYTES;
    }
    MBRT_REQUIRE(workspace_bytes >= need, MBRT_E_INVALID_ARG, "%s: workspace of %lld bytes, %lld needed", op,
                 (long long)workspace_bytes, (long long)need);
    MBRT_REQUIRE(aligned(workspace, 4) && aligned(spec, spec_dtype == F32 ? 8 : 4), MBRT_E_ALIGN,
                 "%s: spectrum and workspace must be aligned to their element", op);
    const int64_t full = kN + (frames - 1) * hop;
    const int64_t ntb = ceil_div(frames, kTF);
    MBRT_REQUIRE(batch * ntb < (int64_t(1) << 31) && batch * out_len < (int64_t(1) << 31) &&
                     full + kN < (int64_t(1) << 31),
                 MBRT_E_SHAPE, "%s: signal too long", op);
    hipStream_t st = as_stream(stream);
    IstftBlockArgs ba{};
    ba.spec = spec;
    ba.w = window;
    ba.part = static_cast<float*>(workspace);
    ba.T = (uint32_t)frames;
    ba.ntb = make_fastdiv((uint32_t)ntb);
    ba.hop = make_fastdiv((uint32_t)hop);
    ba.span = (uint32_t)((kTF - 1) * hop + kN);
    ba.blocks = (uint32_t)(batch * ntb);
    ba.wvec = aligned(window, 8) ? 1 : 0;
    ba.spec_scale = normalized ? std::sqrt((float)kN) : 1.0f;
    if (spec_dtype == F32)
        hipLaunchKernelGGL((istft_block_kernel<kTF, F32>), dim3(ba.blocks), dim3(64 * kTF), 0, st, ba);
    else
        hipLaunchKernelGGL((istft_block_kernel<kTF, BF16>), dim3(ba.blocks), dim3(64 * kTF), 0, st, ba);
    s = check_launch(op);
    if (s != MBRT_OK) return s;
    IstftFinalArgs fa{};
    fa.part = ba.part;
    fa.w = window;
    fa.out = out;
    fa.batch = (uint32_t)batch;
    fa.out_len = (uint32_t)out_len;
    fa.hop = make_fastdiv((uint32_t)hop);
    fa.bhop = make_fastdiv((uint32_t)(kTF * hop));
    fa.span = ba.span;
    fa.ntb = (uint32_t)ntb;
    fa.T = (uint32_t)frames;
    fa.valid = (uint32_t)std::min<int64_t>(out_len, center ? full - kN : full);
    fa.offset = center ? kN / 2 : 0;
    hipLaunchKernelGGL(istft_final_kernel, dim3((unsigned)grid_for(out_len, 256)), dim3(256), 0, st, fa);
    return check_launch(op);
}

}  // namespace

extern "C" {

int mbrt_istft(const void* spec, int spec_dtype, const float* window, float* out, int64_t batch,
               int64_t freq_bins, int64_t frames, int64_t n_fft, int64_t hop, int64_t win_length,
               int64_t window_numel, int center, int normalized, int64_t length, void* workspace,
               int64_t workspace_bytes, mbrt_stream_t stream) {
    if (workspace == nullptr) return set_error(MBRT_E_INVALID_ARG, "mbrt_istft: NULL workspace");
    return istft_impl("mbrt_istft", spec, spec_dtype, window, out, batch, freq_bins, frames, n_fft, hop, win_length,
                      window_numel, center, normalized, length, workspace, workspace_bytes, stream);
}

int mbrt_istft_noalloc(const void* spec, int spec_dtype, const float* window, float* out, int64_t batch,
                       int64_t freq_bins, int64_t frames, int64_t n_fft, int64_t hop, int64_t win_length,
                       int64_t window_numel, int center, int normalized, int64_t length, mbrt_stream_t stream) {
    return istft_impl("mbrt_istft_noalloc", spec, spec_dtype, window, out, batch, freq_bins, frames, n_fft, hop,
                      win_length, window_numel, center, normalized, length, nullptr, 0, stream);
}

}  // extern "C"
