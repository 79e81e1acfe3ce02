// Device-side building blocks shared by every gfx950 kernel of the library:
// dtype-generic vector I/O (16-byte global loads/stores), bf16/f16 round-to-nearest-even
// packing, fast division by run-time invariant integers, and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace mbrt {

enum DT : int { F32 = 0, F16 = 1, I64 = 2, BF16 = 3, I32 = 4 };

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__host__ __device__ constexpr int dt_size(int dt) {
    return dt == F32 ? 4 : dt == I64 ? 8 : dt == I32 ? 4 : 2;
}

// ---- scalar conversions ----------------------------------------------------

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two floats -> two bf16 in one dword (element 0 in the low half).  On gfx950 this is a
// single v_cvt_pk_bf16_f32, which rounds to nearest even and keeps NaN a NaN.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}
__device__ __forceinline__ f32x2 unpack_f16x2(uint32_t w) {
    return __builtin_convertvector(__builtin_bit_cast(f16x2, w), f32x2);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float a) {
    return (uint16_t)(pack_bf16x2(a, 0.0f) & 0xffffu);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float a) {
    return __builtin_bit_cast(uint16_t, (_Float16)a);
}

// Round a float through `dt` storage precision (used where the reference stores an
// intermediate, e.g. the residual sum, before reusing it).
__device__ __forceinline__ float round_through(float v, int dt) {
    if (dt == BF16) return bf16_lo(f32_to_bf16_bits(v));
    if (dt == F16) return (float)(_Float16)v;
    return v;
}

// Round to the nearest bf16 (ties to even) and widen back: an intermediate of the
// bf16-intermediates mode.
__device__ __forceinline__ float bf16r(float v) { return bf16_lo(f32_to_bf16_bits(v)); }

// ---- element loads/stores with a run-time dtype (uniform across the grid) ----

__device__ __forceinline__ float load1(const void* p, int dt, int64_t i) {
    if (dt == F32) return reinterpret_cast<const float*>(p)[i];
    uint32_t h = reinterpret_cast<const uint16_t*>(p)[i];
    if (dt == BF16) return __uint_as_float(h << 16);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ void store1(void* p, int dt, int64_t i, float v) {
    if (dt == F32) {
        reinterpret_cast<float*>(p)[i] = v;
    } else if (dt == BF16) {
        reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
    } else {
        reinterpret_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
    }
}

// 8 consecutive elements starting at element e (caller guarantees 16-byte alignment of
// the 2-byte case and 32-byte alignment of the f32 case, i.e. p 16B-aligned, e % 8 == 0).
__device__ __forceinline__ void load8(const void* p, int dt, int64_t e, float (&f)[8]) {
    if (dt == F32) {
        const u32x4* q = reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(p) + e);
        u32x4 a = q[0], b = q[1];
        f[0] = __uint_as_float(a.x); f[1] = __uint_as_float(a.y);
        f[2] = __uint_as_float(a.z); f[3] = __uint_as_float(a.w);
        f[4] = __uint_as_float(b.x); f[5] = __uint_as_float(b.y);
        f[6] = __uint_as_float(b.z); f[7] = __uint_as_float(b.w);
    } else {
        u32x4 a = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(p) + e);
        if (dt == BF16) {
            f[0] = bf16_lo(a.x); f[1] = bf16_hi(a.x); f[2] = bf16_lo(a.y); f[3] = bf16_hi(a.y);
            f[4] = bf16_lo(a.z); f[5] = bf16_hi(a.z); f[6] = bf16_lo(a.w); f[7] = bf16_hi(a.w);
        } else {
            f32x2 t;
            t = unpack_f16x2(a.x); f[0] = t.x; f[1] = t.y;
            t = unpack_f16x2(a.y); f[2] = t.x; f[3] = t.y;
            t = unpack_f16x2(a.z); f[4] = t.x; f[5] = t.y;
            t = unpack_f16x2(a.w); f[6] = t.x; f[7] = t.y;
        }
    }
}

__device__ __forceinline__ void store8(void* p, int dt, int64_t e, const float (&f)[8]) {
    if (dt == F32) {
        u32x4* q = reinterpret_cast<u32x4*>(reinterpret_cast<float*>(p) + e);
        u32x4 a = {__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                   __float_as_uint(f[3])};
        u32x4 b = {__float_as_uint(f[4]), __float_as_uint(f[5]), __float_as_uint(f[6]),
                   __float_as_uint(f[7])};
        q[0] = a;
        q[1] = b;
    } else {
        u32x4 a;
        if (dt == BF16) {
            a.x = pack_bf16x2(f[0], f[1]); a.y = pack_bf16x2(f[2], f[3]);
            a.z = pack_bf16x2(f[4], f[5]); a.w = pack_bf16x2(f[6], f[7]);
        } else {
            a.x = pack_f16x2(f[0], f[1]); a.y = pack_f16x2(f[2], f[3]);
            a.z = pack_f16x2(f[4], f[5]); a.w = pack_f16x2(f[6], f[7]);
        }
        *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(p) + e) = a;
    }
}

// 4 consecutive elements (p 16B-aligned for f32, 8B-aligned for 2-byte types; e % 4 == 0).
__device__ __forceinline__ void load4(const void* p, int dt, int64_t e, float (&f)[4]) {
    if (dt == F32) {
        u32x4 a = *reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(p) + e);
        f[0] = __uint_as_float(a.x); f[1] = __uint_as_float(a.y);
        f[2] = __uint_as_float(a.z); f[3] = __uint_as_float(a.w);
    } else {
        u32x2 a = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(p) + e);
        if (dt == BF16) {
            f[0] = bf16_lo(a.x); f[1] = bf16_hi(a.x); f[2] = bf16_lo(a.y); f[3] = bf16_hi(a.y);
        } else {
            f32x2 t = unpack_f16x2(a.x); f[0] = t.x; f[1] = t.y;
            t = unpack_f16x2(a.y); f[2] = t.x; f[3] = t.y;
        }
    }
}

__device__ __forceinline__ void store4(void* p, int dt, int64_t e, const float (&f)[4]) {
    if (dt == F32) {
        u32x4 a = {__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                   __float_as_uint(f[3])};
        *reinterpret_cast<u32x4*>(reinterpret_cast<float*>(p) + e) = a;
    } else {
        u32x2 a;
        if (dt == BF16) {
            a.x = pack_bf16x2(f[0], f[1]); a.y = pack_bf16x2(f[2], f[3]);
        } else {
            a.x = pack_f16x2(f[0], f[1]); a.y = pack_f16x2(f[2], f[3]);
        }
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p) + e) = a;
    }
}

// VE consecutive elements at element e: VE = 4 (f32: one 16-byte access; 2-byte types:
// 8 bytes) or VE = 8 (2-byte types: one 16-byte access; f32: two).  Kernels use VE = 4
// whenever an f32 operand is involved so that lane l's bytes follow lane l-1's.
template <int VE>
__device__ __forceinline__ void vload(const void* p, int dt, int64_t e, float (&f)[VE]) {
    if constexpr (VE == 4) load4(p, dt, e, f);
    else load8(p, dt, e, f);
}
template <int VE>
__device__ __forceinline__ void vstore(void* p, int dt, int64_t e, const float (&f)[VE]) {
    if constexpr (VE == 4) store4(p, dt, e, f);
    else store8(p, dt, e, f);
}

// ---- fast division by an invariant 32-bit divisor ------------------------------
// Granlund & Montgomery, "Division by Invariant Integers using Multiplication" (1994),
// round-up variant: q = (umulhi(n, m) + n) >> s with s = ceil(log2 d),
// m = floor(2^32 (2^s - d) / d) + 1.  Exact for every n < 2^32 and 1 <= d < 2^31.
struct FastDiv {
    uint32_t d;
    uint32_t m;
    uint32_t s;
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.d = d;
    uint32_t s = 0;
    while ((1ull << s) < d) ++s;
    f.s = s;
    f.m = (uint32_t)((((1ull << s) - d) << 32) / d + 1);
    return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
    uint64_t t = (uint64_t)__umulhi(n, f.m) + n;
    return (uint32_t)(t >> f.s);
}
__device__ __forceinline__ void fdivmod(uint32_t n, const FastDiv& f, uint32_t& q, uint32_t& r) {
    q = fdiv(n, f);
    r = n - q * f.d;
}

// ---- direct-to-LDS loads and counted waits ---------------------------------------------
// global_load_lds_*: lane i of a wave instruction writes its SIZE bytes at lds + SIZE * i
// (lds is wave-uniform).  Such a load counts in vmcnt like any vector-memory instruction,
// and on gfx9 vmcnt retires in issue order for loads and stores alike, so waiting until
// at most N are outstanding completes everything issued before the last N.
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void global_void;
// Cache-policy operand of those builtins: the non-temporal (nt) bit of gfx940-family
// memory instructions, as __builtin_nontemporal_load sets it on ordinary loads.
constexpr int kCpolNt = 2;
typedef __attribute__((address_space(4))) const int32_t const_i32;

// s_waitcnt vmcnt(N) with expcnt and lgkmcnt left free (gfx9 encoding: vmcnt in bits 3:0
// and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// N ds_read_b64 at LDS byte address addr + OFF0 + i * STEP (i < N), completed before the
// statement ends.  Written as one asm block so that the compiler neither sees these reads
// (it would otherwise wait for every direct-to-LDS load in flight, vmcnt(0), before them:
// it cannot tell one LDS buffer from another) nor touches the registers before the data
// has arrived.  The caller orders them with its own vmcnt wait and barrier.
template <int N, int OFF0, int STEP>
__device__ __forceinline__ void lds_read_b64_n(uint32_t addr, f32x2 (&v)[N]) {
    static_assert(N == 8 || N == 16, "8 or 16 reads");
    static_assert(OFF0 >= 0 && OFF0 + (N - 1) * STEP < 65536, "ds offset is 16 bits");
#define MBRT_DSR(i) "ds_read_b64 %" #i ", %[a] offset:%[o" #i "]\n\t"
#define MBRT_OFF(i) [o##i] "n"(OFF0 + (i) * STEP)
    if constexpr (N == 8) {
        asm volatile(MBRT_DSR(0) MBRT_DSR(1) MBRT_DSR(2) MBRT_DSR(3) MBRT_DSR(4) MBRT_DSR(5) MBRT_DSR(6)
                         MBRT_DSR(7) "s_waitcnt lgkmcnt(0)"
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
                       "=&v"(v[7])
                     : [a] "v"(addr), MBRT_OFF(0), MBRT_OFF(1), MBRT_OFF(2), MBRT_OFF(3), MBRT_OFF(4), MBRT_OFF(5),
                       MBRT_OFF(6), MBRT_OFF(7)
                     : "memory");
    } else {
        asm volatile(MBRT_DSR(0) MBRT_DSR(1) MBRT_DSR(2) MBRT_DSR(3) MBRT_DSR(4) MBRT_DSR(5) MBRT_DSR(6)
                         MBRT_DSR(7) MBRT_DSR(8) MBRT_DSR(9) MBRT_DSR(10) MBRT_DSR(11) MBRT_DSR(12) MBRT_DSR(13)
                             MBRT_DSR(14) MBRT_DSR(15) "s_waitcnt lgkmcnt(0)"
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
                       "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]), "=&v"(v[12]),
                       "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15])
                     : [a] "v"(addr), MBRT_OFF(0), MBRT_OFF(1), MBRT_OFF(2), MBRT_OFF(3), MBRT_OFF(4), MBRT_OFF(5),
                       MBRT_OFF(6), MBRT_OFF(7), MBRT_OFF(8), MBRT_OFF(9), MBRT_OFF(10), MBRT_OFF(11),
                       MBRT_OFF(12), MBRT_OFF(13), MBRT_OFF(14), MBRT_OFF(15)
                     : "memory");
    }
#undef MBRT_DSR
#undef MBRT_OFF
}

// LDS byte address of a __shared__ object.
template <class T>
__device__ __forceinline__ uint32_t lds_addr(const T* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) T*)p;
}

// A wave-uniform load through the scalar data cache (constant address space): the
// address must be the same in every lane.  Used for small read-only tables (indices).
__device__ __forceinline__ int32_t scalar_load_i32(const void* base, int64_t i) {
    // global and constant address spaces share one 64-bit address on AMDGPU
    const const_i32* p = (const const_i32*)(uintptr_t)base;
    return p[i];
}

// MI355X deals the workgroups of a launch to its 8 XCDs round-robin (block p runs on XCD
// p % 8), and each XCD has its own L2.  xcd_tile maps the linear block id p of an n-block
// launch to a tile id so that every XCD walks one contiguous range of tile ids in order:
// neighbouring tiles, which share cache lines at their edges, then meet in one L2 instead
// of being fetched from HBM once per XCD.  The map is a bijection of [0, n).
constexpr uint32_t kXcds = 8;
__device__ __forceinline__ uint32_t xcd_tile(uint32_t p, uint32_t n) {
    const uint32_t x = p % kXcds, i = p / kXcds;
    const uint32_t q = n / kXcds, r = n % kXcds;
    return x < r ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
}

// Runs of G consecutive tiles per XCD, the launch as a whole still sweeping the tiles in
// order: within each group of 8*G blocks, XCD x takes tiles x*G .. x*G+G-1.  Blocks past
// the last whole group keep their own id.  A bijection of [0, n).
template <uint32_t G>
__device__ __forceinline__ uint32_t xcd_runs(uint32_t p, uint32_t n) {
    constexpr uint32_t kGroup = kXcds * G;
    if (G <= 1 || p >= n / kGroup * kGroup) return p;
    const uint32_t base = p / kGroup * kGroup, q = p % kGroup;
    return base + (q % kXcds) * G + q / kXcds;
}

// ---- wave64 reductions -----------------------------------------------------------
// Groups of G consecutive lanes (G in {1,2,4,8,16,32,64}) reduce together and every lane
// of a group receives the group's result.  Steps within a 16-lane row are DPP operand
// modifiers (quad_perm, row_half_mirror, row_mirror) fused into the add/max; the xor-16
// step is a ds_swizzle (BitMode, within 32 lanes); the last step of a full wave reads
// lanes 0 and 32 into scalar registers.  All 64 lanes must be active.

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float swz_xor16(float v) {
    // BitMode: and_mask 0x1f, or_mask 0, xor_mask 0x10 -> offset = (0x10 << 10) | 0x1f
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
__device__ __forceinline__ float lane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if (G >= 2) v += dpp<0xB1>(v);    // quad_perm [1,0,3,2]
    if (G >= 4) v += dpp<0x4E>(v);    // quad_perm [2,3,0,1]
    if (G >= 8) v += dpp<0x141>(v);   // row_half_mirror
    if (G >= 16) v += dpp<0x140>(v);  // row_mirror
    if (G >= 32) v += swz_xor16(v);
    if (G >= 64) v = lane_f(v, 0) + lane_f(v, 32);
    return v;
}

template <int G>
__device__ __forceinline__ float group_max(float v) {
    if (G >= 2) v = fmaxf(v, dpp<0xB1>(v));
    if (G >= 4) v = fmaxf(v, dpp<0x4E>(v));
    if (G >= 8) v = fmaxf(v, dpp<0x141>(v));
    if (G >= 16) v = fmaxf(v, dpp<0x140>(v));
    if (G >= 32) v = fmaxf(v, swz_xor16(v));
    if (G >= 64) v = fmaxf(lane_f(v, 0), lane_f(v, 32));
    return v;
}

// ---- dtype-templated vectors ------------------------------------------------------------
// Vec<DT, VE> holds VE elements of dtype DT as raw registers: load/store move them with
// one 8/16-byte (or two 16-byte) global access without touching the values, so a kernel
// can issue every load before its first use; to_f32/from_f32 convert afterwards.

// Non-temporal global accesses for data a kernel touches exactly once.  Kernels pick a
// policy per operand: bit 0 of an NT argument marks loads non-temporal, bit 1 stores.
template <int NT, class T>
__device__ __forceinline__ T gld(const T* p) {
    if constexpr ((NT & 1) != 0) return __builtin_nontemporal_load(p);
    else return *p;
}
template <int NT, class T>
__device__ __forceinline__ void gst(T* p, T v) {
    if constexpr ((NT & 2) != 0) __builtin_nontemporal_store(v, p);
    else *p = v;
}

template <int DT>
struct DtSize {
    static constexpr int value = DT == F32 ? 4 : 2;
};

template <int DT, int VE>
struct Vec {
    static constexpr int kBytes = VE * DtSize<DT>::value;
    static constexpr int kWords = kBytes / 4;
    uint32_t w[kWords];

    template <int NT = 0>
    __device__ __forceinline__ void load(const void* p, int64_t e) {
        const char* b = reinterpret_cast<const char*>(p) + e * DtSize<DT>::value;
        static_assert(kBytes == 4 || kBytes == 8 || kBytes % 16 == 0, "Vec: unsupported width");
        if constexpr (kBytes == 4) {
            w[0] = gld<NT>(reinterpret_cast<const uint32_t*>(b));
        } else if constexpr (kBytes == 8) {
            const u32x2 t = gld<NT>(reinterpret_cast<const u32x2*>(b));
            w[0] = t.x; w[1] = t.y;
        } else {
#pragma unroll
            for (int q = 0; q < kBytes / 16; ++q) {
                const u32x4 t = gld<NT>(reinterpret_cast<const u32x4*>(b) + q);
                w[4 * q] = t.x; w[4 * q + 1] = t.y; w[4 * q + 2] = t.z; w[4 * q + 3] = t.w;
            }
        }
    }
    template <int NT = 0>
    __device__ __forceinline__ void store(void* p, int64_t e) const {
        char* b = reinterpret_cast<char*>(p) + e * DtSize<DT>::value;
        if constexpr (kBytes == 4) {
            gst<NT>(reinterpret_cast<uint32_t*>(b), w[0]);
        } else if constexpr (kBytes == 8) {
            gst<NT>(reinterpret_cast<u32x2*>(b), u32x2{w[0], w[1]});
        } else {
#pragma unroll
            for (int q = 0; q < kBytes / 16; ++q)
                gst<NT>(reinterpret_cast<u32x4*>(b) + q, u32x4{w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]});
        }
    }
    __device__ __forceinline__ void to_f32(float (&f)[VE]) const {
#pragma unroll
        for (int i = 0; i < kWords; ++i) {
            if constexpr (DT == F32) {
                f[i] = __uint_as_float(w[i]);
            } else if constexpr (DT == BF16) {
                f[2 * i] = bf16_lo(w[i]);
                f[2 * i + 1] = bf16_hi(w[i]);
            } else {
                const f32x2 t = unpack_f16x2(w[i]);
                f[2 * i] = t.x;
                f[2 * i + 1] = t.y;
            }
        }
    }
    __device__ __forceinline__ void from_f32(const float (&f)[VE]) {
#pragma unroll
        for (int i = 0; i < kWords; ++i) {
            if constexpr (DT == F32) w[i] = __float_as_uint(f[i]);
            else if constexpr (DT == BF16) w[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
            else w[i] = pack_f16x2(f[2 * i], f[2 * i + 1]);
        }
    }
};

template <int DT, int NT = 0>
__device__ __forceinline__ float ld1(const void* p, int64_t i) {
    if constexpr (DT == F32) return gld<NT>(reinterpret_cast<const float*>(p) + i);
    const uint32_t h = gld<NT>(reinterpret_cast<const uint16_t*>(p) + i);
    if constexpr (DT == BF16) return __uint_as_float(h << 16);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <int DT, int NT = 0>
__device__ __forceinline__ void st1(void* p, int64_t i, float v) {
    if constexpr (DT == F32) gst<NT>(reinterpret_cast<float*>(p) + i, v);
    else if constexpr (DT == BF16) gst<NT>(reinterpret_cast<uint16_t*>(p) + i, f32_to_bf16_bits(v));
    else gst<NT>(reinterpret_cast<uint16_t*>(p) + i, f32_to_f16_bits(v));
}

// Runs f(std::integral_constant<int, DT>) for a float dtype code known at run time.
template <class Fn>
__host__ __device__ __forceinline__ void with_dt(int dt, Fn f) {
    if (dt == F32) f(std::integral_constant<int, F32>());
    else if (dt == BF16) f(std::integral_constant<int, BF16>());
    else f(std::integral_constant<int, F16>());
}

template <int DT>
__host__ __device__ constexpr int ve_for() { return DT == F32 ? 4 : 8; }

// ---- math ----------------------------------------------------------------------------

__device__ __forceinline__ float fast_exp(float x) { return __expf(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

__device__ __forceinline__ float sigmoidf(float x) { return fast_rcp(1.0f + fast_exp(-x)); }

// Rotary rotation of a pair: (x0, x1) -> (x0 c - x1 s, x0 s + x1 c), each product and the
// sum rounded separately (no FMA contraction), so that every kernel that rotates (the rotary
// kernels, the qkv split, the attention's in-kernel q rotation) rounds alike.
__device__ __forceinline__ void rotate_pair(float x0, float x1, float c, float s, float& y0, float& y1) {
#pragma clang fp contract(off)
    y0 = x0 * c - x1 * s;
    y1 = x0 * s + x1 * c;
}
template <int VE>
__device__ __forceinline__ void rotate(float (&x)[VE], const float (&c)[VE / 2], const float (&s)[VE / 2]) {
#pragma unroll
    for (int i = 0; i < VE / 2; ++i) rotate_pair(x[2 * i], x[2 * i + 1], c[i], s[i], x[2 * i], x[2 * i + 1]);
}

// GELU in the reference's form 0.5 x (1 + erf(x)) (mode 1) and the standard
// 0.5 x (1 + erf(x / sqrt 2)) (mode 2), both written as 0.5 x erfc(-z) so that the
// negative tail keeps full relative precision (1 + erf(z) cancels for z << 0).
__device__ __forceinline__ float gelu_ref(float x) { return 0.5f * x * erfcf(-x); }
__device__ __forceinline__ float gelu_std(float x) { return 0.5f * x * erfcf(-x * 0.70710678118654752440f); }

// erfc(-z) = 1 + erf(z) from Abramowitz & Stegun 7.1.26 (|error in erf| <= 1.5e-7):
// q = (a1 t + ... + a5 t^5) exp(-z^2), t = 1 / (1 + p |z|) approximates erfc(|z|), so
// 1 + erf(z) = q for z < 0 and 2 - q for z >= 0, with no cancellation in the tail.
// Used where the result is rounded to bf16/f16 (8/11-bit significands).
__device__ __forceinline__ float one_plus_erf_as(float z) {
    const float az = fabsf(z);
    const float t = fast_rcp(fmaf(0.3275911f, az, 1.0f));
    float p = fmaf(1.061405429f, t, -1.453152027f);
    p = fmaf(p, t, 1.421413741f);
    p = fmaf(p, t, -0.284496736f);
    p = fmaf(p, t, 0.254829592f);
    p *= t;
    const float q = p * __builtin_amdgcn_exp2f(-az * az * 1.44269504088896341f);
    return z < 0.0f ? q : 2.0f - q;
}
__device__ __forceinline__ float gelu_ref_lowp(float x) { return 0.5f * x * one_plus_erf_as(x); }
__device__ __forceinline__ float gelu_std_lowp(float x) {
    return 0.5f * x * one_plus_erf_as(x * 0.70710678118654752440f);
}

}  // namespace mbrt
