// Device-side building blocks shared by every gfx950 kernel of the library:
// dtype-generic vector I/O (16-byte global loads/stores), bf16/f16 round-to-nearest-even
// packing, fast division by run-time invariant integers, and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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

// ---- wave64 reductions -----------------------------------------------------------
// Groups of G consecutive lanes (G in {1,2,4,8,16,32,64}) reduce together; every lane
// of a group receives the group's result.  xor-butterfly through ds_swizzle/bpermute
// is left to __shfl_xor, which the compiler lowers to DPP where the pattern allows.

template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// ---- math ----------------------------------------------------------------------------

__device__ __forceinline__ float fast_exp(float x) { return __expf(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

__device__ __forceinline__ float sigmoidf(float x) { return fast_rcp(1.0f + fast_exp(-x)); }

// GELU in the reference's form 0.5 x (1 + erf(x)) (mode 1) and the standard
// 0.5 x (1 + erf(x / sqrt 2)) (mode 2).
__device__ __forceinline__ float gelu_ref(float x) { return 0.5f * x * (1.0f + erff(x)); }
__device__ __forceinline__ float gelu_std(float x) {
    return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}

__device__ __forceinline__ float apply_act(float v, int act) {
    switch (act) {
        case 1: return gelu_ref(v);
        case 2: return gelu_std(v);
        case 3: return sigmoidf(v);
        case 4: return tanhf(v);
        default: return v;
    }
}

}  // namespace mbrt
