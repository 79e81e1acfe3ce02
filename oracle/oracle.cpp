// CPU restatement of the reference's tensor-op semantics — TEST INFRASTRUCTURE ONLY
// (see oracle.h).  Citations are paths inside baicai-1145/MBR-CUDA-Tile.
#include "oracle.h"

#include <omp.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstring>
#include <vector>

namespace {

enum { F32 = 0, F16 = 1, I64 = 2, BF16 = 3, I32 = 4 };

int g_threads = 1;

inline uint32_t fbits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float bitsf(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline int esize(int dt) { return dt == F32 || dt == I32 ? 4 : dt == I64 ? 8 : 2; }

// ---- rounding ---------------------------------------------------------------------------

// f32 -> bf16, round to nearest even on the bit pattern; NaN stays a (quiet) NaN.
inline uint16_t f32_to_bf16(float f) {
    uint32_t u = fbits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
inline float bf16_to_f32(uint16_t h) { return bitsf((uint32_t)h << 16); }

// f32 -> IEEE binary16, round to nearest even, with subnormals, overflow to inf.
inline uint16_t f32_to_f16(float f) {
    const uint32_t x = fbits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x0200u | ((ax >> 13) & 0x3ffu) : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // >= 65520 rounds to inf
    if (ax >= 0x38800000u) {                                   // normal binary16
        const uint32_t mant = ax & 0x7fffffu;
        uint32_t h = ((((ax >> 23) - 127u + 15u)) << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
        return (uint16_t)(sign | h);
    }
    if (ax <= 0x33000000u) return (uint16_t)sign;  // <= 2^-25 rounds to zero
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    const int shift = 126 - (int)(ax >> 23);
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return bitsf(sign);
        return (sign ? -1.0f : 1.0f) * std::ldexp((float)m, -24);
    }
    if (e == 31) return bitsf(sign | 0x7f800000u | (m << 13));
    return bitsf(sign | ((e - 15u + 127u) << 23) | (m << 13));
}

// Round a double once to a binary format with p significant bits, minimum normal
// exponent emin and largest finite value maxf (round half to even).
inline double round_fmt(double x, int p, int emin, double maxf) {
    if (!std::isfinite(x) || x == 0.0) return x;
    int e;
    std::frexp(x, &e);
    int lead = e - 1;
    if (lead < emin) lead = emin;
    const double q = std::ldexp(1.0, lead - (p - 1));
    const double r = std::nearbyint(x / q) * q;
    if (std::fabs(r) > maxf) return r > 0 ? INFINITY : -INFINITY;
    return r;
}
inline uint16_t f64_to_bf16(double v) {
    if (std::isnan(v)) return 0x7fc0u;
    return (uint16_t)(fbits((float)round_fmt(v, 8, -126, 3.3895313892515355e38)) >> 16);
}
inline uint16_t f64_to_f16(double v) {
    if (std::isnan(v)) return 0x7e00u;
    return f32_to_f16((float)round_fmt(v, 11, -14, 65504.0));
}

// ---- element access -----------------------------------------------------------------

inline float ld(const void* p, int dt, int64_t i) {
    switch (dt) {
        case F32: return static_cast<const float*>(p)[i];
        case BF16: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
        case F16: return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
        case I64: return (float)static_cast<const int64_t*>(p)[i];
        default: return (float)static_cast<const int32_t*>(p)[i];
    }
}

// store a double with a single rounding to the destination format
inline void st(void* p, int dt, int64_t i, double v) {
    switch (dt) {
        case F32: static_cast<float*>(p)[i] = (float)v; break;
        case BF16: static_cast<uint16_t*>(p)[i] = f64_to_bf16(v); break;
        case F16: static_cast<uint16_t*>(p)[i] = f64_to_f16(v); break;
        case I64: static_cast<int64_t*>(p)[i] = (int64_t)v; break;
        default: static_cast<int32_t*>(p)[i] = (int32_t)v; break;
    }
}
// store a float (the float-pipeline result) with a single rounding
inline void st(void* p, int dt, int64_t i, float v) {
    switch (dt) {
        case F32: static_cast<float*>(p)[i] = v; break;
        case BF16: static_cast<uint16_t*>(p)[i] = f32_to_bf16(v); break;
        case F16: static_cast<uint16_t*>(p)[i] = f32_to_f16(v); break;
        case I64: static_cast<int64_t*>(p)[i] = (int64_t)v; break;
        default: static_cast<int32_t*>(p)[i] = (int32_t)v; break;
    }
}
// One rounding of a double to the nearest bf16, widened back: an intermediate of the
// bf16-intermediates mode (the reference's bf16_round in full-bf16 mode).
inline double rb(double v) { return (double)bf16_to_f32(f64_to_bf16(v)); }

inline float round_through(float v, int dt) {
    if (dt == BF16) return bf16_to_f32(f32_to_bf16(v));
    if (dt == F16) return f16_to_f32(f32_to_f16(v));
    return v;
}

template <class A>
inline A sigmoid(A x) { return A(1) / (A(1) + std::exp(-x)); }

// Activation codes of the C-ABI: 1 GELU 0.5x(1+erf x) (the reference's kernels,
// src/mbr_cuda_tile.cu:5536-5584, 566-583), 2 GELU 0.5x(1+erf(x/sqrt2)), 3 sigmoid
// (5504-5534), 4 tanh (5840-5878).
template <class A>
inline A act(A v, int a) {
    switch (a) {
        case 1: return A(0.5) * v * (A(1) + std::erf(v));
        case 2: return A(0.5) * v * (A(1) + std::erf(v * A(0.70710678118654752440)));
        case 3: return sigmoid(v);
        case 4: return std::tanh(v);
        default: return v;
    }
}

// ---- RNG ------------------------------------------------------------------------------

inline uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
struct Xoshiro {
    uint64_t s[4];
    Xoshiro(uint64_t seed, uint64_t stream) {
        uint64_t sm = seed ^ (stream * 0xd1b54a32d192ed03ull);
        for (auto& v : s) v = splitmix64(sm);
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next() {
        const uint64_t r = rotl(s[1] * 5, 7) * 9;
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
    double uniform() {  // (0, 1)
        return ((double)(next() >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    }
};

}  // namespace

extern "C" {

void orc_set_threads(int n) { g_threads = n > 0 ? n : 1; }
int orc_get_threads(void) { return g_threads; }

void orc_randn(float* out, int64_t n, uint64_t seed, uint64_t stream, double mean, double stddev) {
    Xoshiro g(seed, stream);
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        const double u1 = g.uniform(), u2 = g.uniform();
        const double r = std::sqrt(-2.0 * std::log(u1));
        out[i] = (float)(mean + stddev * r * std::cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(mean + stddev * r * std::sin(two_pi * u2));
    }
}

void orc_randu64(uint64_t* out, int64_t n, uint64_t seed, uint64_t stream) {
    Xoshiro g(seed, stream);
    for (int64_t i = 0; i < n; ++i) out[i] = g.next();
}

void orc_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(in[i]);
}
void orc_bf16_to_f32(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf16_to_f32(in[i]);
}
void orc_f32_to_f16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16(in[i]);
}
void orc_f16_to_f32(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]);
}
void orc_f64_to_bf16(const double* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f64_to_bf16(in[i]);
}

// src/tensor_cuda_tile.cu:87-195: float narrowing rounds to nearest even, float -> int
// truncates, int -> float rounds.
void orc_convert(const void* src, int sdt, void* dst, int ddt, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        if (sdt == I64 || sdt == I32) {
            const int64_t v = sdt == I64 ? static_cast<const int64_t*>(src)[i] : static_cast<const int32_t*>(src)[i];
            if (ddt == I64) static_cast<int64_t*>(dst)[i] = v;
            else if (ddt == I32) static_cast<int32_t*>(dst)[i] = (int32_t)v;
            else st(dst, ddt, i, (float)v);
        } else {
            const float v = ld(src, sdt, i);
            if (ddt == I64) static_cast<int64_t*>(dst)[i] = (int64_t)v;
            else if (ddt == I32) static_cast<int32_t*>(dst)[i] = (int32_t)v;
            else st(dst, ddt, i, v);
        }
    }
}

// src/tensor_cuda_tile.cu:293-339: f32 arithmetic, rounded to the dtype on store.
static inline float binop(float x, float y, int op) {
    switch (op) {
        case 0: return x + y;
        case 1: return x - y;
        case 2: return x * y;
        default: return x / y;
    }
}

void orc_binary(const void* a, const void* b, void* out, int dt, int64_t n, int op) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t i = 0; i < n; ++i) st(out, dt, i, binop(ld(a, dt, i), ld(b, dt, i), op));
}

// src/tensor_cuda_glue.cu:57-114 (broadcast_offset over the output coordinates).
void orc_binary_broadcast(const void* a, const void* b, void* out, int dt, int ndim, const int64_t* shape,
                          const int64_t* sa, const int64_t* sb, int op) {
    int64_t total = 1;
    for (int d = 0; d < ndim; ++d) total *= shape[d];
    for (int64_t i = 0; i < total; ++i) {
        int64_t rem = i, oa = 0, ob = 0;
        for (int d = ndim - 1; d >= 0; --d) {
            const int64_t c = rem % shape[d];
            rem /= shape[d];
            oa += c * sa[d];
            ob += c * sb[d];
        }
        st(out, dt, i, binop(ld(a, dt, oa), ld(b, dt, ob), op));
    }
}

// src/tensor_cuda_glue.cu:146-188: dst[i] = src[sum_d coord_d(i) * stride_d].
void orc_strided_copy(const void* src, void* dst, int es, int ndim, const int64_t* shape, const int64_t* stride) {
    int64_t total = 1;
    for (int d = 0; d < ndim; ++d) total *= shape[d];
    const char* s = static_cast<const char*>(src);
    char* o = static_cast<char*>(dst);
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t i = 0; i < total; ++i) {
        int64_t rem = i, off = 0;
        for (int d = ndim - 1; d >= 0; --d) {
            off += (rem % shape[d]) * stride[d];
            rem /= shape[d];
        }
        std::memcpy(o + i * es, s + off * es, es);
    }
}

// src/tensor_cuda_glue.cu:116-144
void orc_index_select(const void* src, void* dst, int es, int ndim, const int64_t* shape, const int64_t* stride,
                      int sel, const int64_t* idx) {
    int64_t total = 1;
    for (int d = 0; d < ndim; ++d) total *= shape[d];
    const char* s = static_cast<const char*>(src);
    char* o = static_cast<char*>(dst);
    for (int64_t i = 0; i < total; ++i) {
        int64_t rem = i, off = 0;
        for (int d = ndim - 1; d >= 0; --d) {
            int64_t c = rem % shape[d];
            rem /= shape[d];
            if (d == sel) c = idx[c];
            off += c * stride[d];
        }
        std::memcpy(o + i * es, s + off * es, es);
    }
}

// src/tensor_cuda_glue.cu:415-491 (contiguous source; reflect: |c|, 2(n-1)-c, clamp).
void orc_pad(const void* src, void* dst, int dt, int ndim, const int64_t* ss, const int64_t* ds,
             const int64_t* before, float value, int reflect) {
    int64_t total = 1;
    for (int d = 0; d < ndim; ++d) total *= ds[d];
    const int es = esize(dt);
    std::vector<char> pad(es);
    st(pad.data(), dt, 0, value);
    const char* s = static_cast<const char*>(src);
    char* o = static_cast<char*>(dst);
    for (int64_t i = 0; i < total; ++i) {
        int64_t rem = i, lin = 0, pitch = 1;
        bool inside = true;
        for (int d = ndim - 1; d >= 0; --d) {
            int64_t c = rem % ds[d] - before[d];
            rem /= ds[d];
            const int64_t n = ss[d];
            if (reflect) {
                if (c < 0) c = -c;
                if (c >= n) c = 2 * (n - 1) - c;
                c = std::min<int64_t>(std::max<int64_t>(c, 0), n - 1);
            } else {
                inside = inside && c >= 0 && c < n;
            }
            lin += c * pitch;
            pitch *= n;
        }
        std::memcpy(o + i * es, inside ? s + lin * es : pad.data(), es);
    }
}

// Tensor::sum/max over the last dim (src/tensor_cuda_tile.cu:264-291).
void orc_reduce_last(const float* src, float* dst, int64_t outer, int64_t inner, int op, int mode) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t o = 0; o < outer; ++o) {
        const float* p = src + o * inner;
        if (op == 1) {
            float m = -INFINITY;
            for (int64_t i = 0; i < inner; ++i) m = std::max(m, p[i]);
            dst[o] = m;
        } else if (mode == ORC_EXACT) {
            double s = 0;
            for (int64_t i = 0; i < inner; ++i) s += p[i];
            dst[o] = (float)s;
        } else {
            float s = 0;
            for (int64_t i = 0; i < inner; ++i) s += p[i];
            dst[o] = s;
        }
    }
}

// src/tensor_cuda_glue.cu:518-557: sequential over r in f32 (bit-exact definition).
void orc_reduce_general(const float* src, float* dst, int64_t outer, int64_t reduce, int64_t inner, int op) {
    for (int64_t o = 0; o < outer; ++o) {
        for (int64_t i = 0; i < inner; ++i) {
            float v = op == 1 ? -INFINITY : 0.0f;
            for (int64_t r = 0; r < reduce; ++r) {
                const float x = src[(o * reduce + r) * inner + i];
                v = op == 1 ? std::max(v, x) : v + x;
            }
            dst[o * inner + i] = v;
        }
    }
}

// mbr_tile::rms_norm / try_residual_add_rms_norm (src/mbr_cuda_tile.cu:4791-4965, 6297-6417):
// s = round_to_sdt(x + res) (an f32 add, as the reference's add_ / fused kernel), then
// y = s * scale * gamma / sqrt(sum s^2 + eps).
void orc_rms_norm(const void* x, int xdt, const void* res, const void* gamma, int gdt, void* sum_out, int sdt,
                  void* out, int odt, int64_t rows, int64_t dim, float scale, float eps, int mode) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        std::vector<float> s(dim);
        const int64_t base = r * dim;
        for (int64_t d = 0; d < dim; ++d) {
            float v = ld(x, xdt, base + d);
            if (res) {
                v = round_through(v + ld(res, xdt, base + d), sdt);
                if (sum_out) st(sum_out, sdt, base + d, v);
            }
            s[d] = v;
        }
        if (mode == ORC_BF16I) {
            // src/mbr_cuda_tile.cu:4830-4843, 4890-4905
            double ss = 0;
            for (int64_t d = 0; d < dim; ++d) ss += rb(s[d]) * rb(s[d]);
            const double inv = rb(1.0 / std::sqrt(rb(ss) + (double)eps));
            for (int64_t d = 0; d < dim; ++d)
                st(out, odt, base + d, rb(rb(s[d]) * inv * rb(ld(gamma, gdt, d)) * (double)scale));
        } else if (mode == ORC_EXACT) {
            double ss = 0;
            for (int64_t d = 0; d < dim; ++d) ss += (double)s[d] * s[d];
            const double inv = 1.0 / std::sqrt(ss + (double)eps);
            for (int64_t d = 0; d < dim; ++d)
                st(out, odt, base + d, (double)s[d] * inv * (double)ld(gamma, gdt, d) * (double)scale);
        } else {
            float ss = 0;
            for (int64_t d = 0; d < dim; ++d) ss += s[d] * s[d];
            const float inv = scale / std::sqrt(ss + eps);
            for (int64_t d = 0; d < dim; ++d) st(out, odt, base + d, s[d] * inv * ld(gamma, gdt, d));
        }
    }
}

// Linear-layer epilogues add_bias* (src/mbr_cuda_tile.cu:5474-5584), tanh (5840-5878).
void orc_bias_act(const void* x, int xdt, const void* bias, int bdt, void* out, int odt, int64_t rows, int64_t cols,
                  int a, int mode) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < cols; ++c) {
            const int64_t i = r * cols + c;
            if (mode == ORC_EXACT) {
                double v = ld(x, xdt, i);
                if (bias) v += ld(bias, bdt, c);
                st(out, odt, i, act<double>(v, a));
            } else {
                float v = ld(x, xdt, i);
                if (bias) v += ld(bias, bdt, c);
                st(out, odt, i, act<float>(v, a));
            }
        }
    }
}

// glu_last_dim (src/mbr_cuda_tile.cu:5880-5942): out[r,d] = x[r,d] * sigmoid(x[r,H+d]).
void orc_glu(const void* x, int xdt, void* out, int odt, int64_t rows, int64_t half, int mode) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t d = 0; d < half; ++d) {
            const int64_t i = r * 2 * half + d;
            if (mode == ORC_BF16I)  // src/mbr_cuda_tile.cu:5933-5938
                st(out, odt, r * half + d, rb(rb(ld(x, xdt, i)) * rb(sigmoid<double>(rb(ld(x, xdt, i + half))))));
            else if (mode == ORC_EXACT)
                st(out, odt, r * half + d, (double)ld(x, xdt, i) * sigmoid<double>(ld(x, xdt, i + half)));
            else
                st(out, odt, r * half + d, ld(x, xdt, i) * sigmoid<float>(ld(x, xdt, i + half)));
        }
    }
}

// linear_sigmoid epilogue + apply_gates_and_merge_heads (src/mbr_cuda_tile.cu:4603-4789,
// 5504-5534): merged[b, n, h*D + d] = attn(b, h, n, d) * sigmoid(gate[b, n, h]).
void orc_gate_merge(const void* attn, int adt, const void* gate, int gdt, int logit, void* out, int odt, int64_t B,
                    int64_t H, int64_t N, int64_t D, int layout, int mode) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t tok = 0; tok < B * N; ++tok) {
        const int64_t b = tok / N, n = tok % N;
        for (int64_t h = 0; h < H; ++h) {
            const float gl = ld(gate, gdt, tok * H + h);
            const double gd = logit ? sigmoid<double>(gl) : (double)gl;
            const float gf = logit ? sigmoid<float>(gl) : gl;
            for (int64_t d = 0; d < D; ++d) {
                const int64_t src = layout == 0 ? ((b * H + h) * N + n) * D + d : (tok * H + h) * D + d;
                const int64_t dst = (tok * H + h) * D + d;
                if (mode == ORC_BF16I)  // src/mbr_cuda_tile.cu:4743-4746
                    st(out, odt, dst, rb(rb(ld(attn, adt, src)) * rb(gd)));
                else if (mode == ORC_EXACT) st(out, odt, dst, (double)ld(attn, adt, src) * gd);
                else st(out, odt, dst, ld(attn, adt, src) * gf);
            }
        }
    }
}

// scale_softmax* (src/mbr_cuda_tile.cu:5092-5285): z = scale*x; exp(z - max) / sum.
void orc_softmax(const void* in, int idt, void* out, int odt, int64_t rows, int64_t cols, float scale, int mode) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t base = r * cols;
        if (mode == ORC_BF16I) {
            // src/mbr_cuda_tile.cu:5237-5248
            std::vector<double> z(cols);
            double m = -INFINITY;
            for (int64_t c = 0; c < cols; ++c) {
                z[c] = rb(rb(ld(in, idt, base + c)) * (double)scale);
                m = std::max(m, z[c]);
            }
            m = rb(m);
            double s = 0;
            for (int64_t c = 0; c < cols; ++c) s += (z[c] = rb(std::exp(z[c] - m)));
            const double den = rb(s);
            for (int64_t c = 0; c < cols; ++c) st(out, odt, base + c, rb(z[c] / den));
        } else if (mode == ORC_EXACT) {
            std::vector<double> z(cols);
            double m = -INFINITY;
            for (int64_t c = 0; c < cols; ++c) {
                z[c] = (double)scale * ld(in, idt, base + c);
                m = std::max(m, z[c]);
            }
            double s = 0;
            for (int64_t c = 0; c < cols; ++c) s += (z[c] = std::exp(z[c] - m));
            for (int64_t c = 0; c < cols; ++c) st(out, odt, base + c, z[c] / s);
        } else {
            std::vector<float> z(cols);
            float m = -FLT_MAX;
            for (int64_t c = 0; c < cols; ++c) {
                z[c] = scale * ld(in, idt, base + c);
                m = std::max(m, z[c]);
            }
            float s = 0;
            for (int64_t c = 0; c < cols; ++c) s += (z[c] = std::exp(z[c] - m));
            const float inv = 1.0f / s;
            for (int64_t c = 0; c < cols; ++c) st(out, odt, base + c, z[c] * inv);
        }
    }
}

// MelBandRoformer::compute_rotary_cos_sin (src/model_mel_band_roformer.cu:270-300), in f32:
// freq = 1 / theta^(2i/dim), angle = n * freq, cos/sin of the f32 angle.
void orc_rotary_tables(float* cos_t, float* sin_t, int64_t seq, int64_t dim, float theta) {
    const int64_t half = dim / 2;
    for (int64_t n = 0; n < seq; ++n) {
        for (int64_t i = 0; i < half; ++i) {
            const float freq = 1.0f / std::pow(theta, (float)(2 * i) / (float)dim);
            const float angle = (float)n * freq;
            cos_t[n * half + i] = std::cos(angle);
            sin_t[n * half + i] = std::sin(angle);
        }
    }
}

// Interleaved-pair rotary (src/mbr_cuda_tile.cu:3897-4458, 4146-4208):
// (x0, x1) -> (x0 c - x1 s, x0 s + x1 c).  layout 0: [B*H, N, D]; 1: [B, N, H, D].
void orc_rotary(void* q, void* k, int dt, const void* cos_t, const void* sin_t, int tdt, int64_t rows, int64_t n_pos,
                int64_t heads, int64_t D, int layout, int mode) {
    const int64_t half = D / 2;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t n = (layout == 1 ? r / heads : r) % n_pos;
        for (int64_t i = 0; i < half; ++i) {
            float c = ld(cos_t, tdt, n * half + i), s = ld(sin_t, tdt, n * half + i);
            if (mode == ORC_BF16I) {  // src/mbr_cuda_tile.cu:4033-4060 (and its in-place variants)
                c = (float)rb(c);
                s = (float)rb(s);
            }
            for (int t = 0; t < 2; ++t) {
                void* buf = t == 0 ? q : k;
                if (!buf) continue;
                const int64_t e = r * D + 2 * i;
                float x0 = ld(buf, dt, e), x1 = ld(buf, dt, e + 1);
                if (mode == ORC_BF16I) {
                    x0 = (float)rb(x0);
                    x1 = (float)rb(x1);
                    st(buf, dt, e, rb((double)x0 * c - (double)x1 * s));
                    st(buf, dt, e + 1, rb((double)x0 * s + (double)x1 * c));
                } else if (mode == ORC_EXACT) {
                    st(buf, dt, e, (double)x0 * c - (double)x1 * s);
                    st(buf, dt, e + 1, (double)x0 * s + (double)x1 * c);
                } else {
                    st(buf, dt, e, x0 * c - x1 * s);
                    st(buf, dt, e + 1, x0 * s + x1 * c);
                }
            }
        }
    }
}

// split_qkv_heads_rotary (src/mbr_cuda_tile.cu:3897-4068, 4379-4552): [B, N, 3HD] ->
// q, k, v [B, H, out_n, D]; rows n >= N are zero.
void orc_split_qkv(const void* qkv, int idt, const void* cos_t, const void* sin_t, int tdt, void* q, void* k, void* v,
                   int odt, int64_t B, int64_t N, int64_t H, int64_t D, int64_t out_n, int mode) {
    const int64_t half = D / 2;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t h = 0; h < H; ++h)
            for (int64_t n = 0; n < out_n; ++n)
                for (int64_t i = 0; i < half; ++i) {
                    const int64_t e = ((b * H + h) * out_n + n) * D + 2 * i;
                    if (n >= N) {
                        for (void* dst : {q, k, v}) {
                            st(dst, odt, e, 0.0f);
                            st(dst, odt, e + 1, 0.0f);
                        }
                        continue;
                    }
                    const int64_t src = (b * N + n) * 3 * H * D + h * D + 2 * i;
                    float c = ld(cos_t, tdt, n * half + i), s = ld(sin_t, tdt, n * half + i);
                    if (mode == ORC_BF16I) {  // src/mbr_cuda_tile.cu:4033-4060
                        c = (float)rb(c);
                        s = (float)rb(s);
                    }
                    for (int part = 0; part < 3; ++part) {
                        void* dst = part == 0 ? q : part == 1 ? k : v;
                        const float x0 = ld(qkv, idt, src + part * H * D), x1 = ld(qkv, idt, src + part * H * D + 1);
                        if (part == 2) {
                            st(dst, odt, e, x0);
                            st(dst, odt, e + 1, x1);
                        } else if (mode == ORC_BF16I) {
                            const double y0 = rb(x0), y1 = rb(x1);
                            st(dst, odt, e, rb(y0 * c - y1 * s));
                            st(dst, odt, e + 1, rb(y0 * s + y1 * c));
                        } else if (mode == ORC_EXACT) {
                            st(dst, odt, e, (double)x0 * c - (double)x1 * s);
                            st(dst, odt, e + 1, (double)x0 * s + (double)x1 * c);
                        } else {
                            st(dst, odt, e, x0 * c - x1 * s);
                            st(dst, odt, e + 1, x0 * s + x1 * c);
                        }
                    }
                }
}

// Slaney mel scale (librosa.core.convert.hz_to_mel / mel_to_hz, htk=False).
static double hz_to_mel(double f) {
    const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp;
    const double logstep = std::log(6.4) / 27.0;
    if (f >= min_log_hz) return min_log_mel + std::log(f / min_log_hz) / logstep;
    return f / f_sp;
}
static double mel_to_hz(double m) {
    const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp;
    const double logstep = std::log(6.4) / 27.0;
    if (m >= min_log_mel) return min_log_hz * std::exp(logstep * (m - min_log_mel));
    return f_sp * m;
}

// Band layout of MelBandRoformer: support of librosa.filters.mel(sr, n_fft, n_mels) with
// [0][0] and [-1][-1] set to 1; stereo interleaves 2*bin + ch.  The reference consumes
// the result as __precomputed__.freq_indices / num_freqs_per_band / num_bands_per_freq
// and builds the per-freq CSR itself (src/model_mel_band_roformer.cu:79-150).
int64_t orc_mel_bands(double sr, int n_fft, int n_bands, int C, int32_t* freq_indices, int32_t* freqs_per_band,
                      int32_t* bands_per_freq, int32_t* csr_offsets, int32_t* csr_indices) {
    const int bins = n_fft / 2 + 1;
    std::vector<double> fft(bins), melf(n_bands + 2);
    for (int i = 0; i < bins; ++i) fft[i] = (sr / 2.0) * i / (bins - 1);
    const double m0 = hz_to_mel(0.0), m1 = hz_to_mel(sr / 2.0);
    for (int i = 0; i < n_bands + 2; ++i) melf[i] = mel_to_hz(m0 + (m1 - m0) * i / (n_bands + 1));
    std::vector<std::vector<char>> sup(n_bands, std::vector<char>(bins, 0));
    for (int b = 0; b < n_bands; ++b) {
        const double fd0 = melf[b + 1] - melf[b], fd1 = melf[b + 2] - melf[b + 1];
        const double enorm = 2.0 / (melf[b + 2] - melf[b]);
        for (int f = 0; f < bins; ++f) {
            const double lower = -(melf[b] - fft[f]) / fd0;
            const double upper = (melf[b + 2] - fft[f]) / fd1;
            const float w = (float)(std::max(0.0, std::min(lower, upper)) * enorm);  // float32 weights
            sup[b][f] = w > 0.0f;
        }
    }
    sup[0][0] = 1;
    sup[n_bands - 1][bins - 1] = 1;
    int64_t J = 0;
    for (int b = 0; b < n_bands; ++b)
        for (int f = 0; f < bins; ++f) J += sup[b][f] ? C : 0;
    if (!freq_indices) return J;
    int64_t j = 0;
    std::vector<std::vector<int32_t>> by_freq(bins * C);
    for (int b = 0; b < n_bands; ++b) {
        int32_t cnt = 0;
        for (int f = 0; f < bins; ++f) {
            if (!sup[b][f]) continue;
            ++cnt;
            for (int c = 0; c < C; ++c) {
                freq_indices[j] = f * C + c;
                by_freq[f * C + c].push_back((int32_t)j);
                ++j;
            }
        }
        if (freqs_per_band) freqs_per_band[b] = cnt;
    }
    int32_t e = 0;
    for (int fr = 0; fr < bins * C; ++fr) {
        if (bands_per_freq) bands_per_freq[fr] = (int32_t)by_freq[fr].size();
        if (csr_offsets) csr_offsets[fr] = e;
        for (int32_t jj : by_freq[fr]) {
            if (csr_indices) csr_indices[e] = jj;
            ++e;
        }
    }
    if (csr_offsets) csr_offsets[bins * C] = e;
    return J;
}

// gather_freqs_fold_complex (src/mbr_cuda_tile.cu:4554-4601): out[b,t,j,c] = stft[b,idx[j],t,c].
// An index outside [0, F) reads the nearest valid row (the library's contract; the
// reference leaves such indices undefined).
void orc_band_gather(const float* stft, const int32_t* idx, void* out, int odt, int64_t B, int64_t F, int64_t T,
                     int64_t J) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t bt = 0; bt < B * T; ++bt) {
        const int64_t b = bt / T, t = bt % T;
        for (int64_t j = 0; j < J; ++j) {
            const int64_t f = std::min<int64_t>(std::max<int64_t>(idx[j], 0), F - 1);
            const float* s = stft + ((b * F + f) * T + t) * 2;
            const int64_t o = (bt * J + j) * 2;
            st(out, odt, o, s[0]);
            st(out, odt, o + 1, s[1]);
        }
    }
}

// apply_mask_and_scatter (src/mbr_cuda_tile.cu:5586-5803, 7951-8081), written per output:
// out[(b*S+s)*C+ch, bin, t] = (sum_{e in CSR[freq], ascending} stft[b,freq,t] * mask_s[b,t,ind[e]])
//                              / max(count[freq], 1e-8),   freq = bin*C + ch.
void orc_band_mask_merge(const float* stft, const void* const* masks, int mdt, int S, const int32_t* off,
                         const int32_t* ind, const void* cnt, int cdt, void* out, int odt, int64_t B, int64_t F,
                         int64_t T, int64_t J, int64_t C, int mode) {
    const int64_t bins = F / C;
    const float eps = 1.0e-8f;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t bsf = 0; bsf < B * S * F; ++bsf) {
        const int64_t f = bsf % F, bs = bsf / F, s = bs % S, b = bs / S;
        const int64_t bin = f / C, ch = f % C;
        const float cf = ld(cnt, cdt, f);
        const float den = cf > eps ? cf : eps;
        for (int64_t t = 0; t < T; ++t) {
            const float* sv = stft + ((b * F + f) * T + t) * 2;
            const int64_t o = ((((b * S + s) * C + ch) * bins + bin) * T + t) * 2;
            if (mode == ORC_BF16I && odt == BF16) {
                // reduce form, src/mbr_cuda_tile.cu:5771-5799: sum the masks, rounding each sum
                double mr = 0, mm = 0;
                for (int32_t e = off[f]; e < off[f + 1]; ++e) {
                    const int64_t mi = ((b * T + t) * J + ind[e]) * 2;
                    mr = rb(mr + rb(ld(masks[s], mdt, mi)));
                    mm = rb(mm + rb(ld(masks[s], mdt, mi + 1)));
                }
                st(out, odt, o, rb(((double)sv[0] * mr - (double)sv[1] * mm) / den));
                st(out, odt, o + 1, rb(((double)sv[0] * mm + (double)sv[1] * mr) / den));
            } else if (mode == ORC_BF16I) {
                // scatter form, src/mbr_cuda_tile.cu:5702-5717: each entry's value is rounded,
                // then added (here in ascending entry order)
                double ar = 0, ai = 0;
                for (int32_t e = off[f]; e < off[f + 1]; ++e) {
                    const int64_t mi = ((b * T + t) * J + ind[e]) * 2;
                    const double mr = rb(ld(masks[s], mdt, mi)), mm = rb(ld(masks[s], mdt, mi + 1));
                    ar += rb(((double)sv[0] * mr - (double)sv[1] * mm) / den);
                    ai += rb(((double)sv[0] * mm + (double)sv[1] * mr) / den);
                }
                st(out, odt, o, ar);
                st(out, odt, o + 1, ai);
            } else if (mode == ORC_EXACT) {
                double ar = 0, ai = 0;
                for (int32_t e = off[f]; e < off[f + 1]; ++e) {
                    const int64_t mi = ((b * T + t) * J + ind[e]) * 2;
                    const double mr = ld(masks[s], mdt, mi), mm = ld(masks[s], mdt, mi + 1);
                    ar += (double)sv[0] * mr - (double)sv[1] * mm;
                    ai += (double)sv[0] * mm + (double)sv[1] * mr;
                }
                st(out, odt, o, ar / den);
                st(out, odt, o + 1, ai / den);
            } else {
                float ar = 0, ai = 0;
                for (int32_t e = off[f]; e < off[f + 1]; ++e) {
                    const int64_t mi = ((b * T + t) * J + ind[e]) * 2;
                    const float mr = ld(masks[s], mdt, mi), mm = ld(masks[s], mdt, mi + 1);
                    ar += sv[0] * mr - sv[1] * mm;
                    ai += sv[0] * mm + sv[1] * mr;
                }
                const float inv = 1.0f / den;
                st(out, odt, o, ar * inv);
                st(out, odt, o + 1, ai * inv);
            }
        }
    }
    (void)J;
}

// zero_dc (src/mbr_cuda_tile.cu:5805-5838, 8083-8096): bin 0 of [outer, bins, T, 2] := 0.
void orc_zero_dc(void* spec, int dt, int64_t outer, int64_t bins, int64_t T) {
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t i = 0; i < T * 2; ++i) st(spec, dt, o * bins * T * 2 + i, 0.0f);
}

// Attention (src/mbr_cuda_tile.cu:6530-6709): s_ij = scale * q_i . k_j, p = softmax_j(s),
// out_i = sum_j p_ij v_j; scale 0 means 1 / sqrt(D).  EXACT: double throughout, one
// rounding of the output.  FAST: float scores and sums, probabilities rounded to bf16
// before the second product (the reference's bf16 attention), the CPU baseline's pipeline.
void orc_attention(const void* q, const void* k, const void* v, int dt, void* out, int odt, int64_t BH,
                   int64_t nq, int64_t nk, int64_t D, float scale, int mode) {
    const double sc = scale == 0.0f ? 1.0 / std::sqrt((double)D) : (double)scale;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int64_t r = 0; r < BH * nq; ++r) {
        const int64_t bh = r / nq;
        const int64_t qb = r * D, kb0 = bh * nk * D;
        std::vector<double> s((size_t)nk);
        std::vector<float> qf((size_t)D);
        for (int64_t d = 0; d < D; ++d) qf[d] = ld(q, dt, qb + d);
        double m = -INFINITY;
        for (int64_t j = 0; j < nk; ++j) {
            double acc = 0.0;
            if (mode == ORC_EXACT) {
                for (int64_t d = 0; d < D; ++d) acc += (double)qf[d] * (double)ld(k, dt, kb0 + j * D + d);
            } else {
                float fa = 0.0f;
                for (int64_t d = 0; d < D; ++d) fa += qf[d] * ld(k, dt, kb0 + j * D + d);
                acc = fa;
            }
            s[j] = acc * sc;
            m = std::max(m, s[j]);
        }
        double l = 0.0;
        for (int64_t j = 0; j < nk; ++j) {
            s[j] = mode == ORC_EXACT ? std::exp(s[j] - m) : (double)std::exp((float)(s[j] - m));
            l += s[j];
        }
        for (int64_t d = 0; d < D; ++d) {
            double acc = 0.0;
            for (int64_t j = 0; j < nk; ++j) {
                const double p = mode == ORC_EXACT ? s[j] : (double)bf16_to_f32(f32_to_bf16((float)s[j]));
                acc += p * (double)ld(v, dt, kb0 + j * D + d);
            }
            if (mode == ORC_EXACT) st(out, odt, r * D + d, acc / l);
            else st(out, odt, r * D + d, (float)(acc / l));
        }
    }
}

// The reference's arithmetic of P in the time attention (src/mbr_time_attention_cutile.cu:
// 160-180), in double: keys in tiles of 64 (one of its KTile choices); the running max
// m moves to the max of each tile's scaled scores; P = exp(s - m) is rounded once to bf16
// for the P V sum while the row sum l adds the unrounded P; both are rescaled by
// exp(m_old - m_new); out = O / l rounded once to odt.
void orc_attention_ref_p_ex(const void* q, const void* k, const void* v, int dt, void* out, int odt, int64_t BH,
                            int64_t nq, int64_t nk, int64_t D, float scale, double lazy, int sum_rounded) {
    const double sc = scale == 0.0f ? 1.0 / std::sqrt((double)D) : (double)scale;
    const int64_t kTile = 64;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int64_t r = 0; r < BH * nq; ++r) {
        const int64_t bh = r / nq;
        const int64_t qb = r * D, kb0 = bh * nk * D;
        std::vector<double> s((size_t)kTile), o((size_t)D, 0.0);
        double m = -INFINITY, l = 0.0;
        for (int64_t k0 = 0; k0 < nk; k0 += kTile) {
            const int64_t n = std::min(kTile, nk - k0);
            double tm = -INFINITY;
            for (int64_t j = 0; j < n; ++j) {
                double acc = 0.0;
                for (int64_t d = 0; d < D; ++d)
                    acc += (double)ld(q, dt, qb + d) * (double)ld(k, dt, kb0 + (k0 + j) * D + d);
                s[j] = acc * sc;
                tm = std::max(tm, s[j]);
            }
            // the running max moves to the tile's max when that exceeds it by more than
            // `lazy` (0: every tile, the exact running max)
            const double mn = tm > m + lazy ? tm : m;
            const double alpha = std::exp(m - mn);
            l *= alpha;
            for (int64_t d = 0; d < D; ++d) o[d] *= alpha;
            m = mn;
            for (int64_t j = 0; j < n; ++j) {
                const double p = std::exp(s[j] - m);
                const double pb = (double)bf16_to_f32(f64_to_bf16(p));
                l += sum_rounded ? pb : p;
                for (int64_t d = 0; d < D; ++d) o[d] += pb * (double)ld(v, dt, kb0 + (k0 + j) * D + d);
            }
        }
        for (int64_t d = 0; d < D; ++d) st(out, odt, r * D + d, o[d] / l);
    }
}

void orc_attention_ref_p(const void* q, const void* k, const void* v, int dt, void* out, int odt, int64_t BH,
                         int64_t nq, int64_t nk, int64_t D, float scale) {
    orc_attention_ref_p_ex(q, k, v, dt, out, odt, BH, nq, nk, D, scale, 0.0, 0);
}

}  // extern "C"
