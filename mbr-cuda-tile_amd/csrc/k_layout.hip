// Layout kernels: strided copy (permute / contiguous / clone of views), index_select,
// constant and reflect pad, concatenation.  All copies are bit-exact byte moves.
//
// Strided copy strategy (replaces tensor_tile::strided_copy_glue,
// src/tensor_cuda_glue.cu:146-188, 615-638, which divides/modulos every element over
// all dims and uploads its metadata with a synchronous H2D memcpy):
//   1. drop size-1 dims and merge dims that are contiguous in the source;
//   2. if the innermost remaining dim has source stride 1, every output row is a
//      contiguous run in both tensors: copy it with the widest vector (16/8/4/2/1 B)
//      that divides the run, the source row pitches and both base addresses;
//   3. otherwise, if one source dim is unit-stride, stage 64x64-element tiles through
//      LDS so that both the read and the write are coalesced;
//   4. otherwise copy element by element.
// The bf16 [4,801,60,384] <-> [4,60,801,384] permute takes path 2 with 768-byte rows of
// 16-byte vectors.
#include "abi_common.hpp"

#include <algorithm>
#include <cstring>
#include <vector>

namespace mbrt {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxOuter = MBRT_MAX_DIMS;

template <int W>
struct WordOf;
template <> struct WordOf<16> { typedef u32x4 T; };
template <> struct WordOf<8> { typedef u32x2 T; };
template <> struct WordOf<4> { typedef uint32_t T; };
template <> struct WordOf<2> { typedef uint16_t T; };
template <> struct WordOf<1> { typedef uint8_t T; };

// Simplified view of a copy: output is contiguous with shape `shape` (outermost first),
// the source element (c_0..c_{n-1}) lives at sum c_d * stride[d] (elements).
struct Dims {
    int nd = 0;
    int64_t shape[kMaxOuter];
    int64_t stride[kMaxOuter];
};

Dims simplify(const int64_t* shape, const int64_t* stride, int nd) {
    Dims r;
    for (int d = 0; d < nd; ++d) {
        if (shape[d] == 1) continue;
        if (r.nd > 0 && r.stride[r.nd - 1] == stride[d] * shape[d]) {
            r.shape[r.nd - 1] *= shape[d];
            r.stride[r.nd - 1] = stride[d];
        } else {
            r.shape[r.nd] = shape[d];
            r.stride[r.nd] = stride[d];
            ++r.nd;
        }
    }
    if (r.nd == 0) {
        r.nd = 1;
        r.shape[0] = 1;
        r.stride[0] = 1;
    }
    return r;
}

// ---- path 2: contiguous runs --------------------------------------------------------

struct RowCopyArgs {
    const char* src;
    char* dst;
    uint32_t total_vec;      // rows * vectors per row
    FastDiv vpr;             // vectors per row
    int64_t dst_pitch;       // output row pitch in bytes
    int nd;                  // number of outer dims
    FastDiv outer[kMaxOuter];        // outer dim extents, innermost first
    int64_t outer_stride[kMaxOuter]; // source pitch in bytes, innermost first
};

template <int W, int U>
__global__ __launch_bounds__(kThreads) void row_copy_kernel(RowCopyArgs a) {
    typedef typename WordOf<W>::T Word;
    const uint32_t base = blockIdx.x * (kThreads * U) + threadIdx.x;
    Word v[U];
    int64_t dst_off[U];
    // all loads first (index clamped into the copy), then predicated stores
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t i = min(base + u * kThreads, a.total_vec - 1);
        uint32_t row, col;
        fdivmod(i, a.vpr, row, col);
        int64_t off = (int64_t)col * W;
        dst_off[u] = (int64_t)row * a.dst_pitch + (int64_t)col * W;
#pragma unroll
        for (int d = 0; d < kMaxOuter; ++d) {
            if (d < a.nd) {
                uint32_t q, r;
                fdivmod(row, a.outer[d], q, r);
                off += (int64_t)r * a.outer_stride[d];
                row = q;
            }
        }
        v[u] = gld<MBRT_NT_ROW>(reinterpret_cast<const Word*>(a.src + off));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (base + u * kThreads < a.total_vec) gst<MBRT_NT_ROW>(reinterpret_cast<Word*>(a.dst + dst_off[u]), v[u]);
    }
}

// 64-bit fallback for copies of more than 2^32 vectors.
struct RowCopyArgs64 {
    const char* src;
    char* dst;
    int64_t total_vec;
    int64_t vpr;
    int64_t dst_pitch;
    int nd;
    int64_t outer[kMaxOuter];
    int64_t outer_stride[kMaxOuter];
};

template <int W>
__global__ __launch_bounds__(kThreads) void row_copy_kernel64(RowCopyArgs64 a) {
    typedef typename WordOf<W>::T Word;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t step = (int64_t)gridDim.x * kThreads;
    for (; i < a.total_vec; i += step) {
        int64_t row = i / a.vpr;
        const int64_t col_bytes = (i - row * a.vpr) * W;
        const int64_t dst_off = row * a.dst_pitch + col_bytes;
        int64_t off = col_bytes;
        for (int d = 0; d < a.nd; ++d) {
            int64_t q = row / a.outer[d];
            off += (row - q * a.outer[d]) * a.outer_stride[d];
            row = q;
        }
        *reinterpret_cast<Word*>(a.dst + dst_off) = *reinterpret_cast<const Word*>(a.src + off);
    }
}

template <int W>
int launch_row_copy(const char* src, char* dst, const Dims& dm, int esize, int64_t dst_pitch,
                    hipStream_t st) {
    const int64_t run_bytes = dm.shape[dm.nd - 1] * esize;
    const int64_t vpr = run_bytes / W;
    int64_t rows = 1;
    for (int d = 0; d < dm.nd - 1; ++d) rows *= dm.shape[d];
    const int64_t total = rows * vpr;
    bool small = total < (1ll << 31) && vpr < (1ll << 31);  // 32-bit vector indices cannot wrap
    for (int d = 0; d < dm.nd - 1; ++d) small = small && dm.shape[d] < (1ll << 31);
    if (small) {
        RowCopyArgs a;
        a.src = src;
        a.dst = dst;
        a.total_vec = (uint32_t)total;
        a.vpr = make_fastdiv((uint32_t)vpr);
        a.dst_pitch = dst_pitch;
        a.nd = dm.nd - 1;
        for (int d = 0; d < a.nd; ++d) {
            int src_d = dm.nd - 2 - d;
            a.outer[d] = make_fastdiv((uint32_t)dm.shape[src_d]);
            a.outer_stride[d] = dm.stride[src_d] * esize;
        }
        constexpr int U = MBRT_ROW_U;
        int64_t grid = ceil_div(total, (int64_t)kThreads * U);
        hipLaunchKernelGGL((row_copy_kernel<W, U>), dim3((unsigned)grid), dim3(kThreads), 0, st, a);
    } else {
        RowCopyArgs64 a;
        a.src = src;
        a.dst = dst;
        a.total_vec = total;
        a.vpr = vpr;
        a.dst_pitch = dst_pitch;
        a.nd = dm.nd - 1;
        for (int d = 0; d < a.nd; ++d) {
            int src_d = dm.nd - 2 - d;
            a.outer[d] = dm.shape[src_d];
            a.outer_stride[d] = dm.stride[src_d] * esize;
        }
        int64_t grid = std::min<int64_t>(ceil_div(total, kThreads), 1 << 20);
        hipLaunchKernelGGL((row_copy_kernel64<W>), dim3((unsigned)grid), dim3(kThreads), 0, st, a);
    }
    return MBRT_OK;
}

// ---- path 3: LDS-tiled transpose ----------------------------------------------------
// The copy is viewed as out[batch, p, m, q] = in(batch, p, m, q) where q is the
// innermost output dim (source stride sq != 1) and p is the output dim that is
// unit-stride in the source.  A 64x64 tile over (p, q) is read along p (coalesced in
// the source) and written along q (coalesced in the output).  `batch` and `m`
// enumerate the remaining dims (outer to p, and between p and q).

constexpr int kTile = 64;

struct TransposeArgs {
    const char* src;
    char* dst;
    int64_t P, Q;                 // extents of p and q
    int64_t sq;                   // source stride of q (elements); source stride of p is 1
    int64_t out_p_pitch;          // output stride of p (elements) = M * Q
    int nb;                       // number of "other" dims (batch and m together)
    int64_t other_shape[kMaxOuter];
    int64_t other_src_stride[kMaxOuter];
    int64_t other_dst_stride[kMaxOuter];
    int64_t tiles_p, tiles_q;
};

template <int E>
__global__ __launch_bounds__(kThreads) void transpose_kernel(TransposeArgs a) {
    typedef typename WordOf<E>::T Elem;
    __shared__ Elem tile[kTile][kTile + 1];
    int64_t t = blockIdx.x;
    const int64_t tq = t % a.tiles_q;
    t /= a.tiles_q;
    const int64_t tp = t % a.tiles_p;
    t /= a.tiles_p;
    int64_t src_base = 0, dst_base = 0;
    for (int d = a.nb - 1; d >= 0; --d) {
        int64_t c = t % a.other_shape[d];
        t /= a.other_shape[d];
        src_base += c * a.other_src_stride[d];
        dst_base += c * a.other_dst_stride[d];
    }
    const int64_t p0 = tp * kTile, q0 = tq * kTile;
    const int lane = threadIdx.x % kTile;
    const int grp = threadIdx.x / kTile;  // 4 groups of 64
    // read: for each q row of the tile, 64 consecutive p (unit stride in source)
    for (int r = grp; r < kTile; r += kThreads / kTile) {
        int64_t p = p0 + lane, q = q0 + r;
        if (p < a.P && q < a.Q) {
            tile[r][lane] = gld<MBRT_NT_TR>(reinterpret_cast<const Elem*>(a.src) + src_base + q * a.sq + p);
        }
    }
    __syncthreads();
    // write: for each p row of the tile, 64 consecutive q (unit stride in output)
    for (int r = grp; r < kTile; r += kThreads / kTile) {
        int64_t p = p0 + r, q = q0 + lane;
        if (p < a.P && q < a.Q) {
            gst<MBRT_NT_TR>(reinterpret_cast<Elem*>(a.dst) + dst_base + p * a.out_p_pitch + q, tile[lane][r]);
        }
    }
}

// ---- path 4: generic element copy --------------------------------------------------

struct ElemCopyArgs {
    const char* src;
    char* dst;
    int64_t total;
    int nd;
    int64_t shape[kMaxOuter];   // outermost first
    int64_t stride[kMaxOuter];  // elements
};

template <int E>
__global__ __launch_bounds__(kThreads) void elem_copy_kernel(ElemCopyArgs a) {
    typedef typename WordOf<E>::T Elem;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t step = (int64_t)gridDim.x * kThreads;
    for (; i < a.total; i += step) {
        int64_t rem = i, off = 0;
        for (int d = a.nd - 1; d >= 0; --d) {
            int64_t q = rem / a.shape[d];
            off += (rem - q * a.shape[d]) * a.stride[d];
            rem = q;
        }
        reinterpret_cast<Elem*>(a.dst)[i] = reinterpret_cast<const Elem*>(a.src)[off];
    }
}

int launch_elem_copy(const void* src, void* dst, const Dims& dm, int esize, hipStream_t st) {
    ElemCopyArgs a;
    a.src = static_cast<const char*>(src);
    a.dst = static_cast<char*>(dst);
    a.nd = dm.nd;
    a.total = 1;
    for (int d = 0; d < dm.nd; ++d) {
        a.shape[d] = dm.shape[d];
        a.stride[d] = dm.stride[d];
        a.total *= dm.shape[d];
    }
    int64_t grid = std::min<int64_t>(ceil_div(a.total, kThreads), 1 << 20);
    switch (esize) {
        case 1: hipLaunchKernelGGL(elem_copy_kernel<1>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        case 2: hipLaunchKernelGGL(elem_copy_kernel<2>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        case 4: hipLaunchKernelGGL(elem_copy_kernel<4>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        default: hipLaunchKernelGGL(elem_copy_kernel<8>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
    }
    return MBRT_OK;
}

// Try the tiled transpose: needs a unit-stride source dim p that is not the innermost.
bool try_transpose(const void* src, void* dst, const Dims& dm, int esize, hipStream_t st) {
    const int q = dm.nd - 1;
    int p = -1;
    for (int d = 0; d < q; ++d) {
        if (dm.stride[d] == 1) p = d;
    }
    if (p < 0 || dm.shape[p] < 16 || dm.shape[q] < 16) return false;
    TransposeArgs a;
    a.src = static_cast<const char*>(src);
    a.dst = static_cast<char*>(dst);
    a.P = dm.shape[p];
    a.Q = dm.shape[q];
    a.sq = dm.stride[q];
    // output strides (contiguous, outermost first)
    int64_t ostride[kMaxOuter];
    int64_t acc = 1;
    for (int d = dm.nd - 1; d >= 0; --d) {
        ostride[d] = acc;
        acc *= dm.shape[d];
    }
    a.out_p_pitch = ostride[p];
    a.nb = 0;
    for (int d = 0; d < dm.nd; ++d) {
        if (d == p || d == q) continue;
        a.other_shape[a.nb] = dm.shape[d];
        a.other_src_stride[a.nb] = dm.stride[d];
        a.other_dst_stride[a.nb] = ostride[d];
        ++a.nb;
    }
    a.tiles_p = ceil_div(a.P, kTile);
    a.tiles_q = ceil_div(a.Q, kTile);
    int64_t blocks = a.tiles_p * a.tiles_q;
    for (int d = 0; d < a.nb; ++d) blocks *= a.other_shape[d];
    if (blocks > kMaxGridX) return false;
    switch (esize) {
        case 1: hipLaunchKernelGGL(transpose_kernel<1>, dim3((unsigned)blocks), dim3(kThreads), 0, st, a); break;
        case 2: hipLaunchKernelGGL(transpose_kernel<2>, dim3((unsigned)blocks), dim3(kThreads), 0, st, a); break;
        case 4: hipLaunchKernelGGL(transpose_kernel<4>, dim3((unsigned)blocks), dim3(kThreads), 0, st, a); break;
        default: hipLaunchKernelGGL(transpose_kernel<8>, dim3((unsigned)blocks), dim3(kThreads), 0, st, a); break;
    }
    return true;
}

int esize_of(int dt) { return dt_size(dt); }

int validate_meta_dims(const char* op, int nd, const int64_t* shape) {
    MBRT_REQUIRE(nd >= 1 && nd <= MBRT_MAX_DIMS, MBRT_E_INVALID_ARG, "%s: ndim %d out of [1, 8]", op, nd);
    for (int d = 0; d < nd; ++d) {
        MBRT_REQUIRE(shape[d] >= 0, MBRT_E_SHAPE, "%s: negative extent %lld at dim %d", op,
                     (long long)shape[d], d);
    }
    return MBRT_OK;
}

}  // namespace

// Copies `dm` (already simplified) from src to dst.  The output is contiguous except
// that, when the innermost dim is a unit-stride run, consecutive runs may be placed
// `dst_pitch` bytes apart (dst_pitch < 0: packed).
int strided_copy_dims(const void* src, void* dst, int esize, const Dims& dm, int64_t dst_pitch,
                      hipStream_t st) {
    const int64_t inner_stride = dm.stride[dm.nd - 1];
    if (inner_stride == 1) {
        const int64_t run_bytes = dm.shape[dm.nd - 1] * esize;
        if (dst_pitch < 0) dst_pitch = run_bytes;
        uintptr_t align_bits = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) |
                               (uintptr_t)run_bytes | (uintptr_t)dst_pitch;
        for (int d = 0; d < dm.nd - 1; ++d) align_bits |= (uintptr_t)(dm.stride[d] * esize);
        const char* s = (const char*)src;
        char* o = (char*)dst;
        if ((align_bits & 15) == 0) return launch_row_copy<16>(s, o, dm, esize, dst_pitch, st);
        if ((align_bits & 7) == 0) return launch_row_copy<8>(s, o, dm, esize, dst_pitch, st);
        if ((align_bits & 3) == 0) return launch_row_copy<4>(s, o, dm, esize, dst_pitch, st);
        if ((align_bits & 1) == 0) return launch_row_copy<2>(s, o, dm, esize, dst_pitch, st);
        return launch_row_copy<1>(s, o, dm, esize, dst_pitch, st);
    }
    if (try_transpose(src, dst, dm, esize, st)) return MBRT_OK;
    return launch_elem_copy(src, dst, dm, esize, st);
}

}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_strided_copy(const void* src, void* dst, int dtype, const mbrt_strided_meta* meta,
                      mbrt_stream_t stream) {
    MBRT_REQUIRE(meta != nullptr, MBRT_E_INVALID_ARG, "mbrt_strided_copy: meta is NULL");
    MBRT_REQUIRE(is_valid_dt(dtype), MBRT_E_UNSUPPORTED_DTYPE, "mbrt_strided_copy: bad dtype %d", dtype);
    int s = validate_meta_dims("mbrt_strided_copy", meta->ndim, meta->dst_shape);
    if (s != MBRT_OK) return s;
    int64_t total = 1;
    for (int d = 0; d < meta->ndim; ++d) total *= meta->dst_shape[d];
    if (total == 0) return MBRT_OK;
    MBRT_REQUIRE(src != nullptr && dst != nullptr, MBRT_E_INVALID_ARG, "mbrt_strided_copy: NULL pointer");
    Dims dm = simplify(meta->dst_shape, meta->src_strides, meta->ndim);
    s = strided_copy_dims(src, dst, esize_of(dtype), dm, -1, as_stream(stream));
    if (s != MBRT_OK) return s;
    return check_launch("mbrt_strided_copy");
}

}  // extern "C"

// ---- index_select, pads, cat ---------------------------------------------------------

namespace mbrt {
namespace {

struct IndexSelectArgs {
    const char* src;
    char* dst;
    const void* idx;
    int idx_i64;
    int64_t total;
    int nd;
    int sel;
    int64_t shape[kMaxOuter];
    int64_t stride[kMaxOuter];
};

template <int E>
__global__ __launch_bounds__(kThreads) void index_select_kernel(IndexSelectArgs a) {
    typedef typename WordOf<E>::T Elem;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t step = (int64_t)gridDim.x * kThreads;
    for (; i < a.total; i += step) {
        int64_t rem = i, off = 0;
        for (int d = a.nd - 1; d >= 0; --d) {
            int64_t q = rem / a.shape[d];
            int64_t c = rem - q * a.shape[d];
            if (d == a.sel) {
                c = a.idx_i64 ? reinterpret_cast<const int64_t*>(a.idx)[c]
                              : (int64_t)reinterpret_cast<const int32_t*>(a.idx)[c];
            }
            off += c * a.stride[d];
            rem = q;
        }
        reinterpret_cast<Elem*>(a.dst)[i] = reinterpret_cast<const Elem*>(a.src)[off];
    }
}

struct PadArgs {
    const char* src;
    char* dst;
    int64_t total;
    int nd;
    int64_t src_shape[kMaxOuter];
    int64_t dst_shape[kMaxOuter];
    int64_t before[kMaxOuter];
    uint64_t pad_bits;  // the pad value's bit pattern in the element type
    int reflect;
};

template <int E>
__global__ __launch_bounds__(kThreads) void pad_kernel(PadArgs a) {
    typedef typename WordOf<E>::T Elem;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t step = (int64_t)gridDim.x * kThreads;
    for (; i < a.total; i += step) {
        int64_t rem = i, src_lin = 0, src_pitch = 1;
        bool inside = true;
        for (int d = a.nd - 1; d >= 0; --d) {
            int64_t q = rem / a.dst_shape[d];
            int64_t c = rem - q * a.dst_shape[d] - a.before[d];
            rem = q;
            const int64_t n = a.src_shape[d];
            if (a.reflect) {
                if (c < 0) c = -c;
                if (c >= n) c = 2 * (n - 1) - c;
                c = c < 0 ? 0 : (c > n - 1 ? n - 1 : c);
            } else {
                inside = inside && c >= 0 && c < n;
            }
            src_lin += c * src_pitch;
            src_pitch *= n;
        }
        Elem v;
        if (inside) {
            v = reinterpret_cast<const Elem*>(a.src)[src_lin];
        } else {
            v = (Elem)a.pad_bits;
        }
        reinterpret_cast<Elem*>(a.dst)[i] = v;
    }
}

int launch_pad(const void* src, void* dst, int dtype, const mbrt_pad_meta* m, float value,
               int reflect, const char* op, hipStream_t st) {
    MBRT_REQUIRE(m != nullptr, MBRT_E_INVALID_ARG, "%s: meta is NULL", op);
    MBRT_REQUIRE(is_valid_dt(dtype), MBRT_E_UNSUPPORTED_DTYPE, "%s: bad dtype %d", op, dtype);
    int s = validate_meta_dims(op, m->ndim, m->dst_shape);
    if (s != MBRT_OK) return s;
    PadArgs a;
    a.src = static_cast<const char*>(src);
    a.dst = static_cast<char*>(dst);
    a.nd = m->ndim;
    a.total = 1;
    int64_t src_total = 1;
    for (int d = 0; d < m->ndim; ++d) {
        a.src_shape[d] = m->src_shape[d];
        a.dst_shape[d] = m->dst_shape[d];
        a.before[d] = m->pad_before[d];
        a.total *= m->dst_shape[d];
        src_total *= m->src_shape[d];
        MBRT_REQUIRE(m->src_shape[d] >= 0, MBRT_E_SHAPE, "%s: negative source extent", op);
    }
    if (a.total == 0) return MBRT_OK;
    MBRT_REQUIRE(src_total > 0 || !reflect, MBRT_E_SHAPE, "%s: reflect pad of an empty source", op);
    a.reflect = reflect;
    // pad value in the element type (the reference converts the float pad value the same way)
    switch (dtype) {
        case F32: { uint32_t b; std::memcpy(&b, &value, 4); a.pad_bits = b; break; }
        case F16: { _Float16 h = (_Float16)value; uint16_t b; std::memcpy(&b, &h, 2); a.pad_bits = b; break; }
        case BF16: { __bf16 h = (__bf16)value; uint16_t b; std::memcpy(&b, &h, 2); a.pad_bits = b; break; }
        case I64: { int64_t v = (int64_t)value; std::memcpy(&a.pad_bits, &v, 8); break; }
        default: { int32_t v = (int32_t)value; uint32_t b; std::memcpy(&b, &v, 4); a.pad_bits = b; break; }
    }
    if (src_total == 0) a.reflect = 0;
    int64_t grid = std::min<int64_t>(ceil_div(a.total, kThreads), 1 << 20);
    switch (dt_size(dtype)) {
        case 2: hipLaunchKernelGGL(pad_kernel<2>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        case 4: hipLaunchKernelGGL(pad_kernel<4>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        default: hipLaunchKernelGGL(pad_kernel<8>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
    }
    return check_launch(op);
}

}  // namespace
}  // namespace mbrt

extern "C" {

int mbrt_index_select(const void* src, void* dst, int dtype, const void* indices,
                      int index_dtype, int64_t n_idx, int64_t src_dim_size,
                      const mbrt_strided_meta* meta, int select_dim, mbrt_stream_t stream) {
    const char* op = "mbrt_index_select";
    MBRT_REQUIRE(meta != nullptr, MBRT_E_INVALID_ARG, "%s: meta is NULL", op);
    MBRT_REQUIRE(is_valid_dt(dtype), MBRT_E_UNSUPPORTED_DTYPE, "%s: bad dtype %d", op, dtype);
    MBRT_REQUIRE(is_index_dt(index_dtype), MBRT_E_UNSUPPORTED_DTYPE, "%s: indices must be I32/I64", op);
    int s = validate_meta_dims(op, meta->ndim, meta->dst_shape);
    if (s != MBRT_OK) return s;
    MBRT_REQUIRE(select_dim >= 0 && select_dim < meta->ndim, MBRT_E_INVALID_ARG, "%s: select_dim %d", op, select_dim);
    MBRT_REQUIRE(meta->dst_shape[select_dim] == n_idx, MBRT_E_SHAPE,
                 "%s: dst extent %lld != number of indices %lld", op,
                 (long long)meta->dst_shape[select_dim], (long long)n_idx);
    (void)src_dim_size;
    IndexSelectArgs a;
    a.src = static_cast<const char*>(src);
    a.dst = static_cast<char*>(dst);
    a.idx = indices;
    a.idx_i64 = index_dtype == I64;
    a.nd = meta->ndim;
    a.sel = select_dim;
    a.total = 1;
    for (int d = 0; d < meta->ndim; ++d) {
        a.shape[d] = meta->dst_shape[d];
        a.stride[d] = meta->src_strides[d];
        a.total *= meta->dst_shape[d];
    }
    if (a.total == 0) return MBRT_OK;
    hipStream_t st = as_stream(stream);
    int64_t grid = std::min<int64_t>(ceil_div(a.total, kThreads), 1 << 20);
    switch (dt_size(dtype)) {
        case 2: hipLaunchKernelGGL(index_select_kernel<2>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        case 4: hipLaunchKernelGGL(index_select_kernel<4>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
        default: hipLaunchKernelGGL(index_select_kernel<8>, dim3((unsigned)grid), dim3(kThreads), 0, st, a); break;
    }
    return check_launch(op);
}

int mbrt_pad_const(const void* src, void* dst, int dtype, const mbrt_pad_meta* meta, float value,
                   mbrt_stream_t stream) {
    return launch_pad(src, dst, dtype, meta, value, 0, "mbrt_pad_const", as_stream(stream));
}

int mbrt_pad_reflect(const void* src, void* dst, int dtype, const mbrt_pad_meta* meta,
                     mbrt_stream_t stream) {
    return launch_pad(src, dst, dtype, meta, 0.0f, 1, "mbrt_pad_reflect", as_stream(stream));
}

int mbrt_cat(void* out, const mbrt_cat_src* srcs, int n_srcs, int64_t outer_size,
             int64_t total_cat_dim, int64_t inner_bytes, mbrt_stream_t stream) {
    const char* op = "mbrt_cat";
    MBRT_REQUIRE(n_srcs >= 0 && (n_srcs == 0 || srcs != nullptr), MBRT_E_INVALID_ARG, "%s: bad source list", op);
    MBRT_REQUIRE(outer_size >= 0 && total_cat_dim >= 0 && inner_bytes >= 0, MBRT_E_SHAPE, "%s: negative size", op);
    hipStream_t st = as_stream(stream);
    int64_t used = 0;
    for (int i = 0; i < n_srcs; ++i) {
        MBRT_REQUIRE(srcs[i].dim_size >= 0 && srcs[i].dim_offset >= 0 &&
                         srcs[i].dim_offset + srcs[i].dim_size <= total_cat_dim,
                     MBRT_E_SHAPE, "%s: source %d does not fit the concat dim", op, i);
        used += srcs[i].dim_size;
    }
    (void)used;
    for (int i = 0; i < n_srcs; ++i) {
        const int64_t run = srcs[i].dim_size * inner_bytes;
        if (run == 0 || outer_size == 0) continue;
        // one source = a [outer, run] byte matrix copied into [outer, total*inner] at an offset
        Dims dm;
        dm.nd = 2;
        dm.shape[0] = outer_size;
        dm.stride[0] = run;
        dm.shape[1] = run;
        dm.stride[1] = 1;
        char* dst = static_cast<char*>(out) + srcs[i].dim_offset * inner_bytes;
        // [outer, run] source bytes land in rows `total_cat_dim * inner_bytes` apart
        const int64_t dst_pitch = total_cat_dim * inner_bytes;
        int s = strided_copy_dims(srcs[i].ptr, dst, 1, dm, dst_pitch, st);
        if (s != MBRT_OK) return s;
    }
    return check_launch(op);
}

}  // extern "C"
