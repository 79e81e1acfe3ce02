// tensor_tile:: on the C-ABI.  Dtype checks and messages follow the reference's host
// dispatch (src/tensor_cuda_tile.cu:403-595, src/tensor_cuda_glue.cu:561-696); the
// kernels and their alignment handling are libmbrt's.
#include "tensor_tile.h"

#include "abi_call.h"

namespace cudasep::tensor_tile {

namespace {

int code(DType dt) { return (int)dt; }

void require_contiguous(const Tensor& t, const char* op) {
    if (!t.is_contiguous()) throw std::runtime_error(std::string(op) + ": tensor must be contiguous");
}

bool is_f32_or_f16(DType dt) { return dt == DType::Float32 || dt == DType::Float16; }

int binary_code(BinaryOp op) {
    switch (op) {
        case BinaryOp::Add: return MBRT_ADD;
        case BinaryOp::Sub: return MBRT_SUB;
        case BinaryOp::Mul: return MBRT_MUL;
        case BinaryOp::Div: return MBRT_DIV;
    }
    return MBRT_ADD;
}

mbrt_strided_meta to_abi(const StridedCopyMeta& m) {
    mbrt_strided_meta a{};
    a.ndim = m.ndim;
    for (int d = 0; d < kMaxDims; ++d) {
        a.src_strides[d] = d < m.ndim ? m.src_strides[d] : 0;
        a.dst_shape[d] = d < m.ndim ? m.dst_shape[d] : 1;
    }
    return a;
}

mbrt_broadcast_meta to_abi(const BroadcastMeta& m) {
    mbrt_broadcast_meta a{};
    a.ndim = m.ndim;
    for (int d = 0; d < kMaxDims; ++d) {
        a.out_shape[d] = d < m.ndim ? m.out_shape[d] : 1;
        a.a_strides[d] = d < m.ndim ? m.a_strides[d] : 0;
        a.b_strides[d] = d < m.ndim ? m.b_strides[d] : 0;
    }
    return a;
}

mbrt_pad_meta to_abi(const PadMeta& m) {
    mbrt_pad_meta a{};
    a.ndim = m.ndim;
    for (int d = 0; d < kMaxDims; ++d) {
        a.src_shape[d] = d < m.ndim ? m.src_shape[d] : 1;
        a.dst_shape[d] = d < m.ndim ? m.dst_shape[d] : 1;
        a.pad_before[d] = d < m.ndim ? m.pad_before[d] : 0;
    }
    return a;
}

void scalar_op(Tensor& data, int op, float a, float b, const char* name) {
    if (data.numel() == 0) return;
    if (!is_f32_or_f16(data.dtype())) throw std::runtime_error(std::string(name) + ": unsupported dtype");
    require_contiguous(data, name);
    abi_check(mbrt_scalar_op(data.data_ptr(), code(data.dtype()), data.numel(), op, a, b, abi_stream()), name);
}

}  // namespace

void fill(Tensor& dst, float value) {
    if (dst.numel() == 0) return;
    require_contiguous(dst, "fill");
    abi_check(mbrt_fill(dst.data_ptr(), code(dst.dtype()), dst.numel(), (double)value, abi_stream()), "fill");
}

void arange(Tensor& dst, int64_t start) {
    if (dst.numel() == 0) return;
    if (dst.dtype() == DType::BFloat16) throw std::runtime_error("arange: unsupported BF16 dtype");
    require_contiguous(dst, "arange");
    abi_check(mbrt_arange(dst.data_ptr(), code(dst.dtype()), dst.numel(), start, abi_stream()), "arange");
}

void convert_dtype(const Tensor& src, Tensor& dst) {
    if (src.numel() == 0) return;
    const DType in = src.dtype(), out = dst.dtype();
    // the reference converts between Float32 and each other dtype and between Int64 and
    // each float dtype; Float16 <-> BFloat16 has no kernel there
    const bool f16_bf16 = (in == DType::Float16 && out == DType::BFloat16) ||
                          (in == DType::BFloat16 && out == DType::Float16);
    if (in == out || f16_bf16) throw std::runtime_error("to_dtype: unsupported conversion");
    if (dst.numel() != src.numel()) throw std::runtime_error("to_dtype: size mismatch");
    require_contiguous(src, "to_dtype");
    require_contiguous(dst, "to_dtype");
    abi_check(mbrt_convert(src.data_ptr(), code(in), dst.data_ptr(), code(out), src.numel(), abi_stream()),
              "to_dtype");
}

void add_scalar(Tensor& data, float value) { scalar_op(data, MBRT_SCALAR_ADD, value, 0.0f, "add_scalar_"); }
void mul_scalar(Tensor& data, float value) { scalar_op(data, MBRT_SCALAR_MUL, value, 0.0f, "mul_scalar_"); }
void clamp(Tensor& data, float min_value, float max_value) {
    scalar_op(data, MBRT_SCALAR_CLAMP, min_value, max_value, "clamp_");
}

void negate(const Tensor& src, Tensor& dst) {
    if (src.numel() == 0) return;
    if (!is_f32_or_f16(src.dtype())) throw std::runtime_error("negate: unsupported dtype");
    require_contiguous(src, "negate");
    abi_check(mbrt_unary(src.data_ptr(), dst.data_ptr(), code(src.dtype()), src.numel(), MBRT_UNARY_NEG, 0.0f,
                         abi_stream()),
              "negate");
}

void greater_than(const Tensor& src, Tensor& dst, float value) {
    if (src.numel() == 0) return;
    if (!is_f32_or_f16(src.dtype())) throw std::runtime_error("operator>: unsupported dtype");
    require_contiguous(src, "operator>");
    abi_check(mbrt_unary(src.data_ptr(), dst.data_ptr(), code(src.dtype()), src.numel(), MBRT_UNARY_GT, value,
                         abi_stream()),
              "operator>");
}

void binary_same_shape(const Tensor& a, const Tensor& b, Tensor& out, BinaryOp op) {
    if (out.numel() == 0) return;
    abi_check(mbrt_binary(a.data_ptr(), b.data_ptr(), out.data_ptr(), code(a.dtype()), out.numel(), binary_code(op),
                          abi_stream()),
              "binary op");
}

void binary_inplace_same_shape(Tensor& a, const Tensor& b, BinaryOp op) {
    if (a.numel() == 0) return;
    abi_check(mbrt_binary(a.data_ptr(), b.data_ptr(), a.data_ptr(), code(a.dtype()), a.numel(), binary_code(op),
                          abi_stream()),
              "inplace binary op");
}

void binary_glue(const Tensor& a, const Tensor& b, Tensor& out, const BroadcastMeta& meta, BinaryOp op) {
    const mbrt_broadcast_meta m = to_abi(meta);
    abi_check(mbrt_binary_broadcast(a.data_ptr(), b.data_ptr(), out.data_ptr(), code(out.dtype()), &m,
                                    binary_code(op), abi_stream()),
              "binary op");
}

void binary_inplace_glue(Tensor& a, const Tensor& b, const BroadcastMeta& meta, BinaryOp op) {
    // `a` is the output: read it through its own (contiguous) strides
    if (!a.is_contiguous()) throw std::runtime_error("inplace binary op: destination must be contiguous");
    mbrt_broadcast_meta m = to_abi(meta);
    int64_t s = 1;
    for (int d = m.ndim - 1; d >= 0; --d) {
        m.a_strides[d] = m.out_shape[d] == 1 ? 0 : s;
        s *= m.out_shape[d];
    }
    abi_check(mbrt_binary_broadcast(a.data_ptr(), b.data_ptr(), a.data_ptr(), code(a.dtype()), &m, binary_code(op),
                                    abi_stream()),
              "inplace binary op");
}

void index_select_glue(const Tensor& src, Tensor& dst, const Tensor& indices, const StridedCopyMeta& meta,
                       int select_dim) {
    const mbrt_strided_meta m = to_abi(meta);
    const Tensor idx = indices.contiguous();
    abi_check(mbrt_index_select(src.data_ptr(), dst.data_ptr(), code(src.dtype()), idx.data_ptr(), MBRT_I64,
                                idx.numel(), src.size(select_dim), &m, select_dim, abi_stream()),
              "index_select");
}

void strided_copy_glue(const Tensor& src, Tensor& dst, const StridedCopyMeta& meta) {
    const mbrt_strided_meta m = to_abi(meta);
    abi_check(mbrt_strided_copy(src.data_ptr(), dst.data_ptr(), code(src.dtype()), &m, abi_stream()), "contiguous");
}

void pad_const_glue(const Tensor& src, Tensor& dst, const PadMeta& meta, float value) {
    const mbrt_pad_meta m = to_abi(meta);
    abi_check(mbrt_pad_const(src.data_ptr(), dst.data_ptr(), code(src.dtype()), &m, value, abi_stream()), "pad");
}

void pad_reflect_glue(const Tensor& src, Tensor& dst, const PadMeta& meta) {
    const mbrt_pad_meta m = to_abi(meta);
    abi_check(mbrt_pad_reflect(src.data_ptr(), dst.data_ptr(), code(src.dtype()), &m, abi_stream()), "pad_reflect");
}

void cat_glue(char* out, const CatSrcInfo* infos, int n_infos, int64_t outer_size, int64_t total_cat_dim,
              int64_t inner_bytes, int64_t /*max_src_bytes*/) {
    std::vector<mbrt_cat_src> srcs((size_t)n_infos);
    for (int i = 0; i < n_infos; ++i) srcs[i] = mbrt_cat_src{infos[i].ptr, infos[i].dim_size, infos[i].dim_offset};
    abi_check(mbrt_cat(out, srcs.data(), n_infos, outer_size, total_cat_dim, inner_bytes, abi_stream()), "cat");
}

void sum_reduce_last_dim(const Tensor& src, Tensor& dst, int64_t inner_size, int64_t outer_size) {
    abi_check(mbrt_reduce_last_dim((const float*)src.data_ptr(), (float*)dst.data_ptr(), outer_size, inner_size,
                                   MBRT_REDUCE_SUM, abi_stream()),
              "sum");
}

void max_reduce_last_dim(const Tensor& src, Tensor& dst, int64_t inner_size, int64_t outer_size) {
    abi_check(mbrt_reduce_last_dim((const float*)src.data_ptr(), (float*)dst.data_ptr(), outer_size, inner_size,
                                   MBRT_REDUCE_MAX, abi_stream()),
              "max");
}

void sum_reduce_general_glue(const Tensor& src, Tensor& dst, int64_t outer, int64_t reduce, int64_t inner) {
    abi_check(mbrt_reduce_general((const float*)src.data_ptr(), (float*)dst.data_ptr(), outer, reduce, inner,
                                  MBRT_REDUCE_SUM, abi_stream()),
              "sum");
}

void max_reduce_general_glue(const Tensor& src, Tensor& dst, int64_t outer, int64_t reduce, int64_t inner) {
    abi_check(mbrt_reduce_general((const float*)src.data_ptr(), (float*)dst.data_ptr(), outer, reduce, inner,
                                  MBRT_REDUCE_MAX, abi_stream()),
              "max");
}

}  // namespace cudasep::tensor_tile
