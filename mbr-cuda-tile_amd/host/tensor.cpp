// cudasep::Tensor: metadata algebra on the host (views share storage), device work through
// tensor_tile:: and the C-ABI.  Semantics follow src/tensor.cu section by section; the
// line ranges are cited per method.
#include "tensor.h"

#include <algorithm>
#include <iostream>
#include <numeric>
#include <sstream>
#include <stdexcept>

#include "abi_call.h"
#include "memory_pool.h"
#include "tensor_tile.h"

namespace cudasep {

namespace {

hipStream_t stream() { return HipContext::instance().stream(); }

// Copies that the reference makes with synchronous cudaMemcpy: enqueued on the tensor
// stream (after the work that produced the data) and waited for.
void copy_sync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
    if (bytes == 0) return;
    HIP_CHECK(hipMemcpyAsync(dst, src, bytes, kind, stream()));
    HIP_CHECK(hipStreamSynchronize(stream()));
}

int64_t product(const std::vector<int64_t>& s) {
    int64_t n = 1;
    for (int64_t v : s) n *= v;
    return n;
}

tensor_tile::StridedCopyMeta copy_meta(const std::vector<int64_t>& src_strides, const std::vector<int64_t>& shape) {
    if ((int)shape.size() > tensor_tile::kMaxDims) throw std::runtime_error("strided copy: too many dims (max 8)");
    tensor_tile::StridedCopyMeta m{};
    m.ndim = (int)shape.size();
    for (int i = 0; i < m.ndim; ++i) {
        m.src_strides[i] = src_strides[i];
        m.dst_shape[i] = shape[i];
    }
    return m;
}

}  // namespace

// src/tensor.cu:14-23
Tensor::Tensor() : storage_(nullptr), data_(nullptr), numel_(0), dtype_(DType::Float32) {}

std::shared_ptr<void> Tensor::alloc_gpu(size_t bytes) {
    if (bytes == 0) return nullptr;
    void* p = HipMemoryPool::instance().allocate(bytes);
    return std::shared_ptr<void>(p, [](void* q) { HipMemoryPool::instance().deallocate(q); });
}

void Tensor::compute_strides() {
    strides_.assign(shape_.size(), 1);
    for (int i = (int)shape_.size() - 2; i >= 0; --i) strides_[i] = strides_[i + 1] * shape_[i + 1];
}

Tensor Tensor::view_of(std::vector<int64_t> shape, std::vector<int64_t> strides, void* data) const {
    Tensor t;
    t.storage_ = storage_;
    t.data_ = data;
    t.dtype_ = dtype_;
    t.shape_ = std::move(shape);
    t.strides_ = std::move(strides);
    t.numel_ = product(t.shape_);
    return t;
}

// src/tensor.cu:35-41
int64_t Tensor::size(int dim) const {
    if (dim < 0) dim += ndim();
    if (dim < 0 || dim >= ndim()) throw std::out_of_range("Tensor::size: dim out of range");
    return shape_[dim];
}

// src/tensor.cu:43-51: size-1 dims do not constrain their stride
bool Tensor::is_contiguous() const {
    if (numel_ <= 1) return true;
    int64_t expected = 1;
    for (int i = ndim() - 1; i >= 0; --i) {
        if (shape_[i] != 1 && strides_[i] != expected) return false;
        expected *= shape_[i];
    }
    return true;
}

// src/tensor.cu:54-123
Tensor Tensor::empty(std::vector<int64_t> shape, DType dtype) {
    Tensor t;
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    t.numel_ = product(t.shape_);
    if (t.numel_ < 0) throw std::runtime_error("Tensor::empty: negative dimension");
    t.compute_strides();
    t.storage_ = alloc_gpu((size_t)t.numel_ * dtype_size(dtype));
    t.data_ = t.storage_.get();
    return t;
}

Tensor Tensor::zeros(std::vector<int64_t> shape, DType dtype) {
    Tensor t = empty(std::move(shape), dtype);
    if (t.numel_ > 0) HIP_CHECK(hipMemsetAsync(t.data_, 0, (size_t)t.numel_ * dtype_size(dtype), stream()));
    return t;
}

Tensor Tensor::ones(std::vector<int64_t> shape, DType dtype) { return full(std::move(shape), 1.0f, dtype); }

Tensor Tensor::full(std::vector<int64_t> shape, float value, DType dtype) {
    Tensor t = empty(std::move(shape), dtype);
    if (t.numel_ > 0) tensor_tile::fill(t, value);
    return t;
}

Tensor Tensor::from_cpu_f32(const float* data, std::vector<int64_t> shape) {
    Tensor t = empty(std::move(shape), DType::Float32);
    copy_sync(t.data_, data, (size_t)t.numel_ * 4, hipMemcpyHostToDevice);
    return t;
}

Tensor Tensor::from_cpu_f16(const void* data, std::vector<int64_t> shape) {
    Tensor t = empty(std::move(shape), DType::Float16);
    copy_sync(t.data_, data, (size_t)t.numel_ * 2, hipMemcpyHostToDevice);
    return t;
}

Tensor Tensor::from_cpu_i64(const int64_t* data, std::vector<int64_t> shape) {
    Tensor t = empty(std::move(shape), DType::Int64);
    copy_sync(t.data_, data, (size_t)t.numel_ * 8, hipMemcpyHostToDevice);
    return t;
}

// src/tensor.cu:115-122: an empty range gives an empty tensor
Tensor Tensor::arange(int64_t start, int64_t end, DType dtype) {
    const int64_t n = end - start;
    if (n <= 0) return Tensor();
    Tensor t = empty({n}, dtype);
    tensor_tile::arange(t, start);
    return t;
}

// src/tensor.cu:125-145
std::vector<float> Tensor::to_cpu_f32() const {
    if (dtype_ != DType::Float32) return to_f32().to_cpu_f32();
    const Tensor c = contiguous();
    std::vector<float> out((size_t)numel_);
    copy_sync(out.data(), c.data_, (size_t)numel_ * 4, hipMemcpyDeviceToHost);
    return out;
}

void Tensor::copy_from_cpu(const void* src, size_t bytes) { copy_sync(data_, src, bytes, hipMemcpyHostToDevice); }

void Tensor::copy_to_cpu(void* dst, size_t bytes) const { copy_sync(dst, data_, bytes, hipMemcpyDeviceToHost); }

// src/tensor.cu:157-199: one -1 allowed; a non-contiguous source is copied first
Tensor Tensor::reshape(std::vector<int64_t> new_shape) const {
    int neg = -1;
    int64_t prod = 1;
    for (int i = 0; i < (int)new_shape.size(); ++i) {
        if (new_shape[i] == -1) {
            if (neg >= 0) throw std::runtime_error("reshape: only one -1 allowed");
            neg = i;
        } else {
            prod *= new_shape[i];
        }
    }
    if (neg >= 0) new_shape[neg] = prod == 0 ? 0 : numel_ / prod;
    const int64_t n = product(new_shape);
    if (n != numel_)
        throw std::runtime_error("reshape: incompatible sizes " + std::to_string(numel_) + " vs " + std::to_string(n));
    const Tensor src = is_contiguous() ? *this : contiguous();
    Tensor t = src.view_of(std::move(new_shape), {}, src.data_);
    t.compute_strides();
    return t;
}

// src/tensor.cu:202-219 (zero-copy stride reordering)
Tensor Tensor::permute(std::vector<int> dims) const {
    const int nd = ndim();
    if ((int)dims.size() != nd) throw std::runtime_error("permute: dims size mismatch");
    std::vector<int64_t> shape(nd), strides(nd);
    std::vector<bool> seen(nd, false);
    for (int i = 0; i < nd; ++i) {
        int d = dims[i] < 0 ? dims[i] + nd : dims[i];
        if (d < 0 || d >= nd || seen[d]) throw std::runtime_error("permute: invalid dims");
        seen[d] = true;
        shape[i] = shape_[d];
        strides[i] = strides_[d];
    }
    return view_of(std::move(shape), std::move(strides), data_);
}

Tensor Tensor::transpose(int dim0, int dim1) const {
    const int nd = ndim();
    if (dim0 < 0) dim0 += nd;
    if (dim1 < 0) dim1 += nd;
    std::vector<int> dims(nd);
    std::iota(dims.begin(), dims.end(), 0);
    std::swap(dims.at(dim0), dims.at(dim1));
    return permute(dims);
}

// src/tensor.cu:233-251: a contiguous tensor is returned as a shared view
Tensor Tensor::contiguous() const {
    if (is_contiguous()) return *this;
    Tensor out = empty(shape_, dtype_);
    if (numel_ == 0) return out;
    tensor_tile::strided_copy_glue(*this, out, copy_meta(strides_, shape_));
    return out;
}

Tensor Tensor::unsqueeze(int dim) const {
    if (dim < 0) dim += ndim() + 1;
    if (dim < 0 || dim > ndim()) throw std::out_of_range("unsqueeze: dim out of range");
    std::vector<int64_t> s = shape_;
    s.insert(s.begin() + dim, 1);
    return reshape(s);
}

Tensor Tensor::squeeze(int dim) const {
    if (dim < 0) dim += ndim();
    if (dim < 0 || dim >= ndim()) throw std::out_of_range("squeeze: dim out of range");
    if (shape_[dim] != 1) throw std::runtime_error("squeeze: dimension is not 1");
    std::vector<int64_t> s = shape_;
    s.erase(s.begin() + dim);
    return reshape(s);
}

// src/tensor.cu:275-306: size-1 dims broadcast with stride 0
Tensor Tensor::expand(std::vector<int64_t> new_shape) const {
    const int nd = (int)new_shape.size();
    if (nd < ndim()) throw std::runtime_error("expand: cannot reduce dims");
    std::vector<int64_t> ss = shape_, st = strides_;
    while ((int)ss.size() < nd) {
        ss.insert(ss.begin(), 1);
        st.insert(st.begin(), 0);
    }
    std::vector<int64_t> strides(nd);
    for (int d = 0; d < nd; ++d) {
        if (ss[d] == new_shape[d]) strides[d] = st[d];
        else if (ss[d] == 1) strides[d] = 0;
        else throw std::runtime_error("expand: incompatible shape at dim " + std::to_string(d));
    }
    return view_of(std::move(new_shape), std::move(strides), data_);
}

// src/tensor.cu:309-327: clamped bounds, empty range -> Tensor(); the data pointer moves,
// so a slice may lose 16-byte alignment (the kernels check and take their scalar paths)
Tensor Tensor::slice(int dim, int64_t start, int64_t end) const {
    if (dim < 0) dim += ndim();
    if (dim < 0 || dim >= ndim()) throw std::out_of_range("slice: dim out of range");
    if (start < 0) start += shape_[dim];
    if (end < 0) end += shape_[dim];
    start = std::max<int64_t>(start, 0);
    end = std::min<int64_t>(end, shape_[dim]);
    if (start >= end) return Tensor();
    std::vector<int64_t> s = shape_;
    s[dim] = end - start;
    return view_of(std::move(s), strides_, (char*)data_ + start * strides_[dim] * (int64_t)dtype_size(dtype_));
}

// src/tensor.cu:330-356
Tensor Tensor::index_select(int dim, const Tensor& indices) const {
    if (dim < 0) dim += ndim();
    if (indices.dtype() != DType::Int64) throw std::runtime_error("index_select: indices must be Int64");
    std::vector<int64_t> out_shape = shape_;
    out_shape.at(dim) = indices.numel();
    Tensor out = empty(out_shape, dtype_);
    if (out.numel_ == 0) return out;
    tensor_tile::index_select_glue(*this, out, indices, copy_meta(strides_, out_shape), dim);
    return out;
}

// src/tensor.cu:359-414
Tensor Tensor::cat(const std::vector<Tensor>& tensors, int dim) {
    if (tensors.empty()) throw std::runtime_error("cat: empty tensor list");
    const int nd = tensors[0].ndim();
    if (dim < 0) dim += nd;
    const DType dt = tensors[0].dtype();
    std::vector<int64_t> out_shape = tensors[0].shape();
    int64_t total = 0;
    for (const Tensor& t : tensors) {
        if (t.ndim() != nd) throw std::runtime_error("cat: ndim mismatch");
        if (t.dtype() != dt) throw std::runtime_error("cat: dtype mismatch");
        for (int d = 0; d < nd; ++d)
            if (d != dim && t.shape_[d] != out_shape[d]) throw std::runtime_error("cat: shape mismatch");
        total += t.size(dim);
    }
    out_shape[dim] = total;
    Tensor out = empty(out_shape, dt);
    if (out.numel_ == 0) return out;
    int64_t outer = 1, inner = 1;
    for (int d = 0; d < dim; ++d) outer *= out_shape[d];
    for (int d = dim + 1; d < nd; ++d) inner *= out_shape[d];
    const int64_t inner_bytes = inner * (int64_t)dtype_size(dt);
    std::vector<Tensor> keep;
    std::vector<tensor_tile::CatSrcInfo> infos;
    int64_t off = 0, max_bytes = 0;
    for (const Tensor& t : tensors) {
        keep.push_back(t.contiguous());
        infos.push_back({keep.back().data_, t.size(dim), off});
        max_bytes = std::max(max_bytes, outer * t.size(dim) * inner_bytes);
        off += t.size(dim);
    }
    tensor_tile::cat_glue((char*)out.data_, infos.data(), (int)infos.size(), outer, total, inner_bytes, max_bytes);
    return out;
}

Tensor Tensor::stack(const std::vector<Tensor>& tensors, int dim) {
    if (tensors.empty()) throw std::runtime_error("stack: empty tensor list");
    std::vector<Tensor> u;
    u.reserve(tensors.size());
    for (const Tensor& t : tensors) u.push_back(t.unsqueeze(dim));
    return cat(u, dim);
}

// src/tensor.cu:425-456
std::vector<Tensor> Tensor::split(int dim, const std::vector<int64_t>& sizes) const {
    if (dim < 0) dim += ndim();
    int64_t total = 0;
    for (int64_t s : sizes) total += s;
    if (total != shape_.at(dim)) throw std::runtime_error("split: sizes don't sum to dim size");
    std::vector<Tensor> out;
    int64_t off = 0;
    for (int64_t s : sizes) {
        out.push_back(slice(dim, off, off + s));
        off += s;
    }
    return out;
}

std::vector<Tensor> Tensor::unbind(int dim) const {
    if (dim < 0) dim += ndim();
    std::vector<Tensor> out;
    for (int64_t i = 0; i < shape_.at(dim); ++i) out.push_back(slice(dim, i, i + 1).squeeze(dim));
    return out;
}

namespace {
// Pairs (before, after) from the last dim backwards, as torch.nn.functional.pad
// (src/tensor.cu:461-476).
tensor_tile::PadMeta pad_meta(const std::vector<int64_t>& shape, const std::vector<int64_t>& padding,
                              std::vector<int64_t>& out_shape) {
    const int nd = (int)shape.size();
    if (nd > tensor_tile::kMaxDims) throw std::runtime_error("pad: too many dims (max 8)");
    tensor_tile::PadMeta m{};
    m.ndim = nd;
    out_shape = shape;
    for (int d = 0; d < nd; ++d) {
        m.src_shape[d] = shape[d];
        m.pad_before[d] = 0;
    }
    const int pairs = (int)padding.size() / 2;
    for (int i = 0; i < pairs && i < nd; ++i) {
        const int d = nd - 1 - i;
        m.pad_before[d] = padding[2 * i];
        out_shape[d] = shape[d] + padding[2 * i] + padding[2 * i + 1];
    }
    for (int d = 0; d < nd; ++d) m.dst_shape[d] = out_shape[d];
    return m;
}
}  // namespace

Tensor Tensor::pad(const std::vector<int64_t>& padding, float value) const {
    std::vector<int64_t> out_shape;
    const tensor_tile::PadMeta m = pad_meta(shape_, padding, out_shape);
    Tensor out = empty(out_shape, dtype_);
    if (out.numel_ == 0) return out;
    const Tensor src = contiguous();
    tensor_tile::pad_const_glue(src, out, m, value);
    return out;
}

Tensor Tensor::pad_reflect(const std::vector<int64_t>& padding) const {
    std::vector<int64_t> out_shape;
    const tensor_tile::PadMeta m = pad_meta(shape_, padding, out_shape);
    Tensor out = empty(out_shape, dtype_);
    if (out.numel_ == 0) return out;
    const Tensor src = contiguous();
    tensor_tile::pad_reflect_glue(src, out, m);
    return out;
}

// src/tensor.cu:534-542: same dtype is a no-op view
Tensor Tensor::to_dtype(DType new_dtype) const {
    if (new_dtype == dtype_) return *this;
    Tensor out = empty(shape_, new_dtype);
    if (numel_ == 0) return out;
    tensor_tile::convert_dtype(contiguous(), out);
    return out;
}

namespace {

// Right-aligned broadcasting, stride 0 on size-1 dims (src/tensor.cu:548-580).
tensor_tile::BroadcastMeta broadcast_meta(const Tensor& a, const Tensor& b, std::vector<int64_t>& out_shape) {
    const int na = a.ndim(), nb = b.ndim(), nd = std::max(na, nb);
    if (nd > tensor_tile::kMaxDims) throw std::runtime_error("broadcast: too many dims (max 8)");
    tensor_tile::BroadcastMeta m{};
    m.ndim = nd;
    out_shape.assign(nd, 1);
    for (int d = 0; d < nd; ++d) {
        const int ia = na - nd + d, ib = nb - nd + d;
        const int64_t sa = ia >= 0 ? a.shape()[ia] : 1, sb = ib >= 0 ? b.shape()[ib] : 1;
        if (sa != sb && sa != 1 && sb != 1) throw std::runtime_error("broadcast: incompatible shapes");
        out_shape[d] = std::max(sa, sb);
        m.out_shape[d] = out_shape[d];
        m.a_strides[d] = (ia >= 0 && sa != 1) ? a.strides()[ia] : 0;
        m.b_strides[d] = (ib >= 0 && sb != 1) ? b.strides()[ib] : 0;
    }
    return m;
}

template <tensor_tile::BinaryOp OP>
Tensor binary_op(const Tensor& a, const Tensor& b) {
    if (a.dtype() != b.dtype()) throw std::runtime_error("binary op: dtype mismatch");
    if (a.shape() == b.shape() && a.is_contiguous() && b.is_contiguous()) {
        Tensor out = Tensor::empty(a.shape(), a.dtype());
        tensor_tile::binary_same_shape(a, b, out, OP);
        return out;
    }
    std::vector<int64_t> out_shape;
    const tensor_tile::BroadcastMeta m = broadcast_meta(a, b, out_shape);
    Tensor out = Tensor::empty(out_shape, a.dtype());
    if (out.numel() == 0) return out;
    tensor_tile::binary_glue(a, b, out, m, OP);
    return out;
}

// In place: `a` is the output and keeps its shape (src/tensor.cu:583-608, 652-671).
template <tensor_tile::BinaryOp OP>
void binary_op_inplace(Tensor& a, const Tensor& b) {
    if (a.dtype() != b.dtype()) throw std::runtime_error("inplace binary op: dtype mismatch");
    if (a.shape() == b.shape() && a.is_contiguous() && b.is_contiguous()) {
        tensor_tile::binary_inplace_same_shape(a, b, OP);
        return;
    }
    const int na = a.ndim(), nb = b.ndim();
    if (na > tensor_tile::kMaxDims) throw std::runtime_error("broadcast inplace: too many dims");
    if (nb > na) throw std::runtime_error("broadcast inplace: incompatible shapes");
    tensor_tile::BroadcastMeta m{};
    m.ndim = na;
    for (int d = 0; d < na; ++d) {
        const int ib = nb - na + d;
        const int64_t sb = ib >= 0 ? b.shape()[ib] : 1;
        if (a.shape()[d] != sb && sb != 1) throw std::runtime_error("broadcast inplace: incompatible shapes");
        m.out_shape[d] = a.shape()[d];
        m.a_strides[d] = 0;
        m.b_strides[d] = (ib >= 0 && sb != 1) ? b.strides()[ib] : 0;
    }
    if (a.numel() == 0) return;
    tensor_tile::binary_inplace_glue(a, b, m, OP);
}

}  // namespace

Tensor Tensor::operator+(const Tensor& o) const { return binary_op<tensor_tile::BinaryOp::Add>(*this, o); }
Tensor Tensor::operator-(const Tensor& o) const { return binary_op<tensor_tile::BinaryOp::Sub>(*this, o); }
Tensor Tensor::operator*(const Tensor& o) const { return binary_op<tensor_tile::BinaryOp::Mul>(*this, o); }
Tensor Tensor::operator/(const Tensor& o) const { return binary_op<tensor_tile::BinaryOp::Div>(*this, o); }

Tensor Tensor::operator-() const {
    Tensor out = empty(shape_, dtype_);
    if (numel_ == 0) return out;
    tensor_tile::negate(contiguous(), out);
    return out;
}

Tensor& Tensor::add_(const Tensor& o) {
    binary_op_inplace<tensor_tile::BinaryOp::Add>(*this, o);
    return *this;
}

Tensor& Tensor::mul_(const Tensor& o) {
    binary_op_inplace<tensor_tile::BinaryOp::Mul>(*this, o);
    return *this;
}

Tensor& Tensor::add_scalar_(float v) {
    tensor_tile::add_scalar(*this, v);
    return *this;
}

Tensor& Tensor::mul_scalar_(float v) {
    tensor_tile::mul_scalar(*this, v);
    return *this;
}

Tensor& Tensor::clamp_(float lo, float hi) {
    tensor_tile::clamp(*this, lo, hi);
    return *this;
}

Tensor& Tensor::fill_(float v) {
    tensor_tile::fill(*this, v);
    return *this;
}

Tensor Tensor::operator>(float v) const {
    Tensor out = empty(shape_, dtype_);
    if (numel_ == 0) return out;
    tensor_tile::greater_than(contiguous(), out, v);
    return out;
}

namespace {
// src/tensor.cu:702-709
void reduce_dims(const std::vector<int64_t>& s, int dim, int64_t& outer, int64_t& red, int64_t& inner) {
    outer = 1;
    inner = 1;
    for (int d = 0; d < dim; ++d) outer *= s[d];
    red = s[dim];
    for (int d = dim + 1; d < (int)s.size(); ++d) inner *= s[d];
}

std::vector<int64_t> reduced_shape(std::vector<int64_t> s, int dim, bool keepdim) {
    if (keepdim) s[dim] = 1;
    else s.erase(s.begin() + dim);
    if (s.empty()) s.push_back(1);
    return s;
}
}  // namespace

// src/tensor.cu:710-780: non-f32 inputs are converted first; outputs are f32
Tensor Tensor::sum(int dim, bool keepdim) const {
    if (dim < 0) dim += ndim();
    if (dim < 0 || dim >= ndim()) throw std::out_of_range("sum: dim out of range");
    if (dtype_ != DType::Float32) return to_f32().sum(dim, keepdim);
    int64_t outer, red, inner;
    reduce_dims(shape_, dim, outer, red, inner);
    Tensor out = empty(reduced_shape(shape_, dim, keepdim), DType::Float32);
    if (out.numel_ == 0) return out;
    const Tensor src = contiguous();
    if (inner == 1) tensor_tile::sum_reduce_last_dim(src, out, red, outer);
    else tensor_tile::sum_reduce_general_glue(src, out, outer, red, inner);
    return out;
}

Tensor Tensor::mean(int dim, bool keepdim) const {
    if (dim < 0) dim += ndim();
    Tensor s = sum(dim, keepdim);
    s.mul_scalar_(1.0f / (float)shape_[dim]);
    return s;
}

Tensor Tensor::max(int dim, bool keepdim) const {
    if (dim < 0) dim += ndim();
    if (dim < 0 || dim >= ndim()) throw std::out_of_range("max: dim out of range");
    if (dtype_ != DType::Float32) return to_f32().max(dim, keepdim);
    int64_t outer, red, inner;
    reduce_dims(shape_, dim, outer, red, inner);
    Tensor out = empty(reduced_shape(shape_, dim, keepdim), DType::Float32);
    if (out.numel_ == 0) return out;
    const Tensor src = contiguous();
    if (inner == 1) tensor_tile::max_reduce_last_dim(src, out, red, outer);
    else tensor_tile::max_reduce_general_glue(src, out, outer, red, inner);
    return out;
}

// src/tensor.cu:782-816
Tensor Tensor::clone() const {
    Tensor out = empty(shape_, dtype_);
    if (numel_ == 0) return out;
    if (is_contiguous()) {
        HIP_CHECK(hipMemcpyAsync(out.data_, data_, (size_t)numel_ * dtype_size(dtype_), hipMemcpyDeviceToDevice,
                                 stream()));
    } else {
        tensor_tile::strided_copy_glue(*this, out, copy_meta(strides_, shape_));
    }
    return out;
}

void Tensor::copy_from(const Tensor& src) {
    if (numel_ != src.numel_) throw std::runtime_error("copy_from: size mismatch");
    if (dtype_ != src.dtype_) throw std::runtime_error("copy_from: dtype mismatch");
    if (numel_ == 0) return;
    if (!is_contiguous()) throw std::runtime_error("copy_from: destination must be contiguous");
    if (src.is_contiguous()) {
        HIP_CHECK(hipMemcpyAsync(data_, src.data_, (size_t)numel_ * dtype_size(dtype_), hipMemcpyDeviceToDevice,
                                 stream()));
    } else {
        tensor_tile::strided_copy_glue(src, *this, copy_meta(src.strides_, src.shape_));
    }
}

std::string Tensor::shape_str() const {
    std::ostringstream ss;
    ss << "(";
    for (int i = 0; i < ndim(); ++i) ss << (i ? ", " : "") << shape_[i];
    ss << ")";
    return ss.str();
}

void Tensor::print(const std::string& name, int max_elements) const {
    static const char* names[] = {"float32", "float16", "int64", "bfloat16"};
    std::cout << "Tensor";
    if (!name.empty()) std::cout << " \"" << name << "\"";
    std::cout << " shape=" << shape_str() << " dtype=" << names[(int)dtype_] << " numel=" << numel_ << std::endl;
    if (numel_ == 0) {
        std::cout << "  (empty)" << std::endl;
        return;
    }
    const std::vector<float> v = to_cpu_f32();
    const int n = std::min((int)v.size(), max_elements);
    std::cout << "  [";
    for (int i = 0; i < n; ++i) std::cout << (i ? ", " : "") << v[i];
    if ((int)v.size() > max_elements) std::cout << ", ...";
    std::cout << "]" << std::endl;
}

}  // namespace cudasep
