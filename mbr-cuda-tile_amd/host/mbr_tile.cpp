// mbr_tile:: on the C-ABI.  Output dtypes follow the reference's precision policies,
// which read g_quantize_bf16 and the same CUDASEP_* environment switches
// (src/mbr_cuda_tile.cu:103-354); shapes and error messages follow its host dispatch.
#include "mbr_tile.h"

#include <algorithm>
#include <limits>
#include <stdexcept>
#include <string>

#include "abi_call.h"

namespace cudasep::mbr_tile {

namespace {

// ---- policies (src/mbr_cuda_tile.cu:111-354)
bool custom_bf16_path() { return g_quantize_bf16 && !env_flag_enabled("CUDASEP_DISABLE_BF16_CUSTOM_PATH"); }
bool all_bf16_experiments() {
    return g_quantize_bf16 && (custom_bf16_path() || env_flag_enabled("CUDASEP_ALL_BF16_EXPERIMENTS"));
}
bool remaining_bf16_experiments() {
    return g_quantize_bf16 && (custom_bf16_path() || env_flag_enabled("CUDASEP_REMAINING_BF16_EXPERIMENTS"));
}
bool bf16_experiment(const char* name) {
    return g_quantize_bf16 && (all_bf16_experiments() || env_flag_enabled(name));
}
bool remaining_bf16_experiment(const char* name) {
    return bf16_experiment(name) || remaining_bf16_experiments();
}
bool rms_norm_bf16() { return bf16_experiment("CUDASEP_RMS_NORM_BF16"); }
bool gate_merge_bf16() { return bf16_experiment("CUDASEP_GATE_MERGE_BF16"); }
bool gather_bf16_output() { return remaining_bf16_experiment("CUDASEP_GATHER_BF16_OUTPUT"); }
bool mask_scatter_bf16() { return bf16_experiment("CUDASEP_MASK_SCATTER_BF16"); }
bool stft_result_bf16() { return g_quantize_bf16 && env_flag_enabled("CUDASEP_ENABLE_STFT_RESULT_BF16"); }
bool glu_bf16_output() { return bf16_experiment("CUDASEP_GLU_BF16_OUTPUT"); }
bool glu_bf16_input() { return remaining_bf16_experiment("CUDASEP_GLU_BF16_INPUT"); }
bool tanh_bf16_input() { return remaining_bf16_experiment("CUDASEP_TANH_BF16_INPUT"); }
bool freq_attention60_padded() {
    return g_quantize_bf16 && !env_flag_enabled("CUDASEP_DISABLE_FREQ_ATTENTION60_CUTILE_PADDED");
}
// CUDASEP_FULL_BF16_ARITH_EXPERIMENTS under bf16 (full_bf16_arith_enabled,
// src/mbr_cuda_tile.cu:190-192): the reference's kernels then round intermediates (sums of
// squares, row maxima, exponentials, gates, ...) to bf16.  The ops that take the mode hold
// this scope around their C-ABI call, which sets MBRT_ARITH_BF16_INTERMEDIATES on the
// calling thread exactly while the switch is on, and restores the caller's flags after.
class FullBf16Scope {
public:
    FullBf16Scope() : prev_(mbrt_get_arith_flags()) {
        const bool on = g_quantize_bf16 && env_flag_enabled("CUDASEP_FULL_BF16_ARITH_EXPERIMENTS");
        const uint32_t want = on ? (prev_ | MBRT_ARITH_BF16_INTERMEDIATES) : (prev_ & ~(uint32_t)MBRT_ARITH_BF16_INTERMEDIATES);
        if (want != prev_) mbrt_set_arith_flags(want);
    }
    ~FullBf16Scope() { mbrt_set_arith_flags(prev_); }
    FullBf16Scope(const FullBf16Scope&) = delete;
    FullBf16Scope& operator=(const FullBf16Scope&) = delete;

private:
    uint32_t prev_;
};

constexpr int kFreqAttnN = 60;
constexpr int kFreqAttnPadN = 64;
constexpr int kFreqAttnD = 64;

int code(DType dt) { return (int)dt; }
bool is_float(DType dt) { return dt != DType::Int64; }

// gamma, tables, counts: F32 or BF16 are read as they are, F16 is widened once
Tensor f32_or_bf16(const Tensor& t) {
    if (t.dtype() == DType::Float32 || t.dtype() == DType::BFloat16) return t.contiguous();
    return t.to_f32().contiguous();
}

Tensor float_contig(const Tensor& t, const char* op) {
    if (!is_float(t.dtype())) throw std::runtime_error(std::string(op) + ": expected a floating-point tensor");
    return t.contiguous();
}

// Output dtype of the f32 pipelines, which the reference returns as F16 for F16 inputs.
DType f32_pipeline_out(DType in) { return in == DType::Float16 ? DType::Float16 : DType::Float32; }

}  // namespace

bool residual_bf16_enabled() { return remaining_bf16_experiment("CUDASEP_RESIDUAL_BF16"); }
bool bias_bf16_enabled() { return remaining_bf16_experiment("CUDASEP_BIAS_BF16"); }
bool norm_gamma_bf16_enabled() { return g_quantize_bf16 && !env_flag_enabled("CUDASEP_DISABLE_NORM_GAMMA_BF16"); }
bool bands_per_freq_bf16_enabled() {
    return g_quantize_bf16 && !env_flag_enabled("CUDASEP_DISABLE_BANDS_PER_FREQ_BF16");
}
bool rotary_freqs_bf16_enabled() { return g_quantize_bf16 && !env_flag_enabled("CUDASEP_DISABLE_ROTARY_FREQS_BF16"); }
// The reference's predicate (src/mbr_cuda_tile.cu:166-169, 6000-6002): the model takes its
// fused feed-forward branch (src/model_mel_band_roformer.cu:490) only under bf16.  The
// fused op itself, try_residual_add_rms_norm, serves every dtype unless disabled.
bool residual_rms_norm_fused_path_enabled() {
    return g_quantize_bf16 && !env_flag_enabled("CUDASEP_DISABLE_RESIDUAL_RMS_NORM_FUSED");
}

// ---- time-attention context: per-thread indices, -1 when unset ---------------------------

namespace {
thread_local int t_attention_chunk = -1;
thread_local int t_attention_depth = -1;
}  // namespace

void set_time_attention_context_chunk(int chunk_index) { t_attention_chunk = chunk_index; }
void set_time_attention_context_depth(int depth_index) { t_attention_depth = depth_index; }
int time_attention_context_chunk() { return t_attention_chunk; }
int time_attention_context_depth() { return t_attention_depth; }

// ---- normalisation ----------------------------------------------------------------------

Tensor rms_norm(const Tensor& x, const Tensor& gamma, float scale) {
    const Tensor xc = float_contig(x, "mbr_tile::rms_norm");
    const Tensor gf = f32_or_bf16(gamma);
    const int64_t dim = xc.size(xc.ndim() - 1);
    if (gf.numel() != dim) throw std::runtime_error("mbr_tile::rms_norm: gamma size does not match the last dimension");
    const DType odt = rms_norm_bf16() ? DType::BFloat16 : f32_pipeline_out(xc.dtype());
    Tensor out = Tensor::empty(xc.shape(), odt);
    if (xc.numel() == 0) return out;
    FullBf16Scope full_bf16;
    abi_check(mbrt_rms_norm(xc.data_ptr(), code(xc.dtype()), gf.data_ptr(), code(gf.dtype()), out.data_ptr(), code(odt),
                            xc.numel() / dim, dim, scale, 1e-12f, abi_stream()),
              "mbr_tile::rms_norm");
    return out;
}

bool try_residual_add_rms_norm(const Tensor& residual, const Tensor& update, const Tensor& gamma, float scale,
                               Tensor& residual_out, Tensor& normed) {
    if (env_flag_enabled("CUDASEP_DISABLE_RESIDUAL_RMS_NORM_FUSED")) return false;
    if (residual.dtype() != update.dtype() || !is_float(residual.dtype())) return false;
    if (residual.shape() != update.shape() || residual.ndim() == 0 || residual.numel() == 0) return false;
    if (!residual.is_contiguous() || !update.is_contiguous()) return false;
    const int64_t dim = residual.size(residual.ndim() - 1);
    const Tensor gf = f32_or_bf16(gamma);
    if (gf.numel() != dim) return false;
    const DType ndt = rms_norm_bf16() ? DType::BFloat16 : f32_pipeline_out(residual.dtype());
    Tensor sum = Tensor::empty(residual.shape(), residual.dtype());
    Tensor out = Tensor::empty(residual.shape(), ndt);
    FullBf16Scope full_bf16;
    abi_check(mbrt_residual_add_rms_norm(residual.data_ptr(), update.data_ptr(), code(residual.dtype()), gf.data_ptr(),
                                         code(gf.dtype()), sum.data_ptr(), code(residual.dtype()), out.data_ptr(),
                                         code(ndt), residual.numel() / dim, dim, scale, 1e-12f, abi_stream()),
              "mbr_tile::try_residual_add_rms_norm");
    residual_out = sum;
    normed = out;
    return true;
}

// ---- attention plumbing -----------------------------------------------------------------

void split_qkv_heads_rotary(const Tensor& qkv, int heads, int dim_head, const Tensor& cos_freqs,
                            const Tensor& sin_freqs, Tensor& q, Tensor& k, Tensor& v) {
    if ((dim_head % 2) != 0) throw std::runtime_error("mbr_tile::split_qkv_heads_rotary: dim_head must be even");
    const Tensor x = float_contig(qkv, "mbr_tile::split_qkv_heads_rotary");
    const int64_t B = x.size(0), N = x.size(1);
    if (x.ndim() != 3 || x.size(2) != 3LL * heads * dim_head)
        throw std::runtime_error("mbr_tile::split_qkv_heads_rotary: expected qkv [B, N, 3*heads*dim_head]");
    const bool out_bf16 = g_quantize_bf16 && dim_head <= 128;
    const bool pad64 = out_bf16 && x.dtype() == DType::BFloat16 && freq_attention60_padded() && N == kFreqAttnN &&
                       dim_head == kFreqAttnD;
    const int64_t out_n = pad64 ? kFreqAttnPadN : N;
    const DType odt = out_bf16 ? DType::BFloat16 : DType::Float32;
    const Tensor c = f32_or_bf16(cos_freqs), s = f32_or_bf16(sin_freqs);
    if (c.dtype() != s.dtype()) throw std::runtime_error("mbr_tile::split_qkv_heads_rotary: cos/sin dtypes differ");
    if (c.numel() < N * (dim_head / 2) || s.numel() < N * (dim_head / 2))
        throw std::runtime_error("mbr_tile::split_qkv_heads_rotary: cos/sin tables shorter than [N, dim_head/2]");
    q = Tensor::empty({B, (int64_t)heads, out_n, (int64_t)dim_head}, odt);
    k = Tensor::empty({B, (int64_t)heads, out_n, (int64_t)dim_head}, odt);
    v = Tensor::empty({B, (int64_t)heads, out_n, (int64_t)dim_head}, odt);
    if (x.numel() == 0) return;
    FullBf16Scope full_bf16;
    abi_check(mbrt_split_qkv_heads_rotary(x.data_ptr(), code(x.dtype()), c.data_ptr(), s.data_ptr(), code(c.dtype()),
                                          q.data_ptr(), k.data_ptr(), v.data_ptr(), code(odt), B, N, heads, dim_head,
                                          out_n, abi_stream()),
              "mbr_tile::split_qkv_heads_rotary");
}

namespace {
void rotary_inplace(Tensor& q, Tensor* k, const Tensor& cos_freqs, const Tensor& sin_freqs, const char* op) {
    if (q.ndim() != 4 || (k && k->shape() != q.shape()))
        throw std::runtime_error(std::string(op) + ": expected q/k [B, N, heads, dim_head]");
    if (!q.is_contiguous() || (k && !k->is_contiguous()))
        throw std::runtime_error(std::string(op) + ": expected contiguous q/k");
    if (!is_float(q.dtype()) || (k && k->dtype() != q.dtype()))
        throw std::runtime_error(std::string(op) + ": expected floating-point q/k of one dtype");
    const int64_t N = q.size(1), H = q.size(2), D = q.size(3);
    if (cos_freqs.ndim() != 2 || sin_freqs.ndim() != 2 || cos_freqs.size(0) != N || sin_freqs.size(0) != N ||
        cos_freqs.size(1) != D / 2 || sin_freqs.size(1) != D / 2)
        throw std::runtime_error(std::string(op) + ": expected cos/sin [N, dim_head/2]");
    const Tensor c = f32_or_bf16(cos_freqs), s = f32_or_bf16(sin_freqs);
    if (c.dtype() != s.dtype()) throw std::runtime_error(std::string(op) + ": cos/sin dtypes differ");
    if (q.numel() == 0) return;
    FullBf16Scope full_bf16;
    abi_check(mbrt_rotary_inplace(q.data_ptr(), k ? k->data_ptr() : nullptr, code(q.dtype()), c.data_ptr(),
                                  s.data_ptr(), code(c.dtype()), q.numel() / D, N, H, D, MBRT_LAYOUT_BNHD,
                                  abi_stream()),
              op);
}
}  // namespace

void apply_rotary_time_split_contig_inplace(Tensor& q, Tensor& k, const Tensor& cos_freqs, const Tensor& sin_freqs) {
    rotary_inplace(q, &k, cos_freqs, sin_freqs, "mbr_tile::apply_rotary_time_split_contig_inplace");
}

void apply_rotary_time_split_contig_k_only_inplace(Tensor& k, const Tensor& cos_freqs, const Tensor& sin_freqs) {
    rotary_inplace(k, nullptr, cos_freqs, sin_freqs, "mbr_tile::apply_rotary_time_split_contig_k_only_inplace");
}

namespace {
Tensor gate_merge(const Tensor& attn, const Tensor& gates, int heads, int dim_head, bool logits, const char* op) {
    const Tensor a = float_contig(attn, op), g = f32_or_bf16(gates);
    if (a.ndim() != 4 || a.size(1) != heads || a.size(3) != dim_head)
        throw std::runtime_error(std::string(op) + ": expected attn [B, heads, N, dim_head]");
    const int64_t B = a.size(0), N = a.size(2);
    if (g.numel() != B * N * heads) throw std::runtime_error(std::string(op) + ": expected gates [B, N, heads]");
    const DType odt = gate_merge_bf16() ? DType::BFloat16 : DType::Float32;
    Tensor merged = Tensor::empty({B, N, (int64_t)heads * dim_head}, odt);
    if (merged.numel() == 0) return merged;
    FullBf16Scope full_bf16;
    abi_check(mbrt_sigmoid_gate_merge(a.data_ptr(), code(a.dtype()), g.data_ptr(), code(g.dtype()), logits ? 1 : 0,
                                      merged.data_ptr(), code(odt), B, heads, N, dim_head, MBRT_LAYOUT_BHND,
                                      abi_stream()),
              op);
    return merged;
}
}  // namespace

Tensor apply_gates_and_merge_heads(const Tensor& attn, const Tensor& gates, int heads, int dim_head) {
    return gate_merge(attn, gates, heads, dim_head, false, "mbr_tile::apply_gates_and_merge_heads");
}

Tensor apply_gate_logits_and_merge_heads(const Tensor& attn, const Tensor& gate_logits, int heads, int dim_head) {
    return gate_merge(attn, gate_logits, heads, dim_head, true, "mbr_tile::apply_gate_logits_and_merge_heads");
}

Tensor scaled_dot_product_attention(const Tensor& q, const Tensor& k, const Tensor& v, float scale) {
    const char* op = "mbr_tile::scaled_dot_product_attention";
    if (q.ndim() != 4 || k.ndim() != 4 || v.ndim() != 4 || k.shape() != v.shape() || q.size(0) != k.size(0) ||
        q.size(1) != k.size(1) || q.size(3) != k.size(3))
        throw std::runtime_error(std::string(op) + ": expected q [B, H, N, D] and k, v [B, H, N_k, D]");
    auto bf16 = [](const Tensor& t) { return t.dtype() == DType::BFloat16 ? t.contiguous() : t.to_bf16().contiguous(); };
    const Tensor qb = bf16(q), kb = bf16(k), vb = bf16(v);
    const int64_t B = q.size(0), H = q.size(1), N = q.size(2), Nk = k.size(2), D = q.size(3);
    const DType odt = g_quantize_bf16 ? DType::BFloat16 : DType::Float32;
    Tensor out = Tensor::empty({B, H, N, D}, odt);
    if (out.numel() == 0) return out;
    abi_check(mbrt_attention(qb.data_ptr(), kb.data_ptr(), vb.data_ptr(), MBRT_BF16, out.data_ptr(), code(odt), B * H, N,
                             Nk, D, scale, abi_stream()),
              op);
    return out;
}

namespace {
// The reference's split-contig time attention (src/mbr_cuda_tile.cu:6417-6527): q, k, v
// [B, N, H, D] bf16 with unit inner stride, read through their strides.
Tensor split_contig_attention(const char* op, const Tensor& q, const Tensor& k, const Tensor& v, const Tensor* cos_f,
                              const Tensor* sin_f, float scale) {
    if (q.dtype() != DType::BFloat16 || k.dtype() != DType::BFloat16 || v.dtype() != DType::BFloat16)
        throw std::runtime_error(std::string(op) + ": expected BF16 q/k/v");
    if (q.ndim() != 4 || k.shape() != q.shape() || v.shape() != q.shape())
        throw std::runtime_error(std::string(op) + ": expected q/k/v [B, N, H, D] of one shape");
    const int64_t B = q.size(0), N = q.size(1), H = q.size(2), D = q.size(3);
    if (B <= 0 || B * H > std::numeric_limits<int>::max())
        throw std::runtime_error(std::string(op) + ": invalid batch count");
    auto inner = [](const Tensor& t) { return t.strides()[3] == 1 ? t : t.contiguous(); };
    Tensor qb = inner(q), kb = inner(k), vb = inner(v);
    if (kb.strides() != vb.strides()) vb = vb.contiguous(), kb = kb.contiguous();
    Tensor cw, sw;
    if (cos_f) {
        if (cos_f->ndim() != 2 || sin_f->ndim() != 2 || cos_f->size(0) != N || sin_f->size(0) != N ||
            cos_f->size(1) != D / 2 || sin_f->size(1) != D / 2)
            throw std::runtime_error(std::string(op) + ": expected cos/sin [N, D/2]");
        const bool bf = cos_f->dtype() == DType::BFloat16 && sin_f->dtype() == DType::BFloat16;
        cw = bf ? cos_f->contiguous() : (cos_f->dtype() == DType::Float32 ? cos_f->contiguous() : cos_f->to_f32().contiguous());
        sw = bf ? sin_f->contiguous() : (sin_f->dtype() == DType::Float32 ? sin_f->contiguous() : sin_f->to_f32().contiguous());
    }
    Tensor out = Tensor::empty({B, H, N, D}, DType::BFloat16);
    abi_check(mbrt_attention_strided(qb.data_ptr(), kb.data_ptr(), vb.data_ptr(), MBRT_BF16, B, H, N, N, D,
                                     qb.strides()[0], qb.strides()[2], qb.strides()[1], kb.strides()[0],
                                     kb.strides()[2], kb.strides()[1],
                                     cos_f ? cw.data_ptr() : nullptr, cos_f ? sw.data_ptr() : nullptr,
                                     cos_f ? code(cw.dtype()) : MBRT_F32, nullptr, MBRT_F32, 0, out.data_ptr(),
                                     MBRT_BF16, scale, abi_stream()),
              op);
    return out;
}
}  // namespace

Tensor scaled_dot_product_attention_time_split_contig(const Tensor& q, const Tensor& k, const Tensor& v, float scale) {
    return split_contig_attention("mbr_tile::scaled_dot_product_attention_time_split_contig", q, k, v, nullptr,
                                  nullptr, scale);
}

Tensor scaled_dot_product_attention_time_split_contig_q_rotary(const Tensor& q, const Tensor& k, const Tensor& v,
                                                               const Tensor& cos_freqs, const Tensor& sin_freqs,
                                                               float scale) {
    return split_contig_attention("mbr_tile::scaled_dot_product_attention_time_split_contig_q_rotary", q, k, v,
                                  &cos_freqs, &sin_freqs, scale);
}

Tensor softmax_last_dim(const Tensor& x, float scale, DType out_dtype) {
    const Tensor xc = float_contig(x, "mbr_tile::softmax_last_dim");
    Tensor out = Tensor::empty(xc.shape(), out_dtype);
    if (xc.numel() == 0) return out;
    const int64_t cols = xc.size(xc.ndim() - 1);
    FullBf16Scope full_bf16;
    abi_check(mbrt_softmax_rows(xc.data_ptr(), code(xc.dtype()), out.data_ptr(), code(out_dtype), xc.numel() / cols,
                                cols, scale, abi_stream()),
              "mbr_tile::softmax_last_dim");
    return out;
}

void softmax_last_dim_(Tensor& x, float scale) {
    if (!x.is_contiguous()) throw std::runtime_error("mbr_tile::softmax_last_dim_: expected a contiguous tensor");
    if (x.numel() == 0) return;
    const int64_t cols = x.size(x.ndim() - 1);
    FullBf16Scope full_bf16;
    abi_check(mbrt_softmax_rows(x.data_ptr(), code(x.dtype()), x.data_ptr(), code(x.dtype()), x.numel() / cols, cols,
                                scale, abi_stream()),
              "mbr_tile::softmax_last_dim_");
}

// ---- activations ---------------------------------------------------------------------------

Tensor add_bias_activation(const Tensor& x, const Tensor* bias, Activation act, DType out_dtype) {
    const Tensor xc = float_contig(x, "mbr_tile::add_bias_activation");
    Tensor out = Tensor::empty(xc.shape(), out_dtype);
    if (xc.numel() == 0) return out;
    const int64_t cols = xc.size(xc.ndim() - 1);
    Tensor b;
    if (bias) {
        b = f32_or_bf16(*bias);
        if (b.numel() != cols) throw std::runtime_error("mbr_tile::add_bias_activation: bias size mismatch");
    }
    abi_check(mbrt_bias_act(xc.data_ptr(), code(xc.dtype()), bias ? b.data_ptr() : nullptr,
                            bias ? code(b.dtype()) : MBRT_F32, out.data_ptr(), code(out_dtype), xc.numel() / cols, cols,
                            (int)act, abi_stream()),
              "mbr_tile::add_bias_activation");
    return out;
}

// src/mbr_cuda_tile.cu:8098-8121
Tensor tanh_act(const Tensor& x) {
    DType odt;
    if (g_quantize_bf16 && tanh_bf16_input() && x.dtype() == DType::BFloat16) odt = DType::BFloat16;
    else odt = g_quantize_bf16 ? DType::BFloat16 : f32_pipeline_out(x.dtype());
    return add_bias_activation(x, nullptr, Activation::Tanh, odt);
}

// src/mbr_cuda_tile.cu:8123-8165
Tensor glu_last_dim(const Tensor& x) {
    const Tensor xc = float_contig(x, "glu_last_dim");
    const int64_t full = xc.size(xc.ndim() - 1);
    if ((full % 2) != 0) throw std::runtime_error("glu_last_dim: last dimension must be even");
    DType odt;
    if (glu_bf16_input() && glu_bf16_output() && xc.dtype() == DType::BFloat16) odt = DType::BFloat16;
    else odt = glu_bf16_output() ? DType::BFloat16 : f32_pipeline_out(xc.dtype());
    std::vector<int64_t> shape = xc.shape();
    shape.back() = full / 2;
    Tensor out = Tensor::empty(shape, odt);
    if (out.numel() == 0) return out;
    FullBf16Scope full_bf16;
    abi_check(mbrt_glu_last_dim(xc.data_ptr(), code(xc.dtype()), out.data_ptr(), code(odt), xc.numel() / full,
                                full / 2, abi_stream()),
              "glu_last_dim");
    return out;
}

// ---- band split / merge ---------------------------------------------------------------------

// src/mbr_cuda_tile.cu:6215-6241
Tensor gather_freqs_fold_complex(const Tensor& stft_repr, const Tensor& freq_indices) {
    const Tensor s = stft_repr.dtype() == DType::Float32 ? stft_repr.contiguous() : stft_repr.to_f32().contiguous();
    if (s.ndim() != 4 || s.size(3) != 2)
        throw std::runtime_error("mbr_tile::gather_freqs_fold_complex: expected [B, F, T, 2]");
    if (freq_indices.dtype() != DType::Int64)
        throw std::runtime_error("mbr_tile::gather_freqs_fold_complex: freq_indices must be Int64");
    const Tensor idx = freq_indices.contiguous();
    const int64_t B = s.size(0), F = s.size(1), T = s.size(2), J = idx.numel();
    const DType odt = gather_bf16_output() ? DType::BFloat16 : DType::Float32;
    Tensor out = Tensor::empty({B, T, J * 2}, odt);
    if (out.numel() == 0) return out;
    abi_check(mbrt_band_gather((const float*)s.data_ptr(), idx.data_ptr(), MBRT_I64, out.data_ptr(), code(odt), B, F, T,
                               J, abi_stream()),
              "mbr_tile::gather_freqs_fold_complex");
    return out;
}

// src/mbr_cuda_tile.cu:7951-8081.  Every output element is the sum over its freq's bands
// in ascending CSR order, divided by max(count, 1e-8), written once (no zero fill, no
// atomics).  When the reverse index tensors are not a valid CSR for freq_indices (the
// reference reads them only on its bf16-output path), it is rebuilt from freq_indices.
Tensor apply_mask_and_scatter(const Tensor& stft_repr, const std::vector<Tensor>& stem_masks,
                              const Tensor& freq_indices, const Tensor& freq_band_offsets,
                              const Tensor& freq_band_indices, const Tensor& bands_per_freq, int64_t batch,
                              int64_t num_stems, int64_t total_freq, int64_t total_band_freqs, int64_t frames,
                              int64_t audio_channels, int64_t /*max_bands_per_freq*/) {
    const char* op = "mbr_tile::apply_mask_and_scatter";
    if ((int64_t)stem_masks.size() != num_stems) throw std::runtime_error(std::string(op) + ": stem mask count mismatch");
    if (num_stems < 1 || num_stems > 2) throw std::runtime_error(std::string(op) + ": expected one or two stems");
    const bool out_bf16 = stft_result_bf16();
    const bool masks_bf16 = mask_scatter_bf16() || out_bf16;
    const DType mdt = masks_bf16 ? DType::BFloat16 : DType::Float32;
    std::vector<Tensor> masks;
    for (const Tensor& m : stem_masks) {
        Tensor w = m.dtype() == mdt ? m.contiguous() : m.to_dtype(mdt).contiguous();
        if (w.ndim() != 3 || w.size(0) != batch || w.size(1) != frames || w.size(2) != total_band_freqs * 2)
            throw std::runtime_error(std::string(op) + ": expected [B, T, total_band_freqs * 2]");
        masks.push_back(w);
    }
    if (audio_channels < 1 || total_freq % audio_channels != 0)
        throw std::runtime_error(std::string(op) + ": invalid audio channel count");
    if (bands_per_freq.dtype() != DType::Float32 && bands_per_freq.dtype() != DType::BFloat16)
        throw std::runtime_error(std::string(op) + ": expected FP32/BF16 bands_per_freq");
    const Tensor stft = stft_repr.dtype() == DType::Float32 ? stft_repr.contiguous() : stft_repr.to_f32().contiguous();
    if (stft.numel() != batch * total_freq * frames * 2)
        throw std::runtime_error(std::string(op) + ": expected stft [B, total_freq, T, 2]");
    const Tensor counts = bands_per_freq.contiguous();

    Tensor offsets = freq_band_offsets, indices = freq_band_indices;
    const bool csr_ok = offsets.dtype() == DType::Int64 && offsets.numel() == total_freq + 1 &&
                        indices.dtype() == DType::Int64 && indices.numel() == total_band_freqs;
    if (!csr_ok) {
        if (freq_indices.dtype() != DType::Int64 || freq_indices.numel() != total_band_freqs)
            throw std::runtime_error(std::string(op) + ": invalid reverse band index");
        std::vector<int64_t> fi((size_t)total_band_freqs);
        freq_indices.contiguous().copy_to_cpu(fi.data(), fi.size() * 8);
        std::vector<int32_t> fi32(fi.begin(), fi.end()), off((size_t)total_freq + 1), ind((size_t)total_band_freqs);
        abi_check(mbrt_band_csr(fi32.data(), total_band_freqs, total_freq, off.data(), ind.data(), nullptr, nullptr), op);
        std::vector<int64_t> off64(off.begin(), off.end()), ind64(ind.begin(), ind.end());
        offsets = Tensor::from_cpu_i64(off64.data(), {total_freq + 1});
        indices = Tensor::from_cpu_i64(ind64.data(), {std::max<int64_t>(total_band_freqs, 1)});
    } else {
        offsets = offsets.contiguous();
        indices = indices.contiguous();
    }

    const DType odt = out_bf16 ? DType::BFloat16 : DType::Float32;
    Tensor out = Tensor::empty({batch * num_stems * audio_channels, total_freq / audio_channels, frames, 2}, odt);
    if (out.numel() == 0) return out;
    const void* mptr[2] = {masks[0].data_ptr(), masks[num_stems - 1].data_ptr()};
    FullBf16Scope full_bf16;
    abi_check(mbrt_band_mask_merge((const float*)stft.data_ptr(), mptr, code(mdt), (int)num_stems, offsets.data_ptr(),
                                   indices.data_ptr(), MBRT_I64, counts.data_ptr(), code(counts.dtype()),
                                   out.data_ptr(), code(odt), batch, total_freq, frames, total_band_freqs,
                                   audio_channels, abi_stream()),
              op);
    return out;
}

// src/mbr_cuda_tile.cu:8083-8096: bin 0 of every [F, T, 2] plane
void zero_dc(Tensor& complex_spec) {
    if (complex_spec.ndim() < 3) throw std::runtime_error("mbr_tile::zero_dc: expected [.., F, T, 2]");
    if (!complex_spec.is_contiguous()) throw std::runtime_error("mbr_tile::zero_dc: expected a contiguous tensor");
    const int64_t F = complex_spec.size(1), T = complex_spec.size(2);
    if (complex_spec.numel() == 0) return;
    const int64_t outer = complex_spec.numel() / (F * T * 2);
    abi_check(mbrt_zero_dc(complex_spec.data_ptr(), code(complex_spec.dtype()), outer, F, T, abi_stream()),
              "mbr_tile::zero_dc");
}

}  // namespace cudasep::mbr_tile
