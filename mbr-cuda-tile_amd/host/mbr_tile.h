// cudasep::mbr_tile — the memory-bound MelBandRoformer ops of the reference's model
// library (src/mbr_cuda_tile.h), same names, arguments and dtype policies, on libmbrt's
// gfx950 kernels.  The GEMM and fused-attention entry points of that header are outside
// this library; the epilogues they end in (bias + GELU / sigmoid, row softmax) are
// exported as their own functions below.
#pragma once

#include <vector>

#include "tensor.h"

namespace cudasep::mbr_tile {

// ---- precision policies (env switches and g_quantize_bf16, src/mbr_cuda_tile.cu:103-354)
bool residual_bf16_enabled();
bool bias_bf16_enabled();
bool norm_gamma_bf16_enabled();
bool bands_per_freq_bf16_enabled();
bool rotary_freqs_bf16_enabled();
bool residual_rms_norm_fused_path_enabled();

// ---- time-attention context (src/mbr_cuda_tile.h:92-94, src/mbr_cuda_tile.cu:83-84,
// 5988-5994).  Per-thread chunk and depth indices that the application sets around each
// model call (src/inference_app.cpp:32-40) and the model around each time-transformer
// layer (src/model_mel_band_roformer.cu:745-802); -1 means unset.  No op depends on them,
// as in the reference; the getters let a caller read back what it set.
void set_time_attention_context_chunk(int chunk_index);
void set_time_attention_context_depth(int depth_index);
int time_attention_context_chunk();
int time_attention_context_depth();

// ---- normalisation
// y = x * scale * gamma / sqrt(sum x^2 + 1e-12) over the last dim (src/mbr_cuda_tile.cu:6297-6373).
// Output BF16 under the RMS-norm bf16 policy, else F32 (F16 for F16 input).
Tensor rms_norm(const Tensor& x, const Tensor& gamma, float scale);

// residual_out = residual + update (in residual's dtype), normed = rms_norm(residual_out)
// in one pass (src/mbr_cuda_tile.cu:6375-6417).  Unlike the reference, which fuses only
// bf16 rows of 256, every dim and dtype is fused; false is returned only when the fused
// path is disabled (CUDASEP_DISABLE_RESIDUAL_RMS_NORM_FUSED) or the operands do not
// match, and the caller then adds and normalises separately, as in the reference.
bool try_residual_add_rms_norm(const Tensor& residual, const Tensor& update, const Tensor& gamma, float scale,
                               Tensor& residual_out, Tensor& normed);

// ---- attention plumbing
// qkv [B, N, 3*heads*dim_head] -> q, k, v [B, heads, N', dim_head] with rotary on q and k
// (src/mbr_cuda_tile.cu:6058-6213).  N' = 64 for the bf16 N = 60, D = 64 frequency
// attention (zero rows 60..63), else N.
void split_qkv_heads_rotary(const Tensor& qkv, int heads, int dim_head, const Tensor& cos_freqs,
                            const Tensor& sin_freqs, Tensor& q, Tensor& k, Tensor& v);

// In-place rotary on contiguous q, k [B, N, heads, dim_head] with cos/sin [N, dim_head/2]
// (src/mbr_cuda_tile.cu:7454-7584), for any B, N, heads, even dim_head.
void apply_rotary_time_split_contig_inplace(Tensor& q, Tensor& k, const Tensor& cos_freqs, const Tensor& sin_freqs);
void apply_rotary_time_split_contig_k_only_inplace(Tensor& k, const Tensor& cos_freqs, const Tensor& sin_freqs);

// merged[b, n, h*D + d] = attn[b, h, n, d] * gates[b, n, h] (src/mbr_cuda_tile.cu:6243-6295).
Tensor apply_gates_and_merge_heads(const Tensor& attn, const Tensor& gates, int heads, int dim_head);
// Same with the gate logits: sigmoid fused into the merge (linear_sigmoid's epilogue and
// the merge in one pass).
Tensor apply_gate_logits_and_merge_heads(const Tensor& attn, const Tensor& gate_logits, int heads, int dim_head);

// softmax(scale q k^T) v for q [B, H, N, D], k and v [B, H, N_k, D] with D = 64, fused on
// MFMA without the [B*H, N, N_k] score tensor (src/mbr_cuda_tile.cu:6530-6709); scale 0
// means 1/sqrt(D).  Inputs that are not bf16 are converted to bf16 first; the result is
// BF16 under g_quantize_bf16, else F32.
Tensor scaled_dot_product_attention(const Tensor& q, const Tensor& k, const Tensor& v, float scale);

// Time attention straight from the split-contig projection layout: q, k, v [B, N, H, D]
// bf16 (views of the fused qkv are read in place through their strides) -> [B, H, N, D]
// bf16; the _q_rotary form rotates q in the kernel with cos/sin [N, D/2] (F32 or BF16;
// other dtypes go to F32).  src/mbr_cuda_tile.cu:6417-6527, generalised from N = 1301,
// H = 8 and scale 1/8 (0 still means 1/sqrt(D)).  Throws "expected BF16 q/k/v" and
// shape errors as the reference does.
Tensor scaled_dot_product_attention_time_split_contig(const Tensor& q, const Tensor& k, const Tensor& v, float scale);
Tensor scaled_dot_product_attention_time_split_contig_q_rotary(const Tensor& q, const Tensor& k, const Tensor& v,
                                                               const Tensor& cos_freqs, const Tensor& sin_freqs,
                                                               float scale);

// Row softmax of attention scores over the last dim, p = softmax(scale * x), f32
// accumulation (the scale_softmax kernels, src/mbr_cuda_tile.cu:5092-5285).
Tensor softmax_last_dim(const Tensor& x, float scale, DType out_dtype);
void softmax_last_dim_(Tensor& x, float scale);

// ---- activations
// act(x + bias) over the last dim, the linear-layer epilogues (src/mbr_cuda_tile.cu:5474-5584).
enum class Activation { None = 0, GeluRef = 1, GeluStd = 2, Sigmoid = 3, Tanh = 4 };
Tensor add_bias_activation(const Tensor& x, const Tensor* bias, Activation act, DType out_dtype);
Tensor tanh_act(const Tensor& x);
Tensor glu_last_dim(const Tensor& x);

// ---- band split / merge
Tensor gather_freqs_fold_complex(const Tensor& stft_repr, const Tensor& freq_indices);
Tensor apply_mask_and_scatter(const Tensor& stft_repr, const std::vector<Tensor>& stem_masks,
                              const Tensor& freq_indices, const Tensor& freq_band_offsets,
                              const Tensor& freq_band_indices, const Tensor& bands_per_freq, int64_t batch,
                              int64_t num_stems, int64_t total_freq, int64_t total_band_freqs, int64_t frames,
                              int64_t audio_channels, int64_t max_bands_per_freq = 0);
void zero_dc(Tensor& complex_spec);

}  // namespace cudasep::mbr_tile
