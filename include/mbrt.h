/*
 * mbrt.h — C-ABI of the MI355X (gfx950) tensor-op library behind the
 * MelBandRoformer tensor API (Tensor / tensor_tile:: / mbr_tile::).
 *
 * Conventions
 *   - Every entry point returns an int status: MBRT_OK (0) or an MBRT_E_* code.
 *     mbrt_last_error() returns a thread-local message for the last failure
 *     on the calling thread.
 *   - All data pointers are DEVICE pointers (hipMalloc'd or views into such
 *     memory) unless a parameter says "host".  Sizes are element counts.
 *   - The library never allocates or frees memory: the caller owns every buffer.
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*; NULL is the
 *     null stream).  Calls are asynchronous with respect to the host.
 *   - Metadata structs are read on the host during the call and passed to
 *     kernels by value; no device-side metadata buffer exists, so calls on
 *     different streams are independent.
 *   - Inputs must not overlap outputs, except where an entry point documents
 *     in-place operation (out == in).
 *   - Vector (16-byte) paths are chosen only when every pointer and row pitch
 *     involved is suitably aligned; otherwise a scalar path runs.  Alignment is
 *     never an error.
 *
 * Dtype codes equal the reference's DType values (src/tensor.h:17), which are
 * also the .csm tensor ids (src/weights.h:94); MBRT_I32 is added for indices.
 *
 * Reference citations below are paths inside baicai-1145/MBR-CUDA-Tile.
 */
#ifndef MBRT_H
#define MBRT_H

#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define MBRT_API __attribute__((visibility("default")))
#else
#define MBRT_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mbrt_stream_t; /* hipStream_t */

enum mbrt_dtype {
    MBRT_F32 = 0,
    MBRT_F16 = 1,
    MBRT_I64 = 2,
    MBRT_BF16 = 3,
    MBRT_I32 = 4
};

enum mbrt_status {
    MBRT_OK = 0,
    MBRT_E_INVALID_ARG = 1,
    MBRT_E_UNSUPPORTED_DTYPE = 2,
    MBRT_E_SHAPE = 3,
    MBRT_E_ALIGN = 4,
    MBRT_E_HIP = 5
};

#define MBRT_MAX_DIMS 8

/* Same fields as tensor_tile::StridedCopyMeta (src/tensor_cuda_tile.h:9-13).
 * Strides are in elements; dst is contiguous with shape dst_shape. */
typedef struct mbrt_strided_meta {
    int64_t src_strides[MBRT_MAX_DIMS];
    int64_t dst_shape[MBRT_MAX_DIMS];
    int32_t ndim;
} mbrt_strided_meta;

/* Same fields as tensor_tile::BroadcastMeta (src/tensor_cuda_tile.h:15-20). */
typedef struct mbrt_broadcast_meta {
    int64_t out_shape[MBRT_MAX_DIMS];
    int64_t a_strides[MBRT_MAX_DIMS];
    int64_t b_strides[MBRT_MAX_DIMS];
    int32_t ndim;
} mbrt_broadcast_meta;

/* Same fields as tensor_tile::PadMeta (src/tensor_cuda_tile.h:22-27).
 * The source is contiguous with shape src_shape. */
typedef struct mbrt_pad_meta {
    int64_t src_shape[MBRT_MAX_DIMS];
    int64_t dst_shape[MBRT_MAX_DIMS];
    int64_t pad_before[MBRT_MAX_DIMS];
    int32_t ndim;
} mbrt_pad_meta;

/* Same fields as tensor_tile::CatSrcInfo (src/tensor_cuda_tile.h:29-33). */
typedef struct mbrt_cat_src {
    const void* ptr;    /* device pointer to a contiguous source */
    int64_t dim_size;   /* its extent along the concat dim */
    int64_t dim_offset; /* where it starts along the concat dim of the output */
} mbrt_cat_src;

enum mbrt_binary_op { MBRT_ADD = 0, MBRT_SUB = 1, MBRT_MUL = 2, MBRT_DIV = 3 };
enum mbrt_scalar_op { MBRT_SCALAR_ADD = 0, MBRT_SCALAR_MUL = 1, MBRT_SCALAR_CLAMP = 2 };
enum mbrt_unary_op { MBRT_UNARY_NEG = 0, MBRT_UNARY_GT = 1 };
enum mbrt_reduce_op { MBRT_REDUCE_SUM = 0, MBRT_REDUCE_MAX = 1 };
enum mbrt_act {
    MBRT_ACT_NONE = 0,
    MBRT_ACT_GELU_REF = 1, /* 0.5 x (1 + erf(x)): the reference's GELU kernels */
    MBRT_ACT_GELU_STD = 2, /* 0.5 x (1 + erf(x / sqrt 2)): torch nn.GELU() */
    MBRT_ACT_SIGMOID = 3,
    MBRT_ACT_TANH = 4
};
enum mbrt_layout {
    MBRT_LAYOUT_BHND = 0, /* [B, H, N, D]: heads outside tokens */
    MBRT_LAYOUT_BNHD = 1  /* [B, N, H, D]: tokens outside heads */
};

/* ---- library state -------------------------------------------------------- */

/* Message for the last failing call on this thread ("" if none). */
MBRT_API const char* mbrt_last_error(void);
/* ABI version: major * 10000 + minor * 100 + patch. */
MBRT_API int mbrt_version(void);
/* Blocks until all work on `stream` has finished; reports asynchronous errors. */
MBRT_API int mbrt_stream_sync(mbrt_stream_t stream);

/* Arithmetic flags of the calling thread, read by every later call it makes (0 = default).
 * MBRT_ARITH_BF16_INTERMEDIATES is the reference's full-bf16 experiment mode
 * (full_bf16_arith_enabled(), src/mbr_cuda_tile.cu:190-192, which its host dispatch passes
 * to the kernels as `full_bf16`): the ops below round their intermediates to bf16 at the
 * points its kernels do, under the same dtype conditions (each op's comment says which).
 * Ops and dtypes without such a path compute as by default.  The reference reads the
 * switch from the environment; here the caller sets it, and mbr_tile:: does so from
 * CUDASEP_FULL_BF16_ARITH_EXPERIMENTS under bf16.  Unknown bits are rejected. */
enum mbrt_arith_flag { MBRT_ARITH_BF16_INTERMEDIATES = 1 };
MBRT_API int mbrt_set_arith_flags(uint32_t flags);
MBRT_API uint32_t mbrt_get_arith_flags(void);

/* ---- flat element-wise (tensor_tile, src/tensor_cuda_tile.cu) -------------- */

/* dst[i] = value for i < n.  Replaces tensor_tile::fill (src/tensor_cuda_tile.cu:403-420).
 * Writes `value` even where dst held NaN/Inf (the reference's load*0+value yields NaN there). */
MBRT_API int mbrt_fill(void* dst, int dtype, int64_t n, double value, mbrt_stream_t stream);

/* dst[i] = start + i.  Replaces tensor_tile::arange (src/tensor_cuda_tile.cu:422-440);
 * BF16 is rejected as in the reference. */
MBRT_API int mbrt_arange(void* dst, int dtype, int64_t n, int64_t start, mbrt_stream_t stream);

/* dst[i] = (dst_dtype) src[i].  Float narrowing rounds to nearest even; float to
 * integer truncates toward zero.  Replaces tensor_tile::convert_dtype
 * (src/tensor_cuda_tile.cu:442-472); also accepts I32 on either side. */
MBRT_API int mbrt_convert(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n,
                 mbrt_stream_t stream);

/* In place: ADD x+a, MUL x*a, CLAMP min(max(x,a),b).  F32/F16 only, as the
 * reference (tensor_tile::add_scalar/mul_scalar/clamp, src/tensor_cuda_tile.cu:474-521). */
MBRT_API int mbrt_scalar_op(void* data, int dtype, int64_t n, int op, float a, float b,
                   mbrt_stream_t stream);

/* NEG dst=-src; GT dst = src > value ? 1 : 0 in src's dtype (NaN gives 0).
 * F32/F16 only.  Replaces tensor_tile::negate / greater_than (src/tensor_cuda_tile.cu:523-551). */
MBRT_API int mbrt_unary(const void* src, void* dst, int dtype, int64_t n, int op, float value,
               mbrt_stream_t stream);

/* out[i] = a[i] op b[i] for contiguous same-shape operands; out may equal a
 * (in place).  F32/F16/BF16.  Replaces tensor_tile::binary_same_shape and
 * binary_inplace_same_shape (src/tensor_cuda_tile.cu:293-339, 553-577) and the
 * fixed-shape bf16 residual add (src/mbr_residual_cutile.cu:71-94). */
MBRT_API int mbrt_binary(const void* a, const void* b, void* out, int dtype, int64_t n, int op,
                mbrt_stream_t stream);

/* Broadcast binary: out (contiguous, meta->out_shape) = a op b, where a and b are
 * addressed through meta->a_strides / b_strides (0 on broadcast dims).  out may
 * equal a when a is contiguous with out's shape (set a_strides accordingly).
 * Replaces tensor_tile::binary_glue / binary_inplace_glue (src/tensor_cuda_glue.cu:561-602). */
MBRT_API int mbrt_binary_broadcast(const void* a, const void* b, void* out, int dtype,
                          const mbrt_broadcast_meta* meta, int op, mbrt_stream_t stream);

/* ---- layout (tensor_tile glue, src/tensor_cuda_glue.cu) ------------------- */

/* dst (contiguous, meta->dst_shape) = src read through meta->src_strides: permute,
 * contiguous(), clone of a view.  Any dtype; bit-exact.  Replaces
 * tensor_tile::strided_copy_glue (src/tensor_cuda_glue.cu:615-638). */
MBRT_API int mbrt_strided_copy(const void* src, void* dst, int dtype, const mbrt_strided_meta* meta,
                      mbrt_stream_t stream);

/* dst = src gathered along `select_dim` by `indices` (device, I64 or I32, n_idx of
 * them; meta->dst_shape[select_dim] == n_idx).  Indices out of
 * [0, src extent) are the caller's contract, as in the reference.
 * Replaces tensor_tile::index_select_glue (src/tensor_cuda_glue.cu:640-648). */
MBRT_API int mbrt_index_select(const void* src, void* dst, int dtype, const void* indices,
                      int index_dtype, int64_t n_idx, int64_t src_dim_size,
                      const mbrt_strided_meta* meta, int select_dim, mbrt_stream_t stream);

/* Constant pad of a contiguous source.  Replaces tensor_tile::pad_const_glue
 * (src/tensor_cuda_glue.cu:650-657). */
MBRT_API int mbrt_pad_const(const void* src, void* dst, int dtype, const mbrt_pad_meta* meta,
                   float value, mbrt_stream_t stream);

/* Reflect pad: c = |c|; if c >= n then c = 2(n-1) - c; then clamp to [0, n-1].
 * Replaces tensor_tile::pad_reflect_glue (src/tensor_cuda_glue.cu:659-666). */
MBRT_API int mbrt_pad_reflect(const void* src, void* dst, int dtype, const mbrt_pad_meta* meta,
                     mbrt_stream_t stream);

/* Concatenate n_srcs contiguous sources (host array `srcs`) into `out`.
 * Replaces tensor_tile::cat_glue (src/tensor_cuda_glue.cu:668-685). */
MBRT_API int mbrt_cat(void* out, const mbrt_cat_src* srcs, int n_srcs, int64_t outer_size,
             int64_t total_cat_dim, int64_t inner_bytes, mbrt_stream_t stream);

/* ---- reductions (F32 in, F32 out) ----------------------------------------- */

/* dst[o] = reduce_i src[o, i].  Replaces tensor_tile::sum_reduce_last_dim /
 * max_reduce_last_dim (src/tensor_cuda_tile.cu:579-595); no 2048-column limit. */
MBRT_API int mbrt_reduce_last_dim(const float* src, float* dst, int64_t outer, int64_t inner, int op,
                         mbrt_stream_t stream);

/* dst[o, i] = reduce_r src[o, r, i], r ascending (sum and max are bit-identical to
 * a sequential loop).  Replaces tensor_tile::sum_/max_reduce_general_glue
 * (src/tensor_cuda_glue.cu:687-696). */
MBRT_API int mbrt_reduce_general(const float* src, float* dst, int64_t outer, int64_t reduce,
                        int64_t inner, int op, mbrt_stream_t stream);

/* ---- normalisation (mbr_tile, src/mbr_cuda_tile.cu) ------------------------ */

/* out[r, d] = x[r, d] * scale * gamma[d] / sqrt(sum_d x[r, d]^2 + eps), f32 math.
 * x: F32/F16/BF16; gamma: F32/BF16; out: F32/F16/BF16.  Rows are contiguous with
 * pitch `dim`.  Replaces mbr_tile::rms_norm (src/mbr_cuda_tile.cu:6297-6373;
 * kernels 4791-5090), which uses eps = 1e-12.
 * MBRT_ARITH_BF16_INTERMEDIATES, BF16 out (kernels 4815-4843): x, sum x^2, 1/sqrt and
 * gamma are rounded to bf16 and out = bf16(((x * inv) * gamma) * scale). */
MBRT_API int mbrt_rms_norm(const void* x, int x_dtype, const void* gamma, int gamma_dtype, void* out,
                  int out_dtype, int64_t rows, int64_t dim, float scale, float eps,
                  mbrt_stream_t stream);

/* s = residual + update (rounded to sum_dtype, then normalised from the rounded
 * value); sum_out = s; normed = rms_norm(s).  residual/update share in_dtype.
 * sum_out may alias residual (in place) but not update.  Replaces
 * mbr_tile::try_residual_add_rms_norm (src/mbr_cuda_tile.cu:6375-6417; kernels
 * 4877-4965) without its D == 256 / bf16-only restriction.
 * MBRT_ARITH_BF16_INTERMEDIATES, BF16 normed: as mbrt_rms_norm of bf16(s); sum_out
 * keeps sum_dtype. */
MBRT_API int mbrt_residual_add_rms_norm(const void* residual, const void* update, int in_dtype,
                               const void* gamma, int gamma_dtype, void* sum_out,
                               int sum_dtype, void* normed, int normed_dtype, int64_t rows,
                               int64_t dim, float scale, float eps, mbrt_stream_t stream);

/* ---- activations ---------------------------------------------------------- */

/* out[r, c] = act(x[r, c] + bias[c]) for an [rows, cols] matrix (bias may be NULL).
 * x: F32/F16/BF16; bias: F32/BF16; out: F32/F16/BF16; out may equal x when the
 * dtypes match.  Replaces the linear-layer epilogues add_bias*, add_bias_sigmoid*,
 * add_bias_gelu* (src/mbr_cuda_tile.cu:5474-5584) and tanh_act / gelu in place
 * (5840-5878, 3793-3803, 8098-8121). */
MBRT_API int mbrt_bias_act(const void* x, int x_dtype, const void* bias, int bias_dtype, void* out,
                  int out_dtype, int64_t rows, int64_t cols, int act, mbrt_stream_t stream);

/* out[r, d] = x[r, d] * sigmoid(x[r, half_dim + d]) for x [rows, 2 * half_dim].
 * Replaces mbr_tile::glu_last_dim (src/mbr_cuda_tile.cu:8123-8165; kernels 5880-5942).
 * MBRT_ARITH_BF16_INTERMEDIATES, BF16 in and out (5918-5940): the sigmoid is rounded
 * to bf16 before the product. */
MBRT_API int mbrt_glu_last_dim(const void* x, int x_dtype, void* out, int out_dtype, int64_t rows,
                      int64_t half_dim, mbrt_stream_t stream);

/* Sigmoid gate and head merge: merged[b, n, h*D + d] = attn(b, h, n, d) * g(b, n, h)
 * with g = sigmoid(gate) when gate_is_logit, else gate as given.  attn is laid
 * out [B,H,N,D] (MBRT_LAYOUT_BHND, the attention output) or [B,N,H,D]
 * (MBRT_LAYOUT_BNHD); gate is [B, N, H]; merged is [B, N, H*D].  Replaces
 * linear_sigmoid's add_bias_sigmoid epilogue + mbr_tile::apply_gates_and_merge_heads
 * (src/mbr_cuda_tile.cu:7907-7949, 6243-6295; kernels 4603-4789).
 * MBRT_ARITH_BF16_INTERMEDIATES, BF16 attn (4718-4750): g and the product are rounded
 * to bf16, also for an F32 output. */
MBRT_API int mbrt_sigmoid_gate_merge(const void* attn, int attn_dtype, const void* gate,
                            int gate_dtype, int gate_is_logit, void* merged, int out_dtype,
                            int64_t B, int64_t H, int64_t N, int64_t D, int layout,
                            mbrt_stream_t stream);

/* ---- softmax -------------------------------------------------------------- */

/* Row softmax over `cols` with f32 accumulation: z = scale*x; p = exp(z - max z) / sum.
 * in: F32/F16/BF16; out: F32/F16/BF16; out may equal in (same dtype).  Rows are
 * contiguous with pitch `cols`.  Replaces the scale_softmax* kernels
 * (src/mbr_cuda_tile.cu:5092-5285, dispatch 6663-6697) without the 2048-column limit.
 * MBRT_ARITH_BF16_INTERMEDIATES, BF16 in and out (5224-5281): scale * x, the max, each
 * exp, the sum and each quotient are rounded to bf16. */
MBRT_API int mbrt_softmax_rows(const void* in, int in_dtype, void* out, int out_dtype, int64_t rows,
                      int64_t cols, float scale, mbrt_stream_t stream);

/* ---- rotary embedding ----------------------------------------------------- */

/* In-place rotary on q and (optionally, k != NULL) k, both [.., D] rows of dtype
 * `dtype` (F32/BF16/F16).  Pair (2i, 2i+1) at position n becomes
 * (x0 c - x1 s, x0 s + x1 c) with c = cos[n, i], s = sin[n, i], tables
 * [n_pos, D/2] of trig_dtype (F32/BF16).  layout BHND: tensor [B*H, n_pos, D];
 * BNHD: [B, n_pos, H, D].  `rows` = total rows (B*H*n_pos).  Replaces
 * mbr_tile::apply_rotary_time_split_contig_inplace (src/mbr_cuda_tile.cu:7454-7530;
 * kernels 4146-4377), generalised from its fixed [B,1301,8,64] shape.
 * MBRT_ARITH_BF16_INTERMEDIATES, BF16 data: c and s are rounded to bf16 first. */
MBRT_API int mbrt_rotary_inplace(void* q, void* k, int dtype, const void* cos_table,
                        const void* sin_table, int trig_dtype, int64_t rows, int64_t n_pos,
                        int64_t heads, int64_t dim_head, int layout, mbrt_stream_t stream);

/* Split fused qkv [B, N, 3*H*D] into q, k, v [B, H, out_N, D] with rotary on q and
 * k; rows n >= N of a padded output (out_N > N) are zero-filled in q, k and v.
 * Replaces mbr_tile::split_qkv_heads_rotary (src/mbr_cuda_tile.cu:6058-6213;
 * kernels 3897-4068, 4379-4552).
 * MBRT_ARITH_BF16_INTERMEDIATES, BF16 qkv and out (4000-4068): c and s are rounded to
 * bf16 first. */
MBRT_API int mbrt_split_qkv_heads_rotary(const void* qkv, int qkv_dtype, const void* cos_table,
                                const void* sin_table, int trig_dtype, void* q, void* k,
                                void* v, int out_dtype, int64_t B, int64_t N, int64_t H,
                                int64_t D, int64_t out_N, mbrt_stream_t stream);

/* ---- mel band split / merge ----------------------------------------------- */

/* Band gather: out[b, t, j, c] = stft[b, idx[j], t, c] for the interleaved-stereo
 * spectrum stft [B, total_freq, frames, 2] (F32) and idx [n_band_freqs]
 * (I32 or I64); out [B, frames, n_band_freqs, 2] of out_dtype (F32 bit-exact, or
 * BF16).  Replaces mbr_tile::gather_freqs_fold_complex (src/mbr_cuda_tile.cu:6215-6241;
 * kernels 4554-4601). */
MBRT_API int mbrt_band_gather(const float* stft, const void* freq_indices, int index_dtype,
                     void* out, int out_dtype, int64_t B, int64_t total_freq,
                     int64_t frames, int64_t n_band_freqs, mbrt_stream_t stream);

/* Mask multiply + overlap merge.  For every stem s, output row
 * o = (b*num_stems + s)*channels + ch, bin f and frame t (freq = f*channels + ch):
 *   out[o, f, t] = (sum over e in [offsets[freq], offsets[freq+1]) in ascending e of
 *                   stft[b, freq, t] * mask_s[b, t, indices[e]]) / max(count[freq], 1e-8)
 * (complex products).  masks: host array of num_stems (1 or 2) device pointers,
 * each [B, frames, n_band_freqs, 2] of mask_dtype (F32/BF16); offsets
 * [total_freq + 1] and indices [n_band_freqs] are the band-per-freq CSR (I32 or
 * I64, `index_dtype`); counts [total_freq] F32/BF16; out
 * [B*num_stems*channels, total_freq/channels, frames, 2] of out_dtype (F32/BF16).
 * Every output element is written exactly once (no atomics, no pre-zeroing).
 * Replaces mbr_tile::apply_mask_and_scatter (src/mbr_cuda_tile.cu:7951-8081;
 * kernels 5586-5803).
 * MBRT_ARITH_BF16_INTERMEDIATES with BF16 masks (5650-5799): a BF16 out sums the masks
 * first, rounding each partial sum to bf16, then divides stft * sum by the count and
 * rounds; an F32 out adds each entry's bf16-rounded stft * mask / count, in ascending e. */
MBRT_API int mbrt_band_mask_merge(const float* stft, const void* const* masks, int mask_dtype,
                         int num_stems, const void* csr_offsets, const void* csr_indices,
                         int index_dtype, const void* counts, int counts_dtype, void* out,
                         int out_dtype, int64_t B, int64_t total_freq, int64_t frames,
                         int64_t n_band_freqs, int64_t channels, mbrt_stream_t stream);

/* Zero frequency bin 0 of a complex spectrogram [outer, freq_bins, frames, 2]
 * (F32/BF16).  Writes 0 even over NaN/Inf (the reference's load*0 keeps NaN).
 * Replaces mbr_tile::zero_dc (src/mbr_cuda_tile.cu:8083-8096; kernels 5805-5838). */
MBRT_API int mbrt_zero_dc(void* spec, int dtype, int64_t outer, int64_t freq_bins, int64_t frames,
                 mbrt_stream_t stream);

/* ---- fused attention (MFMA) ---------------------------------------------------- */

/* out[bh, i, :] = sum_j softmax_j(scale * q[bh, i, :] . k[bh, j, :]) v[bh, j, :] for bf16
 * q [BH, n_q, head_dim], k and v [BH, n_k, head_dim] (contiguous, 16-byte aligned) and
 * out [BH, n_q, head_dim] of out_dtype (BF16/F32); scale > 0, or 0 for 1/sqrt(head_dim).
 * f32 accumulation and softmax; the probabilities enter the second product as a pair of
 * bf16 values (hi + lo), so the result has f32 accuracy.  head_dim 64 only.  Replaces mbr_tile::scaled_dot_product_attention
 * (src/mbr_cuda_tile.cu:6530-6709) and the time-attention kernels
 * (src/mbr_time_attention_cutile.cu:108-196) for every n_q / n_k, without the [BH, n, n]
 * score tensor. */
MBRT_API int mbrt_attention(const void* q, const void* k, const void* v, int dtype, void* out, int out_dtype,
                            int64_t BH, int64_t n_q, int64_t n_k, int64_t head_dim, float scale,
                            mbrt_stream_t stream);

/* The same attention over strided q, k, v, with optional in-kernel rotary of q and an
 * optional sigmoid-gate head-merge epilogue.  Head (b, h) of B x H, row n, element d sits
 * at q + b*q_batch_stride + h*q_head_stride + n*q_row_stride + d (k and v with the kv
 * strides; every stride a non-negative multiple of 8 elements).  [B, N, H, 64] views of a
 * fused qkv projection are strides (N*3*H*64, 64, 3*H*64).
 *  - rot_cos / rot_sin [n_q, 32] (F32/BF16, NULL for none): q row n is rotated as
 *    mbrt_rotary_inplace would (pairs (2i, 2i+1), f32, rounded to bf16) before use.
 *  - gate [B, n_q, H] (F32/BF16/F16, NULL for none): out is [B, n_q, H*64] with
 *    out[b, n, h*64 + d] = O * g, g = sigmoid(gate) when gate_is_logit, O first rounded
 *    to out_dtype: the result equals mbrt_sigmoid_gate_merge of the plain output.  Without
 *    a gate, out is [B*H, n_q, 64].
 * Replaces mbr_tile::scaled_dot_product_attention_time_split_contig[_q_rotary]
 * (src/mbr_cuda_tile.cu:6417-6527; kernels src/mbr_time_attention_cutile.cu:403-542),
 * generalised from N = 1301 and scale 1/8, and fuses apply_gates_and_merge_heads
 * (src/mbr_cuda_tile.cu:6243-6295) into the epilogue. */
MBRT_API int mbrt_attention_strided(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t H,
                                    int64_t n_q, int64_t n_k, int64_t head_dim, int64_t q_batch_stride,
                                    int64_t q_head_stride, int64_t q_row_stride, int64_t kv_batch_stride,
                                    int64_t kv_head_stride, int64_t kv_row_stride, const void* rot_cos,
                                    const void* rot_sin, int trig_dtype, const void* gate, int gate_dtype,
                                    int gate_is_logit, void* out, int out_dtype, float scale,
                                    mbrt_stream_t stream);

/* Precision of the probabilities P in the attention's second product (O = P V). */
enum mbrt_attn_precision {
    MBRT_ATTN_P_PAIR = 0, /* P as a bf16 hi + lo pair: f32 accuracy (mbrt_attention's default) */
    MBRT_ATTN_P_BF16 = 1, /* the reference's arithmetic: running max per 64-key tile, P
                             rounded once to bf16 for one P V product, the row sum over
                             the unrounded P (src/mbr_time_attention_cutile.cu:160-180) */
    MBRT_ATTN_P_BF16_FAST = 2 /* P rounded once to bf16 as in MBRT_ATTN_P_BF16, but the
                                 running max moves only when a 64-key tile's max exceeds it
                                 by 8 (log2 units), and the row sum adds the rounded P (an
                                 MFMA against ones): the fastest mode, same error size */
};

/* mbrt_attention_strided with the P precision chosen (enum mbrt_attn_precision).
 * MBRT_ATTN_P_BF16 runs one MFMA per key tile instead of two and matches the
 * reference's rounding of P; its output differs from exact attention by ~1e-3 of the
 * output's RMS (one bf16 rounding of every P); MBRT_ATTN_P_BF16_FAST likewise.
 * Replaces the same reference functions as mbrt_attention_strided. */
MBRT_API int mbrt_attention_ex(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t H,
                               int64_t n_q, int64_t n_k, int64_t head_dim, int64_t q_batch_stride,
                               int64_t q_head_stride, int64_t q_row_stride, int64_t kv_batch_stride,
                               int64_t kv_head_stride, int64_t kv_row_stride, const void* rot_cos,
                               const void* rot_sin, int trig_dtype, const void* gate, int gate_dtype,
                               int gate_is_logit, void* out, int out_dtype, float scale, int p_precision,
                               mbrt_stream_t stream);

/* ---- STFT / iSTFT (n_fft = win_length = 2048) --------------------------------- */

/* Hann window of `size` f32 samples, 0.5 (1 - cos(2 pi n / size)) in f32; size 1 gives
 * [1].  Replaces stft_tile::hann_window (src/stft_cuda_tile.cu:514-528). */
MBRT_API int mbrt_hann_window(float* out, int64_t size, mbrt_stream_t stream);

/* Frames of an STFT: padded = length + 2048 when centred, else length;
 * T = (padded - 2048) / hop + 1 (src/stft_cuda_tile.cu:544-551).  0 when padded < 2048,
 * -1 for a negative length or hop < 1.  Host only. */
MBRT_API int64_t mbrt_stft_num_frames(int64_t length, int64_t hop, int center);

/* STFT of `batch` f32 signals [batch, length] with a 2048-sample f32 window:
 * out[b, f, t] (complex, [batch, 1025, T, 2] f32) = sum_n x_pad[b, t hop + n] w[n]
 * exp(-2 pi i f n / 2048), x_pad = x reflect-padded by 1024 on both sides when centred
 * (reflect once about the end samples, then clamp, as Tensor::pad_reflect), times
 * 1/sqrt(2048) when normalized.  Requires n_fft = win_length = window_numel = 2048 and
 * T >= 1 (the reference reads past a non-centred signal shorter than 2048; this is an
 * MBRT_E_SHAPE error here).  Replaces stft_tile::stft (src/stft_cuda_tile.cu:530-598). */
MBRT_API int mbrt_stft(const float* signal, const float* window, float* out, int64_t batch, int64_t length,
                       int64_t n_fft, int64_t hop, int64_t win_length, int64_t window_numel, int center,
                       int normalized, mbrt_stream_t stream);

/* Output length of mbrt_istft: `length` when > 0, else 2048 + (frames - 1) hop, minus 2048
 * when centred.  -1 for frames < 1 or hop < 1.  Host only. */
MBRT_API int64_t mbrt_istft_output_length(int64_t frames, int64_t hop, int center, int64_t length);

/* Workspace mbrt_istft needs, in bytes: the overlap-added partial signal of every block of
 * 8 frames, batch * ceil(frames / 8) * (7 hop + 2048) f32.  -1 for a negative extent or a
 * hop outside 1..2^20. */
MBRT_API int64_t mbrt_istft_workspace_bytes(int64_t batch, int64_t frames, int64_t hop);

/* Inverse STFT of spec [batch, 1025, frames, 2] (F32 or BF16; times sqrt(2048) when
 * normalized): each frame is the real inverse DFT (imaginary parts of bins 0 and 1024
 * ignored) times the window, overlap-added at hop spacing and divided by the window's
 * summed squares where that sum exceeds 1e-8; centred output drops 1024 samples at each
 * end; `length` > 0 trims or zero-fills to that length.  out is [batch,
 * mbrt_istft_output_length(...)] f32.  Frames are summed per sample in frame order within
 * blocks of 8, then the block sums in block order (the reference adds them with atomics),
 * so the result is deterministic.  hop <= 2^20.  Replaces stft_tile::istft
 * (src/stft_cuda_tile.cu:600-717). */
MBRT_API int mbrt_istft(const void* spec, int spec_dtype, const float* window, float* out, int64_t batch,
                        int64_t freq_bins, int64_t frames, int64_t n_fft, int64_t hop, int64_t win_length,
                        int64_t window_numel, int center, int normalized, int64_t length, void* workspace,
                        int64_t workspace_bytes, mbrt_stream_t stream);

/* Bytes of device scratch the library holds on each GPU for mbrt_istft_noalloc. */
#define MBRT_ISTFT_SCRATCH_BYTES (32 * 1024 * 1024)

/* mbrt_istft with no workspace argument and no allocation of any kind: the block partials
 * go to a scratch array the library holds on each GPU (MBRT_ISTFT_SCRATCH_BYTES, enough
 * for mbrt_istft_workspace_bytes(batch, frames, hop) up to that size; larger calls fail
 * with MBRT_E_SHAPE).  Every call on one GPU shares that array, so calls that overlap on
 * one GPU (concurrent streams, threads) race.  Same results as mbrt_istft, bit for bit.
 * No counterpart in the reference: it is for callers that cannot allocate device memory,
 * such as tight serving loops and code under HIP graph capture.  The first call on a GPU
 * looks up that GPU's scratch address (hipGetSymbolAddress): make it outside any capture;
 * later calls issue kernel launches only and can be captured and replayed. */
MBRT_API int mbrt_istft_noalloc(const void* spec, int spec_dtype, const float* window, float* out,
                                int64_t batch, int64_t freq_bins, int64_t frames, int64_t n_fft, int64_t hop,
                                int64_t win_length, int64_t window_numel, int center, int normalized,
                                int64_t length, mbrt_stream_t stream);

/* ---- chunk overlap-add --------------------------------------------------------- */

/* dest[c, offset + i] += src[c, i] * window[i] for c < channels, i < chunk_len, and
 * weight_sum[offset + i] += window[i]; dest is [channels, dest_len], src [channels,
 * chunk_len], all f32.  The product and the sum are rounded separately and each element is
 * written once per call, so calls on one stream accumulate in call order (the reference adds
 * with atomics).  Requires 0 <= offset and offset + chunk_len <= dest_len.  Replaces
 * chunk_tile::accumulate_chunk (src/chunk_cuda_tile.cu:18-42, 61-73). */
MBRT_API int mbrt_chunk_accumulate(float* dest, float* weight_sum, const float* src, const float* window,
                                   int64_t channels, int64_t chunk_len, int64_t dest_len, int64_t offset,
                                   mbrt_stream_t stream);

/* data[c, i] /= weight_sum[i] where weight_sum[i] > 1e-8 (data [channels, length] f32).
 * Replaces chunk_tile::normalize_by_weights (src/chunk_cuda_tile.cu:44-58, 75-83). */
MBRT_API int mbrt_chunk_normalize(float* data, const float* weight_sum, int64_t channels, int64_t length,
                                  mbrt_stream_t stream);

/* Fade window of a chunk (host, `chunk_size` floats): ones, with a linear ramp
 * i / (fade_size - 1) over the first fade_size samples unless `first`, and its mirror over
 * the last fade_size samples unless `last` (fade_size 1: a single 0 at each faded end).
 * Requires 2 fade_size <= chunk_size.  Mirrors process_chunked's window
 * (src/inference_app.cpp:135-148, 201-210).  Host only. */
MBRT_API int mbrt_chunk_fade_window(float* window, int64_t chunk_size, int64_t fade_size, int first, int last);

/* ---- host-side tables (CPU only, no GPU access) ----------------------------- */

/* Band layout of a MelBandRoformer: the support of a Slaney-normalised mel filterbank
 * (librosa.filters.mel(sr, n_fft, n_bands) semantics) with the first bin of band 0 and
 * the last bin of the last band forced on; every bin of a band is repeated for each
 * channel as freq index bin * channels + ch.  Writes *n_band_freqs; when freq_indices
 * (host, `capacity` entries) is not NULL fills it, band after band.  freqs_per_band
 * (host, n_bands entries, may be NULL) gets each band's bin count.  This is the
 * __precomputed__.freq_indices / num_freqs_per_band content that the reference reads
 * from its model file (src/model_mel_band_roformer.cu:79-118). */
MBRT_API int mbrt_mel_band_layout(double sample_rate, int n_fft, int n_bands, int channels,
                                  int32_t* freq_indices, int64_t capacity, int64_t* n_band_freqs,
                                  int32_t* freqs_per_band);

/* Per-freq reverse map of a band layout (host arrays): offsets [total_freq + 1],
 * indices [n_band_freqs] (band-bins of each freq in ascending order), counts
 * [total_freq] as float (may be NULL) and the largest count (may be NULL).  Mirrors
 * MelBandRoformer::load's CSR build (src/model_mel_band_roformer.cu:120-150). */
MBRT_API int mbrt_band_csr(const int32_t* freq_indices, int64_t n_band_freqs, int64_t total_freq,
                           int32_t* offsets, int32_t* indices, float* counts,
                           int32_t* max_bands_per_freq);

/* Rotary tables [seq_len, dim_head/2] (host): f = 1 / theta^(2i/dim_head) and
 * angle = n * f in f32, then cos/sin.  Mirrors MelBandRoformer::compute_rotary_cos_sin
 * (src/model_mel_band_roformer.cu:270-300). */
MBRT_API int mbrt_rotary_tables(float* cos_table, float* sin_table, int64_t seq_len,
                                int64_t dim_head, float theta);

#ifdef __cplusplus
}
#endif

#endif /* MBRT_H */
