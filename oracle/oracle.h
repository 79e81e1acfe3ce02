/*
 * oracle.h — CPU restatement of the reference's tensor-op semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle that the GPU kernels in
 * mbr-cuda-tile_amd/ are held to: it is loaded by tests/, by __graft_entry__.smoke() and
 * by the cpu_baseline leg of bench.py, and nothing in the product links or calls it.
 *
 * Every op is plain host C++ over host buffers, with dtype codes equal to the C-ABI's
 * (F32=0, F16=1, I64=2, BF16=3, I32=4).  Float ops take `mode`:
 *   ORC_EXACT (0): compute in double, round once to the output dtype (round to nearest
 *                  even) — the "exact maths" value used for parity;
 *   ORC_FAST  (1): compute in float with the same operation order as the GPU kernels —
 *                  the loop that is timed as the CPU baseline;
 *   ORC_BF16I (2): the reference's full-bf16 experiment mode: double arithmetic, rounded
 *                  to bf16 at each point where the reference's bf16 kernels round under
 *                  full_bf16 (rms_norm, softmax, glu, gate_merge, rotary, split_qkv,
 *                  band_mask_merge; the cited kernel lines are at each op).  The caller
 *                  picks the dtypes for which the reference takes those kernels.
 * Outer loops are OpenMP-parallel; orc_set_threads() picks the thread count.
 *
 * Each function cites the reference code whose semantics it restates
 * (paths inside baicai-1145/MBR-CUDA-Tile).
 */
#ifndef MBRT_ORACLE_H
#define MBRT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_EXACT = 0, ORC_FAST = 1, ORC_BF16I = 2 };

void orc_set_threads(int n);
int orc_get_threads(void);

/* ---- deterministic inputs: SplitMix64 -> xoshiro256** -> Box-Muller (double) ---- */
void orc_randn(float* out, int64_t n, uint64_t seed, uint64_t stream, double mean, double stddev);
void orc_randu64(uint64_t* out, int64_t n, uint64_t seed, uint64_t stream);

/* ---- storage conversions (bit-level, round to nearest even, NaN stays NaN) -------- */
void orc_f32_to_bf16(const float* in, uint16_t* out, int64_t n);
void orc_bf16_to_f32(const uint16_t* in, float* out, int64_t n);
void orc_f32_to_f16(const float* in, uint16_t* out, int64_t n);
void orc_f16_to_f32(const uint16_t* in, float* out, int64_t n);
void orc_f64_to_bf16(const double* in, uint16_t* out, int64_t n);
/* generic dtype conversion (src/tensor_cuda_tile.cu:87-195, 442-472) */
void orc_convert(const void* src, int sdt, void* dst, int ddt, int64_t n);

/* ---- tensor library (src/tensor_cuda_tile.cu, src/tensor_cuda_glue.cu) ---------- */
void orc_binary(const void* a, const void* b, void* out, int dt, int64_t n, int op);
void orc_binary_broadcast(const void* a, const void* b, void* out, int dt, int ndim, const int64_t* out_shape,
                          const int64_t* a_strides, const int64_t* b_strides, int op);
void orc_strided_copy(const void* src, void* dst, int esize, int ndim, const int64_t* dst_shape,
                      const int64_t* src_strides);
void orc_index_select(const void* src, void* dst, int esize, int ndim, const int64_t* dst_shape,
                      const int64_t* src_strides, int sel, const int64_t* idx);
void orc_pad(const void* src, void* dst, int dt, int ndim, const int64_t* src_shape, const int64_t* dst_shape,
             const int64_t* before, float value, int reflect);
void orc_reduce_last(const float* src, float* dst, int64_t outer, int64_t inner, int op, int mode);
void orc_reduce_general(const float* src, float* dst, int64_t outer, int64_t reduce, int64_t inner, int op);

/* ---- hot-path ops (src/mbr_cuda_tile.cu) -------------------------------------------- */
void orc_rms_norm(const void* x, int xdt, const void* res, const void* gamma, int gdt, void* sum_out, int sdt,
                  void* out, int odt, int64_t rows, int64_t dim, float scale, float eps, int mode);
void orc_bias_act(const void* x, int xdt, const void* bias, int bdt, void* out, int odt, int64_t rows, int64_t cols,
                  int act, int mode);
void orc_glu(const void* x, int xdt, void* out, int odt, int64_t rows, int64_t half, int mode);
void orc_gate_merge(const void* attn, int adt, const void* gate, int gdt, int logit, void* out, int odt, int64_t B,
                    int64_t H, int64_t N, int64_t D, int layout, int mode);
void orc_softmax(const void* in, int idt, void* out, int odt, int64_t rows, int64_t cols, float scale, int mode);
void orc_rotary_tables(float* cos_t, float* sin_t, int64_t seq, int64_t dim_head, float theta);
void orc_rotary(void* q, void* k, int dt, const void* cos_t, const void* sin_t, int tdt, int64_t rows,
                int64_t n_pos, int64_t heads, int64_t dim_head, int layout, int mode);
void orc_split_qkv(const void* qkv, int idt, const void* cos_t, const void* sin_t, int tdt, void* q, void* k,
                   void* v, int odt, int64_t B, int64_t N, int64_t H, int64_t D, int64_t out_n, int mode);

/* ---- mel band split / merge --------------------------------------------------------- */
/* Support of a Slaney mel filterbank (librosa.filters.mel, htk=False, norm="slaney")
 * with [0,0] and [last, last] forced on, as the band layout of MelBandRoformer.
 * Pass NULL arrays to query sizes: returns the number of band-bins J (x channels).
 * freq_indices [J] (stereo index bin*channels+ch), freqs_per_band [n_bands],
 * bands_per_freq [bins*channels], csr_offsets [bins*channels+1], csr_indices [J]. */
int64_t orc_mel_bands(double sr, int n_fft, int n_bands, int channels, int32_t* freq_indices,
                      int32_t* freqs_per_band, int32_t* bands_per_freq, int32_t* csr_offsets,
                      int32_t* csr_indices);
void orc_band_gather(const float* stft, const int32_t* idx, void* out, int odt, int64_t B, int64_t F, int64_t T,
                     int64_t J);
void orc_band_mask_merge(const float* stft, const void* const* masks, int mdt, int S, const int32_t* off,
                         const int32_t* ind, const void* cnt, int cdt, void* out, int odt, int64_t B, int64_t F,
                         int64_t T, int64_t J, int64_t C, int mode);
void orc_zero_dc(void* spec, int dt, int64_t outer, int64_t bins, int64_t T);
void orc_attention(const void* q, const void* k, const void* v, int dt, void* out, int odt, int64_t BH,
                   int64_t nq, int64_t nk, int64_t D, float scale, int mode);
/* the time attention with the reference's rounding of P (src/mbr_time_attention_cutile.cu:160-180) */
void orc_attention_ref_p(const void* q, const void* k, const void* v, int dt, void* out, int odt, int64_t BH,
                         int64_t nq, int64_t nk, int64_t D, float scale);
/* the same with the running max moved only when a 64-key tile's max exceeds it by more
 * than `lazy` (natural-log units; 0 = every tile), and the row sum over the rounded P when
 * sum_rounded (the library's MBRT_ATTN_P_BF16_FAST: lazy = 8 ln 2, sum_rounded = 1) */
void orc_attention_ref_p_ex(const void* q, const void* k, const void* v, int dt, void* out, int odt, int64_t BH,
                            int64_t nq, int64_t nk, int64_t D, float scale, double lazy, int sum_rounded);

#ifdef __cplusplus
}
#endif

#endif
