// Per-kernel launch shapes and cache policies, chosen by measurement on MI355X at the
// MelBandRoformer chunk shapes (T = 801 frames, 60 bands, D = 384, 48060 token rows).
// Every value can be overridden at build time (build.py -D NAME=VALUE) to re-tune.
//
// MBRT_NT_* : non-temporal policy of a kernel's streaming operands, bit 0 = loads,
//             bit 1 = stores.  Operands that are re-read (gamma, bias, gate logits, cos/sin
//             tables) always use ordinary accesses.  Measured with each op's calls back to
//             back (so an op pays for its own write-backs from the 256 MB MALL): uniform
//             policies 0..3 per kernel, the best kept; differences under ~3 % are noise.
#pragma once

#ifndef MBRT_NT_RMS
#define MBRT_NT_RMS 3    // residual add + RMSNorm: x, residual, sum, normed
#endif
#ifndef MBRT_NT_ACT
#define MBRT_NT_ACT 2    // bias + activation (GELU)
#endif
#ifndef MBRT_NT_GLU
#define MBRT_NT_GLU 3
#endif
#ifndef MBRT_NT_GATE
#define MBRT_NT_GATE 3   // sigmoid gate x head merge: attention values, merged output
#endif
#ifndef MBRT_NT_SMR
#define MBRT_NT_SMR 0    // register-resident softmax rows (time attention, 801 columns)
#endif
#ifndef MBRT_NT_SMS
#define MBRT_NT_SMS 3    // LDS-staged short softmax rows (freq attention, 60 columns)
#endif
#ifndef MBRT_NT_SML
#define MBRT_NT_SML 3    // LDS-staged long softmax rows (time attention, 801 columns)
#endif
#ifndef MBRT_NT_ROT
#define MBRT_NT_ROT 3    // rotary q/k
#endif
#ifndef MBRT_NT_ROW
#define MBRT_NT_ROW 3    // row copy (permutes that keep the innermost dim)
#endif
#ifndef MBRT_NT_TR
#define MBRT_NT_TR 0     // LDS tile transpose
#endif
#ifndef MBRT_NT_EW
#define MBRT_NT_EW 0     // convert / unary / scalar / binary vector kernels
#endif
#ifndef MBRT_NT_STFT
#define MBRT_NT_STFT 0   // STFT spectrum stores (bit 1), iSTFT spectrum loads (bit 0)
#endif
#ifndef MBRT_NT_ISTFT
#define MBRT_NT_ISTFT 4  // iSTFT block partials: final-pass loads (bit 0), block stores (bit 1); output stores (bit 2)
#endif
#ifndef MBRT_NT_CHUNK
#define MBRT_NT_CHUNK 3  // chunk accumulate and normalize: chunk and output loads (bit 0), output stores (bit 1)
#endif
#ifndef MBRT_NT_BAND
#define MBRT_NT_BAND 2   // band gather / mask merge: stft, masks, outputs
#endif

#ifndef MBRT_BAND_XCD
#define MBRT_BAND_XCD 8  // band kernels: runs of this many consecutive tiles per XCD (1: launch order)
#endif
#ifndef MBRT_BAND_GATHER_PIPE
#define MBRT_BAND_GATHER_PIPE 1  // band gather: persistent pipelined blocks (1) or one tile per block (0)
#endif
#ifndef MBRT_BAND_GTT
#define MBRT_BAND_GTT 64  // pipelined band gather: frames per tile (32 or 64)
#endif
#ifndef MBRT_BAND_GNW
#define MBRT_BAND_GNW 4  // pipelined band gather: waves per block
#endif
#ifndef MBRT_BAND_GALIGN
#define MBRT_BAND_GALIGN 1  // pipelined band gather: output runs start on 128-byte lines (1) or at the tile (0)
#endif
#ifndef MBRT_BAND_GBPC
#define MBRT_BAND_GBPC 1  // pipelined band gather: persistent blocks per CU
#endif
#ifndef MBRT_BAND_MTF
#define MBRT_BAND_MTF 32  // band merge: freqs per tile (<= 64)
#endif
#ifndef MBRT_BAND_MME
#define MBRT_BAND_MME 64  // band merge: CSR entries staged per chunk (a multiple of 64)
#endif
#ifndef MBRT_BAND_MNW
#define MBRT_BAND_MNW 4  // band merge: waves per block
#endif
#ifndef MBRT_BAND_MERGE_PAIRS
#define MBRT_BAND_MERGE_PAIRS 0  // band merge tile order: pairs of frame tiles within the freq-fastest order (1)
#endif
#ifndef MBRT_BAND_MERGE_TFAST
#define MBRT_BAND_MERGE_TFAST 0  // band merge tile order: frame tiles fastest (1) or freq tiles fastest (0)
#endif
#ifndef MBRT_SM_STAGE_LONG
#define MBRT_SM_STAGE_LONG 1  // softmax rows of 129..1024 elements through LDS when spans align
#endif
#ifndef MBRT_SM_LONG_G
#define MBRT_SM_LONG_G 64  // lanes per staged row of 129..1024 elements when 4-row spans align (64 or 32)
#endif
#ifndef MBRT_SM_STAGE16
#define MBRT_SM_STAGE16 1  // staged softmax: bf16->bf16 / f16->f16 spans kept 2-byte in LDS (1) or as f32 (0)
#endif
#ifndef MBRT_SM_LONG_RPG
#define MBRT_SM_LONG_RPG 1  // staged softmax rows of 129..1024 elements: rows per lane group (block of 4 or 8 rows x this)
#endif
#ifndef MBRT_SM_SHORT_BYTES
#define MBRT_SM_SHORT_BYTES 6144  // staged softmax rows of 33..64: below this many input bytes per 32 rows, 64-row blocks
#endif
#ifndef MBRT_SM_DMA
#define MBRT_SM_DMA 1  // staged softmax: raw spans loaded straight into LDS (direct-to-LDS loads)
#endif
#ifndef MBRT_SM_PAIR_U
#define MBRT_SM_PAIR_U 1  // 2-byte softmax rows of 33..64 (cols % 4 == 0, even row count): row pairs per 16-lane group from registers (0: LDS-staged kernel)
#endif
#ifndef MBRT_NT_SMP
#define MBRT_NT_SMP 3    // softmax row pairs from registers: non-temporal loads (bit 0) and stores (bit 1)
#endif
#ifndef MBRT_SM_PAIR_RCP
#define MBRT_SM_PAIR_RCP 1  // softmax row pairs: 1/sum as v_rcp_f32 (1) or the correctly rounded division (0)
#endif
#ifndef MBRT_SM_PAIR_BPC
#define MBRT_SM_PAIR_BPC 24  // softmax row pairs: blocks per CU of a grid that walks the chunks (0: one chunk per block)
#endif
#ifndef MBRT_SM_SHORT_RPG
#define MBRT_SM_SHORT_RPG 2  // rows per lane group in those blocks
#endif
#ifndef MBRT_ATTN_HEADS_WPC
#define MBRT_ATTN_HEADS_WPC 2  // attention over <= 64 queries and keys: persistent workgroups per CU, each walking heads (0: one head per workgroup)
#endif
#ifndef MBRT_ATTN_NT
#define MBRT_ATTN_NT 0  // attention, one workgroup per query tile: non-temporal q loads (bit 0) and output stores (bit 1); measured: no gain
#endif
#ifndef MBRT_ATTN_HEADS_NT
#define MBRT_ATTN_HEADS_NT 3  // persistent attention over short heads: non-temporal output stores (bit 0) and K/V/Q loads (bit 1)
#endif
#ifndef MBRT_GATE_TPW
#define MBRT_GATE_TPW 4  // gate merge of a head-major [B,H,N,D] input: tokens per run (1: a block step writes whole token rows; measured 4 > 12, 6, 2, 1 by 1 %)
#endif
#ifndef MBRT_ACT_U
#define MBRT_ACT_U 2     // 16-byte groups per thread: bias + activation (GELU)
#endif
#ifndef MBRT_GLU_U
#define MBRT_GLU_U 1     // 16-byte output groups per thread: GLU
#endif
#ifndef MBRT_GATE_U
#define MBRT_GATE_U 2    // 16-byte groups per thread: sigmoid gate x head merge
#endif
#ifndef MBRT_GATE_BPC
#define MBRT_GATE_BPC 16  // sigmoid gate x head merge: blocks per CU of a grid that walks the chunks (0: one chunk per block)
#endif
#ifndef MBRT_CHUNK_CPB
#define MBRT_CHUNK_CPB 4  // chunk accumulate: channels (one wave each) per block over shared positions (0: one channel per grid row)
#endif
#ifndef MBRT_EW_U
#define MBRT_EW_U 4      // 16-byte groups per thread in the elementwise kernels
#endif
#ifndef MBRT_ROW_U
#define MBRT_ROW_U 1     // row-copy vectors per thread
#endif
#ifndef MBRT_RMS_G
#define MBRT_RMS_G 16    // lanes per row for rows of at most 128 16-byte chunks (16 or 32)
#endif
