// cudasep::stft_tile — the reference's STFT header (src/stft_cuda_tile.h), same names,
// arguments, defaults and error messages, on libmbrt's gfx950 kernels.  Only
// n_fft = win_length = 2048 is supported, as in the reference.
#pragma once

#include "tensor.h"

namespace cudasep::stft_tile {

// Periodic Hann window [size] f32 (src/stft_cuda_tile.cu:514-528).
Tensor hann_window(int size);

// signal [L] or [B, L] (any float dtype; computed in f32) -> [B, 1025, T, 2] f32, frames
// reflect-padded by n_fft/2 when centred (src/stft_cuda_tile.cu:530-598).
Tensor stft(const Tensor& signal,
            int n_fft,
            int hop_length,
            int win_length,
            const Tensor& window,
            bool center = true,
            bool normalized = false);

// [B, 1025, T, 2] (BF16 read as is, other dtypes as f32) -> [B, samples] f32
// (src/stft_cuda_tile.cu:600-717).  The window sum of squares is evaluated inside the
// overlap-add kernel, so CUDASEP_DISABLE_ISTFT_WINDOW_SUM_CACHE has nothing to switch.
Tensor istft(const Tensor& complex_spec,
             int n_fft,
             int hop_length,
             int win_length,
             const Tensor& window,
             int64_t length = -1,
             bool center = true,
             bool normalized = false);

}  // namespace cudasep::stft_tile
