// stft_tile:: on the C-ABI (mbrt_hann_window, mbrt_stft, mbrt_istft).  The workspace of
// the iSTFT (its windowed frames) comes from the caching allocator like any tensor.
#include "stft_tile.h"

#include <stdexcept>
#include <string>

#include "abi_call.h"

namespace cudasep::stft_tile {

namespace {

Tensor ensure_f32(const Tensor& x) {
    return x.dtype() == DType::Float32 ? x.contiguous() : x.to_f32().contiguous();
}

int64_t mbrt_code(DType d) { return static_cast<int64_t>(d); }

}  // namespace

Tensor hann_window(int size) {
    Tensor out = Tensor::empty({(int64_t)(size < 0 ? 0 : size)}, DType::Float32);
    if (size <= 0) return out;
    abi_check(mbrt_hann_window(out.data_f32(), size, abi_stream()), "stft_tile::hann_window");
    return out;
}

Tensor stft(const Tensor& signal, int n_fft, int hop_length, int win_length, const Tensor& window, bool center,
            bool normalized) {
    Tensor sig = ensure_f32(signal);
    const Tensor win = ensure_f32(window);
    if (sig.ndim() == 1) sig = sig.reshape({1, sig.size(0)});
    if (sig.ndim() != 2) throw std::runtime_error("stft_tile::stft: expected a [L] or [B, L] signal");
    if (n_fft != 2048 || win_length != 2048 || win.numel() != 2048)
        throw std::runtime_error("custom STFT only supports n_fft=2048, win_length=2048");
    if (hop_length < 1) throw std::runtime_error("stft_tile::stft: hop_length must be positive");
    const int64_t B = sig.size(0), L = sig.size(1);
    const int64_t T = mbrt_stft_num_frames(L, hop_length, center ? 1 : 0);
    if (T < 1) throw std::runtime_error("stft_tile::stft: signal shorter than n_fft");
    Tensor out = Tensor::empty({B, 1025, T, 2}, DType::Float32);
    if (out.numel() == 0) return out;
    abi_check(mbrt_stft(sig.data_f32(), win.data_f32(), out.data_f32(), B, L, n_fft, hop_length, win_length,
                        win.numel(), center ? 1 : 0, normalized ? 1 : 0, abi_stream()),
              "stft_tile::stft");
    return out;
}

Tensor istft(const Tensor& complex_spec, int n_fft, int hop_length, int win_length, const Tensor& window,
             int64_t length, bool center, bool normalized) {
    const Tensor spec =
        complex_spec.dtype() == DType::BFloat16 ? complex_spec.contiguous() : ensure_f32(complex_spec);
    const Tensor win = ensure_f32(window);
    if (spec.ndim() != 4 || spec.size(3) != 2)
        throw std::runtime_error("stft_tile::istft: expected a [B, F, T, 2] spectrum");
    const int64_t B = spec.size(0), F = spec.size(1), T = spec.size(2);
    if (n_fft != 2048 || win_length != 2048 || F != 1025 || win.numel() != 2048)
        throw std::runtime_error("custom iSTFT only supports n_fft=2048, win_length=2048");
    if (hop_length < 1 || T < 1) throw std::runtime_error("stft_tile::istft: bad hop_length or frame count");
    const int64_t n_out = mbrt_istft_output_length(T, hop_length, center ? 1 : 0, length);
    Tensor out = Tensor::empty({B, n_out}, DType::Float32);
    if (out.numel() == 0) return out;
    const int64_t ws_bytes = mbrt_istft_workspace_bytes(B, T, hop_length);
    if (ws_bytes < 0) throw std::runtime_error("stft_tile::istft: hop_length out of range");
    Tensor frames = Tensor::empty({ws_bytes / 4}, DType::Float32);
    abi_check(mbrt_istft(spec.data_ptr(), (int)mbrt_code(spec.dtype()), win.data_f32(), out.data_f32(), B, F, T,
                         n_fft, hop_length, win_length, win.numel(), center ? 1 : 0, normalized ? 1 : 0, length,
                         frames.data_ptr(), ws_bytes, abi_stream()),
              "stft_tile::istft");
    return out;
}

}  // namespace cudasep::stft_tile
