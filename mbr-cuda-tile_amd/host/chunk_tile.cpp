// chunk_tile:: on the C-ABI (mbrt_chunk_accumulate, mbrt_chunk_normalize,
// mbrt_chunk_fade_window) and the chunked-inference driver, host code mirroring
// src/inference_app.cpp:72-232 step for step.
#include "chunk_tile.h"

#include <algorithm>
#include <stdexcept>

#include "abi_call.h"

namespace cudasep::chunk_tile {

void accumulate_chunk(Tensor& dest, Tensor& weight_sum, const Tensor& src, const Tensor& window, int64_t offset) {
    const char* op = "chunk_tile::accumulate_chunk";
    if (dest.dtype() != DType::Float32 || weight_sum.dtype() != DType::Float32 || src.dtype() != DType::Float32 ||
        window.dtype() != DType::Float32)
        throw std::runtime_error(std::string(op) + ": expected f32 tensors");
    if (!dest.is_contiguous() || !weight_sum.is_contiguous())
        throw std::runtime_error(std::string(op) + ": dest and weight_sum must be contiguous");
    const Tensor s = src.contiguous(), w = window.contiguous();
    const int64_t n = s.size(-1), L = dest.size(-1);
    const int64_t channels = n ? s.numel() / n : 0;
    if (w.numel() != n || weight_sum.numel() != L || (L && dest.numel() / L != channels))
        throw std::runtime_error(std::string(op) + ": shapes do not match");
    abi_check(mbrt_chunk_accumulate(dest.data_f32(), weight_sum.data_f32(), s.data_f32(), w.data_f32(), channels, n, L,
                                    offset, abi_stream()),
              op);
}

void normalize_by_weights(Tensor& data, const Tensor& weight_sum) {
    const char* op = "chunk_tile::normalize_by_weights";
    if (data.dtype() != DType::Float32 || weight_sum.dtype() != DType::Float32 || !data.is_contiguous())
        throw std::runtime_error(std::string(op) + ": expected a contiguous f32 tensor and f32 weights");
    const int64_t L = data.size(-1);
    if (L == 0) return;
    const Tensor w = weight_sum.contiguous();
    if (w.numel() != L) throw std::runtime_error(std::string(op) + ": weight_sum length does not match");
    abi_check(mbrt_chunk_normalize(data.data_f32(), w.data_f32(), data.numel() / L, L, abi_stream()), op);
}

std::vector<float> fade_window(int chunk_size, int fade_size, bool first, bool last) {
    std::vector<float> w((size_t)std::max(chunk_size, 0));
    abi_check(mbrt_chunk_fade_window(w.data(), chunk_size, fade_size, first ? 1 : 0, last ? 1 : 0),
              "chunk_tile::fade_window");
    return w;
}

Tensor process_chunked(const Tensor& audio, int chunk_size, int step, int chunk_batch_size,
                       const std::function<Tensor(const Tensor&)>& model_forward,
                       const std::function<void(const std::string&)>& logger) {
    if (chunk_size <= 0 || step <= 0) throw std::runtime_error("process_chunked: chunk_size and step must be positive");
    Tensor mix = audio;
    const int64_t length_init = audio.size(-1);
    const int fade_size = chunk_size / 10;
    const int border = chunk_size - step;
    const bool padded = length_init > 2LL * border && border > 0;
    if (padded) mix = mix.pad_reflect({border, border});

    const int64_t total_samples = mix.size(-1);
    std::vector<int64_t> chunk_starts;
    for (int64_t start = 0; start < total_samples; start += step) chunk_starts.push_back(start);
    const int64_t chunk_count = (int64_t)chunk_starts.size();
    const int effective_batch = std::max(1, (int)std::min<int64_t>((int64_t)chunk_batch_size, chunk_count));
    const bool single_chunk_mode = effective_batch == 1;

    auto prepare_input_chunk = [&](int64_t start, int64_t end) {
        Tensor chunk = mix.slice(-1, start, end);
        const int64_t actual_len = end - start;
        if (actual_len < chunk_size) {
            if (actual_len > chunk_size / 2) chunk = chunk.pad_reflect({0, chunk_size - actual_len});
            else chunk = chunk.pad({0, chunk_size - actual_len}, 0.0f);
        }
        return chunk;
    };
    auto run_group = [&](int64_t group_start, int group_size) {
        if (single_chunk_mode) {
            const int64_t start = chunk_starts[(size_t)group_start];
            return model_forward(prepare_input_chunk(start, std::min<int64_t>(start + chunk_size, total_samples)));
        }
        std::vector<Tensor> inputs;
        for (int local = 0; local < group_size; ++local) {
            const int64_t start = chunk_starts[(size_t)(group_start + local)];
            inputs.push_back(prepare_input_chunk(start, std::min<int64_t>(start + chunk_size, total_samples)));
        }
        return model_forward(Tensor::cat(inputs, 0));
    };

    Tensor first_batch_out = run_group(0, (int)std::min<int64_t>(effective_batch, chunk_count));
    std::vector<int64_t> out_shape = first_batch_out.shape();
    out_shape[0] = 1;
    out_shape.back() = total_samples;

    const std::vector<float> fade = fade_window(chunk_size, fade_size, false, false);
    const Tensor fade_tensor = Tensor::from_cpu_f32(fade.data(), {(int64_t)chunk_size});

    Tensor output = Tensor::zeros(out_shape);
    Tensor weight_sum = Tensor::zeros({total_samples});
    const int64_t num_channels = output.numel() / total_samples;
    output = output.reshape({num_channels, total_samples});

    if (logger) {
        logger("[chunk] start");
        logger("[chunk] size: " + std::to_string(chunk_size));
        logger("[chunk] step: " + std::to_string(step));
        logger("[chunk] count: " + std::to_string(chunk_count));
        logger("[chunk] batch size: " + std::to_string(effective_batch));
    }
    int64_t chunk_index = 0;
    for (int64_t group_start = 0; group_start < chunk_count; group_start += effective_batch) {
        const int group_size = (int)std::min<int64_t>(effective_batch, chunk_count - group_start);
        const Tensor batch_out = group_start == 0 ? first_batch_out : run_group(group_start, group_size);
        for (int local = 0; local < group_size; ++local) {
            const int64_t start = chunk_starts[(size_t)(group_start + local)];
            const int64_t end = std::min<int64_t>(start + chunk_size, total_samples);
            const int64_t actual_len = end - start;
            const bool last_chunk = end >= total_samples;
            ++chunk_index;
            Tensor chunk_out = single_chunk_mode ? batch_out : batch_out.slice(0, local, local + 1).contiguous();
            if (chunk_out.size(-1) > actual_len) chunk_out = chunk_out.slice(-1, 0, actual_len);
            chunk_out = chunk_out.contiguous().reshape({num_channels, actual_len});
            Tensor window = fade_tensor;
            if (fade_size > 0 && (start == 0 || last_chunk)) {
                const std::vector<float> w = fade_window(chunk_size, fade_size, start == 0, last_chunk);
                window = Tensor::from_cpu_f32(w.data(), {(int64_t)chunk_size});
            }
            const Tensor fade_crop = actual_len < chunk_size ? window.slice(0, 0, actual_len).contiguous() : window;
            accumulate_chunk(output, weight_sum, chunk_out, fade_crop, start);
            if (logger && (chunk_index == 1 || chunk_index == chunk_count || (chunk_index % 4) == 0))
                logger("[chunk] completed " + std::to_string(chunk_index) + "/" + std::to_string(chunk_count));
        }
    }
    if (logger) logger("[chunk] merge complete");

    normalize_by_weights(output, weight_sum);
    output = output.reshape(out_shape);
    if (padded) output = output.slice(output.ndim() - 1, border, border + length_init);
    return output;
}

}  // namespace cudasep::chunk_tile
