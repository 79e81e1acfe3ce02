// chunk_tile:: on the C-ABI (mbrt_chunk_accumulate, mbrt_chunk_normalize,
// mbrt_chunk_fade_window) and a chunked-inference driver with the semantics of the
// reference's chunk loop (src/inference_app.cpp:72-232): a chunk plan is built first, then
// the model runs over groups of planned chunks and their outputs are overlap-added.
#include "chunk_tile.h"

#include <algorithm>
#include <stdexcept>

#include "abi_call.h"
#include "mbr_tile.h"

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

namespace {

// How the part of a model input past the signal's end is filled.
enum class TailFill { None, Reflect, Zero };

// One model input of the chunked pass, in samples of the (possibly border-padded) signal.
struct ChunkSpan {
    int64_t offset;   // first sample
    int64_t taken;    // samples taken from the signal, <= chunk size
    TailFill tail;    // fill of [taken, chunk size)
    bool song_start;  // no fade-in: nothing overlaps this chunk's start
    bool song_end;    // no fade-out: this chunk reaches the end of the signal
};

struct ChunkPlan {
    int64_t source_len = 0;  // samples of the caller's signal
    int64_t border = 0;      // reflect border added at both ends (0: none)
    int64_t work_len = 0;    // samples of the bordered signal: the accumulator length
    int per_call = 1;        // chunks stacked into one model call
    std::vector<ChunkSpan> spans;
};

// Semantics of the reference's chunk loop (src/inference_app.cpp:72-232): a border of
// chunk_size - step is reflected onto both ends when the signal is longer than two
// borders; chunks start every `step` samples of the bordered signal; a chunk cut short by
// the end is completed by reflection when it holds more than half a chunk, else by zeros.
ChunkPlan plan_chunks(int64_t length, int chunk_size, int step, int chunk_batch_size) {
    ChunkPlan plan;
    plan.source_len = length;
    const int64_t border = (int64_t)chunk_size - step;
    plan.border = border > 0 && length > 2 * border ? border : 0;
    plan.work_len = length + 2 * plan.border;
    for (int64_t at = 0; at < plan.work_len; at += step) {
        const int64_t taken = std::min<int64_t>(chunk_size, plan.work_len - at);
        const TailFill tail = taken == chunk_size ? TailFill::None
                              : 2 * taken > chunk_size ? TailFill::Reflect
                                                       : TailFill::Zero;
        plan.spans.push_back({at, taken, tail, at == 0, at + taken >= plan.work_len});
    }
    const int64_t n = (int64_t)plan.spans.size();
    plan.per_call = (int)std::max<int64_t>(1, std::min<int64_t>(chunk_batch_size, n));
    return plan;
}

// Sets the reference's per-thread time-attention chunk index for the duration of one model
// call (src/inference_app.cpp:32-40), back to -1 afterwards.
class AttentionChunkScope {
public:
    explicit AttentionChunkScope(int64_t index) { mbr_tile::set_time_attention_context_chunk((int)index); }
    ~AttentionChunkScope() { mbr_tile::set_time_attention_context_chunk(-1); }
    AttentionChunkScope(const AttentionChunkScope&) = delete;
    AttentionChunkScope& operator=(const AttentionChunkScope&) = delete;
};

}  // namespace

Tensor process_chunked(const Tensor& audio, int chunk_size, int step, int chunk_batch_size,
                       const std::function<Tensor(const Tensor&)>& model_forward,
                       const std::function<void(const std::string&)>& logger) {
    if (chunk_size <= 0 || step <= 0) throw std::runtime_error("process_chunked: chunk_size and step must be positive");
    const ChunkPlan plan = plan_chunks(audio.size(-1), chunk_size, step, chunk_batch_size);
    const Tensor signal = plan.border ? audio.pad_reflect({plan.border, plan.border}) : audio;
    const int64_t n_chunks = (int64_t)plan.spans.size();

    // model input of one span: [.., C, chunk_size]
    auto input_of = [&](const ChunkSpan& c) {
        const Tensor part = signal.slice(-1, c.offset, c.offset + c.taken);
        const int64_t fill = chunk_size - c.taken;
        switch (c.tail) {
            case TailFill::Reflect: return part.pad_reflect({0, fill});
            case TailFill::Zero: return part.pad({0, fill}, 0.0f);
            default: return part;
        }
    };
    // the interior fade window is shared; the song's first and last chunks get their own
    const std::vector<float> interior = fade_window(chunk_size, chunk_size / 10, false, false);
    const Tensor interior_w = Tensor::from_cpu_f32(interior.data(), {(int64_t)chunk_size});
    auto window_of = [&](const ChunkSpan& c) {
        Tensor w = interior_w;
        if (chunk_size / 10 > 0 && (c.song_start || c.song_end)) {
            const std::vector<float> edge = fade_window(chunk_size, chunk_size / 10, c.song_start, c.song_end);
            w = Tensor::from_cpu_f32(edge.data(), {(int64_t)chunk_size});
        }
        return c.taken < chunk_size ? w.slice(0, 0, c.taken).contiguous() : w;
    };

    if (logger)
        logger("chunked pass: " + std::to_string(n_chunks) + " chunk(s) of " + std::to_string(chunk_size) +
               " samples every " + std::to_string(step) + ", " + std::to_string(plan.per_call) + " per model call");

    // accumulators, shaped from the first model output: [1, .., work_len] seen as [channels, work_len]
    std::vector<int64_t> result_shape;
    Tensor acc, weights;
    int64_t channels = 0;
    for (int64_t first = 0; first < n_chunks; first += plan.per_call) {
        const int64_t count = std::min<int64_t>(plan.per_call, n_chunks - first);
        Tensor out;
        {
            const AttentionChunkScope scope(first);
            if (count == 1) {
                out = model_forward(input_of(plan.spans[(size_t)first]));
            } else {
                std::vector<Tensor> inputs;
                inputs.reserve((size_t)count);
                for (int64_t i = 0; i < count; ++i) inputs.push_back(input_of(plan.spans[(size_t)(first + i)]));
                out = model_forward(Tensor::cat(inputs, 0));
            }
        }
        if (channels == 0) {
            result_shape = out.shape();
            result_shape.front() = 1;
            result_shape.back() = plan.work_len;
            int64_t per_sample = 1;
            for (size_t d = 0; d + 1 < result_shape.size(); ++d) per_sample *= result_shape[d];
            channels = per_sample;
            acc = Tensor::zeros({channels, plan.work_len});
            weights = Tensor::zeros({plan.work_len});
        }
        for (int64_t i = 0; i < count; ++i) {
            const ChunkSpan& c = plan.spans[(size_t)(first + i)];
            Tensor piece = count == 1 ? out : out.slice(0, i, i + 1).contiguous();
            if (piece.size(-1) > c.taken) piece = piece.slice(-1, 0, c.taken);
            accumulate_chunk(acc, weights, piece.contiguous().reshape({channels, c.taken}), window_of(c), c.offset);
        }
        if (logger)
            logger("chunked pass: " + std::to_string(first + count) + " of " + std::to_string(n_chunks) +
                   " chunk(s) merged");
    }

    normalize_by_weights(acc, weights);
    Tensor result = acc.reshape(result_shape);
    if (plan.border) result = result.slice(result.ndim() - 1, plan.border, plan.border + plan.source_len);
    return result;
}

}  // namespace cudasep::chunk_tile
