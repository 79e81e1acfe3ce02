// cudasep::chunk_tile — the reference's chunk overlap-add (src/chunk_cuda_tile.h) and its
// chunked-inference driver (src/inference_app.cpp:72-232, an internal function there;
// exported here so an application can run it over any model callable).
#pragma once

#include <functional>
#include <string>

#include "tensor.h"

namespace cudasep::chunk_tile {

// dest[c, offset + i] += src[c, i] * window[i]; weight_sum[offset + i] += window[i]
// (src [.., n] f32 seen as [C, n]; dest [.., L] f32 as [C, L]).  Deterministic.
void accumulate_chunk(Tensor& dest,
                      Tensor& weight_sum,
                      const Tensor& src,
                      const Tensor& window,
                      int64_t offset);

// data[c, i] /= weight_sum[i] where weight_sum[i] > 1e-8.
void normalize_by_weights(Tensor& data, const Tensor& weight_sum);

// Linear fade-in / fade-out window of a chunk, omitted at the start of the first chunk and
// the end of the last (host vector).
std::vector<float> fade_window(int chunk_size, int fade_size, bool first, bool last);

// Splits audio [1, C, L] into chunks of chunk_size every `step` samples (reflect-padded by
// chunk_size - step at both ends when long enough; a short last chunk is reflect- or
// zero-padded), runs model_forward on groups of up to chunk_batch_size chunks stacked on
// dim 0, and overlap-adds the outputs [G, ..., chunk_size] with fade windows of
// chunk_size / 10.  Returns [1, ..., L].
Tensor process_chunked(const Tensor& audio, int chunk_size, int step, int chunk_batch_size,
                       const std::function<Tensor(const Tensor&)>& model_forward,
                       const std::function<void(const std::string&)>& logger = {});

}  // namespace cudasep::chunk_tile
