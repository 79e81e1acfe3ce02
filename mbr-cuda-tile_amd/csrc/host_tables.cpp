// Host-side table builders that the reference runs on the CPU when it loads a model:
// the mel band layout (support of the Slaney mel filterbank, as stored in the model file),
// the per-freq CSR reverse map used by the mask merge, and the rotary cos/sin tables.
// None of these touches the GPU; callers upload the results once.
#include <cmath>
#include <cstdint>
#include <vector>

#include "abi_common.hpp"

namespace mbrt {
namespace {

double hz_to_mel_slaney(double f) {
    const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp;
    const double logstep = std::log(6.4) / 27.0;
    return f >= min_log_hz ? min_log_mel + std::log(f / min_log_hz) / logstep : f / f_sp;
}

double mel_to_hz_slaney(double m) {
    const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp;
    const double logstep = std::log(6.4) / 27.0;
    return m >= min_log_mel ? min_log_hz * std::exp(logstep * (m - min_log_mel)) : f_sp * m;
}

// support[b][f]: filter b of a Slaney-normalised triangular mel filterbank over the
// n_fft/2+1 rfft bins is non-zero at bin f (computed in double, tested in float32 as the
// converter stores the weights), with the first bin of the first band and the last bin
// of the last band forced on.
std::vector<std::vector<uint8_t>> mel_support(double sr, int n_fft, int n_bands) {
    const int bins = n_fft / 2 + 1;
    std::vector<double> fft(bins), mel_f(n_bands + 2);
    for (int i = 0; i < bins; ++i) fft[i] = (sr / 2.0) * i / (bins - 1);
    const double lo = hz_to_mel_slaney(0.0), hi = hz_to_mel_slaney(sr / 2.0);
    for (int i = 0; i < n_bands + 2; ++i) mel_f[i] = mel_to_hz_slaney(lo + (hi - lo) * i / (n_bands + 1));
    std::vector<std::vector<uint8_t>> s(n_bands, std::vector<uint8_t>(bins, 0));
    for (int b = 0; b < n_bands; ++b) {
        const double left = mel_f[b + 1] - mel_f[b], right = mel_f[b + 2] - mel_f[b + 1];
        const double norm = 2.0 / (mel_f[b + 2] - mel_f[b]);
        for (int f = 0; f < bins; ++f) {
            const double rise = (fft[f] - mel_f[b]) / left;
            const double fall = (mel_f[b + 2] - fft[f]) / right;
            const double w = std::max(0.0, std::min(rise, fall)) * norm;
            s[b][f] = static_cast<float>(w) > 0.0f;
        }
    }
    s[0][0] = 1;
    s[n_bands - 1][bins - 1] = 1;
    return s;
}

}  // namespace
}  // namespace mbrt

using namespace mbrt;

extern "C" {

int mbrt_mel_band_layout(double sample_rate, int n_fft, int n_bands, int channels, int32_t* freq_indices,
                         int64_t capacity, int64_t* n_band_freqs, int32_t* freqs_per_band) {
    const char* op = "mbrt_mel_band_layout";
    MBRT_REQUIRE(sample_rate > 0 && n_fft >= 2 && n_bands >= 1 && channels >= 1, MBRT_E_INVALID_ARG,
                 "%s: bad parameters", op);
    MBRT_REQUIRE(n_band_freqs != nullptr, MBRT_E_INVALID_ARG, "%s: n_band_freqs is NULL", op);
    const auto sup = mel_support(sample_rate, n_fft, n_bands);
    const int bins = n_fft / 2 + 1;
    int64_t J = 0;
    for (int b = 0; b < n_bands; ++b) {
        int32_t cnt = 0;
        for (int f = 0; f < bins; ++f) cnt += sup[b][f];
        if (freqs_per_band) freqs_per_band[b] = cnt;
        J += (int64_t)cnt * channels;
    }
    *n_band_freqs = J;
    if (freq_indices == nullptr) return MBRT_OK;
    MBRT_REQUIRE(capacity >= J, MBRT_E_SHAPE, "%s: capacity %lld < %lld band-bins", op, (long long)capacity,
                 (long long)J);
    int64_t j = 0;
    for (int b = 0; b < n_bands; ++b)
        for (int f = 0; f < bins; ++f)
            if (sup[b][f])
                for (int c = 0; c < channels; ++c) freq_indices[j++] = f * channels + c;
    return MBRT_OK;
}

int mbrt_band_csr(const int32_t* freq_indices, int64_t n_band_freqs, int64_t total_freq, int32_t* offsets,
                  int32_t* indices, float* counts, int32_t* max_bands_per_freq) {
    const char* op = "mbrt_band_csr";
    MBRT_REQUIRE(n_band_freqs >= 0 && total_freq >= 1, MBRT_E_SHAPE, "%s: bad sizes", op);
    MBRT_REQUIRE(offsets && (n_band_freqs == 0 || (freq_indices && indices)), MBRT_E_INVALID_ARG,
                 "%s: NULL pointer", op);
    std::vector<int32_t> cnt(total_freq, 0);
    for (int64_t j = 0; j < n_band_freqs; ++j) {
        const int32_t f = freq_indices[j];
        MBRT_REQUIRE(f >= 0 && f < total_freq, MBRT_E_SHAPE, "%s: freq index %d out of range", op, f);
        ++cnt[f];
    }
    int32_t mx = 0;
    offsets[0] = 0;
    for (int64_t f = 0; f < total_freq; ++f) {
        offsets[f + 1] = offsets[f] + cnt[f];
        mx = cnt[f] > mx ? cnt[f] : mx;
        if (counts) counts[f] = (float)cnt[f];
    }
    std::vector<int32_t> fill(offsets, offsets + total_freq);
    for (int64_t j = 0; j < n_band_freqs; ++j) indices[fill[freq_indices[j]]++] = (int32_t)j;  // ascending j
    if (max_bands_per_freq) *max_bands_per_freq = mx;
    return MBRT_OK;
}

int mbrt_rotary_tables(float* cos_table, float* sin_table, int64_t seq_len, int64_t dim_head, float theta) {
    const char* op = "mbrt_rotary_tables";
    MBRT_REQUIRE(seq_len >= 0 && dim_head >= 2 && dim_head % 2 == 0, MBRT_E_SHAPE, "%s: bad shape", op);
    MBRT_REQUIRE(seq_len == 0 || (cos_table && sin_table), MBRT_E_INVALID_ARG, "%s: NULL pointer", op);
    const int64_t half = dim_head / 2;
    for (int64_t n = 0; n < seq_len; ++n) {
        for (int64_t i = 0; i < half; ++i) {
            const float freq = 1.0f / std::pow(theta, (float)(2 * i) / (float)dim_head);
            const float angle = (float)n * freq;
            cos_table[n * half + i] = std::cos(angle);
            sin_table[n * half + i] = std::sin(angle);
        }
    }
    return MBRT_OK;
}

}  // extern "C"
