// cudasep::JsonValue and cudasep::ModelWeights — the reference's .csm model-file reader
// (src/weights.h), same names, accessors, coercions and error messages.
//
// MI355X layout: every tensor of a file lives in ONE device allocation (the weight arena,
// each tensor 256-byte aligned), filled by a streamed read through two pinned staging
// buffers whose DMA copies overlap the file reads.  Tensors are views into the arena.
//
// File layout (little-endian), as the reference writes and reads it:
//   "CSM\0" | u32 version (1) | u32 config_len | config JSON |
//   u32 n_tensors | n_tensors x { u32 name_len | name | u32 ndim | i64 shape[ndim] |
//                                 u32 dtype (0 f32, 1 f16, 2 i64, 3 bf16) | raw data }
#pragma once

#include <map>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "tensor.h"

namespace cudasep {

class JsonValue {
public:
    enum Type { Null, Bool, Number, String, Array, Object };

    JsonValue();
    ~JsonValue();
    JsonValue(const JsonValue& other);
    JsonValue(JsonValue&& other) noexcept;
    JsonValue& operator=(const JsonValue& other);
    JsonValue& operator=(JsonValue&& other) noexcept;

    Type type() const { return type_; }
    bool is_null() const { return type_ == Null; }
    bool is_bool() const { return type_ == Bool; }
    bool is_number() const { return type_ == Number; }
    bool is_string() const { return type_ == String; }
    bool is_array() const { return type_ == Array; }
    bool is_object() const { return type_ == Object; }

    // Accessors; throw std::runtime_error on a type mismatch.  as_bool accepts a number
    // (non-zero is true); as_number accepts a string that is entirely a number.
    bool as_bool() const;
    double as_number() const;
    int as_int() const { return (int)as_number(); }
    int64_t as_int64() const { return (int64_t)as_number(); }
    float as_float() const { return (float)as_number(); }
    const std::string& as_string() const;

    size_t size() const;                                    // array or object size
    const JsonValue& operator[](size_t index) const;        // array element
    const JsonValue& operator[](const std::string& key) const;  // object member
    bool has(const std::string& key) const;
    std::vector<std::string> keys() const;                  // object keys, sorted

    // The value of `key`, or `def` when the key is absent.
    int get_int(const std::string& key, int def) const;
    float get_float(const std::string& key, float def) const;
    bool get_bool(const std::string& key, bool def) const;
    std::string get_string(const std::string& key, const std::string& def) const;

    static JsonValue parse(const std::string& json);  // throws "JSON parse error at position N: ..."

    static JsonValue make_bool(bool v);
    static JsonValue make_number(double v);
    static JsonValue make_string(const std::string& v);
    static JsonValue make_array(std::vector<JsonValue> v);
    static JsonValue make_object(std::map<std::string, JsonValue> v);

private:
    Type type_ = Null;
    bool bool_ = false;
    double number_ = 0.0;
    std::string string_;
    std::vector<JsonValue> array_;
    std::unique_ptr<std::map<std::string, JsonValue>> object_;
};

class ModelWeights {
public:
    // Reads every tensor of a .csm file into device memory (one arena).
    static ModelWeights load(const std::string& path);

    const JsonValue& config() const { return config_; }
    const Tensor& get(const std::string& name) const;  // throws "ModelWeights: tensor not found: <name>"
    bool has(const std::string& name) const;
    std::vector<std::string> tensor_names() const;     // sorted
    size_t num_tensors() const { return tensors_.size(); }
    size_t arena_bytes() const { return arena_bytes_; }

    // Every 2-D f32 tensor becomes f16 / bf16 (round to nearest even), as the reference's
    // GEMM preparation does.  The converted tensors are new allocations.
    void convert_linear_weights_to_fp16();
    void convert_linear_weights_to_bf16();

private:
    JsonValue config_;
    std::unordered_map<std::string, Tensor> tensors_;
    size_t arena_bytes_ = 0;
};

// The band tables MelBandRoformer::load builds from the file's __precomputed__ tensors
// (src/model_mel_band_roformer.cu:79-150): the band index list, the per-freq reverse
// index (CSR in ascending band order), and the per-freq band counts as float (bf16 under
// the bands-per-freq bf16 policy), stereo-expanded as freq 2f + ch.
struct MelBandTables {
    Tensor freq_indices;             // i64 [J]
    Tensor freq_band_offsets;        // i64 [total_freq + 1]
    Tensor freq_band_indices;        // i64 [J]
    Tensor num_bands_per_freq;       // f32 / bf16 [total_freq]
    std::vector<int64_t> freq_indices_host;
    std::vector<int64_t> num_freqs_per_band;   // [num_bands]
    std::vector<int64_t> num_bands_per_freq_host;  // [total_freq]
    std::vector<int64_t> band_freq_dims;       // 2 * num_freqs_per_band * channels
    int64_t max_bands_per_freq = 0;
};

MelBandTables load_mel_band_tables(const ModelWeights& weights, int num_bands, int n_fft, bool stereo);

}  // namespace cudasep
