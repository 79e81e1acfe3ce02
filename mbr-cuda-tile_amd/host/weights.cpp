// .csm reader (src/weights.cu:1-562 semantics) with a single device arena per file and a
// double-buffered pinned upload, plus the model's band-table build from the file's
// __precomputed__ tensors (src/model_mel_band_roformer.cu:79-150).
#include "weights.h"

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <stdexcept>

#include "abi_call.h"
#include "mbr_tile.h"

namespace cudasep {

// ---- JsonValue ---------------------------------------------------------------------------

JsonValue::JsonValue() = default;
JsonValue::~JsonValue() = default;
JsonValue::JsonValue(JsonValue&& other) noexcept = default;
JsonValue& JsonValue::operator=(JsonValue&& other) noexcept = default;

JsonValue::JsonValue(const JsonValue& o)
    : type_(o.type_), bool_(o.bool_), number_(o.number_), string_(o.string_), array_(o.array_) {
    if (o.object_) object_ = std::make_unique<std::map<std::string, JsonValue>>(*o.object_);
}

JsonValue& JsonValue::operator=(const JsonValue& o) {
    if (this != &o) {
        JsonValue t(o);
        *this = std::move(t);
    }
    return *this;
}

bool JsonValue::as_bool() const {
    if (type_ == Bool) return bool_;
    if (type_ == Number) return number_ != 0.0;
    throw std::runtime_error("JsonValue: not a bool");
}

double JsonValue::as_number() const {
    if (type_ == Number) return number_;
    if (type_ == String && !string_.empty()) {
        char* end = nullptr;
        errno = 0;
        const double v = std::strtod(string_.c_str(), &end);
        if (end == string_.c_str() + string_.size() && errno == 0) return v;
    }
    throw std::runtime_error("JsonValue: not a number");
}

const std::string& JsonValue::as_string() const {
    if (type_ != String) throw std::runtime_error("JsonValue: not a string");
    return string_;
}

size_t JsonValue::size() const {
    if (type_ == Array) return array_.size();
    if (type_ == Object) return object_->size();
    throw std::runtime_error("JsonValue: size() called on non-container");
}

const JsonValue& JsonValue::operator[](size_t index) const {
    if (type_ != Array) throw std::runtime_error("JsonValue: not an array");
    if (index >= array_.size()) throw std::runtime_error("JsonValue: array index out of range");
    return array_[index];
}

const JsonValue& JsonValue::operator[](const std::string& key) const {
    if (type_ != Object) throw std::runtime_error("JsonValue: not an object");
    auto it = object_->find(key);
    if (it == object_->end()) throw std::runtime_error("JsonValue: key not found: " + key);
    return it->second;
}

bool JsonValue::has(const std::string& key) const { return type_ == Object && object_->count(key) > 0; }

std::vector<std::string> JsonValue::keys() const {
    std::vector<std::string> k;
    if (type_ == Object)
        for (const auto& kv : *object_) k.push_back(kv.first);
    return k;
}

int JsonValue::get_int(const std::string& key, int def) const { return has(key) ? (*this)[key].as_int() : def; }
float JsonValue::get_float(const std::string& key, float def) const {
    return has(key) ? (*this)[key].as_float() : def;
}
bool JsonValue::get_bool(const std::string& key, bool def) const { return has(key) ? (*this)[key].as_bool() : def; }
std::string JsonValue::get_string(const std::string& key, const std::string& def) const {
    return has(key) ? (*this)[key].as_string() : def;
}

JsonValue JsonValue::make_bool(bool v) {
    JsonValue j;
    j.type_ = Bool;
    j.bool_ = v;
    return j;
}
JsonValue JsonValue::make_number(double v) {
    JsonValue j;
    j.type_ = Number;
    j.number_ = v;
    return j;
}
JsonValue JsonValue::make_string(const std::string& v) {
    JsonValue j;
    j.type_ = String;
    j.string_ = v;
    return j;
}
JsonValue JsonValue::make_array(std::vector<JsonValue> v) {
    JsonValue j;
    j.type_ = Array;
    j.array_ = std::move(v);
    return j;
}
JsonValue JsonValue::make_object(std::map<std::string, JsonValue> v) {
    JsonValue j;
    j.type_ = Object;
    j.object_ = std::make_unique<std::map<std::string, JsonValue>>(std::move(v));
    return j;
}

namespace {

// Recursive-descent JSON (RFC 8259) parser.
class JsonReader {
public:
    explicit JsonReader(const std::string& s) : s_(s) {}

    JsonValue document() {
        JsonValue v = value(0);
        ws();
        if (p_ != s_.size()) fail("unexpected trailing characters");
        return v;
    }

private:
    const std::string& s_;
    size_t p_ = 0;

    [[noreturn]] void fail(const std::string& what) const {
        throw std::runtime_error("JSON parse error at position " + std::to_string(p_) + ": " + what);
    }
    void ws() {
        while (p_ < s_.size() && (s_[p_] == ' ' || s_[p_] == '\t' || s_[p_] == '\n' || s_[p_] == '\r')) ++p_;
    }
    char peek() {
        ws();
        if (p_ >= s_.size()) fail("unexpected end of input");
        return s_[p_];
    }
    void expect(char c) {
        if (peek() != c) fail(std::string("expected '") + c + "'");
        ++p_;
    }
    bool literal(const char* w) {
        const size_t n = std::strlen(w);
        if (s_.compare(p_, n, w) != 0) return false;
        p_ += n;
        return true;
    }

    JsonValue value(int depth) {
        if (depth > 512) fail("nesting too deep");
        const char c = peek();
        if (c == '{') return object(depth);
        if (c == '[') return array(depth);
        if (c == '"') return JsonValue::make_string(string());
        if (c == '-' || (c >= '0' && c <= '9')) return number();
        if (literal("true")) return JsonValue::make_bool(true);
        if (literal("false")) return JsonValue::make_bool(false);
        if (literal("null")) return JsonValue();
        fail("unexpected character");
    }

    JsonValue object(int depth) {
        expect('{');
        std::map<std::string, JsonValue> m;
        if (peek() == '}') {
            ++p_;
            return JsonValue::make_object(std::move(m));
        }
        for (;;) {
            if (peek() != '"') fail("expected a member name");
            std::string k = string();
            expect(':');
            m[k] = value(depth + 1);
            const char c = peek();
            ++p_;
            if (c == '}') break;
            if (c != ',') fail("expected ',' or '}'");
        }
        return JsonValue::make_object(std::move(m));
    }

    JsonValue array(int depth) {
        expect('[');
        std::vector<JsonValue> a;
        if (peek() == ']') {
            ++p_;
            return JsonValue::make_array(std::move(a));
        }
        for (;;) {
            a.push_back(value(depth + 1));
            const char c = peek();
            ++p_;
            if (c == ']') break;
            if (c != ',') fail("expected ',' or ']'");
        }
        return JsonValue::make_array(std::move(a));
    }

    unsigned hex4() {
        if (p_ + 4 > s_.size()) fail("short \\u escape");
        unsigned v = 0;
        for (int i = 0; i < 4; ++i) {
            const char h = s_[p_++];
            v <<= 4;
            if (h >= '0' && h <= '9') v |= (unsigned)(h - '0');
            else if (h >= 'a' && h <= 'f') v |= (unsigned)(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') v |= (unsigned)(h - 'A' + 10);
            else fail("bad \\u escape");
        }
        return v;
    }

    static void utf8(std::string& out, unsigned cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }

    std::string string() {
        expect('"');
        std::string out;
        for (;;) {
            if (p_ >= s_.size()) fail("unterminated string");
            const char c = s_[p_++];
            if (c == '"') break;
            if ((unsigned char)c < 0x20) fail("control character in string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p_ >= s_.size()) fail("unterminated escape");
            const char e = s_[p_++];
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    unsigned cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00 && s_.compare(p_, 2, "\\u") == 0) {
                        p_ += 2;
                        const unsigned lo = hex4();
                        if (lo < 0xDC00 || lo > 0xDFFF) fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(out, cp);
                    break;
                }
                default: fail("bad escape");
            }
        }
        return out;
    }

    JsonValue number() {
        ws();
        const size_t b = p_;
        if (s_[p_] == '-') ++p_;
        auto digits = [&]() {
            const size_t d = p_;
            while (p_ < s_.size() && s_[p_] >= '0' && s_[p_] <= '9') ++p_;
            if (p_ == d) fail("expected a digit");
        };
        if (p_ < s_.size() && s_[p_] == '0') ++p_;
        else digits();
        if (p_ < s_.size() && s_[p_] == '.') {
            ++p_;
            digits();
        }
        if (p_ < s_.size() && (s_[p_] == 'e' || s_[p_] == 'E')) {
            ++p_;
            if (p_ < s_.size() && (s_[p_] == '+' || s_[p_] == '-')) ++p_;
            digits();
        }
        const std::string text = s_.substr(b, p_ - b);
        return JsonValue::make_number(std::strtod(text.c_str(), nullptr));
    }
};

}  // namespace

JsonValue JsonValue::parse(const std::string& json) { return JsonReader(json).document(); }

// ---- ModelWeights ------------------------------------------------------------------------

namespace {

struct Entry {
    std::string name;
    std::vector<int64_t> shape;
    DType dtype;
    int64_t file_offset;
    size_t bytes;
    size_t arena_offset;
};

struct File {
    std::FILE* f = nullptr;
    explicit File(const std::string& path) : f(std::fopen(path.c_str(), "rb")) {}
    ~File() {
        if (f) std::fclose(f);
    }
    void read(void* dst, size_t n, const char* what) {
        if (n && std::fread(dst, 1, n, f) != n)
            throw std::runtime_error(std::string("ModelWeights: unexpected EOF reading ") + what);
    }
    uint32_t u32() {
        uint32_t v;
        read(&v, 4, "uint32");
        return v;
    }
    int64_t i64() {
        int64_t v;
        read(&v, 8, "int64");
        return v;
    }
    int64_t tell() { return (int64_t)std::ftell(f); }
    void seek(int64_t off) {
        if (std::fseek(f, (long)off, SEEK_SET) != 0) throw std::runtime_error("ModelWeights: seek failed");
    }
};

constexpr size_t kArenaAlign = 256;
constexpr size_t kStage = size_t(64) << 20;  // bytes per pinned staging buffer

// Streams [entries' data] from the file into the arena through two pinned buffers: the
// file read into one buffer overlaps the DMA of the other.
void upload(File& file, const std::vector<Entry>& entries, char* arena, hipStream_t st) {
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool pending[2] = {false, false};
    for (int k = 0; k < 2; ++k) {
        HIP_CHECK(hipHostMalloc(&stage[k], kStage, hipHostMallocDefault));
        HIP_CHECK(hipEventCreateWithFlags(&done[k], hipEventDisableTiming));
    }
    int k = 0;
    try {
        for (const Entry& e : entries) {
            file.seek(e.file_offset);
            for (size_t off = 0; off < e.bytes; off += kStage) {
                const size_t n = std::min(kStage, e.bytes - off);
                if (pending[k]) HIP_CHECK(hipEventSynchronize(done[k]));
                file.read(stage[k], n, "data");
                HIP_CHECK(hipMemcpyAsync(arena + e.arena_offset + off, stage[k], n, hipMemcpyHostToDevice, st));
                HIP_CHECK(hipEventRecord(done[k], st));
                pending[k] = true;
                k ^= 1;
            }
        }
        HIP_CHECK(hipStreamSynchronize(st));
    } catch (...) {
        (void)hipStreamSynchronize(st);
        for (int j = 0; j < 2; ++j) {
            (void)hipEventDestroy(done[j]);
            (void)hipHostFree(stage[j]);
        }
        throw;
    }
    for (int j = 0; j < 2; ++j) {
        HIP_CHECK(hipEventDestroy(done[j]));
        HIP_CHECK(hipHostFree(stage[j]));
    }
}

}  // namespace

ModelWeights ModelWeights::load(const std::string& path) {
    File file(path);
    if (!file.f) throw std::runtime_error("ModelWeights: cannot open file: " + path);
    std::fseek(file.f, 0, SEEK_END);
    const int64_t file_size = file.tell();
    file.seek(0);

    char magic[4];
    file.read(magic, 4, "data");
    if (magic[0] != 'C' || magic[1] != 'S' || magic[2] != 'M' || magic[3] != '\0')
        throw std::runtime_error("ModelWeights: invalid magic (expected CSM\\0)");
    const uint32_t version = file.u32();
    if (version != 1) throw std::runtime_error("ModelWeights: unsupported version " + std::to_string(version));
    const uint32_t config_len = file.u32();
    std::string config_json(config_len, '\0');
    file.read(&config_json[0], config_len, "data");

    ModelWeights w;
    w.config_ = JsonValue::parse(config_json);

    // Pass 1: the tensor table (data skipped), with each tensor's place in the arena.
    const uint32_t n = file.u32();
    std::cout << "[ModelWeights] Loading " << n << " tensors from " << path << std::endl;
    std::vector<Entry> entries;
    entries.reserve(n);
    size_t arena = 0;
    for (uint32_t i = 0; i < n; ++i) {
        Entry e;
        const uint32_t name_len = file.u32();
        e.name.assign(name_len, '\0');
        file.read(&e.name[0], name_len, "data");
        const uint32_t ndim = file.u32();
        e.shape.resize(ndim);
        int64_t numel = 1;
        for (uint32_t d = 0; d < ndim; ++d) {
            e.shape[d] = file.i64();
            if (e.shape[d] < 0) throw std::runtime_error("ModelWeights: negative dimension for tensor " + e.name);
            // a shape whose element count does not fit int64 cannot describe data in a file
            if (__builtin_mul_overflow(numel, e.shape[d], &numel))
                throw std::runtime_error("ModelWeights: tensor too large: " + e.name);
        }
        const uint32_t dt = file.u32();
        if (dt > 3)
            throw std::runtime_error("ModelWeights: unknown dtype " + std::to_string(dt) + " for tensor " + e.name);
        e.dtype = (DType)dt;
        int64_t nbytes = 0;
        if (__builtin_mul_overflow(numel, (int64_t)dtype_size(e.dtype), &nbytes))
            throw std::runtime_error("ModelWeights: tensor too large: " + e.name);
        e.bytes = (size_t)nbytes;
        e.file_offset = file.tell();
        if (nbytes > file_size - e.file_offset)
            throw std::runtime_error("ModelWeights: unexpected EOF reading data");
        file.seek(e.file_offset + (int64_t)e.bytes);
        e.arena_offset = arena;
        arena += (e.bytes + kArenaAlign - 1) / kArenaAlign * kArenaAlign;
        entries.push_back(std::move(e));
    }

    // Pass 2: one device allocation, filled by a streamed upload; tensors are views into it.
    Tensor arena_t = Tensor::empty({(int64_t)std::max<size_t>(arena / 4, 1)}, DType::Float32);  // arena % 256 == 0
    char* base = static_cast<char*>(arena_t.data_ptr());
    upload(file, entries, base, HipContext::instance().stream());
    w.arena_bytes_ = arena;
    for (Entry& e : entries) {
        Tensor t;
        t.shape_ = e.shape;
        t.dtype_ = e.dtype;
        t.numel_ = 1;
        for (int64_t s : e.shape) t.numel_ *= s;
        t.compute_strides();
        t.storage_ = arena_t.storage_;
        t.data_ = base + e.arena_offset;
        w.tensors_[e.name] = std::move(t);
    }
    std::cout << "[ModelWeights] Loaded " << w.tensors_.size() << " tensors, config keys: "
              << (w.config_.is_object() ? w.config_.size() : 0) << std::endl;
    return w;
}

const Tensor& ModelWeights::get(const std::string& name) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) throw std::runtime_error("ModelWeights: tensor not found: " + name);
    return it->second;
}

bool ModelWeights::has(const std::string& name) const { return tensors_.count(name) > 0; }

std::vector<std::string> ModelWeights::tensor_names() const {
    std::vector<std::string> names;
    names.reserve(tensors_.size());
    for (const auto& kv : tensors_) names.push_back(kv.first);
    std::sort(names.begin(), names.end());
    return names;
}

void ModelWeights::convert_linear_weights_to_fp16() {
    int converted = 0;
    size_t saved = 0;
    for (auto& kv : tensors_) {
        if (kv.second.ndim() == 2 && kv.second.dtype() == DType::Float32) {
            saved += (size_t)kv.second.numel() * 2;
            kv.second = kv.second.to_f16();
            ++converted;
        }
    }
    std::cout << "  [FP16] Pre-converted " << converted << " linear weight tensors (saved " << (saved / 1048576)
              << " MB VRAM)" << std::endl;
}

void ModelWeights::convert_linear_weights_to_bf16() {
    int converted = 0;
    size_t saved = 0;
    for (auto& kv : tensors_) {
        if (kv.second.ndim() == 2 && kv.second.dtype() == DType::Float32) {
            saved += (size_t)kv.second.numel() * 2;
            kv.second = kv.second.to_bf16();
            ++converted;
        }
    }
    std::cout << "  [BF16] Pre-converted " << converted << " linear weight tensors (saved " << (saved / 1048576)
              << " MB VRAM)" << std::endl;
}

// ---- band tables ---------------------------------------------------------------------------

MelBandTables load_mel_band_tables(const ModelWeights& weights, int num_bands, int n_fft, bool stereo) {
    if (!weights.has("__precomputed__.freq_indices"))
        throw std::runtime_error("MelBandRoformer .csm must include precomputed mel band data");
    MelBandTables t;
    t.freq_indices = weights.get("__precomputed__.freq_indices");
    const Tensor& nfpb = weights.get("__precomputed__.num_freqs_per_band");
    const Tensor& nbpf = weights.get("__precomputed__.num_bands_per_freq");
    const int channels = stereo ? 2 : 1;
    const int bins = n_fft / 2 + 1;
    const int total_freq = bins * channels;
    if (t.freq_indices.dtype() != DType::Int64 || nfpb.dtype() != DType::Int64 || nbpf.dtype() != DType::Int64 ||
        nfpb.numel() < num_bands || nbpf.numel() < bins)
        throw std::runtime_error("MelBandRoformer: precomputed mel band tensors have unexpected shapes");

    t.num_freqs_per_band.resize((size_t)num_bands);
    nfpb.copy_to_cpu(t.num_freqs_per_band.data(), (size_t)num_bands * sizeof(int64_t));
    std::vector<int64_t> per_bin((size_t)bins);
    nbpf.copy_to_cpu(per_bin.data(), (size_t)bins * sizeof(int64_t));
    t.num_bands_per_freq_host.resize((size_t)total_freq);
    for (int f = 0; f < bins; ++f)
        for (int c = 0; c < channels; ++c) t.num_bands_per_freq_host[(size_t)(f * channels + c)] = per_bin[(size_t)f];
    t.band_freq_dims.resize((size_t)num_bands);
    for (int b = 0; b < num_bands; ++b) t.band_freq_dims[(size_t)b] = 2 * t.num_freqs_per_band[(size_t)b] * channels;

    const int64_t J = t.freq_indices.numel();
    t.freq_indices_host.resize((size_t)J);
    t.freq_indices.copy_to_cpu(t.freq_indices_host.data(), (size_t)J * sizeof(int64_t));
    std::vector<std::vector<int64_t>> by_freq((size_t)total_freq);
    for (int64_t j = 0; j < J; ++j) {
        const int64_t f = t.freq_indices_host[(size_t)j];
        if (f < 0 || f >= total_freq) throw std::runtime_error("MelBandRoformer: precomputed freq_indices out of range");
        by_freq[(size_t)f].push_back(j);
    }
    std::vector<int64_t> offsets((size_t)total_freq + 1, 0), indices;
    indices.reserve((size_t)J);
    for (int f = 0; f < total_freq; ++f) {
        offsets[(size_t)f] = (int64_t)indices.size();
        t.max_bands_per_freq = std::max<int64_t>(t.max_bands_per_freq, (int64_t)by_freq[(size_t)f].size());
        indices.insert(indices.end(), by_freq[(size_t)f].begin(), by_freq[(size_t)f].end());
    }
    offsets[(size_t)total_freq] = (int64_t)indices.size();
    t.freq_band_offsets = Tensor::from_cpu_i64(offsets.data(), {(int64_t)offsets.size()});
    t.freq_band_indices = Tensor::from_cpu_i64(indices.data(), {(int64_t)indices.size()});
    std::vector<float> counts(t.num_bands_per_freq_host.begin(), t.num_bands_per_freq_host.end());
    t.num_bands_per_freq = Tensor::from_cpu_f32(counts.data(), {(int64_t)total_freq});
    if (mbr_tile::bands_per_freq_bf16_enabled()) t.num_bands_per_freq = t.num_bands_per_freq.to_bf16();
    return t;
}

}  // namespace cudasep
