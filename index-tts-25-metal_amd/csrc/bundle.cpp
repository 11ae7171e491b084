// MIT2 weight bundles: the on-disk format the reference loads its models from
// (vendor/metal-runtime/bundle.cpp:150-293, include/mit2/bundle.hpp) and the IndexTTS
// checks its Weights facade adds on top (src/weights.cpp:9-49).
//
// A bundle is either
//   * a directory holding manifest.json and a weights file (manifest key "weights_file",
//     default weights.bin), or
//   * one file: the weights stream followed by the manifest JSON and a 24-byte footer
//     [u64 manifest offset][u64 manifest size]["MIT2VOIC"] (little-endian).
// The weights stream starts with a 12-byte header: "MIT2", u32 version, u32 alignment,
// which must equal the manifest's.  Each manifest tensor record gives name, shape, dtype,
// offset and nbytes; offsets are multiples of the alignment and lie inside the file.
//
// The file is memory-mapped and never copied on the host: itts_gpt_create_from_bundle
// (runtime.hip) hands the mapped tensors to the decoder, which uploads them.  The
// manifest is read with a small JSON parser of this file's own (objects, arrays,
// strings, integers, literals); the error messages and the order of the checks are the
// reference's, so a caller sees the same exceptions for the same broken bundles.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <fstream>
#include <limits>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "itts_gpt.h"

namespace {

thread_local std::string g_bundle_error;

// ------------------------------------------------------------------ JSON

struct JValue {
    enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
    std::string text;  // string contents, or the literal of a number
    bool flag = false;
    std::vector<JValue> items;
    std::vector<std::pair<std::string, JValue>> members;

    const JValue* member(const std::string& key) const {
        for (const auto& m : members)
            if (m.first == key) return &m.second;
        return nullptr;
    }
};

class JsonReader {
public:
    explicit JsonReader(const std::string& s) : p_(s.data()), end_(s.data() + s.size()) {}
    JValue document() {
        JValue v = value(0);
        skip_space();
        if (p_ != end_) fail("trailing characters");
        return v;
    }

private:
    const char* p_;
    const char* end_;

    [[noreturn]] void fail(const char* what) const { throw std::runtime_error(std::string("invalid manifest JSON: ") + what); }
    void skip_space() {
        while (p_ != end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool take(char c) {
        skip_space();
        if (p_ != end_ && *p_ == c) {
            ++p_;
            return true;
        }
        return false;
    }
    void expect(char c) {
        if (!take(c)) fail("unexpected character");
    }
    static void put_utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) {
            out += static_cast<char>(cp);
        } else if (cp < 0x800) {
            out += static_cast<char>(0xC0 | (cp >> 6));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += static_cast<char>(0xE0 | (cp >> 12));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            out += static_cast<char>(0xF0 | (cp >> 18));
            out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }
    uint32_t hex4() {
        if (end_ - p_ < 4) fail("short \\u escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i, ++p_) {
            const char c = *p_;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
            else fail("bad \\u escape");
        }
        return v;
    }
    std::string string_body() {  // after the opening quote
        std::string out;
        while (true) {
            if (p_ == end_) fail("unterminated string");
            const char c = *p_++;
            if (c == '"') return out;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p_ == end_) fail("unterminated escape");
            const char e = *p_++;
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
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
                        p_ += 2;
                        const uint32_t lo = hex4();
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: fail("bad escape");
            }
        }
    }
    JValue value(int depth) {
        if (depth > 64) fail("nesting too deep");
        skip_space();
        if (p_ == end_) fail("unexpected end");
        JValue v;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = JValue::kObject;
            if (take('}')) return v;
            do {
                skip_space();
                if (p_ == end_ || *p_ != '"') fail("expected a key");
                ++p_;
                std::string key = string_body();
                expect(':');
                v.members.emplace_back(std::move(key), value(depth + 1));
            } while (take(','));
            expect('}');
        } else if (c == '[') {
            ++p_;
            v.kind = JValue::kArray;
            if (take(']')) return v;
            do v.items.push_back(value(depth + 1));
            while (take(','));
            expect(']');
        } else if (c == '"') {
            ++p_;
            v.kind = JValue::kString;
            v.text = string_body();
        } else if (c == '-' || (c >= '0' && c <= '9')) {
            v.kind = JValue::kNumber;
            const char* b = p_;
            while (p_ != end_ && (*p_ == '-' || *p_ == '+' || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || (*p_ >= '0' && *p_ <= '9'))) ++p_;
            v.text.assign(b, p_);
        } else if (end_ - p_ >= 4 && std::strncmp(p_, "true", 4) == 0) {
            p_ += 4;
            v.kind = JValue::kBool;
            v.flag = true;
        } else if (end_ - p_ >= 5 && std::strncmp(p_, "false", 5) == 0) {
            p_ += 5;
            v.kind = JValue::kBool;
        } else if (end_ - p_ >= 4 && std::strncmp(p_, "null", 4) == 0) {
            p_ += 4;
        } else {
            fail("unexpected character");
        }
        return v;
    }
};

// Exact conversions of integer literals (offsets exceed 2^53 only in theory, but a double
// round trip is not needed).
bool parse_u64(const std::string& s, uint64_t& out) {
    if (s.empty()) return false;
    uint64_t v = 0;
    for (const char c : s) {
        if (c < '0' || c > '9') return false;
        const uint64_t d = static_cast<uint64_t>(c - '0');
        if (v > (std::numeric_limits<uint64_t>::max() - d) / 10) return false;
        v = v * 10 + d;
    }
    out = v;
    return true;
}
bool parse_i64(const std::string& s, int64_t& out) {
    const bool neg = !s.empty() && s[0] == '-';
    uint64_t m = 0;
    if (!parse_u64(neg ? s.substr(1) : s, m)) return false;
    if (m > static_cast<uint64_t>(std::numeric_limits<int64_t>::max())) return false;
    out = neg ? -static_cast<int64_t>(m) : static_cast<int64_t>(m);
    return true;
}

// Manifest accessors with the reference's fallbacks and messages (bundle.cpp:38-68).
std::string get_string(const JValue& obj, const std::string& key, const std::string& fallback = "") {
    const JValue* v = obj.member(key);
    return v && v->kind == JValue::kString ? v->text : fallback;
}
uint64_t get_uint(const JValue& obj, const std::string& key) {
    const JValue* v = obj.member(key);
    uint64_t out = 0;
    if (!v || v->kind != JValue::kNumber || !parse_u64(v->text, out)) throw std::runtime_error("missing numeric key " + key);
    return out;
}
std::vector<int64_t> get_shape(const JValue& obj) {
    const JValue* v = obj.member("shape");
    if (!v || v->kind != JValue::kArray) throw std::runtime_error("missing tensor shape");
    std::vector<int64_t> shape;
    for (const auto& d : v->items) {
        int64_t x = 0;
        if (d.kind != JValue::kNumber || !parse_i64(d.text, x)) throw std::runtime_error("missing tensor shape");
        shape.push_back(x);
    }
    return shape;
}

uint32_t read_u32_le(const uint8_t* p) {
    return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8) | (static_cast<uint32_t>(p[2]) << 16) |
           (static_cast<uint32_t>(p[3]) << 24);
}
uint64_t read_u64_le(const uint8_t* p) { return static_cast<uint64_t>(read_u32_le(p)) | (static_cast<uint64_t>(read_u32_le(p + 4)) << 32); }

std::string read_file_text(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("failed to open " + path);
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

// ------------------------------------------------------------------ mapped file

class Mapping {
public:
    explicit Mapping(const std::string& path) {
        fd_ = ::open(path.c_str(), O_RDONLY);
        if (fd_ < 0) throw std::runtime_error("failed to open mapped file: " + path);
        struct stat st {};
        if (::fstat(fd_, &st) != 0) {
            ::close(fd_);
            throw std::runtime_error("failed to stat mapped file: " + path);
        }
        size_ = static_cast<size_t>(st.st_size);
        if (size_ > 0) {
            void* m = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
            if (m == MAP_FAILED) {
                ::close(fd_);
                throw std::runtime_error("failed to mmap file: " + path);
            }
            data_ = static_cast<const uint8_t*>(m);
        }
    }
    ~Mapping() {
        if (data_) ::munmap(const_cast<uint8_t*>(data_), size_);
        if (fd_ >= 0) ::close(fd_);
    }
    Mapping(const Mapping&) = delete;
    Mapping& operator=(const Mapping&) = delete;
    const uint8_t* data() const { return data_; }
    size_t size() const { return size_; }

private:
    int fd_ = -1;
    const uint8_t* data_ = nullptr;
    size_t size_ = 0;
};

constexpr size_t kFooterSize = 24;
constexpr char kFooterMagic[8] = {'M', 'I', 'T', '2', 'V', 'O', 'I', 'C'};

struct TensorRecord {
    std::string name;
    std::vector<int64_t> shape;
    std::string dtype;
    uint64_t offset = 0;
    uint64_t nbytes = 0;
};

}  // namespace

struct itts_bundle {
    std::unique_ptr<Mapping> weights;
    std::vector<TensorRecord> tensors;
    std::unordered_map<std::string, size_t> by_name;

    explicit itts_bundle(const std::string& path, bool require_model) {
        struct stat st {};
        const bool single_file = ::stat(path.c_str(), &st) == 0 && S_ISREG(st.st_mode);
        std::string json;
        if (single_file) {
            weights = std::make_unique<Mapping>(path);
            const size_t size = weights->size();
            if (size < 12 + kFooterSize) throw std::runtime_error("single-file bundle is too small: " + path);
            const uint8_t* footer = weights->data() + size - kFooterSize;
            if (std::memcmp(footer + 16, kFooterMagic, 8) != 0) throw std::runtime_error("single-file bundle footer magic missing: " + path);
            const uint64_t off = read_u64_le(footer), len = read_u64_le(footer + 8);
            if (off > size - kFooterSize || len > size - kFooterSize - off)
                throw std::runtime_error("single-file bundle manifest exceeds file: " + path);
            json.assign(reinterpret_cast<const char*>(weights->data() + off), static_cast<size_t>(len));
        } else {
            json = read_file_text(path + "/manifest.json");
        }
        const JValue doc = JsonReader(json).document();
        const std::string format = get_string(doc, "format");
        if (format != "MIT2") throw std::runtime_error("unsupported bundle format: " + format);
        const uint64_t version = get_uint(doc, "version");
        const uint64_t alignment = get_uint(doc, "alignment");
        const std::string endianness = get_string(doc, "endianness");
        if (version != 1) throw std::runtime_error("unsupported bundle version: " + std::to_string(static_cast<uint32_t>(version)));
        if (static_cast<uint32_t>(alignment) == 0) throw std::runtime_error("bundle alignment must be non-zero");
        if (endianness != "little") throw std::runtime_error("unsupported bundle endianness: " + endianness);
        if (!single_file) weights = std::make_unique<Mapping>(path + "/" + get_string(doc, "weights_file", "weights.bin"));
        const size_t size = weights->size();
        if (size < 12) throw std::runtime_error("weights file is too small for MIT2 header");
        const uint8_t* header = weights->data();
        if (std::memcmp(header, "MIT2", 4) != 0) throw std::runtime_error("weights file has invalid MIT2 magic");
        if (read_u32_le(header + 4) != static_cast<uint32_t>(version)) throw std::runtime_error("weights header version mismatch");
        if (read_u32_le(header + 8) != static_cast<uint32_t>(alignment)) throw std::runtime_error("weights header alignment mismatch");
        const JValue* list = doc.member("tensors");
        if (!list) throw std::runtime_error("manifest missing tensors");
        if (list->kind != JValue::kArray) throw std::runtime_error("invalid tensors array");
        const uint32_t align32 = static_cast<uint32_t>(alignment);
        for (const auto& obj : list->items) {
            if (obj.kind != JValue::kObject) continue;
            TensorRecord t;
            t.name = get_string(obj, "name");
            t.shape = get_shape(obj);
            t.dtype = get_string(obj, "dtype");
            t.offset = get_uint(obj, "offset");
            t.nbytes = get_uint(obj, "nbytes");
            if (t.name.empty()) throw std::runtime_error("tensor record has empty name");
            if (by_name.count(t.name)) throw std::runtime_error("duplicate tensor in manifest: " + t.name);
            if (t.offset % align32 != 0) throw std::runtime_error("tensor offset is not bundle-aligned: " + t.name);
            if (t.nbytes == 0) throw std::runtime_error("tensor has zero bytes: " + t.name);
            if (t.offset > size || t.nbytes > size - t.offset) throw std::runtime_error("tensor extends beyond weights file: " + t.name);
            by_name.emplace(t.name, tensors.size());
            tensors.push_back(std::move(t));
        }
        // itts25::Weights (weights.cpp:9-28).  As there, the model check reads
        // <path>/manifest.json, so a single-file bundle opens only without it.
        if (require_model) {
            std::string text;
            {
                std::ifstream f(path + "/manifest.json", std::ios::binary);
                if (f) {
                    std::ostringstream ss;
                    ss << f.rdbuf();
                    text = ss.str();
                }
            }
            bool is_model = false;
            if (!text.empty()) {
                try {
                    const JValue m = JsonReader(text).document();
                    is_model = target_is_model(m);
                } catch (const std::runtime_error&) {
                }
            }
            if (!is_model) throw std::runtime_error("Expected an IndexTTS 2.5 model bundle");
        }
        for (const auto& t : tensors) {
            const size_t element = t.dtype == "f32" || t.dtype == "u32" ? 4 : 0;
            if (!element) throw std::runtime_error("Initial native backend requires f32/u32: " + t.name);
            size_t count = 1;
            for (const int64_t n : t.shape) {
                if (n <= 0 || static_cast<uint64_t>(n) > std::numeric_limits<size_t>::max() / count)
                    throw std::runtime_error("Invalid shape: " + t.name);
                count *= static_cast<size_t>(n);
            }
            if (count > std::numeric_limits<size_t>::max() / element || count * element != t.nbytes)
                throw std::runtime_error("Tensor size does not match shape: " + t.name);
        }
    }

    // The reference matches "target": "index-tts2.5" anywhere in the manifest text
    // (weights.cpp:12); a manifest names it in "metadata" or at the top level.
    static bool target_is_model(const JValue& v) {
        if (v.kind == JValue::kObject) {
            for (const auto& m : v.members) {
                if (m.first == "target" && m.second.kind == JValue::kString && m.second.text == "index-tts2.5") return true;
                if (target_is_model(m.second)) return true;
            }
        } else if (v.kind == JValue::kArray) {
            for (const auto& i : v.items)
                if (target_is_model(i)) return true;
        }
        return false;
    }

    void describe(size_t i, itts_bundle_tensor* out) const {
        const TensorRecord& t = tensors[i];
        std::memset(out, 0, sizeof(*out));
        out->name = t.name.c_str();
        out->data = weights->data() + t.offset;
        out->ndim = static_cast<int32_t>(t.shape.size());
        for (size_t d = 0; d < t.shape.size() && d < 8; ++d) out->shape[d] = t.shape[d];
        out->dtype = t.dtype == "f32" ? ITTS_DTYPE_F32 : ITTS_DTYPE_U32;
        out->offset = t.offset;
        out->nbytes = t.nbytes;
    }
};

namespace {

template <class F>
int bundle_guard(F&& f) {
    try {
        f();
        return ITTS_OK;
    } catch (const std::invalid_argument& e) {
        g_bundle_error = e.what();
        return ITTS_EINVAL;
    } catch (const std::exception& e) {
        g_bundle_error = e.what();
        return ITTS_ERUNTIME;
    }
}

}  // namespace

extern "C" {

int itts_bundle_open(const char* path, int32_t require_model, itts_bundle** out) {
    if (!out) return ITTS_EINVAL;
    *out = nullptr;
    return bundle_guard([&] {
        if (!path) throw std::invalid_argument("Invalid bundle path");
        *out = new itts_bundle(path, require_model != 0);
    });
}

void itts_bundle_close(itts_bundle* b) { delete b; }

const char* itts_bundle_last_error(void) { return g_bundle_error.c_str(); }

int32_t itts_bundle_count(const itts_bundle* b) { return b ? static_cast<int32_t>(b->tensors.size()) : 0; }

int itts_bundle_tensor_at(const itts_bundle* b, int32_t index, itts_bundle_tensor* out) {
    return bundle_guard([&] {
        if (!b || !out || index < 0 || static_cast<size_t>(index) >= b->tensors.size())
            throw std::invalid_argument("Invalid bundle tensor index");
        b->describe(static_cast<size_t>(index), out);
    });
}

int itts_bundle_find(const itts_bundle* b, const char* name, itts_bundle_tensor* out) {
    return bundle_guard([&] {
        if (!b || !name || !out) throw std::invalid_argument("Invalid bundle lookup");
        const auto it = b->by_name.find(name);
        if (it == b->by_name.end()) throw std::runtime_error(std::string("Missing tensor: ") + name);
        b->describe(it->second, out);
    });
}

}  // extern "C"
