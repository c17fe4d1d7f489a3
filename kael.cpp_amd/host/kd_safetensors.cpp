// kd_safetensors.cpp - safetensors reading for the GPT-2 engine (host only).
//
// A minimal JSON parser of this repository's own (objects, arrays, strings with escapes, numbers,
// literals; strict: trailing text, control characters, bad escapes, lone surrogates and invalid
// UTF-8 are errors), then the reference's header checks (src/io/safetensors.cpp:64-133,258-310)
// over a read-only memory mapping of the file.
#include "kd_safetensors.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <limits>
#include <string_view>
#include <utility>

namespace kd::safetensors {

namespace {

constexpr uint64_t kMaxHeaderBytes = 100'000'000;
constexpr const char* kMetadataKey = "__metadata__";

struct Json {
    enum Kind { Null, Bool, Int, Real, String, Array, Object } kind = Null;
    bool negative = false;   // Int: the value is -magnitude
    uint64_t magnitude = 0;  // Int
    std::string text;        // String
    std::vector<Json> items;                          // Array
    std::vector<std::pair<std::string, Json>> members;  // Object, in document order

    // The member `key` (the last one when a key repeats, as the reference's parser keeps it).
    const Json* member(const std::string& key) const {
        const Json* found = nullptr;
        for (const auto& [k, v] : members)
            if (k == key) found = &v;
        return found;
    }
};

class Parser {
public:
    Parser(const char* begin, const char* end) : p_(begin), end_(end) {}

    bool parse(Json& out) {
        if (!value(out)) return false;
        space();
        return p_ == end_ || fail("text after the JSON value");
    }
    const std::string& error() const { return error_; }

private:
    const char* p_;
    const char* end_;
    int depth_ = 0;
    std::string error_;

    bool fail(const char* what) {
        if (error_.empty()) error_ = what;
        return false;
    }
    void space() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool literal(const char* word) {
        const size_t n = std::strlen(word);
        if (static_cast<size_t>(end_ - p_) < n || std::memcmp(p_, word, n) != 0) return fail("invalid literal");
        p_ += n;
        return true;
    }
    bool value(Json& out) {
        space();
        if (p_ == end_) return fail("unexpected end of the header");
        switch (*p_) {
        case '{': return object(out);
        case '[': return array(out);
        case '"': out.kind = Json::String; return string(out.text);
        case 't': out.kind = Json::Bool; return literal("true");
        case 'f': out.kind = Json::Bool; return literal("false");
        case 'n': out.kind = Json::Null; return literal("null");
        default: return number(out);
        }
    }
    bool object(Json& out) {
        if (++depth_ > 128) return fail("JSON nested too deeply");
        ++p_;
        out.kind = Json::Object;
        space();
        if (p_ < end_ && *p_ == '}') {
            ++p_;
            --depth_;
            return true;
        }
        for (;;) {
            space();
            if (p_ == end_ || *p_ != '"') return fail("expected a member name");
            std::string key;
            if (!string(key)) return false;
            space();
            if (p_ == end_ || *p_ != ':') return fail("expected ':'");
            ++p_;
            Json v;
            if (!value(v)) return false;
            out.members.emplace_back(std::move(key), std::move(v));
            space();
            if (p_ < end_ && *p_ == ',') {
                ++p_;
                continue;
            }
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                --depth_;
                return true;
            }
            return fail("expected ',' or '}'");
        }
    }
    bool array(Json& out) {
        if (++depth_ > 128) return fail("JSON nested too deeply");
        ++p_;
        out.kind = Json::Array;
        space();
        if (p_ < end_ && *p_ == ']') {
            ++p_;
            --depth_;
            return true;
        }
        for (;;) {
            Json v;
            if (!value(v)) return false;
            out.items.push_back(std::move(v));
            space();
            if (p_ < end_ && *p_ == ',') {
                ++p_;
                continue;
            }
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                --depth_;
                return true;
            }
            return fail("expected ',' or ']'");
        }
    }
    static void utf8(std::string& s, uint32_t c) {
        if (c < 0x80) {
            s += static_cast<char>(c);
        } else if (c < 0x800) {
            s += static_cast<char>(0xC0 | (c >> 6));
            s += static_cast<char>(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            s += static_cast<char>(0xE0 | (c >> 12));
            s += static_cast<char>(0x80 | ((c >> 6) & 0x3F));
            s += static_cast<char>(0x80 | (c & 0x3F));
        } else {
            s += static_cast<char>(0xF0 | (c >> 18));
            s += static_cast<char>(0x80 | ((c >> 12) & 0x3F));
            s += static_cast<char>(0x80 | ((c >> 6) & 0x3F));
            s += static_cast<char>(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t& v) {
        if (end_ - p_ < 4) return fail("truncated \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    // One UTF-8 sequence starting at p_ (first byte >= 0x80), copied to s.
    bool utf8_sequence(std::string& s) {
        const auto b0 = static_cast<unsigned char>(*p_);
        int n = 0;
        uint32_t c = 0, least = 0;
        if ((b0 & 0xE0) == 0xC0) n = 1, c = b0 & 0x1F, least = 0x80;
        else if ((b0 & 0xF0) == 0xE0) n = 2, c = b0 & 0x0F, least = 0x800;
        else if ((b0 & 0xF8) == 0xF0) n = 3, c = b0 & 0x07, least = 0x10000;
        else return fail("invalid UTF-8 in a string");
        if (end_ - p_ < n + 1) return fail("invalid UTF-8 in a string");
        for (int i = 1; i <= n; ++i) {
            const auto b = static_cast<unsigned char>(p_[i]);
            if ((b & 0xC0) != 0x80) return fail("invalid UTF-8 in a string");
            c = (c << 6) | (b & 0x3F);
        }
        if (c < least || c > 0x10FFFF || (c >= 0xD800 && c <= 0xDFFF)) return fail("invalid UTF-8 in a string");
        s.append(p_, static_cast<size_t>(n + 1));
        p_ += n + 1;
        return true;
    }
    bool string(std::string& s) {
        ++p_;  // opening quote
        for (;;) {
            if (p_ == end_) return fail("unterminated string");
            const char c = *p_;
            if (c == '"') {
                ++p_;
                return true;
            }
            if (static_cast<unsigned char>(c) < 0x20) return fail("control character in a string");
            if (static_cast<unsigned char>(c) >= 0x80) {
                if (!utf8_sequence(s)) return false;
                continue;
            }
            ++p_;
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ == end_) return fail("unterminated string");
            const char e = *p_++;
            switch (e) {
            case '"': s += '"'; break;
            case '\\': s += '\\'; break;
            case '/': s += '/'; break;
            case 'b': s += '\b'; break;
            case 'f': s += '\f'; break;
            case 'n': s += '\n'; break;
            case 'r': s += '\r'; break;
            case 't': s += '\t'; break;
            case 'u': {
                uint32_t u = 0;
                if (!hex4(u)) return false;
                if (u >= 0xD800 && u <= 0xDBFF) {
                    uint32_t low = 0;
                    if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate in a string");
                    p_ += 2;
                    if (!hex4(low)) return false;
                    if (low < 0xDC00 || low > 0xDFFF) return fail("lone surrogate in a string");
                    u = 0x10000 + ((u - 0xD800) << 10) + (low - 0xDC00);
                } else if (u >= 0xDC00 && u <= 0xDFFF) {
                    return fail("lone surrogate in a string");
                }
                utf8(s, u);
                break;
            }
            default: return fail("bad escape in a string");
            }
        }
    }
    bool number(Json& out) {
        const char* start = p_;
        bool negative = false;
        if (p_ < end_ && *p_ == '-') negative = true, ++p_;
        if (p_ == end_ || *p_ < '0' || *p_ > '9') return fail("invalid value");
        if (*p_ == '0' && p_ + 1 < end_ && p_[1] >= '0' && p_[1] <= '9') return fail("leading zero in a number");
        bool overflow = false;
        uint64_t m = 0;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t digit = static_cast<uint64_t>(*p_ - '0');
            if (m > (std::numeric_limits<uint64_t>::max() - digit) / 10) overflow = true;
            else m = m * 10 + digit;
            ++p_;
        }
        bool integer = true;
        if (p_ < end_ && *p_ == '.') {
            integer = false;
            ++p_;
            if (p_ == end_ || *p_ < '0' || *p_ > '9') return fail("invalid number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integer = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ == end_ || *p_ < '0' || *p_ > '9') return fail("invalid number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        (void)start;
        // an integer too large for 64 bits is a floating-point number, as the reference's parser reads it
        out.kind = integer && !overflow ? Json::Int : Json::Real;
        out.negative = negative;
        out.magnitude = m;
        return true;
    }
};

bool non_negative_integer(const Json& v, const std::string& what, int64_t* out, std::string* error) {
    if (v.kind != Json::Int) {
        *error = what + " must be an integer";
        return false;
    }
    if (v.negative && v.magnitude != 0) {
        *error = what + " must not be negative";
        return false;
    }
    if (v.magnitude > static_cast<uint64_t>(std::numeric_limits<int64_t>::max())) {
        *error = what + " does not fit in int64";
        return false;
    }
    *out = static_cast<int64_t>(v.magnitude);
    return true;
}

int64_t element_bytes(DType d) {
    switch (d) {
    case DType::F64:
    case DType::I64: return 8;
    case DType::Bool: return 1;
    case DType::F16:
    case DType::BF16: return 2;
    default: return 4;
    }
}

bool dtype_from_name(const std::string& name, DType* out) {
    static const std::pair<const char*, DType> kNames[] = {{"F32", DType::F32}, {"F64", DType::F64}, {"I64", DType::I64},
                                                           {"BOOL", DType::Bool}, {"F16", DType::F16},
                                                           {"BF16", DType::BF16}};
    for (const auto& [n, d] : kNames)
        if (name == n) return *out = d, true;
    return false;
}

float half_to_float(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1Fu;
    uint32_t mantissa = h & 0x3FFu;
    uint32_t bits;
    if (exponent == 0x1F) {
        bits = sign | 0x7F800000u | (mantissa << 13);  // infinity or NaN (payload kept)
    } else if (exponent != 0) {
        bits = sign | ((exponent + 112) << 23) | (mantissa << 13);
    } else if (mantissa == 0) {
        bits = sign;  // signed zero
    } else {  // subnormal half: normalise (every half subnormal is a normal float)
        int e = 113;
        while ((mantissa & 0x400u) == 0) {
            mantissa <<= 1;
            --e;
        }
        bits = sign | (static_cast<uint32_t>(e) << 23) | ((mantissa & 0x3FFu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, sizeof f);
    return f;
}

}  // namespace

int64_t Entry::numel() const {
    int64_t n = 1;
    for (const int64_t s : shape) n *= s;
    return n;
}

File::~File() {
    if (map_ != nullptr) ::munmap(map_, map_bytes_);
}

const Entry* File::find(const std::string& name) const {
    const auto it = std::lower_bound(entries_.begin(), entries_.end(), name,
                                     [](const Entry& e, const std::string& n) { return e.name < n; });
    return it != entries_.end() && it->name == name ? &*it : nullptr;
}

std::unique_ptr<File> File::open(const std::string& path, std::string* error, bool* unsupported) {
    *unsupported = false;
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        *error = "cannot open safetensors file " + path;
        return nullptr;
    }
    struct stat st {};
    if (::fstat(fd, &st) != 0) {
        ::close(fd);
        *error = "cannot open safetensors file " + path;
        return nullptr;
    }
    const auto file_size = static_cast<uint64_t>(st.st_size);
    if (file_size < sizeof(uint64_t)) {
        ::close(fd);
        *error = "safetensors file " + path + " is too short";
        return nullptr;
    }
    void* map = ::mmap(nullptr, static_cast<size_t>(file_size), PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map == MAP_FAILED) {
        *error = "cannot map safetensors file " + path;
        return nullptr;
    }
    std::unique_ptr<File> f(new File());
    f->map_ = map;
    f->map_bytes_ = static_cast<size_t>(file_size);
    const auto* bytes = static_cast<const unsigned char*>(map);
    uint64_t header_size = 0;
    for (int i = 7; i >= 0; --i) header_size = (header_size << 8) | bytes[i];  // little-endian
    if (header_size > kMaxHeaderBytes || header_size > file_size - sizeof(uint64_t)) {
        *error = "safetensors header of " + std::to_string(header_size) + " bytes does not fit the file";
        return nullptr;
    }
    const char* text = reinterpret_cast<const char*>(bytes + sizeof(uint64_t));
    Json header;
    Parser parser(text, text + header_size);
    if (!parser.parse(header) || header.kind != Json::Object) {
        *error = "safetensors header of " + path + " is not a JSON object" +
                 (parser.error().empty() ? std::string() : " (" + parser.error() + ")");
        return nullptr;
    }
    // a repeated name keeps its last description, as the reference's parser does
    std::map<std::string, const Json*> described;
    for (const auto& [name, value] : header.members) described[name] = &value;
    for (const auto& [name, value_ptr] : described) {
        const Json& value = *value_ptr;
        if (name == kMetadataKey) {
            if (value.kind != Json::Object) {
                *error = "safetensors metadata is not an object";
                return nullptr;
            }
            for (const auto& [key, v] : value.members) {
                if (v.kind != Json::String) {
                    *error = "safetensors metadata " + key + " is not a string";
                    return nullptr;
                }
                f->metadata_[key] = v.text;  // a repeated key keeps its last value
            }
            continue;
        }
        if (value.kind != Json::Object) {
            *error = "safetensors entry " + name + " is not an object";
            return nullptr;
        }
        const Json* dtype = value.member("dtype");
        const Json* shape = value.member("shape");
        const Json* offsets = value.member("data_offsets");
        if (dtype == nullptr || dtype->kind != Json::String) {
            *error = "safetensors entry " + name + " has no dtype";
            return nullptr;
        }
        if (shape == nullptr || shape->kind != Json::Array) {
            *error = "safetensors entry " + name + " has no shape";
            return nullptr;
        }
        if (offsets == nullptr || offsets->kind != Json::Array || offsets->items.size() != 2) {
            *error = "safetensors entry " + name + " needs two data offsets";
            return nullptr;
        }
        Entry e;
        e.name = name;
        if (!dtype_from_name(dtype->text, &e.dtype)) {
            *unsupported = true;
            *error = "safetensors dtype '" + dtype->text + "' is not supported: F32, F64, I64, BOOL, F16 and BF16 are";
            return nullptr;
        }
        for (const Json& s : shape->items) {
            int64_t n = 0;
            if (!non_negative_integer(s, "a dimension of " + name, &n, error)) return nullptr;
            e.shape.push_back(n);
        }
        if (!non_negative_integer(offsets->items[0], "an offset of " + name, &e.begin, error) ||
            !non_negative_integer(offsets->items[1], "an offset of " + name, &e.end, error))
            return nullptr;
        if (e.begin > e.end) {
            *error = "safetensors entry " + name + " ends before it starts";
            return nullptr;
        }
        // numel x element size without overflow
        int64_t need = element_bytes(e.dtype);
        for (const int64_t s : e.shape) {
            if (s != 0 && need > std::numeric_limits<int64_t>::max() / s) {
                *error = "tensor size in bytes of " + name + " overflows int64";
                return nullptr;
            }
            need *= s;
        }
        if (e.end - e.begin != need) {
            *error = "safetensors entry " + name + " has " + std::to_string(e.end - e.begin) +
                     " bytes but its shape and dtype need " + std::to_string(need);
            return nullptr;
        }
        f->entries_.push_back(std::move(e));
    }
    // the entries tile the data region in order (reference check_layout)
    std::vector<const Entry*> by_offset;
    for (const Entry& e : f->entries_) by_offset.push_back(&e);
    std::sort(by_offset.begin(), by_offset.end(), [](const Entry* a, const Entry* b) {
        return a->begin != b->begin ? a->begin < b->begin : a->end < b->end;
    });
    const auto data_size = static_cast<int64_t>(file_size - sizeof(uint64_t) - header_size);
    int64_t position = 0;
    for (const Entry* e : by_offset) {
        if (e->begin != position) {
            *error = "safetensors entry " + e->name + " starts at " + std::to_string(e->begin) +
                     " but the previous one ended at " + std::to_string(position);
            return nullptr;
        }
        position = e->end;
    }
    if (position != data_size) {
        *error = "safetensors tensors cover " + std::to_string(position) + " bytes but the file has " +
                 std::to_string(data_size);
        return nullptr;
    }
    f->data_ = bytes + sizeof(uint64_t) + header_size;
    for (const Entry& e : f->entries_) {
        if (e.dtype != DType::Bool) continue;
        for (int64_t i = e.begin; i < e.end; ++i) {
            if (f->data_[i] > 1) {
                *error = "safetensors bool tensor " + e.name + " has the byte " + std::to_string(f->data_[i]);
                return nullptr;
            }
        }
    }
    return f;
}

void File::to_f32(const Entry& e, float* out, bool transpose) const {
    const unsigned char* src = data_ + e.begin;
    const int64_t n = e.numel();
    const int64_t rows = transpose ? e.shape[0] : 1, cols = transpose ? e.shape[1] : n;
    const auto value = [&](int64_t k) -> float {
        switch (e.dtype) {
        case DType::F32: {
            float v;
            std::memcpy(&v, src + 4 * k, 4);
            return v;
        }
        case DType::F64: {
            double v;
            std::memcpy(&v, src + 8 * k, 8);
            return static_cast<float>(v);
        }
        case DType::I64: {
            int64_t v;
            std::memcpy(&v, src + 8 * k, 8);
            return static_cast<float>(v);
        }
        case DType::Bool: return src[k] != 0 ? 1.f : 0.f;
        case DType::F16: {
            uint16_t h;
            std::memcpy(&h, src + 2 * k, 2);
            return half_to_float(h);
        }
        case DType::BF16: {
            uint16_t h;
            std::memcpy(&h, src + 2 * k, 2);
            const uint32_t bits = static_cast<uint32_t>(h) << 16;
            float v;
            std::memcpy(&v, &bits, 4);
            return v;
        }
        }
        return 0.f;
    };
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t j = 0; j < cols; ++j) {
            const int64_t k = i * cols + j;
            out[transpose ? j * rows + i : k] = value(k);
        }
}

// The Hugging Face GPT-2 checkpoint's names against kael's module names (the mapping of reference
// src/nn/transformer.cpp:54-91, a format): an optional "transformer." prefix is dropped, a name
// starting with a top-level entry's `from` has it replaced, and a block's name ("h.<i>." ->
// "blocks.<i>.") then has each sub-module's first occurrence renamed.
struct Rename {
    std::string_view from, to;
};
constexpr Rename kTopLevel[] = {
    {"wte.", "token_embedding."}, {"wpe.", "position_embedding."}, {"ln_f.", "ln_final."}, {"h.", "blocks."}};
constexpr Rename kInBlock[] = {{".ln_1.", ".ln1."},           {".ln_2.", ".ln2."},
                               {".attn.c_attn.", ".attn.qkv."}, {".attn.c_proj.", ".attn.proj."},
                               {".mlp.c_fc.", ".mlp.fc1."},     {".mlp.c_proj.", ".mlp.fc2."}};
// The four Conv1D modules (kael's names), whose weights the checkpoint stores [in, out].
constexpr std::string_view kConv1d[] = {".attn.qkv.", ".attn.proj.", ".mlp.fc1.", ".mlp.fc2."};

std::string translated_gpt2_name(std::string name) {
    constexpr std::string_view prefix = "transformer.";
    if (name.starts_with(prefix)) name.erase(0, prefix.size());
    for (const Rename& top : kTopLevel) {
        if (!name.starts_with(top.from)) continue;
        name.replace(0, top.from.size(), top.to);
        if (top.from == "h.") {
            for (const Rename& sub : kInBlock) {
                const auto at = name.find(sub.from);
                if (at != std::string::npos) name.replace(at, sub.from.size(), sub.to);
            }
        }
        break;
    }
    return name;
}

bool stored_transposed(const std::string& name) {
    bool conv1d = false;
    for (const std::string_view module : kConv1d) conv1d = conv1d || name.find(module) != std::string::npos;
    return conv1d && name.ends_with(".weight");
}

}  // namespace kd::safetensors
