// kd_safetensors.h - safetensors reading for the GPT-2 engine (host only, no HIP).
//
// The format (reference src/io/safetensors.cpp:258-318): an 8-byte little-endian header length N,
// N bytes of JSON {"name": {"dtype", "shape", "data_offsets": [begin, end]}, ..., "__metadata__":
// {...}}, then the tensor bytes. Reading follows the reference's checks: the header fits the file
// and is at most 100 MB, every entry has a dtype, a shape of non-negative integers and two
// offsets whose span is exactly numel x element size, and the entries tile the data region in
// order with no gap or overlap. Bool bytes must be 0 or 1.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace kd::safetensors {

enum class DType { F32, F64, I64, Bool, F16, BF16 };

struct Entry {
    std::string name;
    DType dtype;
    std::vector<int64_t> shape;
    int64_t begin = 0, end = 0;  // byte offsets in the data region
    int64_t numel() const;
};

// A validated, memory-mapped safetensors file.
class File {
public:
    ~File();
    File(const File&) = delete;
    File& operator=(const File&) = delete;

    // Opens and checks `path`; nullptr with `*error` set when the file is not a valid safetensors
    // file (`*unsupported` is set when the only problem is a dtype outside F32 F64 I64 BOOL F16 BF16).
    static std::unique_ptr<File> open(const std::string& path, std::string* error, bool* unsupported);

    const std::vector<Entry>& entries() const { return entries_; }  // sorted by name
    const Entry* find(const std::string& name) const;
    const std::map<std::string, std::string>& metadata() const { return metadata_; }

    // The entry's values as float: F32 as stored, F64 / I64 / BOOL converted as kael's copy_ into
    // an f32 tensor converts them (static_cast), F16 / BF16 widened exactly. With `transpose`
    // (2-D entries only) out[j * rows + i] = value[i][j]. `out` holds numel floats.
    void to_f32(const Entry& e, float* out, bool transpose) const;

private:
    File() = default;
    const unsigned char* data_ = nullptr;  // start of the tensor bytes
    void* map_ = nullptr;
    size_t map_bytes_ = 0;
    std::vector<Entry> entries_;
    std::map<std::string, std::string> metadata_;
};

// kael's names for a Hugging Face GPT-2 checkpoint (reference src/nn/transformer.cpp:54-89
// translated_gpt2_name), and whether kael stores the translated weight transposed (HF's Conv1D
// layers keep [in, out]; stored_transposed).
std::string translated_gpt2_name(std::string name);
bool stored_transposed(const std::string& name);

}  // namespace kd::safetensors
