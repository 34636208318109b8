// ttlab::GgufFile -- a read-only, memory-mapped GGUF (version 3) file: metadata
// key/values and tensor descriptors, with tensor data pointing into the mapping.
// The same file format and checks as the reference's GgufFile (gguf.h:13-85,
// gguf.cpp:145-239): little-endian, magic "GGUF", version 3, tensor data at the
// header end rounded up to general.alignment (default 32), every tensor inside the
// file.  Errors are std::runtime_error with the reference's messages.
#pragma once

#include "gguf_source.hpp"  // gguf_row_bytes

#include <cstddef>
#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace ttlab {

// GGUF metadata value types (gguf.h:13-27).
enum class GgufKind : uint32_t {
    u8 = 0, i8 = 1, u16 = 2, i16 = 3, u32 = 4, i32 = 5, f32 = 6, boolean = 7,
    string = 8, array = 9, u64 = 10, i64 = 11, f64 = 12,
};

// GGML tensor type ids used by gpt-oss GGUFs (tensor.h:11-13) plus BF16.
constexpr uint32_t kGgmlF32 = 0, kGgmlQ8_0 = 8, kGgmlBf16 = 30, kGgmlMxfp4 = 39;

struct GgufEntry {
    GgufKind kind{};
    GgufKind element{};          // arrays only
    uint64_t count = 1;          // arrays only
    const uint8_t *raw = nullptr;  // fixed-size value(s)
    std::string_view text;       // strings
    std::vector<std::string_view> strings;  // arrays of strings (the tokenizer's vocabulary)
};

struct GgufTensorInfo {
    std::string_view name;
    std::vector<uint64_t> shape;  // GGML order: the contiguous dimension first
    uint32_t type = 0;
    uint64_t offset = 0;          // from the data section
    const uint8_t *data = nullptr;
    size_t bytes = 0;
};

class GgufFile {
  public:
    explicit GgufFile(const std::string &path);
    ~GgufFile();
    GgufFile(const GgufFile &) = delete;
    GgufFile &operator=(const GgufFile &) = delete;

    uint32_t version() const {
        return version_;
    }
    const std::vector<GgufTensorInfo> &tensors() const {
        return tensors_;
    }
    const GgufEntry *find(std::string_view key) const;
    const GgufTensorInfo *tensor(std::string_view name) const;

    // Typed lookups; a missing key or a value of the wrong kind throws (gguf.cpp:275-336).
    std::string_view string(std::string_view key) const;
    uint64_t integer(std::string_view key) const;
    double number(std::string_view key) const;

  private:
    void parse_header();       // magic, version, key/values, tensor descriptors
    void place_tensor_data();  // data offset, tensor sizes and bounds
    const GgufEntry &require(std::string_view key) const;

    int fd_ = -1;
    size_t size_ = 0;
    const uint8_t *bytes_ = nullptr;
    size_t header_bytes_ = 0;
    uint32_t version_ = 0;
    std::vector<std::pair<std::string_view, GgufEntry>> entries_;
    std::unordered_map<std::string_view, size_t> entry_index_;
    std::vector<GgufTensorInfo> tensors_;
    std::unordered_map<std::string_view, size_t> tensor_index_;
};

}  // namespace ttlab
