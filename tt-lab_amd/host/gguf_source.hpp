// What the gfx950 facades read from a GGUF file, independent of the file class that
// holds it: ttlab::GgufFile, or the reference's own GgufFile / GgufTensor
// (gguf.h:38-44, 47-85), or any class with the same accessors.
//
//  - TensorRef: one tensor descriptor (name, GGML-order shape, type id, data, bytes).
//    tensor_ref(t) builds it from any struct with `name`, `shape`, `type` and `data`
//    members laid out as the reference's GgufTensor; the byte count follows from the
//    shape and the type (tensor.cpp:136-161).
//  - GgufSource: the metadata and tensor lookups a model loader makes.
//    GgufSourceOf<File> adapts any file class whose find / string / integer / number /
//    tensor accessors have the reference's meaning (gguf.h:67-72): find returns a null
//    pointer for a missing key, the typed lookups throw std::runtime_error, tensor
//    returns a null pointer for a missing tensor.
// Host code only.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string_view>

namespace ttlab {

// Bytes of one row (the first dimension) of a tensor of `type` (tensor.cpp:136-157);
// throws for a type the backend does not read.
size_t gguf_row_bytes(uint32_t type, uint64_t n);

struct TensorRef {
    std::string_view name;
    const uint64_t *shape = nullptr;  // GGML order: the contiguous dimension first
    size_t dims = 0;
    uint32_t type = 0;
    const void *data = nullptr;
    size_t bytes = 0;

    // Extent of dimension d (1 past the rank, as the reference's missing dimensions).
    size_t extent(size_t d) const {
        return d < dims ? size_t(shape[d]) : 1;
    }
};

template <class Tensor>
TensorRef tensor_ref(const Tensor &t) {
    TensorRef r;
    r.name = std::string_view(t.name);
    r.shape = t.shape.data();
    r.dims = t.shape.size();
    r.type = uint32_t(t.type);
    r.data = static_cast<const void *>(t.data);
    size_t bytes = r.dims ? gguf_row_bytes(r.type, r.shape[0]) : 0;
    for (size_t d = 1; d < r.dims; ++d) {
        bytes *= size_t(r.shape[d]);
    }
    r.bytes = bytes;
    return r;
}

class GgufSource {
  public:
    virtual ~GgufSource() = default;
    virtual bool has_key(std::string_view key) const = 0;
    virtual std::string_view string(std::string_view key) const = 0;
    virtual uint64_t integer(std::string_view key) const = 0;
    virtual double number(std::string_view key) const = 0;
    // Fills *out and returns true if the file holds the tensor.
    virtual bool tensor(std::string_view name, TensorRef *out) const = 0;
};

template <class File>
class GgufSourceOf final : public GgufSource {
  public:
    explicit GgufSourceOf(const File &file) : file_(file) {}
    bool has_key(std::string_view key) const override {
        return file_.find(key) != nullptr;
    }
    std::string_view string(std::string_view key) const override {
        return std::string_view(file_.string(key));
    }
    uint64_t integer(std::string_view key) const override {
        return uint64_t(file_.integer(key));
    }
    double number(std::string_view key) const override {
        return double(file_.number(key));
    }
    bool tensor(std::string_view name, TensorRef *out) const override {
        const auto *t = file_.tensor(name);
        if (!t) {
            return false;
        }
        *out = tensor_ref(*t);
        return true;
    }

  private:
    const File &file_;
};

}  // namespace ttlab
