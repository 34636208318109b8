// GGUF v3 reader (see gguf.hpp).
//
// Design: one parser walks the header once.  What it needs to know about a
// metadata value -- how many bytes a scalar occupies, whether it is an integer and
// signed, whether it is a float -- comes from one table indexed by the value kind,
// so scalars, arrays of scalars and the typed accessors all share that table instead
// of a switch per kind.  Tensor descriptors are only collected during the walk;
// their data is placed and bounds-checked in a second pass, once the header's end
// and general.alignment are known.  The format rules and error messages are the
// reference's (gguf.cpp:145-239, 275-336), since callers match on them.
#include "gguf.hpp"

#include <array>
#include <cerrno>
#include <cstring>
#include <fcntl.h>
#include <stdexcept>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace ttlab {
namespace {

[[noreturn]] void fail(const std::string &message) {
    throw std::runtime_error(message);
}

// Per value kind (GgufKind order, gguf.h:13-27): scalar width in bytes (0: not a
// fixed-size scalar), integer, signed, floating point.
struct KindTraits {
    uint8_t width;
    bool integer, is_signed, floating;
};
constexpr std::array<KindTraits, 13> kKinds = {{
    {1, true, false, false},   // u8
    {1, true, true, false},    // i8
    {2, true, false, false},   // u16
    {2, true, true, false},    // i16
    {4, true, false, false},   // u32
    {4, true, true, false},    // i32
    {4, false, false, true},   // f32
    {1, false, false, false},  // bool
    {0, false, false, false},  // string
    {0, false, false, false},  // array
    {8, true, false, false},   // u64
    {8, true, true, false},    // i64
    {8, false, false, true},   // f64
}};

const KindTraits &traits(GgufKind kind) {
    return kKinds[size_t(kind)];
}

// A little-endian scalar of `width` bytes as a 64-bit two's-complement value.
uint64_t widen(const uint8_t *p, const KindTraits &t) {
    uint64_t v = 0;
    for (int i = t.width - 1; i >= 0; --i) {
        v = (v << 8) | p[i];
    }
    if (t.is_signed && t.width < 8 && (v >> (8 * t.width - 1)) & 1) {
        v |= ~uint64_t(0) << (8 * t.width);  // sign extension
    }
    return v;
}

// The header walk: a window [at, end) over the mapping that only ever shrinks from
// the front; every read checks the window first.
class HeaderParser {
  public:
    HeaderParser(const uint8_t *begin, size_t size) : begin_(begin), at_(begin), end_(begin + size) {}

    size_t consumed() const {
        return size_t(at_ - begin_);
    }

    const uint8_t *bytes(uint64_t n) {
        if (n > uint64_t(end_ - at_)) {
            fail("truncated GGUF file");
        }
        const uint8_t *p = at_;
        at_ += n;
        return p;
    }

    template <class T>
    T scalar() {
        T v;
        std::memcpy(&v, bytes(sizeof(T)), sizeof(T));
        return v;
    }

    std::string_view text() {
        const uint64_t n = scalar<uint64_t>();
        if (n > uint64_t(end_ - begin_)) {
            fail("GGUF string is too large");
        }
        return {reinterpret_cast<const char *>(bytes(n)), size_t(n)};
    }

    GgufKind kind() {
        const uint32_t raw = scalar<uint32_t>();
        if (raw >= kKinds.size()) {
            fail("unknown GGUF metadata type " + std::to_string(raw));
        }
        return GgufKind(raw);
    }

    // One metadata value of `kind`: scalars and arrays of scalars keep a pointer to
    // their bytes in the mapping; strings and the elements of string arrays (the
    // tokenizer's vocabulary and merges) views into it.
    GgufEntry value(GgufKind kind) {
        GgufEntry e;
        e.kind = kind;
        if (kind == GgufKind::string) {
            e.text = text();
        } else if (kind != GgufKind::array) {
            e.raw = bytes(traits(kind).width);
        } else {
            e.element = this->kind();
            e.count = scalar<uint64_t>();
            if (e.element == GgufKind::array) {
                fail("nested GGUF arrays are invalid");
            }
            if (e.element == GgufKind::string) {
                if (e.count > uint64_t(end_ - at_) / sizeof(uint64_t)) {
                    fail("GGUF string array is too large");
                }
                e.strings.reserve(size_t(e.count));
                for (uint64_t i = 0; i < e.count; ++i) {
                    e.strings.push_back(text());
                }
            } else {
                const uint64_t w = traits(e.element).width;
                if (e.count > uint64_t(end_ - at_) / w) {
                    fail("GGUF array is too large");
                }
                e.raw = bytes(e.count * w);
            }
        }
        return e;
    }

  private:
    const uint8_t *begin_, *at_, *end_;
};

}  // namespace

size_t gguf_row_bytes(uint32_t type, uint64_t n) {
    // elements per block and bytes per block of each supported type (tensor.cpp:136-157)
    uint64_t per = 1, block = 0;
    const char *name = nullptr;
    if (type == kGgmlF32) {
        block = 4;
    } else if (type == kGgmlBf16) {
        block = 2;
    } else if (type == kGgmlQ8_0) {
        per = 32, block = 34, name = "Q8_0";
    } else if (type == kGgmlMxfp4) {
        per = 32, block = 17, name = "MXFP4";
    } else {
        fail("unsupported tensor type " + std::to_string(type));
    }
    if (n % per) {
        fail(std::string(name) + " row is not a multiple of 32");
    }
    return size_t(n / per * block);
}

GgufFile::GgufFile(const std::string &path) {
    fd_ = open(path.c_str(), O_RDONLY);
    if (fd_ < 0) {
        fail("cannot open " + path + ": " + std::strerror(errno));
    }
    struct stat st {};
    if (fstat(fd_, &st) != 0) {
        const std::string why = std::strerror(errno);
        close(fd_);
        fail("cannot stat " + path + ": " + why);
    }
    size_ = size_t(st.st_size);
    void *map = size_ ? mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0) : MAP_FAILED;
    if (map == MAP_FAILED) {
        const std::string why = size_ ? std::strerror(errno) : "empty file";
        close(fd_);
        fail("cannot mmap " + path + ": " + why);
    }
    bytes_ = static_cast<const uint8_t *>(map);
    try {
        parse_header();
        place_tensor_data();
    } catch (...) {
        munmap(const_cast<uint8_t *>(bytes_), size_);
        close(fd_);
        throw;
    }
}

// Pass 1: magic, version, counts, the key/value table and the tensor descriptors.
void GgufFile::parse_header() {
    HeaderParser p(bytes_, size_);
    if (p.scalar<uint32_t>() != 0x46554747u) {  // the bytes "GGUF"
        fail("not a GGUF file");
    }
    version_ = p.scalar<uint32_t>();
    if (version_ != 3) {
        fail("unsupported GGUF version " + std::to_string(version_));
    }
    const uint64_t tensor_count = p.scalar<uint64_t>();
    const uint64_t key_count = p.scalar<uint64_t>();
    if (tensor_count > size_ || key_count > size_) {
        fail("GGUF header counts are too large");
    }
    for (uint64_t i = 0; i < key_count; ++i) {
        const std::string_view key = p.text();
        const GgufKind kind = p.kind();
        if (!entry_index_.emplace(key, entries_.size()).second) {
            fail("duplicate GGUF key: " + std::string(key));
        }
        entries_.emplace_back(key, p.value(kind));
    }
    tensors_.resize(size_t(tensor_count));
    for (uint64_t i = 0; i < tensor_count; ++i) {
        GgufTensorInfo &t = tensors_[size_t(i)];
        t.name = p.text();
        const uint32_t rank = p.scalar<uint32_t>();
        if (rank == 0 || rank > 4) {
            fail("invalid tensor rank");
        }
        t.shape.resize(rank);
        for (uint64_t &extent : t.shape) {
            extent = p.scalar<uint64_t>();
        }
        t.type = p.scalar<uint32_t>();
        t.offset = p.scalar<uint64_t>();
        if (!tensor_index_.emplace(t.name, size_t(i)).second) {
            fail("duplicate tensor: " + std::string(t.name));
        }
    }
    header_bytes_ = p.consumed();
}

// Pass 2: the data section starts at the header's end rounded up to
// general.alignment (default 32); every tensor's bytes must lie inside the file.
void GgufFile::place_tensor_data() {
    uint64_t alignment = 32;
    if (const GgufEntry *a = find("general.alignment")) {
        if (a->kind != GgufKind::u32) {
            fail("general.alignment is not uint32");
        }
        alignment = widen(a->raw, traits(a->kind));
    }
    if (alignment == 0 || (alignment & (alignment - 1)) != 0) {
        fail("invalid GGUF alignment");
    }
    const uint64_t data = (uint64_t(header_bytes_) + alignment - 1) & ~(alignment - 1);
    if (data > size_) {
        fail("GGUF tensor data starts past end of file");
    }
    const uint64_t room = size_ - data;
    for (GgufTensorInfo &t : tensors_) {
        if (t.offset > room) {
            fail("tensor starts past end of GGUF file");
        }
        // bytes = row bytes x the product of the other extents, without overflow
        uint64_t total = gguf_row_bytes(t.type, t.shape[0]);
        for (size_t d = 1; d < t.shape.size(); ++d) {
            if (t.shape[d] != 0 && total > UINT64_MAX / t.shape[d]) {
                fail("tensor " + std::string(t.name) + " is too large");
            }
            total *= t.shape[d];
        }
        if (total > room - t.offset) {
            fail("tensor extends past end of GGUF file");
        }
        t.bytes = size_t(total);
        t.data = bytes_ + data + t.offset;
    }
}

GgufFile::~GgufFile() {
    munmap(const_cast<uint8_t *>(bytes_), size_);
    close(fd_);
}

const GgufEntry *GgufFile::find(std::string_view key) const {
    const auto it = entry_index_.find(key);
    return it == entry_index_.end() ? nullptr : &entries_[it->second].second;
}

const GgufTensorInfo *GgufFile::tensor(std::string_view name) const {
    const auto it = tensor_index_.find(name);
    return it == tensor_index_.end() ? nullptr : &tensors_[it->second];
}

const GgufEntry &GgufFile::require(std::string_view key) const {
    const GgufEntry *e = find(key);
    if (!e) {
        fail("missing GGUF key: " + std::string(key));
    }
    return *e;
}

std::string_view GgufFile::string(std::string_view key) const {
    const GgufEntry &e = require(key);
    if (e.kind != GgufKind::string) {
        fail("GGUF key is not a string: " + std::string(key));
    }
    return e.text;
}

uint64_t GgufFile::integer(std::string_view key) const {
    const GgufEntry &e = require(key);
    const KindTraits &t = traits(e.kind);
    if (!t.integer) {
        fail("GGUF key is not an integer: " + std::string(key));
    }
    return widen(e.raw, t);
}

double GgufFile::number(std::string_view key) const {
    const GgufEntry &e = require(key);
    if (e.kind == GgufKind::f32) {
        float v;
        std::memcpy(&v, e.raw, sizeof v);
        return v;
    }
    if (e.kind == GgufKind::f64) {
        double v;
        std::memcpy(&v, e.raw, sizeof v);
        return v;
    }
    const KindTraits &t = traits(e.kind);
    if (!t.integer) {
        fail("GGUF key is not an integer: " + std::string(key));
    }
    const uint64_t v = widen(e.raw, t);
    return t.is_signed ? double(int64_t(v)) : double(v);
}

}  // namespace ttlab
