// GGUF v3 reader (see gguf.hpp).
#include "gguf.hpp"

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

// Bounds-checked little-endian reads over the mapping.
class Reader {
  public:
    Reader(const uint8_t *p, size_t n) : base_(p), at_(0), size_(n) {}

    template <class T>
    T get() {
        T v;
        std::memcpy(&v, need(sizeof(T)), sizeof(T));
        return v;
    }
    const uint8_t *need(size_t n) {
        if (n > size_ - at_) {
            fail("truncated GGUF file");
        }
        const uint8_t *p = base_ + at_;
        at_ += n;
        return p;
    }
    std::string_view str() {
        const uint64_t n = get<uint64_t>();
        if (n > size_) {
            fail("GGUF string is too large");
        }
        return {reinterpret_cast<const char *>(need(size_t(n))), size_t(n)};
    }
    size_t pos() const {
        return at_;
    }

  private:
    const uint8_t *base_;
    size_t at_, size_;
};

size_t scalar_width(GgufKind kind) {
    switch (kind) {
    case GgufKind::u8:
    case GgufKind::i8:
    case GgufKind::boolean:
        return 1;
    case GgufKind::u16:
    case GgufKind::i16:
        return 2;
    case GgufKind::u32:
    case GgufKind::i32:
    case GgufKind::f32:
        return 4;
    case GgufKind::u64:
    case GgufKind::i64:
    case GgufKind::f64:
        return 8;
    default:
        fail("GGUF value is not a fixed-size primitive");
    }
}

GgufKind kind_of(Reader &r) {
    const uint32_t raw = r.get<uint32_t>();
    if (raw > uint32_t(GgufKind::f64)) {
        fail("unknown GGUF metadata type " + std::to_string(raw));
    }
    return GgufKind(raw);
}

GgufEntry read_entry(Reader &r, GgufKind kind) {
    GgufEntry e;
    e.kind = kind;
    if (kind == GgufKind::string) {
        e.text = r.str();
        return e;
    }
    if (kind != GgufKind::array) {
        e.raw = r.need(scalar_width(kind));
        return e;
    }
    e.element = kind_of(r);
    e.count = r.get<uint64_t>();
    if (e.element == GgufKind::array) {
        fail("nested GGUF arrays are invalid");
    }
    if (e.element == GgufKind::string) {
        for (uint64_t i = 0; i < e.count; ++i) {
            r.str();  // string arrays (the tokenizer vocabulary) are skipped
        }
        return e;
    }
    const size_t w = scalar_width(e.element);
    if (e.count > SIZE_MAX / w) {
        fail("GGUF array is too large");
    }
    e.raw = r.need(size_t(e.count) * w);
    return e;
}

template <class T>
T value_as(const GgufEntry &e) {
    T v;
    std::memcpy(&v, e.raw, sizeof(T));
    return v;
}

}  // namespace

size_t gguf_row_bytes(uint32_t type, uint64_t n) {
    switch (type) {
    case kGgmlF32:
        return size_t(n) * 4;
    case kGgmlBf16:
        return size_t(n) * 2;
    case kGgmlQ8_0:
        if (n % 32) {
            fail("Q8_0 row is not a multiple of 32");
        }
        return size_t(n / 32) * 34;
    case kGgmlMxfp4:
        if (n % 32) {
            fail("MXFP4 row is not a multiple of 32");
        }
        return size_t(n / 32) * 17;
    default:
        fail("unsupported tensor type " + std::to_string(type));
    }
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
        Reader r(bytes_, size_);
        if (r.get<uint32_t>() != 0x46554747u) {  // "GGUF"
            fail("not a GGUF file");
        }
        version_ = r.get<uint32_t>();
        if (version_ != 3) {
            fail("unsupported GGUF version " + std::to_string(version_));
        }
        const uint64_t ntensors = r.get<uint64_t>();
        const uint64_t nkeys = r.get<uint64_t>();
        if (ntensors > size_ || nkeys > size_) {
            fail("GGUF header counts are too large");
        }
        for (uint64_t i = 0; i < nkeys; ++i) {
            const std::string_view key = r.str();
            GgufEntry e = read_entry(r, kind_of(r));
            if (!entry_index_.emplace(key, entries_.size()).second) {
                fail("duplicate GGUF key: " + std::string(key));
            }
            entries_.emplace_back(key, e);
        }
        for (uint64_t i = 0; i < ntensors; ++i) {
            GgufTensorInfo t;
            t.name = r.str();
            const uint32_t dims = r.get<uint32_t>();
            if (dims == 0 || dims > 4) {
                fail("invalid tensor rank");
            }
            for (uint32_t d = 0; d < dims; ++d) {
                t.shape.push_back(r.get<uint64_t>());
            }
            t.type = r.get<uint32_t>();
            t.offset = r.get<uint64_t>();
            if (!tensor_index_.emplace(t.name, tensors_.size()).second) {
                fail("duplicate tensor: " + std::string(t.name));
            }
            tensors_.push_back(std::move(t));
        }
        uint64_t alignment = 32;
        if (const GgufEntry *a = find("general.alignment")) {
            if (a->kind != GgufKind::u32) {
                fail("general.alignment is not uint32");
            }
            alignment = value_as<uint32_t>(*a);
        }
        if (alignment == 0 || (alignment & (alignment - 1)) != 0) {
            fail("invalid GGUF alignment");
        }
        const uint64_t data = (uint64_t(r.pos()) + alignment - 1) & ~(alignment - 1);
        if (data > size_) {
            fail("GGUF tensor data starts past end of file");
        }
        for (GgufTensorInfo &t : tensors_) {
            if (t.offset > size_ - data) {
                fail("tensor starts past end of GGUF file");
            }
            size_t rows = 1;
            for (size_t d = 1; d < t.shape.size(); ++d) {
                if (t.shape[d] != 0 && rows > SIZE_MAX / t.shape[d]) {
                    fail("tensor " + std::string(t.name) + " is too large");
                }
                rows *= size_t(t.shape[d]);
            }
            const size_t row = gguf_row_bytes(t.type, t.shape[0]);
            if (rows != 0 && row > SIZE_MAX / rows) {
                fail("tensor " + std::string(t.name) + " is too large");
            }
            t.bytes = row * rows;
            if (t.bytes > size_ - data - t.offset) {
                fail("tensor extends past end of GGUF file");
            }
            t.data = bytes_ + data + t.offset;
        }
    } catch (...) {
        munmap(const_cast<uint8_t *>(bytes_), size_);
        close(fd_);
        throw;
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

std::string_view GgufFile::string(std::string_view key) const {
    const GgufEntry *e = find(key);
    if (!e) {
        fail("missing GGUF key: " + std::string(key));
    }
    if (e->kind != GgufKind::string) {
        fail("GGUF key is not a string: " + std::string(key));
    }
    return e->text;
}

uint64_t GgufFile::integer(std::string_view key) const {
    const GgufEntry *e = find(key);
    if (!e) {
        fail("missing GGUF key: " + std::string(key));
    }
    switch (e->kind) {
    case GgufKind::u8:
        return value_as<uint8_t>(*e);
    case GgufKind::i8:
        return uint64_t(int64_t(value_as<int8_t>(*e)));
    case GgufKind::u16:
        return value_as<uint16_t>(*e);
    case GgufKind::i16:
        return uint64_t(int64_t(value_as<int16_t>(*e)));
    case GgufKind::u32:
        return value_as<uint32_t>(*e);
    case GgufKind::i32:
        return uint64_t(int64_t(value_as<int32_t>(*e)));
    case GgufKind::u64:
        return value_as<uint64_t>(*e);
    case GgufKind::i64:
        return uint64_t(value_as<int64_t>(*e));
    default:
        fail("GGUF key is not an integer: " + std::string(key));
    }
}

double GgufFile::number(std::string_view key) const {
    const GgufEntry *e = find(key);
    if (!e) {
        fail("missing GGUF key: " + std::string(key));
    }
    if (e->kind == GgufKind::f32) {
        return value_as<float>(*e);
    }
    if (e->kind == GgufKind::f64) {
        return value_as<double>(*e);
    }
    return double(integer(key));
}

}  // namespace ttlab
