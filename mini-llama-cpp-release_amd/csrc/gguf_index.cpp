// GGUF v3 index over a read-only mapping (see gguf_index.h).  The checks and
// messages restate GGUFReader::load (src/gguf.cpp:371-530) and its helpers
// (value rendering src/gguf.cpp:219-345, sizes :160-205, alignment :347-366);
// reads are bounds-checked against the mapping instead of going through a
// stream, so a read past the end fails where the reference's stream read fails.
#include "gguf_index.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <unordered_set>

namespace mlq {

namespace {

// Limits of the reference reader (src/gguf.cpp:51-58).
constexpr uint64_t kDefaultAlignment = 32;
constexpr uint64_t kMaxAlignment = 1024 * 1024;
constexpr uint64_t kMaxStringBytes = 16 * 1024 * 1024;
constexpr uint64_t kMaxMetadataEntries = 1000000;
constexpr uint64_t kMaxTensorEntries = 1000000;
constexpr uint64_t kMaxArrayElements = 10000000;
constexpr uint32_t kMaxTensorDims = 8;
constexpr uint64_t kQuantElems = 32;

enum : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

// Little-endian reader over [p, p + size).
struct Cursor {
    const uint8_t* p;
    uint64_t size;
    uint64_t pos = 0;

    template <typename T>
    bool get(T& v) {
        if (size - pos < sizeof(T)) return false;
        std::memcpy(&v, p + pos, sizeof(T));
        pos += sizeof(T);
        return true;
    }
    bool skip(uint64_t n) {
        if (size - pos < n) return false;
        pos += n;
        return true;
    }
    bool str(std::string& s) {
        uint64_t len = 0;
        if (!get(len) || len > kMaxStringBytes || size - pos < len) return false;
        s.assign(reinterpret_cast<const char*>(p + pos), static_cast<size_t>(len));
        pos += len;
        return true;
    }
};

// Bytes of a fixed-size scalar value type, 0 for the others.
uint64_t scalar_bytes(uint32_t type) {
    switch (type) {
        case kU8: case kI8: case kBool: return 1;
        case kU16: case kI16: return 2;
        case kU32: case kI32: case kF32: return 4;
        case kU64: case kI64: case kF64: return 8;
        default: return 0;
    }
}

bool skip_value(Cursor& c, uint32_t type) {
    if (const uint64_t n = scalar_bytes(type)) return c.skip(n);
    if (type == kString) {
        std::string s;
        return c.str(s);
    }
    if (type == kArray) {
        uint32_t elem = 0;
        uint64_t len = 0;
        if (!c.get(elem) || !c.get(len) || len > kMaxArrayElements) return false;
        for (uint64_t i = 0; i < len; ++i) {
            if (!skip_value(c, elem)) return false;
        }
        return true;
    }
    return false;
}

template <typename T, typename Shown = T>
bool render(Cursor& c, std::ostringstream& os) {
    T v{};
    if (!c.get(v)) return false;
    os << static_cast<Shown>(v);
    return true;
}

bool render_value(Cursor& c, uint32_t type, std::string& out) {
    std::ostringstream os;
    bool ok = false;
    switch (type) {
        case kU8: ok = render<uint8_t, unsigned>(c, os); break;
        case kI8: ok = render<int8_t, int>(c, os); break;
        case kU16: ok = render<uint16_t>(c, os); break;
        case kI16: ok = render<int16_t>(c, os); break;
        case kU32: ok = render<uint32_t>(c, os); break;
        case kI32: ok = render<int32_t>(c, os); break;
        case kF32: ok = render<float>(c, os); break;
        case kU64: ok = render<uint64_t>(c, os); break;
        case kI64: ok = render<int64_t>(c, os); break;
        case kF64: ok = render<double>(c, os); break;
        case kBool: {
            uint8_t v = 0;
            ok = c.get(v);
            if (ok) os << (v ? "true" : "false");
            break;
        }
        case kString:
            return c.str(out);
        case kArray: {
            uint32_t elem = 0;
            uint64_t len = 0;
            if (!c.get(elem) || !c.get(len) || len > kMaxArrayElements) return false;
            os << "[" << len << " x " << gguf_value_label(elem) << "]";
            for (uint64_t i = 0; i < len; ++i) {
                if (!skip_value(c, elem)) return false;
            }
            ok = true;
            break;
        }
        default:
            return false;
    }
    if (ok) out = os.str();
    return ok;
}

bool mul_ok(uint64_t a, uint64_t b, uint64_t& out) {
    if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) return false;
    out = a * b;
    return true;
}

bool add_ok(uint64_t a, uint64_t b, uint64_t& out) {
    if (b > std::numeric_limits<uint64_t>::max() - a) return false;
    out = a + b;
    return true;
}

// Data bytes of a tensor; false when the element count overflows or a block
// type's count is not a whole number of blocks.  Unknown types have size 0.
bool data_bytes(const GgufTensor& t, uint64_t& out) {
    uint64_t n = 1;
    for (uint64_t d : t.dims) {
        if (d == 0 || !mul_ok(n, d, n)) return false;
    }
    uint64_t block = 0;
    switch (t.type) {
        case kGgmlF32: return mul_ok(n, 4, out);
        case kGgmlF16: return mul_ok(n, 2, out);
        case kGgmlQ4_0: block = 18; break;
        case kGgmlQ4_1: block = 20; break;
        case kGgmlQ8_0: block = 34; break;
        default:
            out = 0;
            return true;
    }
    if (n % kQuantElems != 0) return false;
    return mul_ok(n / kQuantElems, block, out);
}

// general.alignment as the reference reads it: the rendered value must parse
// whole as an unsigned integer, be a power of two and at most 1 MiB; 0 marks
// an invalid value.
uint64_t alignment_of(const std::vector<GgufMeta>& meta) {
    uint64_t a = kDefaultAlignment;
    for (const GgufMeta& m : meta) {
        if (m.key != "general.alignment") continue;
        try {
            size_t used = 0;
            a = std::stoull(m.value, &used);
            if (used != m.value.size()) return 0;
        } catch (const std::exception&) {
            return 0;
        }
    }
    if (a == 0 || a > kMaxAlignment || (a & (a - 1)) != 0) return 0;
    return a;
}

}  // namespace

const char* ggml_type_label(uint32_t type) {
    switch (type) {
        case kGgmlF32: return "F32";
        case kGgmlF16: return "F16";
        case kGgmlQ4_0: return "Q4_0";
        case kGgmlQ4_1: return "Q4_1";
        case kGgmlQ8_0: return "Q8_0";
        default: return "UNKNOWN";
    }
}

const char* gguf_value_label(uint32_t type) {
    static const char* const names[] = {"uint8", "int8", "uint16", "int16", "uint32", "int32", "float32",
                                        "bool", "string", "array", "uint64", "int64", "float64"};
    return type <= kF64 ? names[type] : "unknown";
}

GgufIndex::~GgufIndex() { unmap(); }

void GgufIndex::unmap() {
    if (base_ != nullptr) munmap(const_cast<uint8_t*>(base_), size_);
    base_ = nullptr;
    size_ = 0;
}

bool GgufIndex::open(const std::string& path) {
    unmap();
    version = 0;
    n_tensors = n_metadata = data_offset = 0;
    metadata.clear();
    tensors.clear();
    error.clear();

    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        error = "failed to open: " + path;
        return false;
    }
    struct stat st {};
    if (fstat(fd, &st) == 0 && S_ISREG(st.st_mode) && st.st_size > 0) {
        void* m = mmap(nullptr, static_cast<size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
        if (m != MAP_FAILED) {
            base_ = static_cast<const uint8_t*>(m);
            size_ = static_cast<uint64_t>(st.st_size);
        }
    }
    ::close(fd);
    if (base_ == nullptr && S_ISREG(st.st_mode) && st.st_size > 0) {
        error = "failed to open: " + path;
        return false;
    }

    Cursor c{base_, size_};
    if (size_ < 4 || std::memcmp(base_, "GGUF", 4) != 0) {
        error = "invalid GGUF magic";
        return false;
    }
    c.pos = 4;
    if (!c.get(version)) {
        error = "failed to read version";
        return false;
    }
    if (version != 3) {
        error = "unsupported GGUF version: " + std::to_string(version);
        return false;
    }
    if (!c.get(n_tensors) || !c.get(n_metadata)) {
        error = "failed to read header counts";
        return false;
    }
    if (n_tensors > kMaxTensorEntries) {
        error = "too many tensors: " + std::to_string(n_tensors);
        return false;
    }
    if (n_metadata > kMaxMetadataEntries) {
        error = "too many metadata entries: " + std::to_string(n_metadata);
        return false;
    }

    std::unordered_set<std::string> keys;
    metadata.reserve(n_metadata);
    for (uint64_t i = 0; i < n_metadata; ++i) {
        GgufMeta m;
        if (!c.str(m.key)) {
            error = "failed to read metadata key at index " + std::to_string(i);
            return false;
        }
        if (!keys.insert(m.key).second) {
            error = "duplicate metadata key: " + m.key;
            return false;
        }
        if (!c.get(m.type)) {
            error = "failed to read metadata type for key: " + m.key;
            return false;
        }
        m.value_pos = c.pos;
        if (!render_value(c, m.type, m.value)) {
            error = "failed to read metadata value for key: " + m.key;
            return false;
        }
        metadata.push_back(std::move(m));
    }

    tensors.reserve(n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
        GgufTensor t;
        if (!c.str(t.name)) {
            error = "failed to read tensor name at index " + std::to_string(i);
            return false;
        }
        uint32_t nd = 0;
        if (!c.get(nd)) {
            error = "failed to read tensor n_dims for: " + t.name;
            return false;
        }
        if (nd == 0 || nd > kMaxTensorDims) {
            error = "invalid tensor n_dims for: " + t.name;
            return false;
        }
        t.dims.resize(nd);
        for (uint32_t d = 0; d < nd; ++d) {
            if (!c.get(t.dims[d])) {
                error = "failed to read tensor shape for: " + t.name;
                return false;
            }
            if (t.dims[d] == 0) {
                error = "invalid zero tensor dimension for: " + t.name;
                return false;
            }
        }
        if (!c.get(t.type)) {
            error = "failed to read tensor type for: " + t.name;
            return false;
        }
        if (!c.get(t.offset)) {
            error = "failed to read tensor offset for: " + t.name;
            return false;
        }
        tensors.push_back(std::move(t));
    }
    std::unordered_set<std::string> names;
    for (const GgufTensor& t : tensors) {
        if (!names.insert(t.name).second) {
            error = "duplicate tensor name: " + t.name;
            return false;
        }
    }

    const uint64_t align = alignment_of(metadata);
    if (align == 0) {
        error = "invalid general.alignment";
        return false;
    }
    data_offset = c.pos + (align - c.pos % align) % align;
    if (size_ < data_offset) {
        error = "GGUF file ended before tensor data section";
        return false;
    }
    for (GgufTensor& t : tensors) {
        if (!data_bytes(t, t.nbytes)) {
            error = "invalid tensor data size for: " + t.name;
            return false;
        }
        if (t.nbytes == 0) continue;
        uint64_t start = 0, end = 0;
        if (!add_ok(data_offset, t.offset, start)) {
            error = "tensor offset overflow for: " + t.name;
            return false;
        }
        if (!add_ok(start, t.nbytes, end)) {
            error = "tensor data range overflow for: " + t.name;
            return false;
        }
        if (end > size_) {
            error = "tensor data outside file bounds: " + t.name;
            return false;
        }
    }
    return true;
}

const uint8_t* GgufIndex::tensor_data(const GgufTensor& t) const {
    if (t.nbytes == 0 || base_ == nullptr) return nullptr;
    return base_ + data_offset + t.offset;
}

namespace {

const GgufMeta* meta_of(const std::vector<GgufMeta>& meta, const std::string& key) {
    for (const GgufMeta& m : meta) {
        if (m.key == key) return &m;
    }
    return nullptr;
}

template <typename T>
T read_at(const uint8_t* base, uint64_t pos) {
    T v;
    std::memcpy(&v, base + pos, sizeof(T));
    return v;
}

}  // namespace

bool GgufIndex::get_int(const std::string& key, int64_t& out) const {
    const GgufMeta* m = meta_of(metadata, key);
    if (m == nullptr) return false;
    const uint64_t p = m->value_pos;
    switch (m->type) {
        case kU8: out = read_at<uint8_t>(base_, p); return true;
        case kI8: out = read_at<int8_t>(base_, p); return true;
        case kU16: out = read_at<uint16_t>(base_, p); return true;
        case kI16: out = read_at<int16_t>(base_, p); return true;
        case kU32: out = read_at<uint32_t>(base_, p); return true;
        case kI32: out = read_at<int32_t>(base_, p); return true;
        case kU64: out = static_cast<int64_t>(read_at<uint64_t>(base_, p)); return true;
        case kI64: out = read_at<int64_t>(base_, p); return true;
        default: return false;
    }
}

bool GgufIndex::get_float(const std::string& key, double& out) const {
    const GgufMeta* m = meta_of(metadata, key);
    if (m == nullptr) return false;
    if (m->type == kF32) {
        out = static_cast<double>(read_at<float>(base_, m->value_pos));
        return true;
    }
    if (m->type == kF64) {
        out = read_at<double>(base_, m->value_pos);
        return true;
    }
    return false;
}

bool GgufIndex::get_string(const std::string& key, std::string& out) const {
    const GgufMeta* m = meta_of(metadata, key);
    if (m == nullptr || m->type != kString) return false;
    out = m->value;
    return true;
}

bool GgufIndex::get_string_array_size(const std::string& key, uint64_t& out) const {
    const GgufMeta* m = meta_of(metadata, key);
    if (m == nullptr || m->type != kArray) return false;
    if (read_at<uint32_t>(base_, m->value_pos) != kString) return false;
    out = read_at<uint64_t>(base_, m->value_pos + 4);
    return true;
}

int64_t GgufIndex::find(const std::string& name) const {
    for (size_t i = 0; i < tensors.size(); ++i) {
        if (tensors[i].name == name) return static_cast<int64_t>(i);
    }
    return -1;
}

}  // namespace mlq
