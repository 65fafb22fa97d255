// gguf_index.cpp — the GGUF index: mapping, header scan, tensor-table checks, typed metadata reads.
//
// GGUF (versions 2 and 3), little-endian throughout:
//   "GGUF" u32 version  u64 n_tensors  u64 n_metadata
//   n_metadata x { string key, u32 value_type, value }
//   n_tensors  x { string name, u32 rank, u64 dims[rank], u32 ggml_type, u64 offset }
//   padding to general.alignment (default 32), then the data section; each tensor's bytes lie at
//   its offset from the start of that section, and every offset is a multiple of the alignment.
// A string is a u64 length and that many bytes; an array value is u32 element_type, u64 count,
// then the elements.  Plausibility limits (accepted by every real model file): strings up to
// 2^24 bytes, arrays up to 2^26 elements, at most 100 000 keys or tensors, alignment a power of
// two up to 4096.
#include "gguf_index.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <limits>

namespace ei::gguf {

namespace {

constexpr uint32_t kMagicLE = 0x46554747u;  // the bytes "GGUF" as a little-endian u32
constexpr uint64_t kMaxStringBytes = uint64_t(1) << 24;
constexpr uint64_t kMaxArrayElems = uint64_t(1) << 26;
constexpr uint64_t kMaxRecords = 100000;
constexpr uint64_t kDefaultAlignment = 32;

std::string str(std::string_view v) { return std::string(v); }

// ---- value encodings, indexed by ValueType
enum class Class : uint8_t { Unsigned, Signed, Real, Flag, Text, List, Invalid };

struct Encoding {
    Class cls;
    uint8_t width;  // bytes of one value (a string's length field for Text; 0 for List)
};

constexpr Encoding kEncodings[] = {
    {Class::Unsigned, 1}, {Class::Signed, 1}, {Class::Unsigned, 2}, {Class::Signed, 2},  // U8 I8 U16 I16
    {Class::Unsigned, 4}, {Class::Signed, 4}, {Class::Real, 4},    {Class::Flag, 1},    // U32 I32 F32 BOOL
    {Class::Text, 8},     {Class::List, 0},   {Class::Unsigned, 8}, {Class::Signed, 8}, // STRING ARRAY U64 I64
    {Class::Real, 8},                                                                   // F64
};

Encoding encoding_of(uint32_t type) {
    return type < sizeof(kEncodings) / sizeof(kEncodings[0]) ? kEncodings[type] : Encoding{Class::Invalid, 0};
}

bool integer_class(Class c) { return c == Class::Unsigned || c == Class::Signed || c == Class::Flag; }

// an integer (or bool) value stored at p; values an int64 cannot hold, and bools other than 0/1,
// are format errors
int64_t decode_integer(const uint8_t* p, Encoding e) {
    uint64_t raw = 0;
    std::memcpy(&raw, p, e.width);
    switch (e.cls) {
        case Class::Unsigned:
            if (raw > static_cast<uint64_t>(std::numeric_limits<int64_t>::max()))
                throw FormatError("u64 value does not fit an int64");
            return static_cast<int64_t>(raw);
        case Class::Signed: {
            const unsigned unused = 64u - 8u * e.width;  // sign-extend from the stored width
            return static_cast<int64_t>(raw << unused) >> unused;
        }
        case Class::Flag:
            if (raw > 1) throw FormatError("bool value " + std::to_string(raw) + " is neither 0 nor 1");
            return static_cast<int64_t>(raw);
        default:
            throw FormatError("an integer type was expected");
    }
}

double decode_real(const uint8_t* p, Encoding e) {
    if (e.width == 4) {
        float f;
        std::memcpy(&f, p, 4);
        return f;
    }
    double d;
    std::memcpy(&d, p, 8);
    return d;
}

// ---- block formats, indexed by tensor type id (0 bytes: an id this reader does not know)
struct FormatEntry {
    uint32_t id;
    BlockFormat format;
};

constexpr FormatEntry kFormats[] = {
    {kTF32, {1, 4, "F32"}},        {kTF16, {1, 2, "F16"}},        {kTBF16, {1, 2, "BF16"}},
    {kTQ4_0, {32, 18, "Q4_0"}},    {kTQ4_1, {32, 20, "Q4_1"}},    {kTQ5_0, {32, 22, "Q5_0"}},
    {kTQ5_1, {32, 24, "Q5_1"}},    {kTQ8_0, {32, 34, "Q8_0"}},    {kTQ2_K, {256, 84, "Q2_K"}},
    {kTQ3_K, {256, 110, "Q3_K"}},  {kTQ4_K, {256, 144, "Q4_K"}},  {kTQ5_K, {256, 176, "Q5_K"}},
    {kTQ6_K, {256, 210, "Q6_K"}},
};

// ---- bounds-checked forward scan over the mapping
class Scanner {
public:
    Scanner(const uint8_t* base, uint64_t size) : base_(base), size_(size) {}

    uint64_t pos() const { return pos_; }
    const uint8_t* at(uint64_t offset) const { return base_ + offset; }

    // claims the next n bytes and returns their offset
    uint64_t take(uint64_t n) {
        if (n > size_ - pos_) throw FormatError("file ends early (truncated or corrupt)");
        const uint64_t start = pos_;
        pos_ += n;
        return start;
    }

    uint32_t u32() { return load<uint32_t>(); }
    uint64_t u64() { return load<uint64_t>(); }

    std::string_view string() {
        const uint64_t n = u64();
        if (n > kMaxStringBytes) throw FormatError("string length " + std::to_string(n) + " is not plausible");
        const uint64_t start = take(n);
        return {reinterpret_cast<const char*>(base_ + start), static_cast<size_t>(n)};
    }

private:
    template <class T>
    T load() {
        T v;
        std::memcpy(&v, base_ + take(sizeof(T)), sizeof(T));
        return v;
    }

    const uint8_t* base_;
    uint64_t size_;
    uint64_t pos_ = 0;
};

// Measures (and structurally checks) the value of the given type at the scanner's position.
MetaSlot scan_value(Scanner& s, uint32_t type) {
    MetaSlot m;
    m.type = m.elem_type = type;
    const Encoding e = encoding_of(type);
    switch (e.cls) {
        case Class::Invalid:
            throw FormatError("unknown metadata type " + std::to_string(type));
        case Class::Text:
            m.payload = s.pos();
            s.string();
            break;
        case Class::List: {
            m.elem_type = s.u32();
            m.count = s.u64();
            const Encoding ee = encoding_of(m.elem_type);
            if (ee.cls == Class::Invalid || ee.cls == Class::List)
                throw FormatError("array element type " + std::to_string(m.elem_type) +
                                  " is not supported (nested array?)");
            if (m.count > kMaxArrayElems)
                throw FormatError("array of " + std::to_string(m.count) + " elements is too long");
            m.payload = s.pos();
            if (ee.cls == Class::Text) {
                for (uint64_t k = 0; k < m.count; ++k) s.string();
            } else {
                const uint64_t first = s.take(m.count * ee.width);
                if (ee.cls == Class::Flag || (ee.cls == Class::Unsigned && ee.width == 8))
                    for (uint64_t k = 0; k < m.count; ++k) decode_integer(s.at(first + k * ee.width), ee);
            }
            break;
        }
        default:
            m.payload = s.take(e.width);
            if (integer_class(e.cls)) decode_integer(s.at(m.payload), e);
            break;
    }
    m.span = s.pos() - m.payload;
    return m;
}

}  // namespace

const BlockFormat* block_format(uint32_t tensor_type) {
    for (const FormatEntry& f : kFormats)
        if (f.id == tensor_type) return &f.format;
    return nullptr;
}

// ---------------------------------------------------------------- Index

Index::Index(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw FormatError("cannot open " + path + ": " + std::strerror(errno));
    struct stat st {};
    if (::fstat(fd, &st) != 0) {
        const int err = errno;
        ::close(fd);
        throw FormatError("cannot stat " + path + ": " + std::strerror(err));
    }
    if (st.st_size <= 0) {
        ::close(fd);
        throw FormatError(path + " is empty");
    }
    void* p = ::mmap(nullptr, static_cast<size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
    const int err = errno;
    ::close(fd);  // the mapping holds the file open
    if (p == MAP_FAILED) throw FormatError("cannot map " + path + ": " + std::strerror(err));
    map_ = static_cast<const uint8_t*>(p);
    size_ = static_cast<uint64_t>(st.st_size);
    try {
        scan();
    } catch (...) {
        ::munmap(const_cast<uint8_t*>(map_), static_cast<size_t>(size_));
        throw;
    }
}

Index::~Index() { ::munmap(const_cast<uint8_t*>(map_), static_cast<size_t>(size_)); }

void Index::scan() {
    Scanner s(map_, size_);
    if (s.u32() != kMagicLE) throw FormatError("not a GGUF file (wrong magic)");
    version_ = s.u32();
    if (version_ != 2 && version_ != 3)
        throw FormatError("GGUF version " + std::to_string(version_) + " is not supported");
    const uint64_t n_tensors = s.u64();
    const uint64_t n_meta = s.u64();
    if (n_tensors > kMaxRecords || n_meta > kMaxRecords) throw FormatError("tensor or metadata count is not plausible");

    meta_.reserve(static_cast<size_t>(n_meta));
    for (uint64_t k = 0; k < n_meta; ++k) {
        const std::string_view key = s.string();
        MetaSlot m = scan_value(s, s.u32());
        if (m.type == kString) {
            const uint64_t len = m.span - 8;
            text_pool_.emplace_back(reinterpret_cast<const char*>(map_ + m.payload + 8), static_cast<size_t>(len));
            m.text = static_cast<int>(text_pool_.size() - 1);
        }
        if (!meta_.emplace(key, m).second) throw FormatError("metadata key repeated: " + str(key));
    }

    tensors_.resize(static_cast<size_t>(n_tensors));
    for (TensorSlot& t : tensors_) {
        t.name = str(s.string());
        t.rank = s.u32();
        if (t.rank < 1 || t.rank > 4)
            throw FormatError("tensor " + t.name + " has " + std::to_string(t.rank) + " dimensions");
        for (uint32_t d = 0; d < t.rank; ++d) t.dims[d] = s.u64();
        t.type = s.u32();
        t.data_offset = s.u64();
    }
    check_tensor_records();
    place_tensor_data(s.pos());
}

void Index::check_tensor_records() {
    tensor_names_.reserve(tensors_.size());
    for (size_t i = 0; i < tensors_.size(); ++i) {
        TensorSlot& t = tensors_[i];
        t.elements = 1;
        for (uint32_t d = 0; d < t.rank; ++d)
            if (t.dims[d] == 0 || __builtin_mul_overflow(t.elements, t.dims[d], &t.elements))
                throw FormatError("tensor " + t.name + " has a bad shape");
        const BlockFormat* f = block_format(t.type);
        if (!f) throw FormatError("tensor " + t.name + " has unknown type " + std::to_string(t.type));
        if (t.dims[0] % f->elems != 0)
            throw FormatError("tensor " + t.name + ": row length is not a whole number of blocks");
        if (__builtin_mul_overflow(t.elements / f->elems, uint64_t(f->bytes), &t.bytes))
            throw FormatError("tensor " + t.name + " is too large");
        if (!tensor_names_.emplace(std::string_view(t.name), i).second)
            throw FormatError("tensor name repeated: " + t.name);
    }
}

void Index::place_tensor_data(uint64_t header_end) {
    const int64_t a = integer_or("general.alignment", int64_t(kDefaultAlignment));
    if (a <= 0 || a > 4096 || (a & (a - 1)) != 0)
        throw FormatError("alignment " + std::to_string(a) + " is not valid");
    const uint64_t align = static_cast<uint64_t>(a);
    const uint64_t data_start = (header_end + align - 1) & ~(align - 1);
    if (data_start > size_) throw FormatError("data section lies past the end of the file");
    const uint64_t room = size_ - data_start;
    for (TensorSlot& t : tensors_) {
        if (t.data_offset & (align - 1)) throw FormatError("tensor " + t.name + " is not aligned");
        if (t.data_offset > room || t.bytes > room - t.data_offset)
            throw FormatError("tensor " + t.name + " runs past the end of the file");
        t.data = map_ + data_start + t.data_offset;
    }
}

const TensorSlot* Index::tensor(std::string_view name) const {
    const auto it = tensor_names_.find(name);
    return it == tensor_names_.end() ? nullptr : &tensors_[it->second];
}

const MetaSlot* Index::slot(std::string_view key) const {
    const auto it = meta_.find(key);
    return it == meta_.end() ? nullptr : &it->second;
}

int64_t Index::integer(std::string_view key) const {
    const MetaSlot* m = slot(key);
    if (!m) throw FormatError("metadata missing: " + str(key));
    const Encoding e = encoding_of(m->type);
    if (!integer_class(e.cls)) throw FormatError("metadata is not an integer: " + str(key));
    return decode_integer(map_ + m->payload, e);
}

double Index::number(std::string_view key) const {
    const MetaSlot* m = slot(key);
    if (!m) throw FormatError("metadata missing: " + str(key));
    const Encoding e = encoding_of(m->type);
    if (e.cls == Class::Real) return decode_real(map_ + m->payload, e);
    if (integer_class(e.cls)) return static_cast<double>(decode_integer(map_ + m->payload, e));
    throw FormatError("metadata is not a number: " + str(key));
}

const std::string& Index::text(std::string_view key) const {
    const MetaSlot* m = slot(key);
    if (!m) throw FormatError("metadata missing: " + str(key));
    if (m->type != kString) throw FormatError("metadata is not a string: " + str(key));
    return text_pool_[static_cast<size_t>(m->text)];
}

}  // namespace ei::gguf
