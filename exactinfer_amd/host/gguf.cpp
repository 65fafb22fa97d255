// gguf.cpp — GGUF reader over POSIX mmap; the Qwen3 configuration and tensor table.
// Layout of a GGUF file (versions 2 and 3): magic "GGUF", u32 version, u64 tensor count, u64
// metadata count, the metadata pairs (string key, u32 type, value), the tensor infos (string
// name, u32 n_dims, u64 dims[n_dims], u32 type, u64 offset), then the data section, aligned to
// general.alignment (default 32), holding each tensor at its offset.  Strings are a u64 length
// and that many bytes.  The limits below (string and array lengths, counts, dims, alignment) are
// the reference reader's (src/gguf.cpp:203-254), so the two accept and reject the same files.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <limits>

namespace ei {

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read as a little-endian u32
constexpr uint64_t kMaxString = 1ull << 24;
constexpr uint64_t kMaxArray = 1ull << 26;
constexpr uint64_t kMaxCount = 100000;

struct Layout {
    uint32_t block;  // elements per block
    uint32_t bytes;  // bytes per block
    const char* name;
};

bool layout_of(uint32_t t, Layout* l) {
    switch (static_cast<GgmlType>(t)) {
        case GgmlType::F32: *l = {1, 4, "F32"}; return true;
        case GgmlType::F16: *l = {1, 2, "F16"}; return true;
        case GgmlType::BF16: *l = {1, 2, "BF16"}; return true;
        case GgmlType::Q4_0: *l = {32, 18, "Q4_0"}; return true;
        case GgmlType::Q4_1: *l = {32, 20, "Q4_1"}; return true;
        case GgmlType::Q5_0: *l = {32, 22, "Q5_0"}; return true;
        case GgmlType::Q5_1: *l = {32, 24, "Q5_1"}; return true;
        case GgmlType::Q8_0: *l = {32, 34, "Q8_0"}; return true;
        case GgmlType::Q2_K: *l = {256, 84, "Q2_K"}; return true;
        case GgmlType::Q3_K: *l = {256, 110, "Q3_K"}; return true;
        case GgmlType::Q4_K: *l = {256, 144, "Q4_K"}; return true;
        case GgmlType::Q5_K: *l = {256, 176, "Q5_K"}; return true;
        case GgmlType::Q6_K: *l = {256, 210, "Q6_K"}; return true;
    }
    return false;
}

bool checked_mul(uint64_t a, uint64_t b, uint64_t* out) {
    return !__builtin_mul_overflow(a, b, out);
}

// sequential reader over the mapping; every read is bounds-checked
class Cursor {
public:
    Cursor(const uint8_t* base, uint64_t size) : base_(base), size_(size) {}
    uint64_t offset() const { return at_; }
    void require(uint64_t n) const {
        if (n > size_ - at_) throw GgufError("file ends early (truncated or corrupt)");
    }
    template <class T>
    T read() {
        require(sizeof(T));
        T v;
        std::memcpy(&v, base_ + at_, sizeof(T));
        at_ += sizeof(T);
        return v;
    }
    std::string string() {
        const uint64_t n = read<uint64_t>();
        if (n > kMaxString) throw GgufError("string length " + std::to_string(n) + " is not plausible");
        require(n);
        std::string s(reinterpret_cast<const char*>(base_ + at_), static_cast<size_t>(n));
        at_ += n;
        return s;
    }

private:
    const uint8_t* base_;
    uint64_t size_;
    uint64_t at_ = 0;
};

bool integral(GgufType t) {
    return t == GgufType::U8 || t == GgufType::I8 || t == GgufType::U16 || t == GgufType::I16 || t == GgufType::U32 ||
           t == GgufType::I32 || t == GgufType::U64 || t == GgufType::I64 || t == GgufType::BOOL;
}

int64_t read_integer(Cursor& c, GgufType t) {
    switch (t) {
        case GgufType::U8: return c.read<uint8_t>();
        case GgufType::I8: return c.read<int8_t>();
        case GgufType::U16: return c.read<uint16_t>();
        case GgufType::I16: return c.read<int16_t>();
        case GgufType::U32: return c.read<uint32_t>();
        case GgufType::I32: return c.read<int32_t>();
        case GgufType::I64: return c.read<int64_t>();
        case GgufType::U64: {
            const uint64_t v = c.read<uint64_t>();
            if (v > static_cast<uint64_t>(std::numeric_limits<int64_t>::max()))
                throw GgufError("u64 value does not fit an int64");
            return static_cast<int64_t>(v);
        }
        case GgufType::BOOL: {
            const uint8_t b = c.read<uint8_t>();
            if (b > 1) throw GgufError("bool value " + std::to_string(b) + " is neither 0 nor 1");
            return b;
        }
        default: throw GgufError("an integer type was expected");
    }
}

// minimum bytes of one array element (a string's length field), 0 for types an array may not hold
uint64_t min_element_bytes(GgufType t) {
    switch (t) {
        case GgufType::U8: case GgufType::I8: case GgufType::BOOL: return 1;
        case GgufType::U16: case GgufType::I16: return 2;
        case GgufType::U32: case GgufType::I32: case GgufType::F32: return 4;
        case GgufType::U64: case GgufType::I64: case GgufType::F64: case GgufType::STRING: return 8;
        default: return 0;
    }
}

GgufValue read_value(Cursor& c, GgufType t) {
    GgufValue v;
    v.type = t;
    if (integral(t)) {
        v.i = read_integer(c, t);
        v.f = static_cast<double>(v.i);
        return v;
    }
    switch (t) {
        case GgufType::F32: v.f = c.read<float>(); return v;
        case GgufType::F64: v.f = c.read<double>(); return v;
        case GgufType::STRING: v.s = c.string(); return v;
        case GgufType::ARRAY: {
            v.elem = static_cast<GgufType>(c.read<uint32_t>());
            const uint64_t n = c.read<uint64_t>();
            const uint64_t eb = min_element_bytes(v.elem);
            if (eb == 0) throw GgufError("array element type " + std::to_string(static_cast<uint32_t>(v.elem)) +
                                         " is not supported (nested array?)");
            if (n > kMaxArray) throw GgufError("array of " + std::to_string(n) + " elements is too long");
            c.require(n * eb);  // the file must hold at least this much before anything is allocated
            if (v.elem == GgufType::STRING) {
                v.as.reserve(static_cast<size_t>(n));
                for (uint64_t k = 0; k < n; ++k) v.as.push_back(c.string());
            } else if (v.elem == GgufType::F32 || v.elem == GgufType::F64) {
                v.af.reserve(static_cast<size_t>(n));
                for (uint64_t k = 0; k < n; ++k)
                    v.af.push_back(v.elem == GgufType::F32 ? static_cast<double>(c.read<float>()) : c.read<double>());
            } else {
                v.ai.reserve(static_cast<size_t>(n));
                for (uint64_t k = 0; k < n; ++k) v.ai.push_back(read_integer(c, v.elem));
            }
            return v;
        }
        default: throw GgufError("unknown metadata type " + std::to_string(static_cast<uint32_t>(t)));
    }
}

}  // namespace

const char* ggml_type_name(GgmlType t) {
    Layout l;
    return layout_of(static_cast<uint32_t>(t), &l) ? l.name : "?";
}

GgufFile::GgufFile(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw GgufError("cannot open " + path + ": " + std::strerror(errno));
    struct stat st;
    if (::fstat(fd, &st) != 0) {
        const int e = errno;
        ::close(fd);
        throw GgufError("cannot stat " + path + ": " + std::strerror(e));
    }
    size_ = static_cast<uint64_t>(st.st_size);
    if (size_ == 0) {
        ::close(fd);
        throw GgufError(path + " is empty");
    }
    void* p = ::mmap(nullptr, static_cast<size_t>(size_), PROT_READ, MAP_PRIVATE, fd, 0);
    const int e = errno;
    ::close(fd);  // the mapping keeps the file
    if (p == MAP_FAILED) throw GgufError("cannot map " + path + ": " + std::strerror(e));
    map_ = static_cast<const uint8_t*>(p);
    try {
        Cursor c(map_, size_);
        if (c.read<uint32_t>() != kMagic) throw GgufError("not a GGUF file (wrong magic)");
        version_ = c.read<uint32_t>();
        if (version_ != 2 && version_ != 3) throw GgufError("GGUF version " + std::to_string(version_) + " is not supported");
        const uint64_t n_tensors = c.read<uint64_t>();
        const uint64_t n_kv = c.read<uint64_t>();
        if (n_tensors > kMaxCount || n_kv > kMaxCount) throw GgufError("tensor or metadata count is not plausible");

        for (uint64_t k = 0; k < n_kv; ++k) {
            std::string key = c.string();
            const auto t = static_cast<GgufType>(c.read<uint32_t>());
            GgufValue v = read_value(c, t);
            if (!meta_.emplace(key, std::move(v)).second) throw GgufError("metadata key repeated: " + key);
        }

        std::vector<uint64_t> offsets;
        offsets.reserve(static_cast<size_t>(n_tensors));
        tensors_.reserve(static_cast<size_t>(n_tensors));
        for (uint64_t k = 0; k < n_tensors; ++k) {
            GgufTensor t;
            t.name = c.string();
            const uint32_t nd = c.read<uint32_t>();
            if (nd == 0 || nd > 4) throw GgufError("tensor " + t.name + " has " + std::to_string(nd) + " dimensions");
            t.numel = 1;
            for (uint32_t d = 0; d < nd; ++d) {
                const uint64_t n = c.read<uint64_t>();
                if (n == 0 || !checked_mul(t.numel, n, &t.numel)) throw GgufError("tensor " + t.name + " has a bad shape");
                t.ne.push_back(n);
            }
            const uint32_t ty = c.read<uint32_t>();
            Layout l;
            if (!layout_of(ty, &l)) throw GgufError("tensor " + t.name + " has unknown type " + std::to_string(ty));
            t.type = static_cast<GgmlType>(ty);
            if (t.ne[0] % l.block != 0) throw GgufError("tensor " + t.name + ": row length is not a whole number of blocks");
            if (!checked_mul(t.numel / l.block, l.bytes, &t.nbytes)) throw GgufError("tensor " + t.name + " is too large");
            offsets.push_back(c.read<uint64_t>());
            if (!by_name_.emplace(t.name, tensors_.size()).second) throw GgufError("tensor name repeated: " + t.name);
            tensors_.push_back(std::move(t));
        }

        const int64_t a = get_int_or("general.alignment", 32);
        if (a <= 0 || a > 4096 || (a & (a - 1)) != 0) throw GgufError("alignment " + std::to_string(a) + " is not valid");
        const uint64_t align = static_cast<uint64_t>(a);
        const uint64_t data_start = (c.offset() + align - 1) / align * align;
        if (data_start > size_) throw GgufError("data section lies past the end of the file");
        const uint64_t data_bytes = size_ - data_start;
        for (size_t k = 0; k < tensors_.size(); ++k) {
            GgufTensor& t = tensors_[k];
            const uint64_t off = offsets[k];
            if (off % align != 0) throw GgufError("tensor " + t.name + " is not aligned");
            if (off > data_bytes || t.nbytes > data_bytes - off) throw GgufError("tensor " + t.name + " runs past the end of the file");
            t.data = map_ + data_start + off;
        }
    } catch (...) {
        ::munmap(const_cast<uint8_t*>(map_), static_cast<size_t>(size_));
        map_ = nullptr;
        throw;
    }
}

GgufFile::~GgufFile() {
    if (map_) ::munmap(const_cast<uint8_t*>(map_), static_cast<size_t>(size_));
}

const GgufValue* GgufFile::find(const std::string& key) const {
    const auto it = meta_.find(key);
    return it == meta_.end() ? nullptr : &it->second;
}

const GgufTensor* GgufFile::tensor(const std::string& name) const {
    const auto it = by_name_.find(name);
    return it == by_name_.end() ? nullptr : &tensors_[it->second];
}

const GgufTensor& GgufFile::require_tensor(const std::string& name) const {
    if (const GgufTensor* t = tensor(name)) return *t;
    throw GgufError("tensor missing: " + name);
}

int64_t GgufFile::get_int(const std::string& key) const {
    const GgufValue* v = find(key);
    if (!v) throw GgufError("metadata missing: " + key);
    if (!integral(v->type)) throw GgufError("metadata is not an integer: " + key);
    return v->i;
}

double GgufFile::get_float(const std::string& key) const {
    const GgufValue* v = find(key);
    if (!v) throw GgufError("metadata missing: " + key);
    if (v->type != GgufType::F32 && v->type != GgufType::F64 && !integral(v->type))
        throw GgufError("metadata is not a number: " + key);
    return v->f;
}

const std::string& GgufFile::get_str(const std::string& key) const {
    const GgufValue* v = find(key);
    if (!v) throw GgufError("metadata missing: " + key);
    if (v->type != GgufType::STRING) throw GgufError("metadata is not a string: " + key);
    return v->s;
}

int64_t GgufFile::get_int_or(const std::string& key, int64_t def) const { return find(key) ? get_int(key) : def; }

double GgufFile::get_float_or(const std::string& key, double def) const { return find(key) ? get_float(key) : def; }

// ------------------------------------------------------------------ Qwen3
Qwen3Config qwen3_config(const GgufFile& g) {
    const std::string arch = g.get_str("general.architecture");
    if (arch != "qwen3") throw std::runtime_error("unsupported architecture: " + arch + " (qwen3 only)");
    const std::string p = arch + ".";
    Qwen3Config c;
    c.n_layer = static_cast<int>(g.get_int(p + "block_count"));
    c.n_embd = static_cast<int>(g.get_int(p + "embedding_length"));
    c.n_ff = static_cast<int>(g.get_int(p + "feed_forward_length"));
    c.n_head = static_cast<int>(g.get_int(p + "attention.head_count"));
    c.n_head_kv = static_cast<int>(g.get_int_or(p + "attention.head_count_kv", c.n_head));
    // (a head count <= 0 is rejected below either way; dividing by it is not attempted)
    c.head_dim = static_cast<int>(g.get_int_or(p + "attention.key_length", c.n_head > 0 ? c.n_embd / c.n_head : 0));
    if (g.get_int_or(p + "attention.value_length", c.head_dim) != c.head_dim)
        throw std::runtime_error("key_length != value_length is not supported");
    c.rope_dim = static_cast<int>(g.get_int_or(p + "rope.dimension_count", c.head_dim));
    c.rope_base = g.get_float_or(p + "rope.freq_base", 10000.0);
    c.eps = static_cast<float>(g.get_float_or(p + "attention.layer_norm_rms_epsilon", 1e-6));
    c.n_ctx_train = static_cast<int>(g.get_int_or(p + "context_length", 0));
    const bool ok = c.n_layer > 0 && c.n_layer <= 512 && c.n_embd > 0 && c.n_head > 0 && c.n_head_kv > 0 &&
                    c.n_head % c.n_head_kv == 0 && c.head_dim > 0 && c.head_dim % 2 == 0 && c.rope_dim <= c.head_dim &&
                    c.rope_dim % 2 == 0 && c.n_ff > 0;
    if (!ok) throw std::runtime_error("invalid model configuration");
    if (g.find(p + "rope.scaling.type") && g.get_str(p + "rope.scaling.type") != "none")
        throw std::runtime_error("RoPE scaling is not supported yet");
    return c;
}

namespace {

void check_shape(const GgufTensor& t, std::initializer_list<uint64_t> want) {
    if (t.ne != std::vector<uint64_t>(want)) {
        std::string s = "tensor " + t.name + " has shape [";
        for (size_t i = 0; i < t.ne.size(); ++i) s += (i ? "," : "") + std::to_string(t.ne[i]);
        s += "], expected [";
        size_t i = 0;
        for (uint64_t v : want) s += (i++ ? "," : "") + std::to_string(v);
        throw std::runtime_error(s + "]");
    }
}

bool computable(GgmlType t) {
    return t == GgmlType::F32 || t == GgmlType::F16 || t == GgmlType::BF16 || t == GgmlType::Q8_0 ||
           t == GgmlType::Q4_K || t == GgmlType::Q6_K;
}

}  // namespace

Qwen3Tensors qwen3_tensors(const GgufFile& g, Qwen3Config& c) {
    const uint64_t E = static_cast<uint64_t>(c.n_embd), F = static_cast<uint64_t>(c.n_ff);
    const uint64_t D = static_cast<uint64_t>(c.head_dim);
    const uint64_t QD = D * static_cast<uint64_t>(c.n_head), KD = D * static_cast<uint64_t>(c.n_head_kv);
    Qwen3Tensors m;
    m.tok_embd = &g.require_tensor("token_embd.weight");
    if (m.tok_embd->ne.size() != 2 || m.tok_embd->ne[0] != E) throw std::runtime_error("token_embd has a bad shape");
    c.n_vocab = static_cast<int>(m.tok_embd->ne[1]);
    m.output = g.tensor("output.weight");
    if (!m.output) m.output = m.tok_embd;  // tied embedding
    check_shape(*m.output, {E, static_cast<uint64_t>(c.n_vocab)});
    m.output_norm = &g.require_tensor("output_norm.weight");
    check_shape(*m.output_norm, {E});
    for (int l = 0; l < c.n_layer; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        for (const char* bias : {"attn_q.bias", "attn_k.bias", "attn_v.bias", "attn_output.bias"})
            if (g.tensor(b + bias)) throw std::runtime_error("unexpected bias tensor: " + b + bias);
        Qwen3Layer L;
        L.wq = &g.require_tensor(b + "attn_q.weight");
        check_shape(*L.wq, {E, QD});
        L.wk = &g.require_tensor(b + "attn_k.weight");
        check_shape(*L.wk, {E, KD});
        L.wv = &g.require_tensor(b + "attn_v.weight");
        check_shape(*L.wv, {E, KD});
        L.wo = &g.require_tensor(b + "attn_output.weight");
        check_shape(*L.wo, {QD, E});
        L.gate = &g.require_tensor(b + "ffn_gate.weight");
        check_shape(*L.gate, {E, F});
        L.up = &g.require_tensor(b + "ffn_up.weight");
        check_shape(*L.up, {E, F});
        L.down = &g.require_tensor(b + "ffn_down.weight");
        check_shape(*L.down, {F, E});
        L.attn_norm = &g.require_tensor(b + "attn_norm.weight");
        check_shape(*L.attn_norm, {E});
        L.ffn_norm = &g.require_tensor(b + "ffn_norm.weight");
        check_shape(*L.ffn_norm, {E});
        L.q_norm = &g.require_tensor(b + "attn_q_norm.weight");
        check_shape(*L.q_norm, {D});
        L.k_norm = &g.require_tensor(b + "attn_k_norm.weight");
        check_shape(*L.k_norm, {D});
        for (const GgufTensor* t : {L.wq, L.wk, L.wv, L.wo, L.gate, L.up, L.down, L.attn_norm, L.ffn_norm, L.q_norm,
                                    L.k_norm})
            if (!computable(t->type))
                throw std::runtime_error(std::string("tensor type not supported yet: ") + ggml_type_name(t->type) +
                                         " (" + t->name + ")");
        m.layers.push_back(L);
    }
    return m;
}

}  // namespace ei
