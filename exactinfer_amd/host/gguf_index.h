// gguf_index.h — an index over a memory-mapped GGUF file, and the Qwen3 schema checked against it.
//
// The index is built in one scan over the file's header region.  Nothing is decoded into values
// during the scan: each metadata entry becomes a slot (type ids, element count, and the byte span
// its payload occupies in the mapping) that typed accessors decode on demand through a table of
// value encodings; each tensor record becomes a slot holding its shape, GGML type, byte size and
// a view of its data inside the mapping.  Structural checks (lengths, counts, ranks) run while
// scanning, because the scan cannot continue past a bad one; the semantic checks of the tensor
// table (shapes, types, block divisibility, unique names, alignment, extents) run afterwards over
// the slots.  Every error is a FormatError naming what was wrong.
//
// It serves the role of the reference's el::Gguf (src/gguf.h:55-84, src/gguf.cpp:203-306), which
// maps the file with Win32 calls and does not build on Linux, and accepts and rejects the same
// classes of file.  qwen3_config() covers read_config / read_tensors (src/model.cpp:38-103).
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace ei::gguf {

struct FormatError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// Metadata value type ids, as numbered by the GGUF format.
enum ValueType : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7, kString = 8, kArray = 9,
    kU64 = 10, kI64 = 11, kF64 = 12,
};

// GGML tensor type ids, as numbered by the GGUF format.
enum TensorType : uint32_t {
    kTF32 = 0, kTF16 = 1, kTQ4_0 = 2, kTQ4_1 = 3, kTQ5_0 = 6, kTQ5_1 = 7, kTQ8_0 = 8, kTQ2_K = 10, kTQ3_K = 11,
    kTQ4_K = 12, kTQ5_K = 13, kTQ6_K = 14, kTBF16 = 30,
};

// Storage of one GGML type: elements per block, bytes per block, display name.
struct BlockFormat {
    uint32_t elems;
    uint32_t bytes;
    const char* name;
};
// nullptr for a type id this reader does not know
const BlockFormat* block_format(uint32_t tensor_type);

// Where a metadata value lies in the file and how it is encoded.
struct MetaSlot {
    uint32_t type = 0;       // ValueType of the entry
    uint32_t elem_type = 0;  // element ValueType of an array (the entry's own type otherwise)
    uint64_t count = 1;      // elements of an array, 1 for a scalar
    uint64_t payload = 0;    // file offset of the value (an array's first element)
    uint64_t span = 0;       // bytes from payload to the end of the value
    int text = -1;           // a string scalar's index in the index's text pool
};

struct TensorSlot {
    std::string name;
    uint32_t type = 0;                 // TensorType
    uint32_t rank = 0;                 // 1..4
    uint64_t dims[4] = {1, 1, 1, 1};   // dims[0] is the contiguous row length; unused ones are 1
    uint64_t elements = 0;
    uint64_t bytes = 0;
    uint64_t data_offset = 0;          // from the start of the data section, as recorded
    const uint8_t* data = nullptr;     // inside the mapping
};

class Index {
public:
    explicit Index(const std::string& path);
    ~Index();
    Index(const Index&) = delete;
    Index& operator=(const Index&) = delete;

    uint32_t version() const { return version_; }
    const std::vector<TensorSlot>& tensors() const { return tensors_; }
    const TensorSlot* tensor(std::string_view name) const;  // nullptr when absent
    const MetaSlot* slot(std::string_view key) const;       // nullptr when absent

    // Typed reads of scalar metadata.  Missing keys and values of another kind raise FormatError
    // ("metadata missing: k", "metadata is not an integer: k", ... ).  number() also reads integers.
    int64_t integer(std::string_view key) const;
    double number(std::string_view key) const;
    const std::string& text(std::string_view key) const;
    int64_t integer_or(std::string_view key, int64_t fallback) const { return slot(key) ? integer(key) : fallback; }
    double number_or(std::string_view key, double fallback) const { return slot(key) ? number(key) : fallback; }

private:
    void scan();
    void check_tensor_records();
    void place_tensor_data(uint64_t header_end);

    const uint8_t* map_ = nullptr;
    uint64_t size_ = 0;
    uint32_t version_ = 0;
    std::unordered_map<std::string_view, MetaSlot> meta_;  // keys view the mapping
    std::vector<std::string> text_pool_;
    std::vector<TensorSlot> tensors_;
    std::unordered_map<std::string_view, size_t> tensor_names_;  // views TensorSlot::name
};

// Qwen3 hyper-parameters; n_vocab comes from the embedding's shape.
struct Qwen3Config {
    int n_layer = 0, n_embd = 0, n_ff = 0, n_head = 0, n_head_kv = 0, head_dim = 0, rope_dim = 0, n_ctx_train = 0,
        n_vocab = 0;
    double rope_base = 0.0;
    float eps = 0.0f;
};

// Reads the "qwen3.*" hyper-parameters and checks the whole tensor table against them (every
// tensor of every block present, with the shape the configuration implies and a GGML type the
// reference computes with; no bias tensors).  FormatError on any mismatch.
Qwen3Config qwen3_config(const Index& file);

}  // namespace ei::gguf
