// gguf.h — a read-only, bounds-checked GGUF model-file reader over POSIX mmap, and the Qwen3
// configuration / tensor table the attention path needs from it.
//
// Same interface and error behaviour as the reference's reader (class el::Gguf,
// src/gguf.h:55-84; src/gguf.cpp:203-306), which maps the file with Win32 calls and does not build
// on Linux.  The file is untrusted input: every length, count, dimension and offset is checked
// against the mapping, and a malformed file raises GgufError; tensor data is not copied (views
// into the mapping, valid while the GgufFile lives).  qwen3_config and qwen3_tensors restate
// read_config / read_tensors (src/model.cpp:38-103).
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace ei {

struct GgufError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// GGML tensor element types the reader knows the block layout of (GGUF's type ids)
enum class GgmlType : uint32_t {
    F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8,
    Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, BF16 = 30,
};
const char* ggml_type_name(GgmlType t);

// GGUF metadata value types (GGUF's type ids)
enum class GgufType : uint32_t {
    U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, BOOL = 7, STRING = 8, ARRAY = 9,
    U64 = 10, I64 = 11, F64 = 12,
};

struct GgufValue {
    GgufType type = GgufType::U8;
    GgufType elem = GgufType::U8;      // element type of an ARRAY
    int64_t i = 0;                     // integers and bools
    double f = 0.0;                    // floats (and integers, converted)
    std::string s;                     // STRING
    std::vector<int64_t> ai;           // integer arrays
    std::vector<double> af;            // float arrays
    std::vector<std::string> as;       // string arrays
};

struct GgufTensor {
    std::string name;
    GgmlType type = GgmlType::F32;
    std::vector<uint64_t> ne;  // dimensions; ne[0] is contiguous in memory (the row length)
    uint64_t numel = 0;
    uint64_t nbytes = 0;
    const uint8_t* data = nullptr;

    uint64_t rows() const { return numel / ne[0]; }
};

class GgufFile {
public:
    explicit GgufFile(const std::string& path);
    ~GgufFile();
    GgufFile(const GgufFile&) = delete;
    GgufFile& operator=(const GgufFile&) = delete;

    uint32_t version() const { return version_; }
    const std::unordered_map<std::string, GgufValue>& meta() const { return meta_; }
    const std::vector<GgufTensor>& tensors() const { return tensors_; }

    const GgufValue* find(const std::string& key) const;        // nullptr when absent
    const GgufTensor* tensor(const std::string& name) const;    // nullptr when absent
    const GgufTensor& require_tensor(const std::string& name) const;

    // required keys (GgufError when absent or of another kind)
    int64_t get_int(const std::string& key) const;
    double get_float(const std::string& key) const;
    const std::string& get_str(const std::string& key) const;
    int64_t get_int_or(const std::string& key, int64_t def) const;
    double get_float_or(const std::string& key, double def) const;

private:
    const uint8_t* map_ = nullptr;
    uint64_t size_ = 0;
    uint32_t version_ = 0;
    std::unordered_map<std::string, GgufValue> meta_;
    std::vector<GgufTensor> tensors_;
    std::unordered_map<std::string, size_t> by_name_;
};

// ------------------------------------------------------------------ Qwen3
struct Qwen3Config {
    int n_layer = 0, n_embd = 0, n_ff = 0, n_head = 0, n_head_kv = 0, head_dim = 0, rope_dim = 0;
    double rope_base = 10000.0;
    float eps = 1e-6f;
    int n_ctx_train = 0;
    int n_vocab = 0;
};

struct Qwen3Layer {
    const GgufTensor *wq, *wk, *wv, *wo, *gate, *up, *down, *attn_norm, *ffn_norm, *q_norm, *k_norm;
};

struct Qwen3Tensors {
    const GgufTensor* tok_embd = nullptr;
    const GgufTensor* output = nullptr;  // the embedding when the file ties them
    const GgufTensor* output_norm = nullptr;
    std::vector<Qwen3Layer> layers;
};

// the hyper-parameters of a qwen3 file (read_config, src/model.cpp:38-65); n_vocab is set by
// qwen3_tensors from the embedding's shape
Qwen3Config qwen3_config(const GgufFile& g);
// the tensor table with every shape checked (read_tensors, src/model.cpp:67-103); element types
// are those the reference computes with (F32, F16, BF16, Q8_0, Q4_K, Q6_K)
Qwen3Tensors qwen3_tensors(const GgufFile& g, Qwen3Config& c);

}  // namespace ei
