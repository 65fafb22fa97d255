// qwen3_schema.cpp — the Qwen3 model contract, stated as tables and checked against a GGUF index.
//
// Three tables carry the contract: the hyper-parameters (key, destination, fallback when the
// file leaves the key out), the sanity conditions the configuration must meet, and the tensors
// of each block with their shapes written as symbolic extents of the configuration.  The key
// names, fallbacks and shapes are the model contract the reference engine reads
// (src/model.cpp:38-103); the checking code is table-driven.
#include <climits>
#include <cstdio>
#include <initializer_list>

#include "gguf_index.h"

namespace ei::gguf {

namespace {

using Cfg = Qwen3Config;

// ---- hyper-parameters under "qwen3."; a fallback reads only fields of earlier rows
struct IntParam {
    const char* key;
    int Cfg::*field;
    int (*fallback)(const Cfg&);  // nullptr: the key is required
};

const IntParam kIntParams[] = {
    {"block_count", &Cfg::n_layer, nullptr},
    {"embedding_length", &Cfg::n_embd, nullptr},
    {"feed_forward_length", &Cfg::n_ff, nullptr},
    {"attention.head_count", &Cfg::n_head, nullptr},
    {"attention.head_count_kv", &Cfg::n_head_kv, [](const Cfg& c) { return c.n_head; }},
    {"attention.key_length", &Cfg::head_dim, [](const Cfg& c) { return c.n_head > 0 ? c.n_embd / c.n_head : 0; }},
    {"rope.dimension_count", &Cfg::rope_dim, [](const Cfg& c) { return c.head_dim; }},
    {"context_length", &Cfg::n_ctx_train, [](const Cfg&) { return 0; }},
};

// ---- conditions a usable configuration meets
bool (*const kSane[])(const Cfg&) = {
    [](const Cfg& c) { return c.n_layer > 0 && c.n_layer <= 512; },
    [](const Cfg& c) { return c.n_embd > 0 && c.n_ff > 0; },
    [](const Cfg& c) { return c.n_head > 0 && c.n_head_kv > 0 && c.n_head % c.n_head_kv == 0; },
    [](const Cfg& c) { return c.head_dim > 0 && c.head_dim % 2 == 0; },
    [](const Cfg& c) { return c.rope_dim >= 0 && c.rope_dim <= c.head_dim && c.rope_dim % 2 == 0; },
};

// ---- tensor shapes as symbolic extents
enum Extent : uint8_t { kAbsent, kEmbd, kFF, kQWidth, kKVWidth, kHeadDim, kVocab };

uint64_t extent(Extent e, const Cfg& c) {
    switch (e) {
        case kEmbd: return uint64_t(c.n_embd);
        case kFF: return uint64_t(c.n_ff);
        case kQWidth: return uint64_t(c.n_head) * uint64_t(c.head_dim);
        case kKVWidth: return uint64_t(c.n_head_kv) * uint64_t(c.head_dim);
        case kHeadDim: return uint64_t(c.head_dim);
        case kVocab: return uint64_t(c.n_vocab);
        default: return 0;
    }
}

struct TensorRule {
    const char* suffix;  // after "blk.<i>."
    Extent row;          // dims[0], the contiguous row length
    Extent rows;         // dims[1]; kAbsent for a vector
};

// one block, in the order its tensors are used by a forward pass
const TensorRule kBlock[] = {
    {"attn_norm.weight", kEmbd, kAbsent},     {"attn_q.weight", kEmbd, kQWidth},
    {"attn_k.weight", kEmbd, kKVWidth},       {"attn_v.weight", kEmbd, kKVWidth},
    {"attn_q_norm.weight", kHeadDim, kAbsent}, {"attn_k_norm.weight", kHeadDim, kAbsent},
    {"attn_output.weight", kQWidth, kEmbd},   {"ffn_norm.weight", kEmbd, kAbsent},
    {"ffn_gate.weight", kEmbd, kFF},          {"ffn_up.weight", kEmbd, kFF},
    {"ffn_down.weight", kFF, kEmbd},
};

// a block must not carry these (the engine computes no attention biases)
const char* const kNotInBlock[] = {"attn_q.bias", "attn_k.bias", "attn_v.bias", "attn_output.bias"};

// element types the engine computes with
const uint32_t kComputable[] = {kTF32, kTF16, kTBF16, kTQ8_0, kTQ4_K, kTQ6_K};

std::string dims_text(std::initializer_list<uint64_t> d) {
    std::string s = "[";
    for (uint64_t v : d) s += (s.size() > 1 ? "," : "") + std::to_string(v);
    return s + "]";
}

std::string dims_text(const TensorSlot& t) {
    std::string s = "[";
    for (uint32_t i = 0; i < t.rank; ++i) s += (i ? "," : "") + std::to_string(t.dims[i]);
    return s + "]";
}

void expect_shape(const TensorSlot& t, uint64_t row, uint64_t rows /* 0: a vector */) {
    const bool ok = rows == 0 ? (t.rank == 1 && t.dims[0] == row) : (t.rank == 2 && t.dims[0] == row && t.dims[1] == rows);
    if (!ok)
        throw FormatError("tensor " + t.name + " has shape " + dims_text(t) + ", expected " +
                          (rows == 0 ? dims_text({row}) : dims_text({row, rows})));
}

const TensorSlot& need(const Index& f, const std::string& name) {
    if (const TensorSlot* t = f.tensor(name)) return *t;
    throw FormatError("tensor missing: " + name);
}

void read_hyperparameters(const Index& f, Cfg& c) {
    const std::string arch = f.text("general.architecture");
    if (arch != "qwen3") throw FormatError("unsupported architecture: " + arch + " (qwen3 only)");
    for (const IntParam& p : kIntParams) {
        const std::string key = std::string("qwen3.") + p.key;
        const int64_t v = f.slot(key) || !p.fallback ? f.integer(key) : p.fallback(c);
        if (v < INT_MIN || v > INT_MAX) throw FormatError("invalid model configuration (" + key + " out of range)");
        c.*p.field = static_cast<int>(v);
    }
    if (f.integer_or("qwen3.attention.value_length", c.head_dim) != c.head_dim)
        throw FormatError("key_length != value_length is not supported");
    c.rope_base = f.number_or("qwen3.rope.freq_base", 10000.0);
    c.eps = static_cast<float>(f.number_or("qwen3.attention.layer_norm_rms_epsilon", 1e-6));
    for (auto sane : kSane)
        if (!sane(c)) throw FormatError("invalid model configuration");
    if (f.slot("qwen3.rope.scaling.type") && f.text("qwen3.rope.scaling.type") != "none")
        throw FormatError("RoPE scaling is not supported yet");
}

void check_tensor_table(const Index& f, Cfg& c) {
    const TensorSlot& embd = need(f, "token_embd.weight");
    if (embd.rank != 2 || embd.dims[0] != uint64_t(c.n_embd) || embd.dims[1] > uint64_t(INT_MAX))
        throw FormatError("token_embd has a bad shape");
    c.n_vocab = static_cast<int>(embd.dims[1]);
    const TensorSlot* head = f.tensor("output.weight");
    expect_shape(head ? *head : embd, extent(kEmbd, c), extent(kVocab, c));  // absent: tied to the embedding
    expect_shape(need(f, "output_norm.weight"), extent(kEmbd, c), 0);

    for (int l = 0; l < c.n_layer; ++l) {
        const std::string blk = "blk." + std::to_string(l) + ".";
        for (const char* s : kNotInBlock)
            if (f.tensor(blk + s)) throw FormatError("unexpected bias tensor: " + blk + s);
        for (const TensorRule& r : kBlock) {
            const TensorSlot& t = need(f, blk + r.suffix);
            expect_shape(t, extent(r.row, c), extent(r.rows, c));
            bool computable = false;
            for (uint32_t ty : kComputable) computable |= t.type == ty;
            if (!computable) {
                const BlockFormat* bf = block_format(t.type);
                throw FormatError(std::string("tensor type not supported yet: ") + (bf ? bf->name : "?") + " (" +
                                  t.name + ")");
            }
        }
    }
}

}  // namespace

Qwen3Config qwen3_config(const Index& file) {
    Qwen3Config c;
    read_hyperparameters(file, c);
    check_tensor_table(file, c);
    return c;
}

}  // namespace ei::gguf
