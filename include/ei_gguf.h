/*
 * ei_gguf.h — C ABI of the GGUF model-file reader in libei_attn.so
 * (exactinfer_amd/host/gguf_index.{h,cpp}, qwen3_schema.cpp): the Qwen3 weights the attention
 * path's callers feed it come from these files.
 *
 * Replaces the reference's el::Gguf (src/gguf.h:55-84, src/gguf.cpp:203-306; Win32-only there)
 * and read_config / read_tensors (src/model.cpp:38-103).  Conventions are those of ei_attn.h:
 * int status (EI_OK or an EI_ERR_* code) with the message from ei_last_error(); nothing throws
 * across the boundary.  A malformed or unsupported file is EI_ERR_ARG.  Tensor data pointers
 * point into the read-only file mapping and stay valid until ei_gguf_close.
 */
#ifndef EI_GGUF_H
#define EI_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ei_gguf ei_gguf;

/* Maps and parses the file (bounds-checked: lengths, counts, shapes, alignment and tensor
 * extents must lie inside it).  NULL on failure, with the reason in ei_last_error(). */
ei_gguf* ei_gguf_open(const char* path);
void ei_gguf_close(ei_gguf* g);

int ei_gguf_version(const ei_gguf* g);
long ei_gguf_n_tensors(const ei_gguf* g);
/* Tensor `index` (file order): name, GGML type id, dimensions (ne[0] contiguous; unused entries
 * of ne[4] set to 1), data pointer and byte size.  Any output pointer may be NULL. */
int ei_gguf_tensor(const ei_gguf* g, long index, const char** name, int* type, int* n_dims, uint64_t* ne,
                   const void** data, uint64_t* nbytes);
long ei_gguf_find_tensor(const ei_gguf* g, const char* name); /* index, or -1 when absent */

/* Metadata by key: integers (and bools), numbers (floats, or integers converted), strings.
 * EI_ERR_ARG when the key is absent or holds another kind. */
int ei_gguf_get_int(const ei_gguf* g, const char* key, int64_t* out);
int ei_gguf_get_float(const ei_gguf* g, const char* key, double* out);
int ei_gguf_get_str(const ei_gguf* g, const char* key, const char** out);

/* Qwen3 hyper-parameters, validated against the tensor table (every attention, feed-forward and
 * norm tensor present with the shape the configuration implies and a type the reference
 * computes with), as read_config + read_tensors do. */
typedef struct {
    int n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim, rope_dim, n_ctx_train, n_vocab;
    double rope_base;
    float eps;
} ei_qwen3_config;
int ei_gguf_qwen3_config(const ei_gguf* g, ei_qwen3_config* out);

#ifdef __cplusplus
}
#endif

#endif /* EI_GGUF_H */
