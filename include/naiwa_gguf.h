/*
 * naiwa_gguf.h -- read-only GGUF reader for the routed-expert stacks.
 *
 * The reference loads its experts from GGUF checkpoints through candle's GGUF
 * reader (the fork's model builder, src/load.rs:414-452 checks the header and
 * tensor types) and slices each stacked [E, N, K] projection per expert with
 * expert_range (src/moe/expert.rs:123-145).  This reader maps a GGUF file
 * (versions 2 and 3) read-only, validates every offset against the file, and
 * exposes the tensors and metadata; naiwa_gguf_expert_stack gives one layer's
 * blk.<layer>.ffn_{gate,up,down}_exps.weight with the same per-expert stride,
 * ready to be copied into pinned host stacks and uploaded into slot banks.
 *
 * File layout (little-endian): "GGUF", version u32, tensor count u64, metadata
 * count u64; metadata (key string, value type u32, value); tensor infos (name
 * string, n_dims u32, dims u64 x n_dims (ne0 fastest), type u32, offset u64);
 * then, at the next multiple of general.alignment (default 32), the data.  A
 * string is a u64 length and its bytes.
 *
 * Status codes: NAIWA_OK, NAIWA_E_INVALID (arguments), NAIWA_E_IO (the file
 * cannot be opened or mapped), NAIWA_E_FORMAT (malformed or unsupported file),
 * NAIWA_E_NOT_FOUND (no such tensor or key), NAIWA_E_UNSUPPORTED (a tensor
 * whose type has no known block size, or not an expert stack).
 */
#ifndef NAIWA_GGUF_H
#define NAIWA_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct naiwa_gguf naiwa_gguf;

typedef struct naiwa_gguf_tensor {
    const char* name;  /* NUL-terminated, valid until naiwa_gguf_close */
    int n_dims;
    int64_t dims[4];   /* ne0 (fastest) .. ne3; unused dims are 1 */
    int dtype;         /* GGML type id */
    uint64_t offset;   /* byte offset of the data in the file */
    uint64_t bytes;    /* storage bytes; 0 when the type's block size is unknown */
    const void* data;  /* the mapped bytes (read-only), or NULL when bytes is 0 */
} naiwa_gguf_tensor;

/* One layer's stacked projection [E, N, K]: expert e's bytes are
 * [e * expert_bytes, (e + 1) * expert_bytes) of data. */
typedef struct naiwa_expert_stack {
    const void* data;
    int experts, n, k, dtype;
    uint64_t expert_bytes; /* n * (k / block) * type size */
} naiwa_expert_stack;

#define NAIWA_PROJ_GATE 0 /* blk.<layer>.ffn_gate_exps.weight */
#define NAIWA_PROJ_UP   1 /* blk.<layer>.ffn_up_exps.weight   */
#define NAIWA_PROJ_DOWN 2 /* blk.<layer>.ffn_down_exps.weight */

int naiwa_gguf_open(const char* path, naiwa_gguf** out);
int naiwa_gguf_close(naiwa_gguf* f);
int naiwa_gguf_version(const naiwa_gguf* f, uint32_t* version);
int naiwa_gguf_alignment(const naiwa_gguf* f, uint64_t* alignment);
int naiwa_gguf_tensor_count(const naiwa_gguf* f, int* n);
int naiwa_gguf_tensor_at(const naiwa_gguf* f, int i, naiwa_gguf_tensor* out);
int naiwa_gguf_find(const naiwa_gguf* f, const char* name, naiwa_gguf_tensor* out);
/* Metadata: an integer value of any integer or bool type (NAIWA_E_FORMAT for a
 * negative value or another type); a string value copied NUL-terminated into
 * buf (NAIWA_E_INVALID when cap is too small; *len = its length). */
int naiwa_gguf_meta_u64(const naiwa_gguf* f, const char* key, uint64_t* value);
int naiwa_gguf_meta_string(const naiwa_gguf* f, const char* key, char* buf, int cap, int* len);
/* Block size (values) and bytes of a GGML type id; 0 / 0 when unknown. */
int naiwa_ggml_type_size(int dtype, int* block, int* bytes);
/* proj: NAIWA_PROJ_GATE / UP / DOWN.  The tensor must have 3 dims (or a 4th of
 * 1) and ne0 a multiple of its type's block. */
int naiwa_gguf_expert_stack(const naiwa_gguf* f, int layer, int proj, naiwa_expert_stack* out);

#ifdef __cplusplus
}
#endif
#endif
