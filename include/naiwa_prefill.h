/*
 * naiwa_prefill.h -- the whole-layer prefill stream: a prompt chunk's MoE layers
 * run over expert stacks that live in pinned host memory, each layer's stacks
 * uploaded into one of `depth` device layer buffers on a copy stream while the
 * previous layer's grouped GEMM runs (the reference's PrefillStream,
 * src/prefill_stream.rs:342-1693), and the memory plan that picks the chunk
 * and the number of layer buffers (src/prefill_stream.rs:122-310).
 *
 * On MI355X a model of this class usually fits in HBM, and then the resident
 * naiwa_moe_prefill is the path; the stream serves experts that do not.
 */
#ifndef NAIWA_PREFILL_H
#define NAIWA_PREFILL_H

#include "naiwa_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- the memory plan (pure host arithmetic) ----------------------------- */

/* Device bytes a prompt chunk of `rows` rows needs beside the layer buffers:
 * 32 MiB + 354 KiB a row (chunk_scratch, src/prefill_stream.rs:122-137;
 * NAIWA_CHUNK_FIXED_MIB / NAIWA_CHUNK_PER_ROW_KIB override the constants). */
uint64_t naiwa_prefill_chunk_scratch(int rows);
/* The shape estimate: 160 MiB + 680 MiB per 1024 rows of one 256-row MoE
 * batch, plus 24 KiB a row (activation_bytes, src/prefill_stream.rs:139-143). */
uint64_t naiwa_prefill_activation_bytes(int chunk);

/* plan_with_lend_depth (src/prefill_stream.rs:205-310): the largest chunk on
 * the 256-row grid up to min(ceiling, 8192) whose scratch, one layer buffer
 * and the head (max(512 MiB, free / 8), or NAIWA_PREFILL_SLACK_MIB) fit in
 * free - kv_reserve; then the deepest stride in [2, max_depth] (max_depth
 * clamped to 1..4) that the same chunk affords while leaving the decode
 * reserve (700 MiB, NAIWA_DECODE_RESERVE_MIB) free, else 1.  With `borrowing`
 * the buffers are ranges of a cache pool of `lend_bytes`: the chunk pays only
 * its scratch and min(head, 256 MiB), and stride = lend_bytes / layer_bytes
 * clamped to [1, min(max_depth, NAIWA_DEPTH_CAP or 2)].
 * *stride = *chunk = 0 when nothing fits (the reference's None). */
int naiwa_prefill_plan(uint64_t free_bytes, uint64_t layer_bytes, int ceiling, int borrowing, uint64_t kv_reserve,
                       uint64_t lend_bytes, int max_depth, int* stride, int* chunk);

/* ---- the stream ---------------------------------------------------------- */

typedef struct naiwa_prefill_stream_desc {
    int n_layers;
    int num_experts;              /* experts in each layer's host stacks (shared experts may be appended) */
    int hidden, inter;
    int dtype_gate, dtype_up, dtype_down;
    const void* const* host_gate; /* [n_layers] pinned stacks [E, I, H]; expert e at e * expert bytes */
    const void* const* host_up;   /* [n_layers] [E, I, H] */
    const void* const* host_down; /* [n_layers] [E, H, I] */
    int depth;                    /* device layer buffers, 1..4 (the plan's stride) */
} naiwa_prefill_stream_desc;

typedef struct naiwa_prefill_stream_stats {
    uint64_t uploads;      /* layer uploads queued */
    uint64_t upload_bytes; /* bytes they moved host -> device */
    uint64_t forwards;     /* naiwa_prefill_stream_forward calls */
} naiwa_prefill_stream_stats;

typedef struct naiwa_prefill_stream naiwa_prefill_stream;

/* Allocates `depth` layer buffers (one bank per projection, num_experts slots
 * each) and keeps the host pointers; `copy_stream` carries the uploads. */
int naiwa_prefill_stream_create(const naiwa_prefill_stream_desc* d, int64_t copy_stream, naiwa_prefill_stream** out);
/* Waits for the device, then frees the buffers. */
int naiwa_prefill_stream_destroy(naiwa_prefill_stream* ps);

/* One MoE layer of a chunk (PrefillStream::forward, src/prefill_stream.rs:1362-1693):
 * queue `layer`'s upload into buffer layer % depth unless it is there, queue
 * the uploads of layers layer + 1 .. layer + depth - 1 into their buffers
 * (each after the last kernel that read that buffer), make `stream` wait for
 * `layer`'s upload, run naiwa_moe_prefill over the buffer with expert ids as
 * slot ids, and record the buffer's read fence.  Arguments after `layer` are
 * naiwa_moe_prefill's.  Layers are normally visited in order; any order is
 * correct. */
int naiwa_prefill_stream_forward(naiwa_prefill_stream* ps, int layer, const void* x, const uint32_t* expert_ids,
                                 const float* w, int T, int k, int act, float* out, int flags, int64_t stream);

/* The device banks that hold `layer` (valid once a forward of it was queued),
 * e.g. for a caller's own kernels on the same stream order. */
int naiwa_prefill_stream_banks(const naiwa_prefill_stream* ps, int layer, naiwa_bank* gate, naiwa_bank* up,
                               naiwa_bank* down);
int naiwa_prefill_stream_stats_read(const naiwa_prefill_stream* ps, naiwa_prefill_stream_stats* out);

#ifdef __cplusplus
}
#endif
#endif
