/*
 * naiwa_cached.h -- one MoE layer's decode step over a partial expert cache.
 *
 * The counterpart of the reference's CachedExperts::forward for decode rows
 * (src/moe/decode.rs:241-381 with the stages of src/moe/stages/): route on the
 * device, read the top-k back, split hits from misses with the host policy
 * (include/naiwa_policy.h), stream the chosen misses over PCIe into the
 * staging-ring slots of the layer's banks (src/moe/stages/dma_miss.rs:58-202),
 * run the expert kernel over resident + staged slots, then promote staged
 * experts into the cache (src/moe/cached_layer.rs:892-1051).  The lookahead
 * (src/moe/cached_layer.rs:1236-1300, src/moe/stages/preload.rs:18-111) loads
 * the next layer's predicted experts into its cache while this layer computes.
 *
 * Slot layout of each projection's bank: slots [0, usable) are the cache,
 * slots [usable, usable + ring_len) hold the staging ring's positions, so a
 * ring slot NAIWA_STAGING_RING_FIRST + p is bank slot usable + p (the
 * reference's `slot - bank.first` for its ring bank).
 *
 * Misses the ring does not take run on the CPU, as in the reference
 * (src/moe/stages/cpu_miss.rs:73-162): the step publishes x to mapped host
 * memory, a CPU job on a one-thread executor computes those pairs from the
 * host expert stacks (naiwa_cpu_moe_decode), and its result comes back through
 * a result doorbell that the device waits for on the stream and adds last:
 * resident, then staged, then CPU (src/moe/decode.rs:371-381).
 */
#ifndef NAIWA_CACHED_H
#define NAIWA_CACHED_H

#include "naiwa_moe.h"
#include "naiwa_policy.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct naiwa_cached_layer_desc {
    const float* router;      /* device [E, H] f32 */
    const float* router_bias; /* device [E] f32 or null */
    naiwa_bank gate, up, down; /* device banks, slots >= usable + ring length */
    const void* host_gate;    /* pinned host bytes of expert 0's gate projection */
    const void* host_up;
    const void* host_down;
    int num_experts, top_k, hidden, inter, usable, mode, act;
    /* Bytes between consecutive experts in the host stacks.  0: each projection
     * is a stacked [E, N, K] tensor of its own (expert e at host_p + e * that
     * projection's bytes, the GGUF layout).  Otherwise every projection's
     * expert e is at host_p + e * host_expert_stride.  When an expert's gate,
     * up and down are adjacent both in the host stacks (host_up = host_gate +
     * gate bytes, host_down = host_up + up bytes) and in every slot (up.base =
     * gate.base + gate bytes, down.base = up.base + up bytes, one common slot
     * stride), an upload is one copy of the whole expert. */
    int64_t host_expert_stride;
} naiwa_cached_layer_desc;

/* Per-step report of naiwa_cached_layer_forward. */
typedef struct naiwa_cached_step {
    int hits;        /* (row, k) pairs served from a cache slot */
    int staged;      /* pairs served from a staging slot */
    int staged_experts; /* distinct experts uploaded this step */
    int promoted;    /* experts copied staging -> cache */
    int64_t pcie_bytes;
    int preload_waits; /* 1 when the expert kernel waited for a lookahead claim */
    int cpu;         /* pairs computed on the CPU (the reference's misses) */
} naiwa_cached_step;

/* Host expert stacks for the CPU expert path: expert e's projection p at
 * p + e * p_stride (0: that projection's own bytes, the GGUF [E, N, K] layout);
 * gate and up are [inter, hidden], down [hidden, inter]; Q4_K or Q8_0. */
typedef struct naiwa_host_experts {
    const void* gate;
    const void* up;
    const void* down;
    int64_t gate_stride, up_stride, down_stride;
    int gate_dtype, up_dtype, down_dtype;
    int num_experts, hidden, inter;
} naiwa_host_experts;

/* The reference's CPU expert contract, fused_moe_decode
 * (src/moe/stages/cpu_miss.rs:13-20, :45): xs f32 [rows, hidden]; ids / w
 * [rows, width] row-major, weight-0 entries skipped (padding); pass 1 computes
 * act(gate . x) * (up . x) once per distinct (expert, row), pass 2 writes
 * out[row] = sum over the row's entries in order of w * (down . h) (f32
 * [rows, hidden]).  f32 activations, weights dequantised on the fly; host
 * threads of a persistent pool (one call at a time runs on it).  Synchronous;
 * no device memory is touched.  NAIWA_E_BAD_ID for an id >= num_experts. */
int naiwa_cpu_moe_decode(const naiwa_host_experts* ex, const float* xs, const uint32_t* ids, const float* w,
                         int rows, int width, int act, float* out);

/* Per-call report of the lookahead (src/moe/cached_layer.rs:1262-1295). */
typedef struct naiwa_lookahead_step {
    int predicted;   /* distinct experts in the prediction */
    int resident;    /* of those, already published in a cache slot */
    int loads;       /* admitted into an empty slot (CacheStats::lookahead_loads) */
    int swaps;       /* loaded over an LRU resident (CacheStats::swaps) */
    int64_t pcie_bytes; /* bytes the loads and swaps upload */
} naiwa_lookahead_step;

typedef struct naiwa_cached_layer naiwa_cached_layer;

/* The layer keeps a pointer to `ring` (shared by layers of one shape, as the
 * reference shares its ring) and owns a naiwa_cache of `usable` slots. */
int naiwa_cached_layer_create(const naiwa_cached_layer_desc* d, naiwa_ring* ring, int ring_len,
                              int64_t copy_stream, naiwa_cached_layer** out);
int naiwa_cached_layer_destroy(naiwa_cached_layer* L);
/* The layer's policy state (owned by the layer). */
int naiwa_cached_layer_cache(naiwa_cached_layer* L, naiwa_cache** out);

/* Fill: admit `expert` into an empty cache slot, upload it and publish it once
 * the copy is done (synchronous).  *slot_out = -1 when not admitted. */
int naiwa_cached_layer_fill(naiwa_cached_layer* L, int expert, int* slot_out);

/* Profile seeding before the first token (src/moe/provider.rs:214-256): the
 * first round(usable * fill_share) experts of `experts` (one layer's profile
 * ranking, best first; fill_share is the reference's NAIWA_PROFILE_FILL,
 * 1 by default) are admitted in order -- an expert already resident, one
 * past the model, or one that finds no empty slot uses its place in the
 * budget and is skipped -- uploaded on the copy stream, and published after
 * one synchronisation.  *filled = experts placed. */
int naiwa_cached_layer_seed(naiwa_cached_layer* L, const uint32_t* experts, int n, float fill_share, int* filled);

/* One decode step: x bf16 [rows, H] -> out f32 [rows, H], all on `stream`.
 * Staged uploads are one kernel reading the host stacks through their device
 * mapping when they are mapped pinned memory, else DMA copies
 * (naiwa_cached_layer_set_upload_path).
 * The routing comes back through a mapped doorbell (the role of the
 * reference's TopkDoorbell, src/doorbell/d2h/topk.rs:20-125): the device
 * writes the top-k into fine-grained host memory as 64-bit words tagged with
 * the step's sequence number, and the host spins until every word carries the
 * tag (at most 10 s, else NAIWA_E_TIMEOUT) instead of synchronising the
 * stream.  Steps of one layer are ordered even when each
 * is queued on another stream (a step waits for the previous step's last
 * read of the layer's buffers).  Staged uploads complete into the staged
 * expert pass as naiwa_cached_layer_set_upload_sync chooses.  Misses left
 * out of the ring run on the CPU (naiwa_cpu_moe_decode on the library's
 * executor) while the device computes the resident and staged pairs; the
 * device waits for their result doorbell (bounded, naiwa_doorbell_set_wait_limit_us)
 * and adds it last.  A CPU job that failed is reported (NAIWA_E_DEVICE, or
 * its own code) by the layer's next call, before that call changes any state.
 * pcie_frac, promote_cap and min_hits are the reference's --pcie-frac,
 * NAIWA_PROMOTE_CAP and NAIWA_PROMOTE_MIN_HITS; info->cpu counts the CPU pairs. */
int naiwa_cached_layer_forward(naiwa_cached_layer* L, const void* x, int rows, float* out, float pcie_frac,
                               int promote_cap, uint64_t min_hits, int64_t stream, naiwa_cached_step* info);

/* How staged uploads complete into the expert pass (per layer):
 *  NAIWA_UPLOAD_SYNC_EVENT: an event recorded on the copy stream after the
 *    uploads, which the compute stream waits for;
 *  NAIWA_UPLOAD_SYNC_POLL (the default): the copy stream raises a device flag behind the
 *    uploads (doorbell_poll_signal) and one wave on the compute stream polls it
 *    (the persistent-wave doorbell of the reference's device waits,
 *    src/doorbell/doorbell.cu:105-149).  The poll is bounded
 *    (naiwa_doorbell_set_wait_limit_us): a wait that runs out leaves that
 *    step's output invalid and is counted in the layer's mapped doorbell; the
 *    layer's next forward returns NAIWA_E_TIMEOUT for it before it changes
 *    any state, and naiwa_cached_layer_upload_timeouts reads the count. */
#define NAIWA_UPLOAD_SYNC_EVENT 0
#define NAIWA_UPLOAD_SYNC_POLL 1
int naiwa_cached_layer_set_upload_sync(naiwa_cached_layer* L, int mode);
int naiwa_cached_layer_upload_timeouts(const naiwa_cached_layer* L, uint32_t* count);

/* How staged uploads travel (per layer; CopyStream::queue_async,
 * src/copy_stream.rs:387-409):
 *  NAIWA_UPLOAD_PATH_KERNEL (the default): when the host stacks are mapped
 *    pinned memory, one batched copy kernel on the copy stream reads every
 *    staged expert through the host mapping; the expert pass runs once, after
 *    the uploads (a kernel beside the copy kernel ends with it);
 *  NAIWA_UPLOAD_PATH_DMA: hipMemcpyAsync on the copy stream (the SDMA
 *    engines), one range per expert when slots and stacks are expert-
 *    contiguous; the cache-slot pairs run while the uploads land and the
 *    staged pairs accumulate after them, the same bits either way.
 * Pageable or unmapped stacks always take DMA copies. */
#define NAIWA_UPLOAD_PATH_KERNEL 0
#define NAIWA_UPLOAD_PATH_DMA 1
int naiwa_cached_layer_set_upload_path(naiwa_cached_layer* L, int path);

/* Misses the ring does not take go to the CPU (1, the default) or, with 0, a
 * step that would leave any miss unstaged is refused with NAIWA_E_UNSUPPORTED
 * before the policy is touched (naiwa_cache_plan decides; no tick, hit count or
 * ring position moves).  No counterpart in the reference, whose misses always
 * may go to the CPU; for hosts that keep every expert computation on the GPU. */
int naiwa_cached_layer_set_cpu_misses(naiwa_cached_layer* L, int on);

/* prefetch_predicted (src/moe/cached_layer.rs:1262-1300) for layer `next` on
 * the activation x bf16 [rows, H] of the layer before it: next's router ranks
 * the experts by its logits, router_bias included (the reference's routers
 * have no bias term: without one this is its raw-logit ranking,
 * src/moe/cached_layer.rs:1245-1259), the rows' top-k are merged by
 * naiwa_union_by_votes, and each predicted expert is
 * admitted into an empty cache slot or, while swaps < lookahead_swaps * rows
 * (the reference's --lookahead-swaps, default 2), replaces the LRU resident
 * outside the prediction.  The uploads run on next's copy stream after the
 * last step that read next's slots; the slots are published at once and
 * next's following forward waits for the claim event recorded after them
 * before its expert kernel (src/moe/cached_layer.rs:808-819).  Synchronises
 * `stream` once for the prediction read-back. */
int naiwa_cached_layer_prefetch(naiwa_cached_layer* next, const void* x, int rows, int lookahead_swaps,
                                int64_t stream, naiwa_lookahead_step* info);

/* naiwa_cached_layer_forward of L plus naiwa_cached_layer_prefetch of `next`
 * on the same x with one routing read-back: next's router is queued beside
 * L's, and next's uploads after L's expert kernel, so they overlap L's
 * compute (the reference's Preload stage, src/moe/stages/preload.rs:18-111).
 * next != L and has L's hidden size and top_k (NAIWA_E_INVALID otherwise). */
int naiwa_cached_layer_forward_ahead(naiwa_cached_layer* L, naiwa_cached_layer* next, int lookahead_swaps,
                                     const void* x, int rows, float* out, float pcie_frac, int promote_cap,
                                     uint64_t min_hits, int64_t stream, naiwa_cached_step* info,
                                     naiwa_lookahead_step* ahead);

/* One decode step through a stack of cached layers, in order: for each layer the
 * partial-cache step (naiwa_cached_layer_forward) on x bf16 [rows, H] into y f32
 * [rows, H], then x = bf16(x + y) (naiwa_residual_add_bf16), all on `stream`.
 * With lookahead_swaps >= 0 every layer but the last also predicts and loads the
 * next layer's experts (naiwa_cached_layer_forward_ahead).  No counterpart in the
 * reference, where the model's own layer loop calls each layer's forward
 * (src/moe/cached_layer.rs:524-531): a host that drives the layers itself calls the
 * per-layer entry points.  Every layer has the same hidden size.  *total sums the
 * layers' step reports and *ahead_total their lookahead reports (either may be NULL). */
int naiwa_cached_stack_forward(naiwa_cached_layer* const* layers, int n_layers, void* x, int rows, float* y,
                               float pcie_frac, int promote_cap, uint64_t min_hits, int lookahead_swaps,
                               int64_t stream, naiwa_cached_step* total, naiwa_lookahead_step* ahead_total);

/* The last lookahead's prediction for this layer, in vote order. */
int naiwa_cached_layer_predicted(const naiwa_cached_layer* L, uint32_t* ids, int capacity, int* n_out);

/* The last forward's routing: ids and weights [rows, k] (host copies). */
int naiwa_cached_layer_routing(const naiwa_cached_layer* L, uint32_t* ids, float* w, int capacity);

#ifdef __cplusplus
}
#endif
#endif
