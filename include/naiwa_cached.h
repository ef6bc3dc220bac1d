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
 * Misses the ring cannot take run on the CPU in the reference; this library
 * has no product CPU expert path, so a step that leaves any miss unstaged
 * fails with NAIWA_E_UNSUPPORTED (use pcie_frac 1 and a ring at least as long
 * as the step's distinct misses).
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
    const void* host_gate;    /* pinned stacked [E, I, H] bytes (expert e at e * expert bytes) */
    const void* host_up;
    const void* host_down;
    int num_experts, top_k, hidden, inter, usable, mode, act;
} naiwa_cached_layer_desc;

/* Per-step report of naiwa_cached_layer_forward. */
typedef struct naiwa_cached_step {
    int hits;        /* (row, k) pairs served from a cache slot */
    int staged;      /* pairs served from a staging slot */
    int staged_experts; /* distinct experts uploaded this step */
    int promoted;    /* experts copied staging -> cache */
    int64_t pcie_bytes;
    int preload_waits; /* 1 when the expert kernel waited for a lookahead claim */
} naiwa_cached_step;

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

/* One decode step: x bf16 [rows, H] -> out f32 [rows, H], all on `stream`
 * except the routing read-back, which synchronises it (the reference's
 * top-k round trip).  pcie_frac, promote_cap and min_hits are the
 * reference's --pcie-frac, NAIWA_PROMOTE_CAP and NAIWA_PROMOTE_MIN_HITS. */
int naiwa_cached_layer_forward(naiwa_cached_layer* L, const void* x, int rows, float* out, float pcie_frac,
                               int promote_cap, uint64_t min_hits, int64_t stream, naiwa_cached_step* info);

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
 * next != L and has L's hidden size. */
int naiwa_cached_layer_forward_ahead(naiwa_cached_layer* L, naiwa_cached_layer* next, int lookahead_swaps,
                                     const void* x, int rows, float* out, float pcie_frac, int promote_cap,
                                     uint64_t min_hits, int64_t stream, naiwa_cached_step* info,
                                     naiwa_lookahead_step* ahead);

/* The last lookahead's prediction for this layer, in vote order. */
int naiwa_cached_layer_predicted(const naiwa_cached_layer* L, uint32_t* ids, int capacity, int* n_out);

/* The last forward's routing: ids and weights [rows, k] (host copies). */
int naiwa_cached_layer_routing(const naiwa_cached_layer* L, uint32_t* ids, float* w, int capacity);

#ifdef __cplusplus
}
#endif
#endif
