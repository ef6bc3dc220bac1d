/*
 * naiwa_cached.h -- one MoE layer's decode step over a partial expert cache.
 *
 * The counterpart of the reference's CachedExperts::forward for decode rows
 * (src/moe/decode.rs:241-381 with the stages of src/moe/stages/): route on the
 * device, read the top-k back, split hits from misses with the host policy
 * (include/naiwa_policy.h), stream the chosen misses over PCIe into the
 * staging-ring slots of the layer's banks (src/moe/stages/dma_miss.rs:58-202),
 * run the expert kernel over resident + staged slots, then promote staged
 * experts into the cache (src/moe/cached_layer.rs:892-1051).
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
} naiwa_cached_step;

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

/* One decode step: x bf16 [rows, H] -> out f32 [rows, H], all on `stream`
 * except the routing read-back, which synchronises it (the reference's
 * top-k round trip).  pcie_frac, promote_cap and min_hits are the
 * reference's --pcie-frac, NAIWA_PROMOTE_CAP and NAIWA_PROMOTE_MIN_HITS. */
int naiwa_cached_layer_forward(naiwa_cached_layer* L, const void* x, int rows, float* out, float pcie_frac,
                               int promote_cap, uint64_t min_hits, int64_t stream, naiwa_cached_step* info);

/* The last forward's routing: ids and weights [rows, k] (host copies). */
int naiwa_cached_layer_routing(const naiwa_cached_layer* L, uint32_t* ids, float* w, int capacity);

#ifdef __cplusplus
}
#endif
#endif
