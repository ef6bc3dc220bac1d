/*
 * naiwa_policy.h -- host-side expert-cache policy of the MoE decode path.
 *
 * The reference keeps this logic in Rust under the layer lock; here it is C++
 * behind a C ABI, bit-exact with the reference's rules so a host that drives
 * the device kernels reproduces the same residency decisions step by step.
 * Everything here is host memory and host time: no call touches the GPU.
 *
 *   naiwa_cache_*           CachedLayer state and its policy:
 *                           Route::submit split    src/moe/stages/route.rs:19-158
 *                           fill_candidate         src/moe/cached_layer.rs:344-355
 *                           lru_victim             src/moe/cached_layer.rs:401-410
 *                           admit / replace        src/moe/cached_layer.rs:1056-1101
 *                           load_reserved publish  src/moe/cached_layer.rs:1103-1160
 *                           promote_staged pick    src/moe/cached_layer.rs:892-1051
 *   naiwa_top_k_ids         src/moe/cached_layer.rs:357-363
 *   naiwa_union_by_votes    src/moe/cached_layer.rs:367-379
 *   naiwa_streamed_misses   src/moe/cached_layer.rs:381-398
 *   naiwa_ring_*            StagingRing            src/moe/staging.rs:23-120
 *   naiwa_cache_stage       stage_misses selection src/moe/stages/dma_miss.rs:58-202
 *   naiwa_stats_*           CacheStats             src/stats/cache.rs:7-33
 *   naiwa_profile_*         Profile                src/moe/profile.rs:50-112
 *
 * Return values: NAIWA_OK (0) or a negative NAIWA_E_* code (naiwa_moe.h).
 * A cache object is not thread-safe by itself; the reference serialises the
 * same state with its layer mutex, and callers here do the same.
 */
#ifndef NAIWA_POLICY_H
#define NAIWA_POLICY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Slot ids at or above this value name staging-ring slots (src/moe/staging.rs:23). */
#define NAIWA_STAGING_RING_FIRST (1 << 30)

typedef struct naiwa_cache naiwa_cache;

/* One layer's expert cache: `slots` slots of which the first `usable` may hold
 * experts, every slot empty, tick 0, hit counts 0. */
int naiwa_cache_create(int num_experts, int slots, int usable, naiwa_cache** out);
int naiwa_cache_destroy(naiwa_cache* c);

/* Route::submit: tick += 1, then for every (row, j) in row-major order
 * hit_counts[id] += 1; the first published slot holding id is a hit (its
 * last_use = tick), otherwise a miss.  slot_out[row * k + j] = the slot, or -1
 * for a miss.  An id >= num_experts fails the whole call (NAIWA_E_BAD_ID)
 * before any state changes, as the reference bails. */
int naiwa_cache_route(naiwa_cache* c, const uint32_t* ids, int rows, int k, int32_t* slot_out);

/* fill_candidate: the expert with the most hits that is not in a slot (ties to
 * the lowest id); *found = 0 when every slot holds an expert or every expert
 * is placed. */
int naiwa_cache_fill_candidate(const naiwa_cache* c, int* expert_out, int* found);

/* lru_victim: the published resident outside `protect` with the smallest
 * (last_use, expert), as (expert, slot); *found = 0 when none. */
int naiwa_cache_lru_victim(const naiwa_cache* c, const int32_t* protect, int n_protect, int* expert_out,
                           int* slot_out, int* found);

/* admit: reserve the first empty slot in [0, usable) for `expert` (unpublished
 * until naiwa_cache_publish).  *slot_out = -1 when the expert is already in a
 * slot or no slot is empty. */
int naiwa_cache_admit(naiwa_cache* c, int expert, int* slot_out);

/* replace: unpublish the LRU victim outside `protect` and reserve its slot for
 * `expert`; *slot_out = -1 when the expert is already in a slot or no victim. */
int naiwa_cache_replace(naiwa_cache* c, int expert, const int32_t* protect, int n_protect, int* slot_out);

/* The reserved slot's copy finished: publish it with last_use = tick. */
int naiwa_cache_publish(naiwa_cache* c, int slot);
/* The reserved slot's copy failed: free it. */
int naiwa_cache_unreserve(naiwa_cache* c, int slot);

/* promote_staged selection: the staged experts in id order, each once; skip
 * those already in a slot and those with hit_counts < min_hits; target the
 * first empty usable slot, else the published usable slot with the smallest
 * (last_use, slot) among those with last_use < tick; at most `cap`.  Each pick
 * is reserved (expert set, unpublished); the caller copies staging -> slot on
 * the compute stream and then publishes.  Writes n_out pairs. */
int naiwa_cache_promote_pick(naiwa_cache* c, const uint32_t* staged, int n_staged, int cap, uint64_t min_hits,
                             int32_t* expert_out, int32_t* slot_out, int* n_out);

/* Per-expert device table: slot of each published expert, -1 otherwise. */
int naiwa_cache_slot_table(const naiwa_cache* c, int32_t* slot_of_expert);

/* State inspection (tests, mirrors): per slot expert (-1 empty), published,
 * last_use; hit counts; tick. */
int naiwa_cache_slot_state(const naiwa_cache* c, int slot, int* expert, int* published, uint64_t* last_use);
int naiwa_cache_hit_counts(const naiwa_cache* c, uint64_t* out);
int naiwa_cache_tick(const naiwa_cache* c, uint64_t* tick);
/* Replace the hit counts (expert-profile seeding, src/moe/profile.rs). */
int naiwa_cache_seed_hits(naiwa_cache* c, const uint64_t* counts);
/* Put an expert straight into a slot as published (warm-up / profile seeding). */
int naiwa_cache_place(naiwa_cache* c, int expert, int slot, uint64_t last_use);

/* top_k_ids: indices of the k largest logits by the IEEE total order, largest
 * first, ties to the lowest index; min(k, n) written. */
int naiwa_top_k_ids(const float* logits, int n, int k, uint32_t* out, int* n_out);

/* union_by_votes: every id in the rankings once, by votes desc, best rank asc,
 * id asc.  rankings = concatenation, lens[i] = length of ranking i. */
int naiwa_union_by_votes(const uint32_t* rankings, const int* lens, int n_rankings, uint32_t* out, int out_cap,
                         int* n_out);

/* streamed_misses: the distinct missed ids (pairs in row-major order), their
 * router weights summed per id in that order in f32, take = min(ceil(frac *
 * distinct), cap), ranked by weight desc (total order) then id asc. */
int naiwa_streamed_misses(const uint32_t* ids, const float* w, int n, float frac, int cap, uint32_t* out,
                          int* n_out);

/* The staging ring: `len` slots borrowed round-robin. */
typedef struct naiwa_ring naiwa_ring;
int naiwa_staging_ring_slots(void); /* 16, the reference's fixed ring size */
int naiwa_ring_create(int len, naiwa_ring** out);
int naiwa_ring_destroy(naiwa_ring* r);
/* acquire: start = cursor; cursor = (cursor + n) % len.  n <= len. */
int naiwa_ring_acquire(naiwa_ring* r, int n, int* start);

/* stage_misses selection: from the misses of a routed step (slot_io == -1 for
 * a miss, as naiwa_cache_route writes), choose naiwa_streamed_misses(frac,
 * ring length), acquire that many ring slots, and turn every miss of a chosen
 * id into a hit on NAIWA_STAGING_RING_FIRST + its ring position (in slot_io).
 * chosen_out[i] is staged into ring position pos_out[i]; the caller uploads
 * it there before any kernel reads the step. */
int naiwa_cache_stage(naiwa_ring* r, const uint32_t* ids, const float* w, int rows, int k, float frac,
                      int32_t* slot_io, uint32_t* chosen_out, int32_t* pos_out, int* n_chosen);

/* A step's split without doing it: what naiwa_cache_route followed by
 * naiwa_cache_stage (ring of ring_len slots) would report for these ids and
 * weights -- pairs on a published slot, pairs of the misses chosen for the
 * ring, the chosen experts, and the pairs left to the CPU -- with no state
 * changed (tick, hit counts, last_use and the ring cursor stay as they are).
 * No counterpart in the reference; the partial-cache step checks with it
 * before it commits a step it could not finish. */
typedef struct naiwa_step_plan {
    int hits, staged, staged_experts, cpu;
} naiwa_step_plan;
int naiwa_cache_plan(const naiwa_cache* c, int ring_len, const uint32_t* ids, const float* w, int rows, int k,
                     float frac, naiwa_step_plan* out);

/* The expert-cache profile (src/moe/profile.rs:50-112): a file of (layer,
 * expert) pairs ranked best first ("STRP", u32 version 1, layers, experts,
 * slots, n, then n u16 pairs; the trailing rank table is not read).  Each
 * layer keeps its own pairs in rank order; pairs with layer >= num_layers or
 * expert >= num_experts are dropped, and a repeated pair is kept once.
 * Errors: NAIWA_E_IO (cannot open), NAIWA_E_FORMAT (no magic / shorter than
 * its header, or a truncated ranking), NAIWA_E_UNSUPPORTED (version != 1). */
typedef struct naiwa_profile naiwa_profile;
int naiwa_profile_read(const char* path, int num_layers, int num_experts, naiwa_profile** out);
int naiwa_profile_destroy(naiwa_profile* p);
/* This layer's experts, best first (a layer the profile lacks: none). */
int naiwa_profile_layer(const naiwa_profile* p, int layer, uint32_t* experts, int capacity, int* n_out);
/* Pairs kept after the filter, and the file's own header sizes (any may be null). */
int naiwa_profile_info(const naiwa_profile* p, int* pairs, uint32_t* file_layers, uint32_t* file_experts,
                       uint32_t* file_pairs);

/* CacheStats (src/stats/cache.rs:7-33), process-wide. */
typedef struct naiwa_cache_stats {
    uint64_t hits, promotions, misses, staged, lookahead_loads, swaps, lookahead_dropped, sync_waits,
        pcie_misses, pcie_bytes, result_stalls;
} naiwa_cache_stats;
int naiwa_stats_read(naiwa_cache_stats* out, int reset);
/* Add to the counters (a caller that moves experts records what it did). */
int naiwa_stats_add(const naiwa_cache_stats* delta);

#ifdef __cplusplus
}
#endif
#endif
