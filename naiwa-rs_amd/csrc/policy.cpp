// Host-side expert-cache policy (include/naiwa_policy.h): residency state of
// one MoE layer's slot cache and the rules that move experts in and out of it.
// Pure host code; every decision is a deterministic function of the state and
// the routed ids, like the reference's (src/moe/cached_layer.rs,
// src/moe/stages/route.rs, src/moe/stages/dma_miss.rs, src/moe/staging.rs).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/naiwa_moe.h"
#include "../../include/naiwa_policy.h"

namespace {

struct Slot {
    int expert = -1;        // -1: empty
    bool published = false; // a copy has completed: kernels may read it
    uint64_t last_use = 0;
};

// IEEE-754 total order key of an f32 (the order of Rust's f32::total_cmp).
int32_t total_key(float f) {
    int32_t k;
    std::memcpy(&k, &f, 4);
    return k ^ (int32_t)((uint32_t)(k >> 31) >> 1);
}

bool in_list(const int32_t* list, int n, int v) {
    for (int i = 0; i < n; ++i)
        if (list[i] == v) return true;
    return false;
}

std::mutex g_stats_mu;
naiwa_cache_stats g_stats{};

} // namespace

struct naiwa_cache {
    int num_experts = 0;
    int usable = 0;
    uint64_t tick = 0;
    std::vector<Slot> slots;
    std::vector<uint64_t> hit_counts;

    int slot_of(int expert) const { // any slot holding the expert, published or reserved
        for (size_t s = 0; s < slots.size(); ++s)
            if (slots[s].expert == expert) return (int)s;
        return -1;
    }
    int published_slot_of(int expert) const {
        for (size_t s = 0; s < slots.size(); ++s)
            if (slots[s].expert == expert && slots[s].published) return (int)s;
        return -1;
    }
    int first_empty_usable() const {
        for (int s = 0; s < usable; ++s)
            if (slots[s].expert < 0) return s;
        return -1;
    }
    // (expert, slot) of the published resident outside protect with the
    // smallest (last_use, expert)
    bool lru(const int32_t* protect, int n_protect, int* expert, int* slot) const {
        bool found = false;
        for (size_t s = 0; s < slots.size(); ++s) {
            const Slot& x = slots[s];
            if (x.expert < 0 || !x.published || in_list(protect, n_protect, x.expert)) continue;
            if (!found || x.last_use < slots[*slot].last_use ||
                (x.last_use == slots[*slot].last_use && x.expert < *expert)) {
                *expert = x.expert;
                *slot = (int)s;
                found = true;
            }
        }
        return found;
    }
};

struct naiwa_ring {
    int len = 0;
    int cursor = 0;
};

extern "C" {

int naiwa_cache_create(int num_experts, int slots, int usable, naiwa_cache** out) {
    if (!out || num_experts <= 0 || slots < 0 || usable < 0 || usable > slots) return NAIWA_E_INVALID;
    naiwa_cache* c = new (std::nothrow) naiwa_cache;
    if (!c) return NAIWA_E_NOMEM;
    c->num_experts = num_experts;
    c->usable = usable;
    c->slots.assign((size_t)slots, Slot{});
    c->hit_counts.assign((size_t)num_experts, 0);
    *out = c;
    return NAIWA_OK;
}

int naiwa_cache_destroy(naiwa_cache* c) {
    delete c;
    return NAIWA_OK;
}

int naiwa_cache_route(naiwa_cache* c, const uint32_t* ids, int rows, int k, int32_t* slot_out) {
    if (!c || rows < 0 || k <= 0 || (rows > 0 && (!ids || !slot_out))) return NAIWA_E_INVALID;
    const int n = rows * k;
    for (int i = 0; i < n; ++i)
        if (ids[i] >= (uint32_t)c->num_experts) return NAIWA_E_BAD_ID;
    const uint64_t tick = ++c->tick;
    for (int i = 0; i < n; ++i) {
        const int id = (int)ids[i];
        c->hit_counts[id] += 1;
        const int s = c->published_slot_of(id);
        if (s >= 0) c->slots[s].last_use = tick;
        slot_out[i] = s;
    }
    return NAIWA_OK;
}

int naiwa_cache_fill_candidate(const naiwa_cache* c, int* expert_out, int* found) {
    if (!c || !expert_out || !found) return NAIWA_E_INVALID;
    *found = 0;
    bool all_taken = true;
    for (const Slot& s : c->slots) all_taken &= s.expert >= 0;
    if (all_taken) return NAIWA_OK;
    std::vector<char> taken((size_t)c->num_experts, 0);
    for (const Slot& s : c->slots)
        if (s.expert >= 0 && s.expert < c->num_experts) taken[s.expert] = 1;
    for (int e = 0; e < c->num_experts; ++e) {
        if (taken[e]) continue;
        if (!*found || c->hit_counts[e] > c->hit_counts[*expert_out]) { // ties keep the lower id
            *expert_out = e;
            *found = 1;
        }
    }
    return NAIWA_OK;
}

int naiwa_cache_lru_victim(const naiwa_cache* c, const int32_t* protect, int n_protect, int* expert_out,
                           int* slot_out, int* found) {
    if (!c || !expert_out || !slot_out || !found || n_protect < 0 || (n_protect > 0 && !protect))
        return NAIWA_E_INVALID;
    *found = c->lru(protect, n_protect, expert_out, slot_out) ? 1 : 0;
    return NAIWA_OK;
}

int naiwa_cache_admit(naiwa_cache* c, int expert, int* slot_out) {
    if (!c || !slot_out) return NAIWA_E_INVALID;
    if (expert < 0 || expert >= c->num_experts) return NAIWA_E_BAD_ID;
    *slot_out = -1;
    if (c->slot_of(expert) >= 0) return NAIWA_OK;
    const int s = c->first_empty_usable();
    if (s < 0) return NAIWA_OK;
    c->slots[s].expert = expert;
    c->slots[s].published = false;
    *slot_out = s;
    return NAIWA_OK;
}

int naiwa_cache_replace(naiwa_cache* c, int expert, const int32_t* protect, int n_protect, int* slot_out) {
    if (!c || !slot_out || n_protect < 0 || (n_protect > 0 && !protect)) return NAIWA_E_INVALID;
    if (expert < 0 || expert >= c->num_experts) return NAIWA_E_BAD_ID;
    *slot_out = -1;
    if (c->slot_of(expert) >= 0) return NAIWA_OK;
    int victim = -1, s = -1;
    if (!c->lru(protect, n_protect, &victim, &s)) return NAIWA_OK;
    c->slots[s].expert = expert;
    c->slots[s].published = false;
    *slot_out = s;
    return NAIWA_OK;
}

int naiwa_cache_publish(naiwa_cache* c, int slot) {
    if (!c || slot < 0 || slot >= (int)c->slots.size() || c->slots[slot].expert < 0) return NAIWA_E_INVALID;
    c->slots[slot].published = true;
    c->slots[slot].last_use = c->tick;
    return NAIWA_OK;
}

int naiwa_cache_unreserve(naiwa_cache* c, int slot) {
    if (!c || slot < 0 || slot >= (int)c->slots.size()) return NAIWA_E_INVALID;
    c->slots[slot].expert = -1;
    c->slots[slot].published = false;
    return NAIWA_OK;
}

int naiwa_cache_promote_pick(naiwa_cache* c, const uint32_t* staged, int n_staged, int cap, uint64_t min_hits,
                             int32_t* expert_out, int32_t* slot_out, int* n_out) {
    if (!c || !n_out || n_staged < 0 || cap < 0 || (n_staged > 0 && !staged) ||
        (cap > 0 && (!expert_out || !slot_out)))
        return NAIWA_E_INVALID;
    *n_out = 0;
    for (int i = 0; i < n_staged; ++i)
        if (staged[i] >= (uint32_t)c->num_experts) return NAIWA_E_BAD_ID;
    if (cap == 0 || n_staged == 0) return NAIWA_OK;
    std::vector<uint32_t> order(staged, staged + n_staged);
    std::sort(order.begin(), order.end());
    int promoted = 0;
    for (size_t i = 0; i < order.size() && promoted < cap; ++i) {
        if (i > 0 && order[i] == order[i - 1]) continue; // each staged expert once
        const int e = (int)order[i];
        if (c->slot_of(e) >= 0) continue;                 // already resident or reserved
        if (c->hit_counts[e] < min_hits) continue;        // not asked for often enough
        int s = c->first_empty_usable();
        if (s < 0) {
            // the least recently used usable slot that this step did not read
            for (int t = 0; t < c->usable; ++t) {
                const Slot& x = c->slots[t];
                if (x.expert < 0 || !x.published || x.last_use >= c->tick) continue;
                if (s < 0 || x.last_use < c->slots[s].last_use) s = t; // ties keep the lower slot
            }
        }
        if (s < 0) continue;
        c->slots[s].expert = e;
        c->slots[s].published = false;
        expert_out[promoted] = e;
        slot_out[promoted] = s;
        ++promoted;
    }
    *n_out = promoted;
    return NAIWA_OK;
}

int naiwa_cache_slot_table(const naiwa_cache* c, int32_t* slot_of_expert) {
    if (!c || !slot_of_expert) return NAIWA_E_INVALID;
    for (int e = 0; e < c->num_experts; ++e) slot_of_expert[e] = -1;
    for (size_t s = 0; s < c->slots.size(); ++s) {
        const Slot& x = c->slots[s];
        if (x.expert >= 0 && x.published) slot_of_expert[x.expert] = (int32_t)s;
    }
    return NAIWA_OK;
}

int naiwa_cache_slot_state(const naiwa_cache* c, int slot, int* expert, int* published, uint64_t* last_use) {
    if (!c || slot < 0 || slot >= (int)c->slots.size()) return NAIWA_E_INVALID;
    if (expert) *expert = c->slots[slot].expert;
    if (published) *published = c->slots[slot].published ? 1 : 0;
    if (last_use) *last_use = c->slots[slot].last_use;
    return NAIWA_OK;
}

int naiwa_cache_hit_counts(const naiwa_cache* c, uint64_t* out) {
    if (!c || !out) return NAIWA_E_INVALID;
    std::copy(c->hit_counts.begin(), c->hit_counts.end(), out);
    return NAIWA_OK;
}

int naiwa_cache_seed_hits(naiwa_cache* c, const uint64_t* counts) {
    if (!c || !counts) return NAIWA_E_INVALID;
    std::copy(counts, counts + c->num_experts, c->hit_counts.begin());
    return NAIWA_OK;
}

int naiwa_cache_tick(const naiwa_cache* c, uint64_t* tick) {
    if (!c || !tick) return NAIWA_E_INVALID;
    *tick = c->tick;
    return NAIWA_OK;
}

int naiwa_cache_place(naiwa_cache* c, int expert, int slot, uint64_t last_use) {
    if (!c || slot < 0 || slot >= (int)c->slots.size()) return NAIWA_E_INVALID;
    if (expert < 0 || expert >= c->num_experts) return NAIWA_E_BAD_ID;
    const int other = c->slot_of(expert);
    if (other >= 0 && other != slot) return NAIWA_E_INVALID;
    c->slots[slot].expert = expert;
    c->slots[slot].published = true;
    c->slots[slot].last_use = last_use;
    return NAIWA_OK;
}

int naiwa_top_k_ids(const float* logits, int n, int k, uint32_t* out, int* n_out) {
    if (n < 0 || k < 0 || (n > 0 && !logits) || (k > 0 && n > 0 && !out)) return NAIWA_E_INVALID;
    std::vector<uint32_t> ids((size_t)n);
    for (int i = 0; i < n; ++i) ids[i] = (uint32_t)i;
    std::stable_sort(ids.begin(), ids.end(), [&](uint32_t a, uint32_t b) {
        const int32_t ka = total_key(logits[a]), kb = total_key(logits[b]);
        return ka != kb ? ka > kb : a < b;
    });
    const int m = std::min(k, n);
    std::copy(ids.begin(), ids.begin() + m, out);
    if (n_out) *n_out = m;
    return NAIWA_OK;
}

int naiwa_union_by_votes(const uint32_t* rankings, const int* lens, int n_rankings, uint32_t* out, int out_cap,
                         int* n_out) {
    if (n_rankings < 0 || (n_rankings > 0 && !lens) || !n_out) return NAIWA_E_INVALID;
    struct Entry {
        uint32_t id;
        int votes;
        int best;
    };
    std::vector<Entry> seen;
    size_t pos = 0;
    for (int r = 0; r < n_rankings; ++r) {
        if (lens[r] < 0 || (lens[r] > 0 && !rankings)) return NAIWA_E_INVALID;
        for (int i = 0; i < lens[r]; ++i) {
            const uint32_t id = rankings[pos + i];
            auto it = std::find_if(seen.begin(), seen.end(), [&](const Entry& x) { return x.id == id; });
            if (it == seen.end()) {
                seen.push_back({id, 1, i});
            } else {
                it->votes += 1;
                it->best = std::min(it->best, i);
            }
        }
        pos += (size_t)lens[r];
    }
    std::sort(seen.begin(), seen.end(), [](const Entry& a, const Entry& b) {
        if (a.votes != b.votes) return a.votes > b.votes;
        if (a.best != b.best) return a.best < b.best;
        return a.id < b.id;
    });
    if ((int)seen.size() > out_cap || (!seen.empty() && !out)) return NAIWA_E_INVALID;
    for (size_t i = 0; i < seen.size(); ++i) out[i] = seen[i].id;
    *n_out = (int)seen.size();
    return NAIWA_OK;
}

int naiwa_streamed_misses(const uint32_t* ids, const float* w, int n, float frac, int cap, uint32_t* out,
                          int* n_out) {
    if (n < 0 || (n > 0 && (!ids || !w)) || !n_out || cap < 0) return NAIWA_E_INVALID;
    *n_out = 0;
    if (!(frac > 0.0f) || cap == 0) return NAIWA_OK;
    // per-id sums in order of first appearance, each summed in row-major order
    std::vector<std::pair<uint32_t, float>> weight;
    for (int i = 0; i < n; ++i) {
        auto it = std::find_if(weight.begin(), weight.end(), [&](const auto& x) { return x.first == ids[i]; });
        if (it == weight.end()) weight.push_back({ids[i], w[i]});
        else it->second += w[i];
    }
    const size_t take = std::min((size_t)std::ceil(frac * (float)weight.size()), (size_t)cap);
    std::sort(weight.begin(), weight.end(), [](const auto& a, const auto& b) {
        const int32_t ka = total_key(a.second), kb = total_key(b.second);
        return ka != kb ? ka > kb : a.first < b.first;
    });
    if (take > 0 && !out) return NAIWA_E_INVALID;
    for (size_t i = 0; i < take && i < weight.size(); ++i) out[i] = weight[i].first;
    *n_out = (int)std::min(take, weight.size());
    return NAIWA_OK;
}

int naiwa_staging_ring_slots(void) { return 16; }

int naiwa_ring_create(int len, naiwa_ring** out) {
    if (!out || len <= 0) return NAIWA_E_INVALID;
    naiwa_ring* r = new (std::nothrow) naiwa_ring;
    if (!r) return NAIWA_E_NOMEM;
    r->len = len;
    *out = r;
    return NAIWA_OK;
}

int naiwa_ring_destroy(naiwa_ring* r) {
    delete r;
    return NAIWA_OK;
}

int naiwa_ring_acquire(naiwa_ring* r, int n, int* start) {
    if (!r || !start || n < 0 || n > r->len) return NAIWA_E_INVALID;
    *start = r->cursor;
    r->cursor = (r->cursor + n) % r->len;
    return NAIWA_OK;
}

int naiwa_cache_stage(naiwa_ring* r, const uint32_t* ids, const float* w, int rows, int k, float frac,
                      int32_t* slot_io, uint32_t* chosen_out, int32_t* pos_out, int* n_chosen) {
    if (!r || !n_chosen || rows < 0 || k <= 0 || (rows > 0 && (!ids || !w || !slot_io))) return NAIWA_E_INVALID;
    *n_chosen = 0;
    const int n = rows * k;
    std::vector<uint32_t> mid;
    std::vector<float> mw;
    for (int i = 0; i < n; ++i)
        if (slot_io[i] < 0) {
            mid.push_back(ids[i]);
            mw.push_back(w[i]);
        }
    std::vector<uint32_t> chosen((size_t)r->len);
    int nc = 0;
    int rc = naiwa_streamed_misses(mid.data(), mw.data(), (int)mid.size(), frac, r->len, chosen.data(), &nc);
    if (rc) return rc;
    if (nc == 0) return NAIWA_OK;
    if (!chosen_out || !pos_out) return NAIWA_E_INVALID;
    int start = 0;
    if ((rc = naiwa_ring_acquire(r, nc, &start))) return rc;
    for (int i = 0; i < nc; ++i) {
        chosen_out[i] = chosen[i];
        pos_out[i] = (start + i) % r->len;
    }
    for (int i = 0; i < n; ++i) {
        if (slot_io[i] >= 0) continue;
        for (int j = 0; j < nc; ++j)
            if (ids[i] == chosen[j]) {
                slot_io[i] = NAIWA_STAGING_RING_FIRST + pos_out[j];
                break;
            }
    }
    *n_chosen = nc;
    return NAIWA_OK;
}

int naiwa_cache_plan(const naiwa_cache* c, int ring_len, const uint32_t* ids, const float* w, int rows, int k,
                     float frac, naiwa_step_plan* out) {
    if (!c || !out || ring_len < 0 || rows < 0 || k <= 0 || (rows > 0 && (!ids || !w))) return NAIWA_E_INVALID;
    *out = naiwa_step_plan{};
    const int n = rows * k;
    for (int i = 0; i < n; ++i)
        if (ids[i] >= (uint32_t)c->num_experts) return NAIWA_E_BAD_ID;
    // the split of naiwa_cache_route (published slot or miss) and the choice of
    // naiwa_cache_stage (streamed_misses over the misses), with no state touched
    std::vector<uint32_t> mid;
    std::vector<float> mw;
    for (int i = 0; i < n; ++i) {
        if (c->published_slot_of((int)ids[i]) >= 0) {
            ++out->hits;
        } else {
            mid.push_back(ids[i]);
            mw.push_back(w[i]);
        }
    }
    std::vector<uint32_t> chosen((size_t)std::max(ring_len, 1));
    int nc = 0;
    int rc = naiwa_streamed_misses(mid.data(), mw.data(), (int)mid.size(), frac, ring_len, chosen.data(), &nc);
    if (rc) return rc;
    out->staged_experts = nc;
    for (uint32_t e : mid) {
        if (std::find(chosen.begin(), chosen.begin() + nc, e) != chosen.begin() + nc)
            ++out->staged;
        else
            ++out->cpu;
    }
    return NAIWA_OK;
}

int naiwa_stats_read(naiwa_cache_stats* out, int reset) {
    if (!out) return NAIWA_E_INVALID;
    std::lock_guard<std::mutex> lock(g_stats_mu);
    *out = g_stats;
    if (reset) g_stats = naiwa_cache_stats{};
    return NAIWA_OK;
}

int naiwa_stats_add(const naiwa_cache_stats* d) {
    if (!d) return NAIWA_E_INVALID;
    std::lock_guard<std::mutex> lock(g_stats_mu);
    g_stats.hits += d->hits;
    g_stats.promotions += d->promotions;
    g_stats.misses += d->misses;
    g_stats.staged += d->staged;
    g_stats.lookahead_loads += d->lookahead_loads;
    g_stats.swaps += d->swaps;
    g_stats.lookahead_dropped += d->lookahead_dropped;
    g_stats.sync_waits += d->sync_waits;
    g_stats.pcie_misses += d->pcie_misses;
    g_stats.pcie_bytes += d->pcie_bytes;
    g_stats.result_stalls += d->result_stalls;
    return NAIWA_OK;
}

} // extern "C"
