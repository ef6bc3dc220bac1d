// Stable counting sort of keys into segments, by one block of 256 threads.
//
// Used by naiwa_moe_gather (keys = expert ids) and by the decode path (keys =
// cache slots, entries with router weight 0 left out).  Entries are grouped
// by key in ascending key order and keep their flat index order inside a
// group, so the permutation is the same on every run and equals the CPU
// counting sort bit for bit.
#pragma once

#include "common.h"

#define NAIWA_SEG_THREADS 256
#define NAIWA_SEG_MAX_KEYS 4096

// LDS: hist[NAIWA_SEG_MAX_KEYS] + per-wave key counts of one chunk + scan scratch.
struct NaiwaSegSmem {
    uint32_t hist[NAIWA_SEG_MAX_KEYS];
    uint16_t wcnt[NAIWA_SEG_THREADS / 64][NAIWA_SEG_MAX_KEYS]; // zero between chunks
    uint32_t part[NAIWA_SEG_THREADS];
    uint32_t bad;
};

// keys[n]; weights (may be null): an entry with weight 0 is skipped.
// Outputs (each may be null): perm[valid entries], offsets[nkeys + 1],
// seg_count[1], seg_key[segments], seg_begin[segments + 1], bad[1].
__device__ inline void naiwa_segment(NaiwaSegSmem& sm, const uint32_t* keys, const float* weights,
                                     int n, int nkeys, uint32_t* perm, uint32_t* offsets,
                                     int* seg_count, uint32_t* seg_key, uint32_t* seg_begin,
                                     int* bad) {
    const int tid = threadIdx.x;
    for (int b = tid; b < nkeys; b += NAIWA_SEG_THREADS) {
        sm.hist[b] = 0;
#pragma unroll
        for (int w = 0; w < NAIWA_SEG_THREADS / 64; ++w) sm.wcnt[w][b] = 0;
    }
    if (tid == 0) sm.bad = 0;
    __syncthreads();
    for (int i = tid; i < n; i += NAIWA_SEG_THREADS) {
        const uint32_t k = keys[i];
        if (k >= (uint32_t)nkeys) {
            atomicAdd(&sm.bad, 1u);
        } else if (!weights || weights[i] != 0.0f) {
            atomicAdd(&sm.hist[k], 1u);
        }
    }
    __syncthreads();
    // Exclusive scan of (count | nonempty << 17) over the keys: each thread
    // owns a contiguous run of ceil(nkeys/256) keys.
    const int per = (nkeys + NAIWA_SEG_THREADS - 1) / NAIWA_SEG_THREADS;
    const int k0 = tid * per, k1 = min(nkeys, k0 + per);
    uint32_t local = 0;
    for (int k = k0; k < k1; ++k) local += sm.hist[k] | ((sm.hist[k] ? 1u : 0u) << 17);
    sm.part[tid] = local;
    __syncthreads();
    // Hillis-Steele inclusive scan of the 256 run totals.
    for (int off = 1; off < NAIWA_SEG_THREADS; off <<= 1) {
        const uint32_t v = tid >= off ? sm.part[tid - off] : 0u;
        __syncthreads();
        sm.part[tid] += v;
        __syncthreads();
    }
    uint32_t run = tid ? sm.part[tid - 1] : 0u;
    const uint32_t total = sm.part[NAIWA_SEG_THREADS - 1];
    const uint32_t nvalid = total & 0x1ffffu, nseg = total >> 17;
    for (int k = k0; k < k1; ++k) {
        const uint32_t cnt = sm.hist[k];
        const uint32_t start = run & 0x1ffffu, segi = run >> 17;
        if (offsets) offsets[k] = start;
        if (cnt && seg_key) {
            seg_key[segi] = (uint32_t)k;
            seg_begin[segi] = start;
        }
        run += cnt | ((cnt ? 1u : 0u) << 17);
        sm.hist[k] = start; // becomes the running fill position
    }
    if (tid == 0) {
        if (offsets) offsets[nkeys] = nvalid;
        if (seg_count) *seg_count = (int)nseg;
        if (seg_begin) seg_begin[nseg] = nvalid;
        if (bad) *bad = (int)sm.bad;
    }
    __syncthreads();
    // Stable scatter, one chunk of 256 entries at a time.  An entry's rank among
    // the chunk's entries of its key = its rank inside its wave (one ballot per
    // distinct key of the wave) + the counts of that key in the lower waves.
    const int lane = tid & 63, wave = tid >> 6;
    const uint64_t below = (1ull << lane) - 1ull;
    for (int c0 = 0; c0 < n; c0 += NAIWA_SEG_THREADS) {
        const int i = c0 + tid;
        uint32_t k = 0xffffffffu;
        if (i < n) {
            const uint32_t kk = keys[i];
            if (kk < (uint32_t)nkeys && (!weights || weights[i] != 0.0f)) k = kk;
        }
        uint32_t rank = 0, lead_cnt = 0; // lead_cnt: the wave's count of k, on the key's first lane
        uint64_t todo = __ballot(k != 0xffffffffu);
        while (todo) {
            const int first = __ffsll((long long)todo) - 1;
            const uint32_t key = (uint32_t)__builtin_amdgcn_readlane((int)k, first);
            const uint64_t same = __ballot(k == key);
            if (k == key) rank = (uint32_t)__popcll(same & below);
            if (lane == first) lead_cnt = (uint32_t)__popcll(same);
            todo &= ~same;
        }
        if (lead_cnt) sm.wcnt[wave][k] = (uint16_t)lead_cnt;
        __syncthreads();
        if (k != 0xffffffffu) {
#pragma unroll
            for (int w = 0; w < NAIWA_SEG_THREADS / 64; ++w)
                if (w < wave) rank += sm.wcnt[w][k];
            if (perm) perm[sm.hist[k] + rank] = (uint32_t)i;
        }
        __syncthreads();
        if (lead_cnt) {
            atomicAdd(&sm.hist[k], lead_cnt);
            sm.wcnt[wave][k] = 0;
        }
        __syncthreads();
    }
}

// The same segmentation as naiwa_segment for at most 64 entries, by one wave with
// no LDS scratch: lane i ranks entry i against every other entry (a stable sort by
// key: lower key, or the same key at a lower index, comes first), so the outputs are
// naiwa_segment's bit for bit.  Every lane of the wave calls it; the outputs are
// written by the lanes that own them (perm[nvalid], seg_key/seg_begin[segments],
// seg_begin[segments], seg_count, bad).
__device__ inline void naiwa_segment_small(const uint32_t* keys, const float* weights, int n, int nkeys,
                                           uint32_t* perm, int* seg_count, uint32_t* seg_key, uint32_t* seg_begin,
                                           int* bad) {
    const int lane = threadIdx.x & 63;
    uint32_t k = 0xffffffffu; // invalid: past the keys, weight 0, or no entry
    bool isbad = false;
    if (lane < n) {
        const uint32_t kk = keys[lane];
        isbad = kk >= (uint32_t)nkeys;
        if (!isbad && (!weights || weights[lane] != 0.0f)) k = kk;
    }
    const bool valid = k != 0xffffffffu;
    // pass 1: rank among the valid entries, entries of lower keys, first occurrence
    uint32_t pos = 0, below_key = 0, seg_below = 0;
    bool first = valid;
    for (int j = 0; j < n; ++j) {
        const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)k, j);
        if (kj == 0xffffffffu) continue;
        if (kj < k) {
            ++pos;
            ++below_key;
        } else if (kj == k && j < lane) {
            ++pos;
            first = false;
        }
    }
    // pass 2: distinct keys below this one (first occurrences of lower keys)
    const uint64_t fm = __ballot(first);
    for (int j = 0; j < n; ++j)
        if ((fm >> j) & 1ull)
            if ((uint32_t)__builtin_amdgcn_readlane((int)k, j) < k) ++seg_below;
    const uint64_t vmask = __ballot(valid), fmask = __ballot(first);
    const int nvalid = __popcll(vmask), nseg = __popcll(fmask);
    if (valid) perm[pos] = (uint32_t)lane;
    if (first) {
        seg_key[seg_below] = k;
        seg_begin[seg_below] = below_key;
    }
    const int nbad = __popcll(__ballot(isbad));
    if (lane == 0) {
        seg_begin[nseg] = (uint32_t)nvalid;
        *seg_count = nseg;
        if (bad) *bad = nbad;
    }
}
