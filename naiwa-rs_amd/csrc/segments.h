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

// LDS: hist[NAIWA_SEG_MAX_KEYS] + chunk[NAIWA_SEG_THREADS] + scan scratch.
struct NaiwaSegSmem {
    uint32_t hist[NAIWA_SEG_MAX_KEYS];
    uint32_t chunk[NAIWA_SEG_THREADS];
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
    for (int b = tid; b < nkeys; b += NAIWA_SEG_THREADS) sm.hist[b] = 0;
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
    // Stable scatter, one chunk of 256 entries at a time.
    for (int c0 = 0; c0 < n; c0 += NAIWA_SEG_THREADS) {
        const int i = c0 + tid;
        uint32_t k = 0xffffffffu;
        if (i < n) {
            const uint32_t kk = keys[i];
            if (kk < (uint32_t)nkeys && (!weights || weights[i] != 0.0f)) k = kk;
        }
        sm.chunk[tid] = k;
        __syncthreads();
        uint32_t rank = 0;
        bool last = true;
        if (k != 0xffffffffu) {
            for (int j = 0; j < tid; ++j) rank += sm.chunk[j] == k;
            for (int j = tid + 1; j < NAIWA_SEG_THREADS; ++j)
                if (sm.chunk[j] == k) { last = false; break; }
            if (perm) perm[sm.hist[k] + rank] = (uint32_t)i;
        }
        __syncthreads();
        if (k != 0xffffffffu && last) sm.hist[k] += rank + 1;
        __syncthreads();
    }
}
