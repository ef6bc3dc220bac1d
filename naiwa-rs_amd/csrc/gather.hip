// naiwa_moe_gather: the token->expert gather as a stable counting sort by
// expert id.  The reference groups hits per bank in row-major order
// (src/moe/stages/gpu.rs:100-133); here every (token, k) pair of a step is
// grouped by expert id, ties kept in flat index order, so the permutation and
// the per-expert offsets are bit-exact against the CPU counting sort.
#include "segments.h"

namespace {

__global__ void __launch_bounds__(NAIWA_SEG_THREADS)
gather_kernel(const uint32_t* ids, int n, int E, uint32_t* perm, uint32_t* offsets, int* bad) {
    __shared__ NaiwaSegSmem sm;
    naiwa_segment(sm, ids, nullptr, n, E, perm, offsets, nullptr, nullptr, nullptr, bad);
}

// The same stable counting sort with one block per expert id e: its segment
// starts at the number of valid ids below e, and its entries keep their flat
// order by a block-wide running count of (id == e) over chunks of 256 entries.
// O(n) per block, all ids in parallel: for many entries and few ids (a prefill
// chunk's routing) it replaces the one-block sort's serial chunks.
constexpr int kExpertThreads = 256;

constexpr int kIdsPerThread = 32; // ids a thread keeps in registers (calls of up to 8192 entries)

template <bool CACHED>
__global__ void __launch_bounds__(kExpertThreads)
gather_by_id_kernel(const uint32_t* ids, int n, int E, uint32_t* perm, uint32_t* offsets, int* bad) {
    __shared__ uint32_t wsum[kExpertThreads / 64];
    __shared__ uint32_t wsum2[kExpertThreads / 64];
    const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // entry tid + 256 r: its id, read once (CACHED: all of this thread's loads issued
    // together, then kept for the second pass)
    uint32_t cache[CACHED ? kIdsPerThread : 1];
    if (CACHED) {
#pragma unroll
        for (int r = 0; r < kIdsPerThread; ++r) {
            const int i = tid + kExpertThreads * r;
            cache[r] = i < n ? ids[i] : 0u;
        }
    }
    // valid ids below e, and ids outside [0, E) (block 0 reports them)
    uint32_t below = 0, outside = 0;
    auto count = [&](uint32_t v) {
        below += v < (uint32_t)e;
        outside += v >= (uint32_t)E;
    };
    if constexpr (CACHED) {
#pragma unroll
        for (int r = 0; r < kIdsPerThread; ++r)
            if (tid + kExpertThreads * r < n) count(cache[r]);
    } else {
        for (int i = tid; i < n; i += kExpertThreads) count(ids[i]);
    }
    for (int m = 32; m >= 1; m >>= 1) {
        below += __shfl_xor(below, m, 64);
        outside += __shfl_xor(outside, m, 64);
    }
    if (lane == 0) {
        wsum[wave] = below;
        wsum2[wave] = outside;
    }
    __syncthreads();
    uint32_t start = 0, nbad = 0;
#pragma unroll
    for (int w = 0; w < kExpertThreads / 64; ++w) {
        start += wsum[w];
        nbad += wsum2[w];
    }
    __syncthreads();
    const uint64_t lower = (1ull << lane) - 1ull;
    uint32_t run = 0;
    // entries in chunks of 256: each block-wide chunk keeps the positions stable
    auto chunk = [&](int i, uint32_t v) {
        const bool mine = i < n && v == (uint32_t)e;
        const uint64_t m = __ballot(mine);
        if (lane == 0) wsum[wave] = (uint32_t)__popcll(m);
        __syncthreads();
        uint32_t before = run;
#pragma unroll
        for (int w = 0; w < kExpertThreads / 64; ++w) {
            if (w < wave) before += wsum[w];
            run += wsum[w];
        }
        if (mine && perm) perm[start + before + (uint32_t)__popcll(m & lower)] = (uint32_t)i;
        __syncthreads();
    };
    if constexpr (CACHED) {
#pragma unroll
        for (int r = 0; r < kIdsPerThread; ++r) {
            if (kExpertThreads * r >= n) break; // uniform
            chunk(tid + kExpertThreads * r, cache[r]);
        }
    } else {
        for (int c0 = 0; c0 < n; c0 += kExpertThreads) {
            const int i = c0 + tid;
            chunk(i, i < n ? ids[i] : 0u);
        }
    }
    if (tid == 0) {
        offsets[e] = start;
        if (e == E - 1) offsets[E] = start + run;
        if (e == 0 && bad) *bad = (int)nbad;
    }
}

} // namespace

extern "C" int naiwa_moe_gather(const uint32_t* ids, int n, int E, uint32_t* perm_out,
                                uint32_t* offsets_out, int* bad_out, int64_t stream) {
    if (n < 0 || n > 65536 || E <= 0 || E > NAIWA_SEG_MAX_KEYS) return NAIWA_E_INVALID;
    if (!offsets_out || (n > 0 && (!ids || !perm_out))) return NAIWA_E_INVALID;
    // one block per id while that stays cheap (every block reads all n ids), else one block
    if (n > NAIWA_SEG_THREADS && (int64_t)n * E <= (int64_t)1 << 24) {
        if (n <= kExpertThreads * kIdsPerThread)
            gather_by_id_kernel<true><<<E, kExpertThreads, 0, (hipStream_t)stream>>>(ids, n, E, perm_out,
                                                                                    offsets_out, bad_out);
        else
            gather_by_id_kernel<false><<<E, kExpertThreads, 0, (hipStream_t)stream>>>(ids, n, E, perm_out,
                                                                                     offsets_out, bad_out);
    } else
        gather_kernel<<<1, NAIWA_SEG_THREADS, 0, (hipStream_t)stream>>>(ids, n, E, perm_out, offsets_out,
                                                                         bad_out);
    return naiwa_hip_rc(hipGetLastError());
}
