// NAIWA_STACK_FUSED: one persistent kernel runs a whole decode step through
// every MoE layer, x <- bf16(x + MoE_l(x)).
//
// One workgroup of 512 threads per CU (8 waves, two per SIMD), every
// workgroup resident.  Per layer:
//   A  route   every workgroup polls the layer's logits and activations and
//              routes redundantly and identically: for one token, wave 0 polls
//              the logits while the other waves stage x; every wave counts, for
//              each expert, the keys above it in one slice of the experts; wave
//              0 adds the counts, takes the top k and groups the pairs by slot
//              (its weights follow while the gate/up rows load);
//   B  gate/up the (segment, row pair) items are dealt out evenly.  A wave
//              gathers its items' gate and up row pairs into LDS with coalesced
//              16-byte DMA pieces, then 32 lanes per item take one 144-byte Q4_K
//              block's half (both rows at once, each activation word feeding
//              two dots); h goes out as tagged pairs of 16-bit values, then one
//              tagged done word per workgroup.  The down rows and next router
//              columns of the workgroup's first output chunk are DMA'd into LDS
//              meanwhile;
//   C  down    each workgroup owns 8-feature output chunks: it waits for every
//              done word, reads all h once, dots every (feature, pair), adds the
//              pairs of each token in ascending slot order (no atomics),
//              applies the residual, publishes its x chunk and its int64 partial
//              sums of the next layer's router logits; 16 leader workgroups add
//              every chunk's partials for their experts and publish the logits.
//
// There is no grid barrier.  Every value one workgroup hands to another (x,
// h, done words, router partials, logits) is a 64-bit word (tag << 32) |
// payload written with one device-coherent store, where the tag names the
// launch and the layer.  A consumer loads the words it needs and reloads those
// whose tag is not yet current.  Every wait is bounded; a timeout is counted
// and makes every later wait give up at once, so a grid that cannot be
// co-resident drains instead of hanging.  Reuse is safe without barriers: a
// workgroup can only reach layer l+1 after seeing layer l+1's logits, which
// need every chunk's layer-l partials, which each workgroup produces after its
// last layer-l read of h and of the logits; x alternates between two buffers,
// since idle workgroups may still read x_l while chunk owners publish x_{l+1}.
// vmcnt counts stores as well as loads, so the stores that end phase C come
// from the waves that do not poll right after it.
//
// Router logits: each chunk of 8 features is an f32 fma chain rounded to
// int64 with 32 fractional bits, and the chunks are added as integers.
// Integer addition is associative, so the logits (and the top-k) are bit-
// identical to the CPU oracle's however the chunks are distributed.
#include <algorithm>
#include <type_traits>
#include <mutex>
#include <stdlib.h>
#include <string.h>
#include <vector>

#include "router.h"
#include "rowdot.h"
#include "workspace.h"

namespace {

typedef unsigned long long u64;

constexpr int kThreads = 512;             // 8 waves (two per SIMD), 32 groups of 16 lanes
constexpr int kGroups = kThreads / NAIWA_GROUP;
constexpr int kMaxRows = 8;               // tokens per step served by this kernel
constexpr int kMaxK = 8;                  // routed experts per token
constexpr int kMaxPairs = kMaxRows * kMaxK;
constexpr int kMaxE = 256;
constexpr int kLeaders = 16;              // workgroups that add the router partials
constexpr int kChunk = NAIWA_ROUTER_CHUNK; // output features per phase-C chunk
constexpr int kMaxChunks = 4;             // chunks per workgroup
constexpr int kCPairs = 32;               // h vectors staged per phase-C pass, at most
constexpr int kTraceSlots = 24;
constexpr int kMaxLayers = 128;           // layer descriptors kept in LDS (tags hold layer + 1 < 256)
constexpr int kXG = 8;                    // activation groups (4 values) per thread per poll round
constexpr int kHG = 4;                    // h groups (4 values, 2 words) per thread per poll round
constexpr int kCB = 2;                    // down rows per group in flight (general path)
constexpr int kDU8 = 3;                   // Q4_K down from LDS: units per lane of an 8-lane row group

struct LayerDev {
    const float* router;
    const uint8_t* gate;
    const uint8_t* up;
    const uint8_t* down;
    int64_t gate_stride, up_stride, down_stride;
    const int32_t* slot_of;
    int32_t slots;
    int32_t pad;
};

struct Params {
    const LayerDev* layers;
    int n_layers, rows, H, I, E, k, mode, act;
    uint16_t* x;                 // [rows, H] bf16: layer-0 input, last layer's output
    u64* xt;                     // [2][rows][H/2] tagged bf16 pairs (x of layer l in buffer l & 1)
    u64* h;                      // [kMaxPairs][I/2] tagged pairs of 16-bit values (down format)
    u64* part;                   // [rows * E][chunk owners][2] tagged int64 halves
    u64* logits;                 // [rows * E] tagged f32
    u64* done;                   // [grid] tagged: the workgroup's h words of the layer are stored
    int* status;                 // [0] wait timeouts, [1] missing experts
    uint32_t* ids_out;           // [n_layers, rows, k] or null
    float* w_out;
    float* y_out;                // [n_layers, rows, H] f32 MoE outputs before the residual, or null
    uint64_t spin_limit;         // wall-clock ticks before a wait gives up
    uint32_t seq;                // launch number; tag of layer l = seq << 8 | (l + 1)
    unsigned long long* trace;   // optional [grid][n_layers + 1][kTraceSlots] phase timestamps
    int bitems;                  // Q4_K gate/up: (segment, row pair) items per LDS round
    int hpairs;                  // h vectors staged per phase-C pass
    int dpre;                    // Q4_K down: pairs whose rows are prefetched into LDS (0 = none)
    int hwb_bytes;               // LDS shared by the phase-B gate/up rounds and the phase-C h staging
    int trace_layer;             // the layer being traced (diagnostics)
};

// One diagnostic value of this workgroup for a layer (row n_layers: the
// prologue), when tracing; anything outside the trace buffer is dropped.
__device__ __forceinline__ void trace_put(const Params& p, int layer, int slot, unsigned long long v) {
    if (!p.trace || layer < 0 || layer > p.n_layers || slot < 0 || slot >= kTraceSlots) return;
    p.trace[((size_t)blockIdx.x * (p.n_layers + 1) + layer) * kTraceSlots + slot] = v;
}
// Phase timestamps (s_memrealtime, one device-wide clock) of every workgroup, when tracing.
__device__ __forceinline__ void mark(const Params& p, int layer, int slot) {
    if (!p.trace || threadIdx.x != 0) return;
    trace_put(p, layer, slot, wall_clock64());
}

// The same, recorded by the first lane of the calling wave.
__device__ __forceinline__ void mark_wave(const Params& p, int layer, int slot) {
    if (!p.trace || (threadIdx.x & 63) != 0) return;
    trace_put(p, layer, slot, wall_clock64());
}

struct Smem {
    alignas(16) u64 key[kMaxRows][kMaxE + 2];  // ranking keys: ordered logit bits << 32 | ~expert
    float lg[kMaxRows][kMaxE];
    int32_t rcnt[kThreads / 64][kMaxE]; // one-token ranking: counts per wave's key slice
    int32_t slot_tab[kMaxE];
    uint32_t top_ids[kMaxRows][kMaxK];
    float top_ex[kMaxRows][kMaxK];
    float exv[kMaxPairs];
    uint32_t pair_slot[kMaxPairs]; // slot of pair p = t*k + j
    float pair_w[kMaxPairs];
    uint32_t sorted[kMaxPairs];    // valid pairs in (slot, p) order
    uint32_t srt_slot[kMaxPairs];
    uint32_t srt_tok[kMaxPairs];   // token of sorted position i
    uint32_t seg_begin[kMaxPairs + 1];
    uint32_t seg_slot[kMaxPairs];
    int nseg;
    float partial[kChunk][kMaxPairs];
    float xown[kMaxChunks][kMaxRows][kChunk]; // this workgroup's chunks of x (bf16 values)
};

typedef __attribute__((address_space(1))) u64 gu64;
__device__ __forceinline__ u64 ld64(const u64* p) {
    return __hip_atomic_load((const gu64*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st64(u64* p, u64 v) {
    __hip_atomic_store((gu64*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 tagged(uint32_t tag, uint32_t v) { return ((u64)tag << 32) | v; }

// 16 bytes from global memory straight into LDS (no registers; counted by
// vmcnt): lane i of the wave writes wave_base + 16 * i.  Both addresses must be
// 16-byte aligned, and wave_base must be the same in every active lane.
// Issued as inline assembly so that the compiler does not track it: it would
// otherwise wait for every outstanding DMA (vmcnt(0)) before any later LDS read
// that may alias one, which made the gate/up compute wait for the down-row
// prefetch issued ahead of it.  Every read of DMA'd data here follows an
// explicit vmcnt wait of the wave that issued it (and a barrier where another
// wave reads it).  M0 is a reserved register, so the compiler warns that the
// clobber is not honoured: this is sound only while nothing else in the kernel
// keeps a value in M0 (no LDS DMA builtins, no relative-indexing moves), which
// the generated assembly shows and must keep showing after changes here.
__device__ __forceinline__ void lds_dma16(const void* src, void* wave_base) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane(
        (uint32_t)(size_t)(__attribute__((address_space(3))) void*)wave_base);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(src), "s"(lds) : "memory", "m0");
}
// The same with the non-temporal hint, for expert rows: each is read once per token,
// so they need not displace the router columns, activations and exchange words from
// the caches (1,213 -> 1,232 tok/s).
__device__ __forceinline__ void lds_dma16_nt(const void* src, void* wave_base) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane(
        (uint32_t)(size_t)(__attribute__((address_space(3))) void*)wave_base);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :: "v"(src), "s"(lds) : "memory", "m0");
}

__device__ __forceinline__ bool tag_ok(u64 w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
__device__ __forceinline__ uint32_t layer_tag(const Params& p, int l) { return (p.seq << 8) | (uint32_t)(l + 1); }

// Bounded-wait bookkeeping: false once this wait has run past spin_limit (the
// timeout is counted) or any wait anywhere has (status[0] != 0).
struct Poll {
    uint64_t t0 = 0;
    unsigned n = 0;
};
__device__ inline bool poll_continue(const Params& p, Poll& s) {
    if (s.n++ == 0) {
        s.t0 = wall_clock64();
        return true;
    }
    if ((s.n & 7) == 0) {
        if (__hip_atomic_load(&p.status[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
        if (wall_clock64() - s.t0 > p.spin_limit) {
            atomicAdd(&p.status[0], 1);
            return false;
        }
    }
    return true;
}

// Tagged loads of N words: addr(j) gives word j's address, or null for none.
template <int N, class F>
__device__ __forceinline__ void issue_tagged(u64 (&w)[N], const F& addr, uint32_t tag) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const u64* a = addr(j);
        w[j] = a ? ld64(a) : tagged(tag, 0u);
    }
}
// Reload the words whose tag is not current until all are (or the wait gives up).
template <int N, class F>
__device__ inline unsigned wait_tagged(u64 (&w)[N], const F& addr, uint32_t tag, const Params& p) {
    Poll s;
    while (true) {
        bool ok = true;
#pragma unroll
        for (int j = 0; j < N; ++j) ok &= tag_ok(w[j], tag);
        if (ok || !poll_continue(p, s)) return s.n;
#pragma unroll
        for (int j = 0; j < N; ++j)
            if (!tag_ok(w[j], tag)) w[j] = ld64(addr(j));
    }
}

// Sum over aligned groups of W lanes of an exact int64.
template <int W>
__device__ __forceinline__ long long group_sum_i64(long long v) {
    if (W >= 2) v += naiwa_dpp_i64<0xB1>(v);
    if (W >= 4) v += naiwa_dpp_i64<0x4E>(v);
    if (W >= 8) v += naiwa_dpp_i64<0x141>(v);
    if (W >= 16) v += naiwa_dpp_i64<0x140>(v);
#pragma unroll
    for (int m = 16; m < W; m <<= 1) v += __shfl_xor(v, m, W);
    return v;
}

// The output-feature chunk handled at position p (= workgroup + j * workgroups).
// Workgroups are dealt to the XCDs round-robin, so position p runs on XCD p % 8;
// this mapping gives the 4 chunks that share a 128-byte line of every router
// row (4 x 8 f32) to workgroups of one XCD, which then fetches the line once.
__device__ __forceinline__ int chunk_at(int p, int nchunks) {
    if (nchunks % 32) return p;
    const int x = p & 7, r = p >> 3;
    return (((r >> 2) << 3) + x) * 4 + (r & 3);
}

// The thread that owns router item slot 0 of the partials: the upper half of
// the workgroup first, so that the waves polling right after phase C (the
// leaders' reduction on the lower waves, wave 0's logits) have no stores of
// their own in flight (vmcnt counts stores too, so a load's wait would include
// them).
__device__ __forceinline__ int item_thread() { return (threadIdx.x + kThreads / 2) % kThreads; }

// Publish this workgroup's router partials for layer tag `tag`: item it of
// chunk owner b at part[(b * items + it) * 2 ...], so that an owner writes
// whole cache lines (its items are contiguous) and a leader reads, per owner,
// one contiguous run of its own items.
template <int PPT>
__device__ inline void store_partials(const Params& p, const long long* acc, int nprod, uint32_t tag) {
    const int items = p.rows * p.E;
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        const int it = item_thread() + j * kThreads;
        if (it < items) {
            u64* dst = p.part + ((size_t)blockIdx.x * items + it) * 2;
            st64(dst, tagged(tag, (uint32_t)(unsigned long long)acc[j]));
            st64(dst + 1, tagged(tag, (uint32_t)((unsigned long long)acc[j] >> 32)));
        }
    }
}

// Leader bid adds, for its experts (its items: every token's logit of each),
// the partials of every chunk owner and publishes the logits (tagged f32).
// Thread t takes item t % n and the owners t / n, t / n + kThreads / n, ...:
// consecutive threads read consecutive words of one owner's run.  The int64
// sums are added across threads with LDS atomics (exact, so in any order).
constexpr int kLeadItemsMax = kMaxRows * kMaxE / kLeaders;
__device__ inline void leader_reduce(const Params& p, int nprod, uint32_t tag) {
    __shared__ long long lacc[kLeadItemsMax];
    const int nlead = min(kLeaders, (int)gridDim.x);
    const int epl = (p.E + nlead - 1) / nlead;
    const int e0 = blockIdx.x * epl;
    const int ne = max(0, min(epl, p.E - e0));
    const int n = p.rows * ne;
    if (n <= 0) return;
    const int tid = threadIdx.x, items = p.rows * p.E;
    // barriers that wait for LDS only: the upper waves' partial stores may still be
    // in flight, and waiting for them would delay the loads below
    auto lds_barrier = [] {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    if (tid < n) lacc[tid] = 0;
    lds_barrier();
    const int per = kThreads / n;            // threads per item
    const bool act = tid < per * n;
    const int li = act ? tid % n : 0, ob = act ? tid / n : 0;
    const size_t idx = (size_t)(li / ne) * p.E + e0 + li % ne;
    long long s = 0;
#pragma unroll 1
    for (int b0 = ob; b0 < nprod; b0 += 8 * per) {
        u64 w[16];
        auto addr = [&](int j) -> const u64* {
            const int b = b0 + (j >> 1) * per;
            return (act && b < nprod) ? p.part + ((size_t)b * items + idx) * 2 + (j & 1) : nullptr;
        };
        issue_tagged(w, addr, tag);
        const unsigned polls = wait_tagged(w, addr, tag, p);
        if (p.trace && threadIdx.x == 0 && b0 == ob) {
            mark(p, p.trace_layer, 19);
            trace_put(p, p.trace_layer, 20, polls);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
            s += (long long)(((u64)(uint32_t)w[2 * j + 1] << 32) | (uint32_t)w[2 * j]);
    }
    if (act) atomicAdd((unsigned long long*)&lacc[li], (unsigned long long)s);
    lds_barrier();
    if (tid < n) {
        const size_t gi = (size_t)(tid / ne) * p.E + e0 + tid % ne;
        st64(&p.logits[gi], tagged(tag, __float_as_uint(naiwa_router_fix_to_f32(lacc[tid]))));
    }
}

// Router partials of one chunk for every (token, expert) item: W8(e) gives the
// chunk's 8 router weights of expert e, xv[t] the chunk's activations.
template <int PPT, int AS, class F>
__device__ __forceinline__ void router_chunk_accumulate(const Params& p, const F& W8, const float (*xv)[kChunk],
                                                        long long* acc) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        const int it = item_thread() + j * kThreads;
        if (it < p.rows * p.E) {
            const int t = it / p.E, e = it % p.E;
            acc[j] += naiwa_router_chunk<AS>(W8(e), xv[t]);
        }
    }
}

// Order-preserving 64-bit ranking key: larger key = earlier in (logit desc, id asc).
__device__ __forceinline__ u64 rank_key(float f, int e) {
    const uint32_t u = __float_as_uint(f + 0.0f); // -0 -> +0, which compare equal as floats
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((u64)o << 32) | (uint32_t)~(uint32_t)e;
}
__device__ __forceinline__ float readlane_f32(float v, int ln) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), ln));
}

// Wave 0, one lane per (token, rank) pair q = t * k + j (inp: q < rows * k):
// slot lookup, the routing outputs, and the grouping of valid pairs by slot
// (sorted by (slot, q); a segment per distinct slot).
__device__ inline void group_pairs(const Params& p, Smem& sm, const LayerDev& L, int l, int lane, bool inp, int t,
                                   uint32_t e, float w) {
    const int npairs = p.rows * p.k;
    const int q = lane;
    const int32_t s = inp ? (L.slot_of ? sm.slot_tab[e] : (int32_t)e) : -1;
    const bool ok = inp && s >= 0 && s < L.slots;
    if (inp && !ok && blockIdx.x == 0) atomicAdd(&p.status[1], 1);
    if (inp && blockIdx.x == 0 && p.ids_out) {
        p.ids_out[(size_t)l * npairs + q] = e;
        p.w_out[(size_t)l * npairs + q] = w;
    }
    const bool valid = ok && w != 0.0f;
    // sort key (slot, pair); invalid pairs sort last
    const uint32_t key = valid ? (((uint32_t)s << 6) | (uint32_t)q) : 0xFFFFFFFFu;
    int rank = 0;
    for (int o = 0; o < npairs; ++o) rank += (uint32_t)__builtin_amdgcn_readlane((int)key, o) < key;
    sm.pair_slot[q] = valid ? (uint32_t)s : 0u;
    sm.pair_w[q] = valid ? w : 0.0f;
    if (valid) {
        sm.sorted[rank] = (uint32_t)q;
        sm.srt_slot[rank] = (uint32_t)s;
        sm.srt_tok[rank] = (uint32_t)t;
    }
    const unsigned long long valids = __ballot(valid);
    const int nvalid = __popcll(valids);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // lane r looks at sorted position r: a segment starts where the slot changes
    const bool start = lane < nvalid && (lane == 0 || sm.srt_slot[lane] != sm.srt_slot[lane - 1]);
    const unsigned long long starts = __ballot(start);
    if (start) {
        const int si = __popcll(starts & ((1ull << lane) - 1ull));
        sm.seg_begin[si] = (uint32_t)lane;
        sm.seg_slot[si] = sm.srt_slot[lane];
    }
    if (lane == 0) {
        const int ns = __popcll(starts);
        sm.seg_begin[ns] = (uint32_t)nvalid;
        sm.nseg = ns;
    }
}

__device__ __forceinline__ u64 readlane_u64(u64 v, int ln) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, ln);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), ln);
    return ((u64)hi << 32) | lo;
}

// One token (rows == 1), wave 0: poll the E logits (lane l holds experts
// l + 64 j) and the slot table; their ranking keys, logits and slots go to LDS.
__device__ inline void poll_one_row(const Params& p, Smem& sm, const LayerDev& L, int l, uint32_t tag, int lane) {
    constexpr int KPL = kMaxE / 64;
    const int E = p.E;
    u64 lw[KPL];
    auto laddr = [&](int j) -> const u64* {
        const int e = lane + 64 * j;
        return e < E ? p.logits + e : nullptr;
    };
    issue_tagged(lw, laddr, tag);
    int32_t st[KPL];
#pragma unroll
    for (int j = 0; j < KPL; ++j)
        st[j] = (L.slot_of && lane + 64 * j < E) ? naiwa_ld<int32_t, NAIWA_AS_GLOBAL>(L.slot_of + lane + 64 * j) : 0;
    wait_tagged(lw, laddr, tag, p);
    mark_wave(p, l, 10);
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
        const int e = lane + 64 * j;
        if (e < E) {
            const float f = __uint_as_float((uint32_t)lw[j]);
            sm.lg[0][e] = f;
            sm.key[0][e] = rank_key(f, e);
            if (L.slot_of) sm.slot_tab[e] = st[j];
        }
    }
}

// One token, every wave: the number of keys above each key that lie in this
// wave's slice of the experts (one slice per wave, at most 64 keys, one per
// lane), broadcast one key at a time from the lane holding it.  KPL: keys per lane.
template <int KPL>
__device__ inline void rank_slice(const Params& p, Smem& sm, int wave, int lane) {
    constexpr int NW = kThreads / 64;
    const int E = p.E;
    const int per = (E + NW - 1) / NW, s0 = wave * per, ns = max(0, min(E, s0 + per) - s0);
    const u64 ks = lane < ns ? sm.key[0][s0 + lane] : 0ull;
    u64 mine[KPL];
    int cnt[KPL];
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
        mine[j] = lane + 64 * j < E ? sm.key[0][lane + 64 * j] : 0ull;
        cnt[j] = 0;
    }
    for (int s = 0; s < ns; ++s) {
        const u64 K = readlane_u64(ks, s);
#pragma unroll
        for (int j = 0; j < KPL; ++j) cnt[j] += K > mine[j];
    }
#pragma unroll
    for (int j = 0; j < KPL; ++j)
        if (lane + 64 * j < E) sm.rcnt[wave][lane + 64 * j] = cnt[j];
}

// One token, wave 0: the grouping of its k pairs (lane q = pair q = the rank-q
// expert e, inp: q < k) by slot, all in registers: each pair's position in
// (slot, q) order and its predecessor's slot come from the other lanes' keys,
// one readlane each.  A pair is grouped when its expert has a slot; its weight
// comes later (weigh_one_row), and a zero weight is skipped at the combine.
__device__ inline void group_pairs_one(const Params& p, Smem& sm, const LayerDev& L, int lane, bool inp, uint32_t e) {
    const int k = p.k;
    const int q = lane;
    const int32_t s = inp ? (L.slot_of ? sm.slot_tab[e] : (int32_t)e) : -1;
    const bool valid = inp && s >= 0 && s < L.slots;
    if (inp && !valid && blockIdx.x == 0) atomicAdd(&p.status[1], 1);
    const uint32_t key = valid ? (((uint32_t)s << 6) | (uint32_t)q) : 0xFFFFFFFFu; // invalid pairs sort last
    int rank = 0;
    long long pk = -1; // the largest key below this one
#pragma unroll
    for (int o = 0; o < kMaxK; ++o) {
        const uint32_t ko = (uint32_t)__builtin_amdgcn_readlane((int)key, o);
        if (o < k && ko < key) {
            ++rank;
            pk = max(pk, (long long)ko);
        }
    }
    const bool start = valid && (rank == 0 || (uint32_t)(pk >> 6) != (uint32_t)s);
    // segment index: the starts that sort before this one
    const uint32_t sk = start ? key : 0xFFFFFFFFu;
    int si = 0;
#pragma unroll
    for (int o = 0; o < kMaxK; ++o) si += o < k && (uint32_t)__builtin_amdgcn_readlane((int)sk, o) < key;
    const int nvalid = __popcll(__ballot(valid));
    const int nseg = __popcll(__ballot(start));
    sm.pair_slot[q] = valid ? (uint32_t)s : 0u;
    if (valid) {
        sm.sorted[rank] = (uint32_t)q;
        sm.srt_slot[rank] = (uint32_t)s;
        sm.srt_tok[rank] = 0u;
    }
    if (start) {
        sm.seg_begin[si] = (uint32_t)rank;
        sm.seg_slot[si] = (uint32_t)s;
    }
    if (lane == 0) {
        sm.seg_begin[nseg] = (uint32_t)nvalid;
        sm.nseg = nseg;
    }
}

// One token, wave 0, after every wave's key-slice counts: the rank of each
// expert (lane l: experts l + 64 j), the top k through LDS (lane j takes the
// rank-j expert: my_e, its logit my_f), then the grouping of the pairs.
template <int KPL>
__device__ inline void route_one_row(const Params& p, Smem& sm, const LayerDev& L, int l, int lane, uint32_t& my_e,
                                     float& my_f) {
    const int E = p.E, k = p.k;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
        const int e = lane + 64 * j;
        if (e < E) {
            int r = 0;
#pragma unroll
            for (int w = 0; w < kThreads / 64; ++w) r += sm.rcnt[w][e];
            if (r < k) {
                sm.top_ids[0][r] = (uint32_t)e;
                sm.top_ex[0][r] = sm.lg[0][e];
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const bool inp = lane < k;
    my_e = inp ? sm.top_ids[0][lane] : 0u;
    my_f = inp ? sm.top_ex[0][lane] : 0.0f;
    mark_wave(p, l, 22);
    group_pairs_one(p, sm, L, lane, inp, my_e);
    mark_wave(p, l, 12);
}

// One token, wave 0: the routing weights of the k pairs (denominators summed in
// rank order, or in expert order over all E for the softmax-without-
// renormalisation mode, as the oracle sums them) into pair_w, and the routing
// outputs.  Runs while the gate/up rows are on their way; pair_w is first read
// in phase C.
__device__ inline void weigh_one_row(const Params& p, Smem& sm, int l, int lane, uint32_t my_e, float my_f) {
    const int E = p.E, k = p.k;
    const bool inp = lane < k;
    const float mx = readlane_f32(my_f, 0);
    const float ex = inp ? expf(my_f - mx) : 0.0f;
    float denom = 0.0f;
    if (p.mode == NAIWA_ROUTE_SOFTMAX_TOPK) {
        constexpr int KA = kMaxE / 64;
        float ea[KA];
#pragma unroll
        for (int j = 0; j < KA; ++j) ea[j] = lane + 64 * j < E ? expf(sm.lg[0][lane + 64 * j] - mx) : 0.0f;
#pragma unroll
        for (int j = 0; j < KA; ++j)
            for (int ln = 0; ln < 64 && 64 * j + ln < E; ++ln) denom += readlane_f32(ea[j], ln);
    } else {
#pragma unroll
        for (int o = 0; o < kMaxK; ++o) denom += o < k ? readlane_f32(ex, o) : 0.0f;
    }
    const float w = inp ? ex / denom : 0.0f;
    if (inp) sm.pair_w[lane] = w;
    if (inp && blockIdx.x == 0 && p.ids_out) {
        p.ids_out[(size_t)l * k + lane] = my_e;
        p.w_out[(size_t)l * k + lane] = w;
    }
    mark_wave(p, l, 11);
}

// ---------------------------------------------------------------------------
// Q4_K gate/up with one 144-byte block per lane
// ---------------------------------------------------------------------------

// Scales and mins of one Q4_K block header (ggml get_scale_min_k4), one per byte.
struct Q4Scales {
    float d, dmin;
    uint32_t sc_lo, m_lo, sc_hi, m_hi;
};
__device__ __forceinline__ Q4Scales q4k_scales(const uint4& hd) {
    Q4Scales s;
    s.d = naiwa_f16_to_f32(hd.x & 0xffffu);
    s.dmin = naiwa_f16_to_f32(hd.x >> 16);
    s.sc_lo = hd.y & 0x3F3F3F3Fu;                                    // sc0..sc3
    s.m_lo = hd.z & 0x3F3F3F3Fu;                                     // m0..m3
    s.sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);    // sc4..sc7
    s.m_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u); // m4..m7
    return s;
}
// Chunk c (64 values: sub-blocks 2c, 2c+1) of a block: d*(sc0*qlo + sc1*qhi) - dmin*(m0*slo + m1*shi),
// with qlo = alo - 128*slo (alo / ahi: dots of the nibbles + 128 offset).
__device__ __forceinline__ float q4k_chunk(const Q4Scales& s, int c, float alo, float ahi, float slo, float shi) {
    const uint32_t scw = c < 2 ? s.sc_lo : s.sc_hi, mw = c < 2 ? s.m_lo : s.m_hi;
    const int sh = (c & 1) * 16;
    const float sc0 = (float)((scw >> sh) & 0xFFu), sc1 = (float)((scw >> (sh + 8)) & 0xFFu);
    const float m0 = (float)((mw >> sh) & 0xFFu), m1 = (float)((mw >> (sh + 8)) & 0xFFu);
    return s.d * (sc0 * (alo - 128.0f * slo) + sc1 * (ahi - 128.0f * shi)) - s.dmin * (m0 * slo + m1 * shi);
}

// Dots of chunks c0 and c0 + 1 (64 values each) of two Q4_K blocks (rows A and
// B, 9 x 16 bytes each in LDS) with the same staged activations: words = the
// block's 128 bf16 pair words, sums = its 16 sums of 16.  Each activation word
// is loaded once and feeds both rows.
__device__ __forceinline__ void q4k_block_dot2(const uint8_t* A8, const uint8_t* B8, const uint32_t* words,
                                               const float* sums, int c0, float& ra, float& rb) {
    auto A = [&](int j) { return naiwa_ld<uint4, NAIWA_AS_LDS>(A8 + 16 * j); };
    auto B = [&](int j) { return naiwa_ld<uint4, NAIWA_AS_LDS>(B8 + 16 * j); };
    const Q4Scales sa = q4k_scales(A(0)), sb = q4k_scales(B(0));
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
        const int c = c0 + cc;
        // the chunk's 32 activation words, all loads in flight before the first use
        uint4 x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = reinterpret_cast<const uint4*>(words + 32 * c)[i];
        const float4 sv = reinterpret_cast<const float4*>(sums)[c];
        const uint4 qa0 = A(1 + 2 * c), qa1 = A(2 + 2 * c), qb0 = B(1 + 2 * c), qb1 = B(2 + 2 * c);
        const uint32_t wa[8] = {qa0.x, qa0.y, qa0.z, qa0.w, qa1.x, qa1.y, qa1.z, qa1.w};
        const uint32_t wb[8] = {qb0.x, qb0.y, qb0.z, qb0.w, qb1.x, qb1.y, qb1.z, qb1.w};
        float alo = 0.0f, ahi = 0.0f, blo = 0.0f, bhi = 0.0f;
        const NaiwaNib nc = naiwa_nib_consts();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t xl[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
            const uint32_t xh[4] = {x[4 + i].x, x[4 + i].y, x[4 + i].z, x[4 + i].w};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t qa = wa[2 * i + h], qb = wb[2 * i + h];
                alo = naiwa_dot2_bf16(naiwa_nib(qa, nc), xl[2 * h], alo);
                blo = naiwa_dot2_bf16(naiwa_nib(qb, nc), xl[2 * h], blo);
                alo = naiwa_dot2_bf16(naiwa_nib(qa >> 8, nc), xl[2 * h + 1], alo);
                blo = naiwa_dot2_bf16(naiwa_nib(qb >> 8, nc), xl[2 * h + 1], blo);
                ahi = naiwa_dot2_bf16(naiwa_nib(qa >> 4, nc), xh[2 * h], ahi);
                bhi = naiwa_dot2_bf16(naiwa_nib(qb >> 4, nc), xh[2 * h], bhi);
                ahi = naiwa_dot2_bf16(naiwa_nib(qa >> 12, nc), xh[2 * h + 1], ahi);
                bhi = naiwa_dot2_bf16(naiwa_nib(qb >> 12, nc), xh[2 * h + 1], bhi);
            }
        }
        const float slo = sv.x + sv.y, shi = sv.z + sv.w;
        ra += q4k_chunk(sa, c, alo, ahi, slo, shi);
        rb += q4k_chunk(sb, c, blo, bhi, slo, shi);
        // keep the scheduler from hoisting every chunk's loads at once
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The dot of chunks c0 and c0 + 1 of one Q4_K block: the row-A half of
// q4k_block_dot2, the same operations in the same order.
__device__ __forceinline__ void q4k_block_dot1(const uint8_t* A8, const uint32_t* words, const float* sums, int c0,
                                               float& ra) {
    auto A = [&](int j) { return naiwa_ld<uint4, NAIWA_AS_LDS>(A8 + 16 * j); };
    const Q4Scales sa = q4k_scales(A(0));
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
        const int c = c0 + cc;
        uint4 x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = reinterpret_cast<const uint4*>(words + 32 * c)[i];
        const float4 sv = reinterpret_cast<const float4*>(sums)[c];
        const uint4 qa0 = A(1 + 2 * c), qa1 = A(2 + 2 * c);
        const uint32_t wa[8] = {qa0.x, qa0.y, qa0.z, qa0.w, qa1.x, qa1.y, qa1.z, qa1.w};
        float alo = 0.0f, ahi = 0.0f;
        const NaiwaNib nc = naiwa_nib_consts();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t xl[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
            const uint32_t xh[4] = {x[4 + i].x, x[4 + i].y, x[4 + i].z, x[4 + i].w};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t qa = wa[2 * i + h];
                alo = naiwa_dot2_bf16(naiwa_nib(qa, nc), xl[2 * h], alo);
                alo = naiwa_dot2_bf16(naiwa_nib(qa >> 8, nc), xl[2 * h + 1], alo);
                ahi = naiwa_dot2_bf16(naiwa_nib(qa >> 4, nc), xh[2 * h], ahi);
                ahi = naiwa_dot2_bf16(naiwa_nib(qa >> 12, nc), xh[2 * h + 1], ahi);
            }
        }
        const float slo = sv.x + sv.y, shi = sv.z + sv.w;
        ra += q4k_chunk(sa, c, alo, ahi, slo, shi);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Wait until at most n of this wave's vector memory operations are
// outstanding (they complete in issue order, LDS DMA included); n above 15
// waits for 15, which is stricter.
__device__ __forceinline__ void vm_wait_at_most(int n) {
#define NAIWA_VMW(k) case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
    switch (n) {
        NAIWA_VMW(0) NAIWA_VMW(1) NAIWA_VMW(2) NAIWA_VMW(3) NAIWA_VMW(4) NAIWA_VMW(5) NAIWA_VMW(6)
        NAIWA_VMW(7) NAIWA_VMW(8) NAIWA_VMW(9) NAIWA_VMW(10) NAIWA_VMW(11) NAIWA_VMW(12) NAIWA_VMW(13)
        NAIWA_VMW(14)
        default: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
    }
#undef NAIWA_VMW
}

// h of every token of the segment for intermediate rows r, r + 1 (pair q),
// with the item's rows in LDS: [gate row r][gate row r + 1][up row r][up row r + 1]
// (rb bytes each), on 32 lanes: lane il = 16 u + 8 h + b takes chunks 2h, 2h + 1
// of block b of the gate rows (u = 0) or of the up rows (u = 1), both rows at
// once; rows of at most 8 blocks (H <= 2048).  The two results go out as one
// tagged word in the down projection's 16-bit format DD.
template <int DD>
__device__ inline void q4_pair_compute(const Params& p, const Smem& sm, const uint8_t* dyn, int xstage, int q,
                                       int nb, int il, const uint8_t* item, int64_t rb, uint32_t tag) {
    const int I2 = p.I / 2, H = p.H, k = p.k;
    const int s = q / I2, r = 2 * (q % I2);
    const int b = (int)sm.seg_begin[s], e = (int)sm.seg_begin[s + 1];
    const int b0 = il & 7, c0 = (il >> 2) & 2;
    const uint8_t* A = item + (il >= 16 ? 2 * rb : 0) + b0 * NAIWA_Q4_K_BYTES;
    for (int tt = b; tt < e; ++tt) {
        const int t = (int)sm.sorted[tt] / k;
        const uint32_t* words = (const uint32_t*)(dyn + t * xstage);   // 132 words per block (padded)
        const float* sums = (const float*)(words + H / 2 + 4 * nb);
        float g0 = 0.0f, g1 = 0.0f;   // this lane's share of row r and row r + 1
        if (b0 < nb) q4k_block_dot2(A, A + rb, words + b0 * 132, sums + b0 * 16, c0, g0, g1);
        // lanes 0-15: gate . x, lanes 16-31: up . x (one DPP row each); then the
        // up row takes the gate sums from the last lane of the gate row
        g0 = naiwa_group_sum<16>(g0);
        g1 = naiwa_group_sum<16>(g1);
        const float ga = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                       0, __builtin_bit_cast(int, g0), 0x142, 0xA, 0xF, false));
        const float gb = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                       0, __builtin_bit_cast(int, g1), 0x142, 0xA, 0xF, false));
        const float h0 = naiwa_act(p.act, ga) * g0;
        const float h1 = naiwa_act(p.act, gb) * g1;
        if (il == 16)
            st64(&p.h[(size_t)tt * I2 + r / 2],
                 tagged(tag, Fmt<DD>::to16(h0) | (Fmt<DD>::to16(h1) << 16)));
    }
}

// One token per segment: row r of the item (its gate and up rows r) was
// waited for by the caller; row r + 1 may still be landing, with `later` of
// the wave's memory operations issued after it.  Row r is dotted first, then
// the wait, then row r + 1: the same per-row arithmetic as q4_pair_compute.
template <int DD>
__device__ inline void q4_pair_compute_split(const Params& p, const Smem& sm, const uint8_t* dyn, int xstage, int q,
                                             int nb, int il, const uint8_t* item, int64_t rb, uint32_t tag,
                                             int later) {
    const int I2 = p.I / 2, H = p.H, k = p.k;
    const int s = q / I2, r = 2 * (q % I2);
    const int tt = (int)sm.seg_begin[s];
    if ((int)sm.seg_begin[s + 1] - tt != 1) { // not one token in the segment: everything landed first
        vm_wait_at_most(later);
        q4_pair_compute<DD>(p, sm, dyn, xstage, q, nb, il, item, rb, tag);
        return;
    }
    const int b0 = il & 7, c0 = (il >> 2) & 2;
    const uint8_t* A = item + (il >= 16 ? 2 * rb : 0) + b0 * NAIWA_Q4_K_BYTES;
    const int t = (int)sm.sorted[tt] / k;
    const uint32_t* words = (const uint32_t*)(dyn + t * xstage);
    const float* sums = (const float*)(words + H / 2 + 4 * nb);
    float g0 = 0.0f, g1 = 0.0f;
    if (b0 < nb) q4k_block_dot1(A, words + b0 * 132, sums + b0 * 16, c0, g0);
    vm_wait_at_most(later);
    if (b0 < nb) q4k_block_dot1(A + rb, words + b0 * 132, sums + b0 * 16, c0, g1);
    g0 = naiwa_group_sum<16>(g0);
    g1 = naiwa_group_sum<16>(g1);
    const float ga = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                   0, __builtin_bit_cast(int, g0), 0x142, 0xA, 0xF, false));
    const float gb = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                   0, __builtin_bit_cast(int, g1), 0x142, 0xA, 0xF, false));
    const float h0 = naiwa_act(p.act, ga) * g0;
    const float h1 = naiwa_act(p.act, gb) * g1;
    if (il == 16)
        st64(&p.h[(size_t)tt * I2 + r / 2], tagged(tag, Fmt<DD>::to16(h0) | (Fmt<DD>::to16(h1) << 16)));
}

// ---------------------------------------------------------------------------
// Q8_0 gate/up with 16 lanes per row pair (units of two blocks)
// ---------------------------------------------------------------------------
template <int DG, int DD>
__device__ inline void unit_pair(const Params& p, const Smem& sm, const LayerDev& L, const uint8_t* dyn,
                                 int q, int xstage, int64_t rb, int nu, int lr, uint32_t tag) {
    constexpr int UM = Umax<DG>::v;
    const int I = p.I, H = p.H, k = p.k, I2 = I / 2;
    const int s = q / I2, r = 2 * (q % I2);
    const uint32_t slot = sm.seg_slot[s];
    const int b = (int)sm.seg_begin[s], e = (int)sm.seg_begin[s + 1];
    for (int tt = b; tt < e; ++tt) {
        const int t = (int)sm.sorted[tt] / k;
        const uint32_t* words = (const uint32_t*)(dyn + t * xstage);
        const float* sums = (const float*)(words + H / 2);
        float hv[2];
#pragma unroll 1
        for (int rr = 0; rr < 2; ++rr) {
            const uint8_t* grow = L.gate + (int64_t)slot * L.gate_stride + (int64_t)(r + rr) * rb;
            const uint8_t* urow = L.up + (int64_t)slot * L.up_stride + (int64_t)(r + rr) * rb;
            float ag = 0.0f, au = 0.0f;
            for (int base = lr; base < nu; base += NAIWA_GROUP * UM) {
                typename Fmt<DG>::Frag fg[UM], fu[UM];
#pragma unroll
                for (int i = 0; i < UM; ++i) {
                    const int u = base + NAIWA_GROUP * i;
                    if (u < nu) {
                        fg[i] = Fmt<DG>::template load<NAIWA_AS_GLOBAL>(grow, u);
                        fu[i] = Fmt<DG>::template load<NAIWA_AS_GLOBAL>(urow, u);
                    }
                }
#pragma unroll
                for (int i = 0; i < UM; ++i) {
                    const int u = base + NAIWA_GROUP * i;
                    if (u < nu) {
                        ag += Fmt<DG>::dot(fg[i], u, words, sums);
                        au += Fmt<DG>::dot(fu[i], u, words, sums);
                    }
                }
            }
            const float gv = naiwa_group_sum<NAIWA_GROUP>(ag);
            const float uv = naiwa_group_sum<NAIWA_GROUP>(au);
            hv[rr] = naiwa_act(p.act, gv) * uv;
        }
        if (lr == 0)
            st64(&p.h[(size_t)tt * I2 + r / 2],
                 tagged(tag, Fmt<DD>::to16(hv[0]) | (Fmt<DD>::to16(hv[1]) << 16)));
    }
}

// Stage 4 consecutive values v[0..3] of group gg of a vector in the dot
// layout of DT (pair words + sums over the format's span); every lane of the
// wave must call it (the sums use DPP), with `in` false for no group.
// PAD: 4 words of padding after every 256 values (128 words), so the lanes
// of a group that read 8 different blocks hit 8 different LDS bank sets.
template <int DT, bool PAD = false>
__device__ __forceinline__ void stage_group(float v0, float v1, float v2, float v3, bool in, int gg, uint8_t* vec,
                                            int k) {
    constexpr int gpg = Fmt<DT>::kSumSpan / 4;
    float part = 0.0f;
    if (in) {
        const uint32_t h0 = Fmt<DT>::to16(v0), h1 = Fmt<DT>::to16(v1), h2 = Fmt<DT>::to16(v2),
                       h3 = Fmt<DT>::to16(v3);
        uint32_t* words = (uint32_t*)vec + (PAD ? 4 * (gg >> 6) : 0);
        words[2 * gg] = h0 | (h2 << 16);
        words[2 * gg + 1] = h1 | (h3 << 16);
        part = (Fmt<DT>::from16(h0) + Fmt<DT>::from16(h1)) + (Fmt<DT>::from16(h2) + Fmt<DT>::from16(h3));
    }
    part = naiwa_group_sum<gpg>(part);
    if (in && (gg % gpg) == 0)
        ((float*)((uint32_t*)vec + k / 2 + (PAD ? 4 * (k / NAIWA_QK_K) : 0)))[gg / gpg] = part;
}

// LDS bytes of one staged activation vector of the fused kernel (Q4_K: padded).
__host__ __device__ inline int fused_xstage(int dt, int h) {
    return naiwa_stage_bytes(dt, h) + (dt == NAIWA_Q4_K ? 16 * (h / NAIWA_QK_K) : 0);
}

// Poll the tagged h vectors of sorted positions [v0, v0 + nv) (I/2 words each,
// two 16-bit values of format DD per word; vector v at h + v * I/2) and stage
// them: words at hw[v * I/2 ...] in the dot layout of DD, sums of kSumSpan
// values at hs[v * I/kSumSpan ...].
template <int DD>
__device__ inline void stage_h(const Params& p, int v0, int nv, uint32_t* hw, float* hs, uint32_t tag) {
    constexpr int gpg = Fmt<DD>::kSumSpan / 4;
    const int gpv = p.I / 4, total = nv * gpv;
    const u64* src = p.h + (size_t)v0 * (p.I / 2);
    for (int g0 = 0; g0 < total; g0 += kHG * kThreads) {
        u64 w[2 * kHG];
        auto addr = [&](int j) -> const u64* {
            const int g = g0 + threadIdx.x + (j >> 1) * kThreads;
            return g < total ? src + 2 * g + (j & 1) : nullptr;
        };
        issue_tagged(w, addr, tag);
        const unsigned polls = wait_tagged(w, addr, tag, p);
        if (p.trace && threadIdx.x == 0) {
            mark(p, p.trace_layer, 17);
            trace_put(p, p.trace_layer, 18, polls);
        }
#pragma unroll
        for (int j = 0; j < kHG; ++j) {
            const int g = g0 + threadIdx.x + j * kThreads;
            const bool in = g < total;
            const uint32_t A = (uint32_t)w[2 * j], B = (uint32_t)w[2 * j + 1]; // (h0, h1), (h2, h3)
            float part = 0.0f;
            if (in) {
                hw[2 * g] = (A & 0xffffu) | (B << 16);
                hw[2 * g + 1] = (A >> 16) | (B & 0xffff0000u);
                part = (Fmt<DD>::from16(A & 0xffffu) + Fmt<DD>::from16(A >> 16)) +
                       (Fmt<DD>::from16(B & 0xffffu) + Fmt<DD>::from16(B >> 16));
            }
            part = naiwa_group_sum<gpg>(part);
            if (in && (g % gpg) == 0) hs[g / gpg] = part;
        }
    }
}

// One wave: poll the tagged h vector of sorted position v (I/2 words) and stage
// it like stage_h (words at hw[v * I/2 ...], sums at hs[v * I/kSumSpan ...]).
template <int DD>
__device__ inline void stage_h_wave(const Params& p, int v, uint32_t* hw, float* hs, uint32_t tag, int lane) {
    constexpr int gpg = Fmt<DD>::kSumSpan / 4;
    constexpr int G = 3; // 4-value groups per lane per round (I = 768: one round)
    const int gpv = p.I / 4;
    const u64* src = p.h + (size_t)v * (p.I / 2);
    uint32_t* hwv = hw + (size_t)v * (p.I / 2);
    float* hsv = hs + (size_t)v * (p.I / Fmt<DD>::kSumSpan);
    for (int g0 = 0; g0 < gpv; g0 += 64 * G) {
        u64 w[2 * G];
        auto addr = [&](int j) -> const u64* {
            const int g = g0 + lane + (j >> 1) * 64;
            return g < gpv ? src + 2 * g + (j & 1) : nullptr;
        };
        issue_tagged(w, addr, tag);
        wait_tagged(w, addr, tag, p);
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const int g = g0 + lane + j * 64;
            const bool in = g < gpv;
            const uint32_t A = (uint32_t)w[2 * j], B = (uint32_t)w[2 * j + 1]; // (h0, h1), (h2, h3)
            float part = 0.0f;
            if (in) {
                hwv[2 * g] = (A & 0xffffu) | (B << 16);
                hwv[2 * g + 1] = (A >> 16) | (B & 0xffff0000u);
                part = (Fmt<DD>::from16(A & 0xffffu) + Fmt<DD>::from16(A >> 16)) +
                       (Fmt<DD>::from16(B & 0xffffu) + Fmt<DD>::from16(B >> 16));
            }
            part = naiwa_group_sum<gpg>(part);
            if (in && (g % gpg) == 0) hsv[g / gpg] = part;
        }
    }
}

// Model shapes with an instantiation of their own (the launch checks the sizes).
template <int SH> struct FixedShape;
template <> struct FixedShape<1> { // Qwen3-30B-A3B: hidden 2048, 128 experts, top-8, intermediate 768
    static constexpr int H = 2048, I = 768, E = 128, k = 8;
};

// The pointer, as a value the compiler cannot see through: address math on it
// is then redone inside the layer loop instead of being hoisted out and kept
// live in registers across all layers.
template <class T>
__device__ __forceinline__ T* opaque(T* ptr) {
    asm volatile("" : "+s"(ptr));
    return ptr;
}

// MR: the largest rows (tokens per step) this instantiation serves, 1 or kMaxRows;
// it sizes the per-thread (token, expert) item arrays.  SH: 0 for any shape, or a
// FixedShape whose routing sizes the kernel then knows at compile time: the routing
// loops unroll and their bounds and addresses fold to constants, so fewer scalar
// values are live across the layer loop.  The scalar registers overflow into vector
// lanes in this kernel, and every reload of a spilled value is a v_readlane; at the
// Qwen3-30B-A3B shape this took the bs1 token from 786-805 to 769-773 us.  TR: false
// compiles the phase marks out (the trace buffer is then never written): 755-770 ->
// 745-748 us, for the same reason.
template <int DG, int DD, int MR, int SH, bool TR>
__global__ void __launch_bounds__(kThreads)
stack_kernel(Params p) {
    if constexpr (MR == 1) p.rows = 1;
    if constexpr (!TR) p.trace = nullptr;
    if constexpr (SH != 0) {
        // only the expert count and top k: with the hidden and intermediate sizes fixed
        // too, the unrolled loops spill vector registers to scratch
        p.E = FixedShape<SH>::E;
        p.k = FixedShape<SH>::k;
    }
    constexpr int PPT = (MR * kMaxE + kThreads - 1) / kThreads; // router items per thread
    constexpr int XG = MR == 1 ? 2 : kXG;                       // activation groups per thread per round
    extern __shared__ __align__(16) uint8_t dyn[];
    __shared__ Smem sm;
    __shared__ LayerDev layers_lds[kMaxLayers];
    const int tid = threadIdx.x, grp = tid / NAIWA_GROUP, lr = tid % NAIWA_GROUP;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = gridDim.x, bid = blockIdx.x;
    const int H = p.H, I = p.I, E = p.E, k = p.k, rows = p.rows;
    const int npairs = rows * k;
    const int xstage = fused_xstage(DG, H);
    const int nchunks = H / kChunk;
    const int nprod = min(G, nchunks);        // workgroups that own chunks
    const int nlead = min(kLeaders, G);
    const int64_t rb = naiwa_row_bytes(DG == NAIWA_Q8_0_ODD ? NAIWA_Q8_0 : DG, H);
    const int64_t drb = naiwa_row_bytes(DD == NAIWA_Q8_0_ODD ? NAIWA_Q8_0 : DD, I);
    const int nb = H / NAIWA_QK_K;            // Q4_K blocks per gate/up row
    const int nu = Fmt<DG>::units(H);
    const int dnu = Fmt<DD>::units(I);
    const int gpt_h = H / 4;                  // 4-value groups per token
    const int half_h = H / 2;                 // tagged words per token
    const int nlog = rows * E;
    // after the activations, one region serves the gate/up rounds of phase B (wb) and the
    // h staging of phase C (hw, hs): a barrier separates the last read of one from the
    // first write of the other, in a layer and across layers
    uint8_t* const hdyn = dyn + rows * xstage;
    uint8_t* const wb = hdyn;                       // gate/up rounds
    uint32_t* const hw = (uint32_t*)hdyn;           // [hpairs][I/2] words
    float* const hs = (float*)(hdyn + (size_t)p.hpairs * I * 2); // [hpairs][I / kSumSpan] sums
    uint8_t* const dbuf = hdyn + p.hwb_bytes;       // prefetched down rows: [pair][kChunk][drb]
    float* const rbuf = (float*)(dbuf + (size_t)p.dpre * kChunk * drb); // next router columns [E][kChunk]

    // ---- prologue: layer descriptors into LDS; own chunks of x; layer-0 logits ----
    p.trace_layer = p.n_layers; // the prologue's row of the trace
    mark(p, p.n_layers, 0);
    for (int i = tid; i < p.n_layers * (int)(sizeof(LayerDev) / 8); i += kThreads)
        reinterpret_cast<unsigned long long*>(layers_lds)[i] =
            reinterpret_cast<const unsigned long long*>(p.layers)[i];
    {
        const uint32_t tag0 = layer_tag(p, 0);
        if (tid < rows * kChunk / 2) {
            const int t = tid / (kChunk / 2), pi = tid % (kChunk / 2);
            for (int cp = bid, ci = 0; cp < nchunks; cp += G, ++ci) {
                const int c = chunk_at(cp, nchunks);
                // written before the launch; each workgroup reads only its own chunks
                const uint32_t pr = *reinterpret_cast<const uint32_t*>(p.x + (size_t)t * H + c * kChunk + 2 * pi);
                sm.xown[ci][t][2 * pi] = naiwa_bf16_to_f32(pr & 0xffffu);
                sm.xown[ci][t][2 * pi + 1] = naiwa_bf16_to_f32(pr >> 16);
                st64(&p.xt[(size_t)t * half_h + c * (kChunk / 2) + pi], tagged(tag0, pr));
            }
        }
        __syncthreads();
        if (bid < nprod) {
            long long acc[PPT];
#pragma unroll
            for (int j = 0; j < PPT; ++j) acc[j] = 0;
            const float* W = layers_lds[0].router;
            for (int cp = bid, ci = 0; cp < nchunks; cp += G, ++ci) {
                const int f0 = chunk_at(cp, nchunks) * kChunk;
                router_chunk_accumulate<PPT, NAIWA_AS_GLOBAL>(p, [&](int e) { return W + (size_t)e * H + f0; }, sm.xown[ci], acc);
            }
            store_partials<PPT>(p, acc, nprod, tag0);
        }
        mark(p, p.n_layers, 1);
        if (bid < nlead) leader_reduce(p, nprod, tag0);
        mark(p, p.n_layers, 2);
    }

    for (int l = 0; l < p.n_layers; ++l) {
        p.h = opaque(p.h);
        p.trace_layer = l;
        p.part = opaque(p.part);
        p.logits = opaque(p.logits);
        p.xt = opaque(p.xt);
        p.x = opaque(p.x);
        const LayerDev L = layers_lds[l];
        const uint32_t tag = layer_tag(p, l);
        const bool last = l + 1 == p.n_layers;
        const uint32_t tag_next = layer_tag(p, l + 1);
        const u64* xt_l = p.xt + (size_t)(l & 1) * rows * half_h;

        // ---- A: poll logits + activations, rank, weights, segments ----
        const int ngroups = rows * gpt_h;
        uint32_t r_e = 0; // one token: wave 0 lane j's rank-j expert and its logit
        float r_f = 0.0f;
        // one token: the weights, computed by wave 0 once its gate/up loads are out
        auto weigh = [&]() {
            if constexpr (MR == 1)
                if (wave == 0) weigh_one_row(p, sm, l, lane, r_e, r_f);
        };
        if constexpr (MR == 1) {
            // wave 0 routes the token while waves 1-7 poll and stage its activations
            if (wave == 0) {
                poll_one_row(p, sm, L, l, tag, lane);
            } else {
                constexpr int NT = kThreads - 64;
                const int tx = tid - 64;
                for (int g0 = 0; g0 < ngroups; g0 += XG * NT) {
                    u64 xw[2 * XG];
                    auto xaddr = [&](int j) -> const u64* {
                        const int g = g0 + tx + (j >> 1) * NT;
                        return g < ngroups ? xt_l + 2 * g + (j & 1) : nullptr;
                    };
                    issue_tagged(xw, xaddr, tag);
                    wait_tagged(xw, xaddr, tag, p);
#pragma unroll
                    for (int j = 0; j < XG; ++j) {
                        const int g = g0 + tx + j * NT;
                        const bool in = g < ngroups;
                        const uint32_t a = (uint32_t)xw[2 * j], b = (uint32_t)xw[2 * j + 1];
                        stage_group<DG, DG == NAIWA_Q4_K>(naiwa_bf16_to_f32(a & 0xffffu), naiwa_bf16_to_f32(a >> 16),
                                                          naiwa_bf16_to_f32(b & 0xffffu), naiwa_bf16_to_f32(b >> 16),
                                                          in, in ? g : 0, dyn, H);
                    }
                }
                if (wave == 1) mark_wave(p, l, 13);
            }
            __syncthreads();
            mark(p, l, 0);
            if (E <= 128)
                rank_slice<2>(p, sm, wave, lane);
            else
                rank_slice<kMaxE / 64>(p, sm, wave, lane);
            __syncthreads();
            mark(p, l, 1);
            if (wave == 0) {
                if (E <= 128)
                    route_one_row<2>(p, sm, L, l, lane, r_e, r_f);
                else
                    route_one_row<kMaxE / 64>(p, sm, L, l, lane, r_e, r_f);
            }
        } else {
            for (int g0 = 0; g0 < ngroups; g0 += XG * kThreads) {
                u64 xw[2 * XG];
                auto xaddr = [&](int j) -> const u64* {
                    const int g = g0 + tid + (j >> 1) * kThreads;
                    if (g >= ngroups) return nullptr;
                    return xt_l + (size_t)(g / gpt_h) * half_h + 2 * (g % gpt_h) + (j & 1);
                };
                issue_tagged(xw, xaddr, tag);
                if (g0 == 0) {
                    u64 lw[PPT];
                    auto laddr = [&](int j) -> const u64* {
                        const int i = tid + j * kThreads;
                        return i < nlog ? p.logits + i : nullptr;
                    };
                    issue_tagged(lw, laddr, tag);
                    if (L.slot_of && tid < E) sm.slot_tab[tid] = naiwa_ld<int32_t, NAIWA_AS_GLOBAL>(L.slot_of + tid);
                    wait_tagged(lw, laddr, tag, p);
#pragma unroll
                    for (int j = 0; j < PPT; ++j) {
                        const int i = tid + j * kThreads;
                        if (i < nlog) {
                            const float f = __uint_as_float((uint32_t)lw[j]);
                            sm.lg[i / E][i % E] = f;
                            sm.key[i / E][i % E] = rank_key(f, i % E);
                        }
                    }
                    if ((E & 1) && tid < rows) sm.key[tid][E] = 0; // pad: below every real key
                }
                wait_tagged(xw, xaddr, tag, p);
#pragma unroll
                for (int j = 0; j < XG; ++j) {
                    const int g = g0 + tid + j * kThreads;
                    const bool in = g < ngroups;
                    const int t = in ? g / gpt_h : 0, gg = in ? g % gpt_h : 0;
                    const uint32_t a = (uint32_t)xw[2 * j], b = (uint32_t)xw[2 * j + 1];
                    stage_group<DG, DG == NAIWA_Q4_K>(naiwa_bf16_to_f32(a & 0xffffu), naiwa_bf16_to_f32(a >> 16),
                                                      naiwa_bf16_to_f32(b & 0xffffu), naiwa_bf16_to_f32(b >> 16),
                                                      in, gg, dyn + t * xstage, H);
                }
            }
            __syncthreads();
            mark(p, l, 0);
            {
                // rank of every (token, expert): the number of keys above its own;
                // tpi lanes per item split the comparisons
                const int items = rows * E;
                const int tpi = items * 4 <= kThreads ? 4 : (items * 2 <= kThreads ? 2 : 1);
                const int sub = tid % tpi;
                const int half_e = (E + 1) / 2;
                for (int it = tid / tpi; it < (items + (kThreads / tpi) - 1) / (kThreads / tpi) * (kThreads / tpi);
                     it += kThreads / tpi) {
                    const bool in = it < items;
                    const int t = in ? it / E : 0, e = in ? it % E : 0;
                    const u64 me = sm.key[t][e];
                    const ulonglong2* kv = reinterpret_cast<const ulonglong2*>(sm.key[t]);
                    int cnt = 0;
                    if (in) {
                        // 8 key pairs in flight per batch; a zero key is below every real key
#pragma unroll 4
                        for (int o = sub; o < half_e; o += tpi) {
                            const ulonglong2 v = kv[o];
                            cnt += (v.x > me) + (v.y > me);
                        }
                    }
                    if (tpi >= 2) cnt += __builtin_amdgcn_update_dpp(0, cnt, 0xB1, 0xF, 0xF, true);
                    if (tpi >= 4) cnt += __builtin_amdgcn_update_dpp(0, cnt, 0x4E, 0xF, 0xF, true);
                    if (in && sub == 0 && cnt < k) {
                        sm.top_ids[t][cnt] = (uint32_t)e;
                        sm.top_ex[t][cnt] = sm.lg[t][e];
                    }
                }
            }
            __syncthreads();
            mark(p, l, 1);
            if (wave == 0) {
                // weights (denominators summed in rank order, as the oracle does), then
                // slots and the grouping of valid pairs: one pair per lane
                const int q = lane;
                const bool inp = q < npairs;
                const int t = inp ? q / k : 0, j = inp ? q % k : 0;
                const float mx = sm.top_ex[t][0];
                const uint32_t e = inp ? sm.top_ids[t][j] : 0u;
                const float ex = inp ? expf(sm.top_ex[t][j] - mx) : 0.0f;
                sm.exv[q] = ex;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                float denom = 0.0f;
                if (inp) {
                    if (p.mode == NAIWA_ROUTE_SOFTMAX_TOPK) {
                        for (int o = 0; o < E; ++o) denom += expf(sm.lg[t][o] - mx);
                    } else {
                        for (int o = 0; o < k; ++o) denom += sm.exv[t * k + o];
                    }
                }
                group_pairs(p, sm, L, l, lane, inp, t, e, inp ? ex / denom : 0.0f);
            }
        }
        __syncthreads();
        const int nseg = sm.nseg;
        const int nvalid = (int)sm.seg_begin[nseg];
        mark(p, l, 2);
        if (threadIdx.x == 0) trace_put(p, l, 23, clock64()); // shader clock beside the real-time one

        // ---- B: gate/up ----
        const int total = nseg * (I / 2);        // (segment, row pair) items
        const int per = (total + G - 1) / G;
        const int q0 = bid * per, q1 = min(total, q0 + per);
        const bool owner = bid < nchunks;
        const int I2 = I / 2;
        // down rows of the first chunk for the first pairs: they depend on the
        // routing only, so they are on their way during gate/up and the h wait
        const int npre = owner ? min(p.dpre, nvalid) : 0;
        // (and the next layer's router columns of the first chunk, for its partials)
        // (returns the number of DMA instructions this wave issued)
        auto prefetch_down = [&]() -> int {
            if (!owner) return 0;
            int n = 0;
            const int f0 = chunk_at(bid, nchunks) * kChunk;
            const int span = kChunk * (int)drb / 16; // 16-byte pieces of kChunk consecutive rows
            for (int v = wave; v < npre; v += kThreads / 64) {
                const uint8_t* src = L.down + (int64_t)sm.pair_slot[sm.sorted[v]] * L.down_stride + (int64_t)f0 * drb;
                uint8_t* dst = dbuf + (size_t)v * kChunk * drb;
                for (int c = 0; c * 64 < span; ++c, ++n)
                    if (c * 64 + lane < span) lds_dma16_nt(src + (c * 64 + lane) * 16, dst + c * 1024);
            }
            if (!last) {
                // expert e's 8 columns (two 16-byte pieces) land at rbuf[e * kChunk]
                const float* Wn = layers_lds[l + 1].router;
                const int rpieces = 2 * E;
                for (int c = wave; c * 64 < rpieces; c += kThreads / 64, ++n) {
                    const int pc = c * 64 + lane;
                    if (pc < rpieces) lds_dma16(Wn + (size_t)(pc >> 1) * H + f0 + 4 * (pc & 1), rbuf + c * 256);
                }
            }
            return n;
        };
        if constexpr (DG == NAIWA_Q4_K) {
            // rounds of up to p.bitems items: the gate and up row pairs of each item
            // are gathered into LDS with coalesced 16-byte DMA pieces by the wave
            // that computes it, so each wave waits for its own pieces only.  Items i
            // and i + 8 of a round go to wave (i + 1) % 8, on its two 32-lane halves:
            // wave 0, which also computes the routing weights, gets the last ones
            const int pair_pieces = (int)(rb / 8);       // two rows, 16-byte pieces
            const size_t item_bytes = 4 * (size_t)rb;
            const int half = (tid >> 5) & 1, il = tid & 31;
            const int wslot = (wave + 7) % 8;
            const int my_item = wslot + 8 * half;
            for (int r0 = q0; r0 < q1 && MR == 1; r0 += p.bitems) {
                // one token: rows r of the wave's items (gate and up) go out first, then
                // rows r + 1, and the wave dots rows r while rows r + 1 are landing
                const int nr = min(p.bitems, q1 - r0);
                const int row_pieces = (int)(rb / 16);
                int n1 = 0; // DMA instructions of the rows r + 1
                for (int rr = 0; rr < 2; ++rr) {
                    for (int i = wslot; i < nr; i += kThreads / 64) {
                        const int q = r0 + i;
                        const uint32_t slot = sm.seg_slot[q / I2];
                        const int64_t roff = (int64_t)(2 * (q % I2) + rr) * rb;
                        const uint8_t* g = L.gate + (int64_t)slot * L.gate_stride + roff;
                        const uint8_t* u = L.up + (int64_t)slot * L.up_stride + roff;
                        uint8_t* dst = wb + (size_t)i * item_bytes + (size_t)rr * rb;
                        for (int c = 0; c * 64 < row_pieces; ++c) {
                            if (c * 64 + lane < row_pieces) {
                                lds_dma16_nt(g + (c * 64 + lane) * 16, dst + c * 1024);
                                lds_dma16_nt(u + (c * 64 + lane) * 16, dst + 2 * rb + c * 1024);
                            }
                            n1 += 2 * rr;
                        }
                    }
                }
                if (r0 == q0) weigh();
                vm_wait_at_most(n1); // rows r have landed (later operations only make it stricter)
                int npf = 0;
                if (r0 == q0) {
                    mark(p, l, 3);
                    mark_wave(p, l, 21);
                    npf = prefetch_down();
                }
                if (my_item < nr)
                    q4_pair_compute_split<DD>(p, sm, dyn, xstage, r0 + my_item, nb, il, wb + my_item * item_bytes, rb,
                                              tag, npf);
                else
                    vm_wait_at_most(npf); // the wave's own pieces land before the region is reused
            }
            for (int r0 = q0; r0 < q1 && MR != 1; r0 += p.bitems) {
                const int nr = min(p.bitems, q1 - r0);
                for (int i = wslot; i < nr; i += kThreads / 64) {
                    const int q = r0 + i;
                    const uint32_t slot = sm.seg_slot[q / I2];
                    const int64_t roff = (int64_t)(2 * (q % I2)) * rb;
                    const uint8_t* g = L.gate + (int64_t)slot * L.gate_stride + roff;
                    const uint8_t* u = L.up + (int64_t)slot * L.up_stride + roff;
                    uint8_t* dst = wb + (size_t)i * item_bytes;
                    for (int c = 0; c * 64 < pair_pieces; ++c) {
                        if (c * 64 + lane < pair_pieces) {
                            lds_dma16_nt(g + (c * 64 + lane) * 16, dst + c * 1024);
                            lds_dma16_nt(u + (c * 64 + lane) * 16, dst + 2 * rb + c * 1024);
                        }
                    }
                }
                if (r0 == q0) weigh();
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                if (r0 == q0) {
                    mark(p, l, 3);
                    mark_wave(p, l, 21); // every wave: the last one to land wins
                    prefetch_down();
                }
                if (my_item < nr)
                    q4_pair_compute<DD>(p, sm, dyn, xstage, r0 + my_item, nb, il, wb + my_item * item_bytes, rb, tag);
            }
            mark_wave(p, l, 16); // every wave: the last one to store wins
            if (q0 >= q1) {
                weigh();
                mark(p, l, 3);
                prefetch_down();
            }
        } else {
            weigh();
            mark(p, l, 3);
            prefetch_down();
#pragma unroll 1
            for (int q = q0 + grp; q < q1; q += kGroups) unit_pair<DG, DD>(p, sm, L, dyn, q, xstage, rb, nu, lr, tag);
        }
        // every h word of this workgroup is issued: say so with one tagged word,
        // right behind them (a consumer still checks every h word's tag, so the
        // done word only needs to follow the stores, not their completion)
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (tid == 0 && q0 < q1) st64(&p.done[bid], tagged(tag, 0u));
        mark(p, l, 4);

        // ---- C: down + ordered combine + residual + next layer's router partials ----
        if (owner) {
            long long racc[PPT];
#pragma unroll
            for (int j = 0; j < PPT; ++j) racc[j] = 0;
            u64* xt_next = p.xt + (size_t)((l + 1) & 1) * rows * half_h;
            // before reading all of h, wait (cheaply) for the done word of every
            // workgroup with gate/up items.  The full read below still checks every
            // word's tag; this only keeps the polling traffic small while the last
            // producers are still computing.
            // (wave 0 alone polls, four words per lane per round: fewer loads in flight)
            // one token with one pair per segment, every down row prefetched and one
            // output chunk per workgroup: wave v takes pair v alone -- the done words of
            // its own producers, its h, its 8 rows -- so the pairs whose producers finish
            // first are dotted while the last ones are still computing
            const bool pair_waves = MR == 1 && DD == NAIWA_Q4_K && nchunks <= G && nvalid == nseg &&
                                    nvalid <= kThreads / 64 && npre >= nvalid && dnu <= 8 * kDU8 &&
                                    I2 / max(per, 1) + 2 <= 64;
            if (!pair_waves) {
                const int nprod_h = (total + per - 1) / per;
                if (wave == 0) {
                    for (int b0 = 0; b0 < nprod_h; b0 += 256) {
                        u64 v[4];
                        auto addr = [&](int j) -> const u64* {
                            const int b2 = b0 + lane + 64 * j;
                            return b2 < nprod_h ? p.done + b2 : nullptr;
                        };
                        issue_tagged(v, addr, tag);
                        wait_tagged(v, addr, tag, p);
                    }
                }
                __syncthreads();
                mark(p, l, 14);
            }
            for (int cp = bid, ci = 0; cp < nchunks; cp += G, ++ci) {
                const int c = chunk_at(cp, nchunks);
                const int f0 = c * kChunk;
                if constexpr (MR == 1 && DD == NAIWA_Q4_K) {
                    if (pair_waves && wave < nvalid) {
                        const int v = wave; // sorted position = segment
                        // the producers of this pair's items: workgroups [v I2 / per, ((v + 1) I2 - 1) / per]
                        const int b_lo = v * I2 / per, b_hi = ((v + 1) * I2 - 1) / per;
                        u64 dw[1];
                        auto daddr = [&](int) -> const u64* { return b_lo + lane <= b_hi ? p.done + b_lo + lane : nullptr; };
                        issue_tagged(dw, daddr, tag);
                        wait_tagged(dw, daddr, tag, p);
                        if (wave == 0) mark_wave(p, l, 14);
                        stage_h_wave<DD>(p, v, hw, hs, tag, lane);
                        // this wave's prefetched rows (it issued pair v's) and its h staging
                        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                        if (wave == 0) mark_wave(p, l, 5);
                        __builtin_amdgcn_sched_barrier(0);
                        // 8-lane group fi: output feature fi of the chunk
                        const int fi = lane >> 3, l8 = lane & 7;
                        const uint8_t* drow = dbuf + (size_t)(v * kChunk + fi) * drb;
                        const uint32_t* words = hw + (size_t)v * (I / 2);
                        const float* sums = hs + (size_t)v * (I / Fmt<DD>::kSumSpan);
                        float acc = 0.0f;
#pragma unroll 1
                        for (int u = l8; u < dnu; u += 8)
                            acc += Fmt<DD>::dot(Fmt<DD>::template load<NAIWA_AS_LDS>(drow, u), u, words, sums);
                        const float dv = naiwa_group_sum<8>(acc);
                        if (l8 == 0) {
                            const float w = sm.pair_w[sm.sorted[v]];
                            sm.partial[fi][v] = w != 0.0f ? dv * w : 0.0f;
                        }
                    }
                }
                for (int b0 = 0; !pair_waves && b0 < nvalid; b0 += p.hpairs) {
                    const int nbp = min(p.hpairs, nvalid - b0);
                    if (ci > 0 || b0 > 0) __syncthreads(); // the previous pass's dots read hdyn
                    stage_h<DD>(p, b0, nbp, hw, hs, tag);
                    mark(p, l, 15);
                    // the prefetched rows have landed (vmcnt also counts LDS DMA)
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    __syncthreads();
                    // this pass's rows come from LDS when they were prefetched
                    const bool from_lds = ci == 0 && b0 == 0 && nbp <= npre;
                    mark(p, l, 5);
                    // dots of every (feature, pair) row with the pair's h: AS says
                    // where the rows are read from (global memory, or the LDS prefetch)
                    auto dots = [&](auto as) {
                        constexpr int AS = decltype(as)::value;
                        constexpr int DUM = 2;
                        const int nit = kChunk * nbp;
                        for (int it0 = grp; it0 < nit; it0 += kGroups * kCB) {
                            typename Fmt<DD>::Frag frg[kCB][DUM];
                            float acc[kCB];
#pragma unroll
                            for (int j = 0; j < kCB; ++j) acc[j] = 0.0f;
                            for (int base = lr; base < dnu; base += NAIWA_GROUP * DUM) {
#pragma unroll
                                for (int j = 0; j < kCB; ++j) {
                                    const int it = min(it0 + j * kGroups, nit - 1);
                                    const int fi = it % kChunk, pi = it / kChunk;
                                    const uint8_t* drow =
                                        AS == NAIWA_AS_LDS
                                            ? dbuf + (size_t)(pi * kChunk + fi) * drb
                                            : L.down + (int64_t)sm.pair_slot[sm.sorted[b0 + pi]] * L.down_stride +
                                                  (int64_t)(f0 + fi) * drb;
#pragma unroll
                                    for (int i = 0; i < DUM; ++i) {
                                        const int u = base + NAIWA_GROUP * i;
                                        if (u < dnu) frg[j][i] = Fmt<DD>::template load<AS>(drow, u);
                                    }
                                }
#pragma unroll
                                for (int j = 0; j < kCB; ++j) {
                                    const int it = min(it0 + j * kGroups, nit - 1);
                                    const uint32_t* words = hw + (size_t)(it / kChunk) * (I / 2);
                                    const float* sums = hs + (size_t)(it / kChunk) * (I / Fmt<DD>::kSumSpan);
#pragma unroll
                                    for (int i = 0; i < DUM; ++i) {
                                        const int u = base + NAIWA_GROUP * i;
                                        if (u < dnu) acc[j] += Fmt<DD>::dot(frg[j][i], u, words, sums);
                                    }
                                }
                            }
#pragma unroll
                            for (int j = 0; j < kCB; ++j) {
                                const int it = it0 + j * kGroups;
                                const float v = naiwa_group_sum<NAIWA_GROUP>(acc[j]);
                                if (it < nit && lr == 0) {
                                    // a zero weight contributes nothing, whatever the dot
                                    const float w = sm.pair_w[sm.sorted[b0 + it / kChunk]];
                                    sm.partial[it % kChunk][b0 + it / kChunk] = w != 0.0f ? v * w : 0.0f;
                                }
                            }
                        }
                    };
                    if constexpr (DD == NAIWA_Q4_K) {
                        if (from_lds && kChunk * nbp <= kThreads / 8 && dnu <= 8 * kDU8) {
                            // one 8-lane group per (feature, pair) row, at most kDU8 units
                            // (32 values) per lane: every lane busy at I = 768 (24 units)
                            const int g8 = tid >> 3, l8 = tid & 7;
                            const bool in = g8 < kChunk * nbp;
                            const int fi = in ? g8 % kChunk : 0, pi = in ? g8 / kChunk : 0;
                            const uint8_t* drow = dbuf + (size_t)(pi * kChunk + fi) * drb;
                            const uint32_t* words = hw + (size_t)pi * (I / 2);
                            const float* sums = hs + (size_t)pi * (I / Fmt<DD>::kSumSpan);
                            typename Fmt<DD>::Frag frg[kDU8];
#pragma unroll
                            for (int i = 0; i < kDU8; ++i)
                                if (in && l8 + 8 * i < dnu) frg[i] = Fmt<DD>::template load<NAIWA_AS_LDS>(drow, l8 + 8 * i);
                            float acc = 0.0f;
#pragma unroll
                            for (int i = 0; i < kDU8; ++i)
                                if (in && l8 + 8 * i < dnu) acc += Fmt<DD>::dot(frg[i], l8 + 8 * i, words, sums);
                            const float v = naiwa_group_sum<8>(acc);
                            if (in && l8 == 0) {
                                const float w = sm.pair_w[sm.sorted[b0 + pi]];
                                sm.partial[fi][b0 + pi] = w != 0.0f ? v * w : 0.0f;
                            }
                        } else if (from_lds) {
                            dots(std::integral_constant<int, NAIWA_AS_LDS>());
                        } else {
                            dots(std::integral_constant<int, NAIWA_AS_GLOBAL>());
                        }
                    } else {
                        dots(std::integral_constant<int, NAIWA_AS_GLOBAL>());
                    }
                }
                // prefetched pieces have landed even when no pass ran (no valid pair)
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
                mark(p, l, 6);
                if (tid < rows * kChunk) {
                    // ascending slot order per token, then the residual in f32 and the bf16 store value
                    const int t = tid / kChunk, fi = tid % kChunk;
                    float y = 0.0f;
#pragma unroll 1
                    for (int i0 = 0; i0 < nvalid; i0 += 8) {
                        float pv[8];
                        uint32_t tk[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const int i = i0 + j;
                            pv[j] = i < nvalid ? sm.partial[fi][i] : 0.0f;   // w * (down . h)
                            tk[j] = i < nvalid ? sm.srt_tok[i] : 0xFFFFFFFFu;
                        }
#pragma unroll
                        for (int j = 0; j < 8; ++j) y += tk[j] == (uint32_t)t ? pv[j] : 0.0f;
                    }
                    if (p.y_out) p.y_out[((size_t)l * rows + t) * H + f0 + fi] = y;
                    sm.xown[ci][t][fi] = naiwa_bf16_to_f32(naiwa_f32_to_bf16(sm.xown[ci][t][fi] + y));
                }
                __syncthreads();
                // the chunk's x words go out from the last wave (see item_thread)
                const int xs = tid - (kThreads - 64);
                if (xs >= 0 && xs < rows * kChunk / 2) {
                    const int t = xs / (kChunk / 2), pi = xs % (kChunk / 2);
                    const uint32_t pr = naiwa_f32_to_bf16(sm.xown[ci][t][2 * pi]) |
                                        (naiwa_f32_to_bf16(sm.xown[ci][t][2 * pi + 1]) << 16);
                    if (last)
                        *(__attribute__((address_space(1))) uint32_t*)(p.x + (size_t)t * H + f0 + 2 * pi) = pr;
                    else
                        st64(&xt_next[(size_t)t * half_h + c * (kChunk / 2) + pi], tagged(tag_next, pr));
                }
                mark(p, l, 7);
                if (!last && ci == 0) {
                    // the first chunk's columns were prefetched into LDS
                    router_chunk_accumulate<PPT, NAIWA_AS_LDS>(p, [&](int e) { return rbuf + e * kChunk; },
                                                              sm.xown[ci], racc);
                } else if (!last) {
                    const float* Wn = layers_lds[l + 1].router;
                    router_chunk_accumulate<PPT, NAIWA_AS_GLOBAL>(p, [&](int e) { return Wn + (size_t)e * H + f0; },
                                                             sm.xown[ci], racc);
                }
            }
            if (!last) store_partials<PPT>(p, racc, nprod, tag_next);
        }
        mark(p, l, 8);
        if (!last && bid < nlead) leader_reduce(p, nprod, tag_next);
        mark(p, l, 9);
        // LDS reuse across layers (dyn, sm) is ordered by this barrier
        __syncthreads();
    }
}

__global__ void zero_u32(unsigned int* ptr, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) ptr[i] = 0u;
}

// Before a launch: fold the previous launch's counters (words 0, 1) into the running
// totals (words 2, 3) and clear them; a launch's own wait timeout makes its later waits
// give up, so the per-launch word starts at zero.
__global__ void roll_status(int* st) {
    if (threadIdx.x == 0) {
        st[2] += st[0];
        st[3] += st[1];
        st[0] = 0;
        st[1] = 0;
    }
}

// The outputs of two one-token launches ([2][layers][k] ids and weights, [2][layers][H]
// MoE outputs) into the caller's [layers][2][...] layout; block (l, t).
__global__ void __launch_bounds__(256) interleave_tokens(const uint32_t* ids_t, const float* w_t, const float* y_t,
                                                         int L, int k, int H, uint32_t* ids, float* w, float* y) {
    const size_t src = (size_t)blockIdx.y * L + blockIdx.x, dst = (size_t)blockIdx.x * 2 + blockIdx.y;
    if (ids)
        for (int j = threadIdx.x; j < k; j += 256) {
            ids[dst * k + j] = ids_t[src * k + j];
            w[dst * k + j] = w_t[src * k + j];
        }
    if (y)
        for (int h = threadIdx.x; h < H; h += 256) y[dst * H + h] = y_t[src * H + h];
}

// Per device: the layer-descriptor sets uploaded so far, and the completion of the
// last fused launch.  A set never changes once uploaded (a new descriptor list gets
// its own set, copied on the launch stream), so a launch still queued on another
// stream keeps reading what it was given; the least recently used of kMaxSets sets
// is freed only after its last launch has completed.  Fused launches share the
// device's exchange scratch and each occupies every CU, so each one waits for the
// previous one, whatever stream either came from.
struct DescSet {
    std::vector<LayerDev> desc;
    LayerDev* dev = nullptr;    // device copy
    LayerDev* host = nullptr;   // pinned source of the upload (kept with the set)
    hipEvent_t ready = nullptr; // after the upload
    hipEvent_t used = nullptr;  // after the last launch that read it
    uint64_t stamp = 0;
};
struct FusedDev {
    std::mutex mu;
    std::vector<DescSet> sets;
    uint64_t clock = 0;
    hipEvent_t done = nullptr;  // after the last fused launch
    bool have_done = false;
};
constexpr size_t kMaxSets = 8;
FusedDev g_fused[64]; // per device (the launch checks dev < 64)

void free_set(DescSet& d) {
    if (d.used) (void)hipEventSynchronize(d.used);
    if (d.dev) (void)hipFree(d.dev);
    if (d.host) (void)hipHostFree(d.host);
    for (hipEvent_t ev : {d.ready, d.used})
        if (ev) (void)hipEventDestroy(ev);
    d = DescSet{};
}

// The set holding `desc` on this device (uploaded on `st` if new), ready on `st`.
int desc_set(FusedDev& f, const std::vector<LayerDev>& desc, hipStream_t st, DescSet** out) {
    const size_t bytes = desc.size() * sizeof(LayerDev);
    for (DescSet& d : f.sets)
        if (d.desc.size() == desc.size() && memcmp(d.desc.data(), desc.data(), bytes) == 0) {
            d.stamp = ++f.clock;
            *out = &d;
            return naiwa_hip_rc(hipStreamWaitEvent(st, d.ready, 0));
        }
    if (f.sets.size() >= kMaxSets) {
        auto lru = std::min_element(f.sets.begin(), f.sets.end(),
                                    [](const DescSet& a, const DescSet& b) { return a.stamp < b.stamp; });
        free_set(*lru);
        f.sets.erase(lru);
    }
    DescSet d;
    d.desc = desc;
    int rc = 0;
    if ((rc = naiwa_hip_rc(hipMalloc(&d.dev, bytes))) || (rc = naiwa_hip_rc(hipHostMalloc(&d.host, bytes, 0))) ||
        (rc = naiwa_hip_rc(hipEventCreateWithFlags(&d.ready, hipEventDisableTiming))) ||
        (rc = naiwa_hip_rc(hipEventCreateWithFlags(&d.used, hipEventDisableTiming)))) {
        free_set(d);
        return rc;
    }
    memcpy(d.host, desc.data(), bytes);
    if ((rc = naiwa_hip_rc(hipMemcpyAsync(d.dev, d.host, bytes, hipMemcpyHostToDevice, st))) ||
        (rc = naiwa_hip_rc(hipEventRecord(d.ready, st)))) {
        (void)hipStreamSynchronize(st);
        free_set(d);
        return rc;
    }
    d.stamp = ++f.clock;
    f.sets.push_back(std::move(d));
    *out = &f.sets.back();
    return NAIWA_OK;
}

template <int DG, int DD, int MR, int SH, bool TR>
int launch(const Params& prm, int blocks, size_t lds, hipStream_t st) {
    auto fn = stack_kernel<DG, DD, MR, SH, TR>;
    Params copy = prm;
    void* args[] = {&copy};
    hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    // The grid never exceeds the blocks every CU can hold at once (checked
    // against the occupancy above), so a plain launch is resident when the
    // device is not shared; the bounded waits keep it safe when it is, and the
    // status counters report it.  (A cooperative launch, where the runtime
    // checks residency, measured about 20 us slower per step and is not used.)
    e = hipLaunchKernel((const void*)fn, dim3(blocks), dim3(kThreads), args, (unsigned)lds, st);
    return naiwa_hip_rc(e);
}

template <int DG, int DD, int MR, int SH, bool TR>
int occupancy(size_t lds, int* per_cu) {
    return naiwa_hip_rc(hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, stack_kernel<DG, DD, MR, SH, TR>,
                                                                     kThreads, lds));
}

// The instantiation for (gate/up format, down format, rows class): op(fn) on it.
// sh: the FixedShape the sizes match (0: none); trace: the phase marks are wanted.
// The fixed-shape kernel has a traced and an untraced instantiation; the others
// test for a trace buffer at run time.
template <int MR, class Op>
int with_kernel(int fg, int fd, int sh, bool trace, const Op& op) {
    if constexpr (MR == 1)
        if (sh == 1 && fg == NAIWA_Q4_K && fd == NAIWA_Q4_K)
            return trace ? op.template run<NAIWA_Q4_K, NAIWA_Q4_K, 1, 1, true>()
                         : op.template run<NAIWA_Q4_K, NAIWA_Q4_K, 1, 1, false>();
    if (fg == NAIWA_Q4_K && fd == NAIWA_Q4_K) return op.template run<NAIWA_Q4_K, NAIWA_Q4_K, MR, 0, true>();
    if (fg == NAIWA_Q4_K && fd == NAIWA_Q8_0) return op.template run<NAIWA_Q4_K, NAIWA_Q8_0, MR, 0, true>();
    if (fg == NAIWA_Q4_K && fd == NAIWA_Q8_0_ODD) return op.template run<NAIWA_Q4_K, NAIWA_Q8_0_ODD, MR, 0, true>();
    if (fg == NAIWA_Q8_0 && fd == NAIWA_Q8_0) return op.template run<NAIWA_Q8_0, NAIWA_Q8_0, MR, 0, true>();
    if (fg == NAIWA_Q8_0 && fd == NAIWA_Q8_0_ODD) return op.template run<NAIWA_Q8_0, NAIWA_Q8_0_ODD, MR, 0, true>();
    return NAIWA_E_UNSUPPORTED;
}

struct OccupancyOp {
    size_t lds;
    int* per_cu;
    template <int DG, int DD, int MR, int SH, bool TR>
    int run() const { return occupancy<DG, DD, MR, SH, TR>(lds, per_cu); }
};

struct LaunchOp {
    const Params* prm;
    int blocks;
    size_t lds;
    hipStream_t st;
    template <int DG, int DD, int MR, int SH, bool TR>
    int run() const { return launch<DG, DD, MR, SH, TR>(*prm, blocks, lds, st); }
};

} // namespace

static int g_fused_blocks_per_cu = 1;
static bool g_trace_enabled = false;
static int g_trace_layers = 0;
static int g_trace_blocks = 0;

// Phase timestamps of the fused kernel (diagnostic): when on, every block
// records s_memrealtime ticks at each phase boundary of every layer.
extern "C" int naiwa_stack_trace_enable(int on) {
    g_trace_enabled = on != 0;
    return NAIWA_OK;
}

// Copies the last traced launch's timestamps: [blocks][n_layers + 1][24] u64
// ticks (the extra layer row is the prologue).  Synchronizes the device.
extern "C" int naiwa_stack_trace_read(uint64_t* out, int capacity, int* n_layers, int* blocks) {
    int rc = 0;
    if (!g_trace_layers) return NAIWA_E_NOT_FOUND;
    const size_t n = (size_t)g_trace_blocks * (g_trace_layers + 1) * kTraceSlots;
    if (!out || capacity < 0 || (size_t)capacity < n) return NAIWA_E_INVALID;
    void* t = naiwa_scratch(NAIWA_SCRATCH_FUSED_TRACE, n * 8, &rc);
    if (!t) return rc;
    if (n_layers) *n_layers = g_trace_layers;
    if (blocks) *blocks = g_trace_blocks;
    return naiwa_hip_rc(hipMemcpy(out, t, n * 8, hipMemcpyDeviceToHost));
}

extern "C" int naiwa_stack_set_blocks_per_cu(int n) {
    if (n < 1 || n > 8) return NAIWA_E_INVALID;
    g_fused_blocks_per_cu = n;
    return NAIWA_OK;
}

namespace {
constexpr size_t kStatusOff = 0;   // status words at the start of the sync scratch
constexpr int kMaxDev = 64;
// Per device: the launch counter behind the tags, and how many bytes of the
// tagged scratch are known to hold no current-looking tag (zeroed since the
// buffer was allocated and since the counter last wrapped).
uint32_t g_seq[kMaxDev];
size_t g_tag_clean[kMaxDev];
std::mutex g_seq_mu;
}

// Status of every fused launch since the last read: waits that gave up after their
// 2 s bound, and routed experts that had no resident slot.  Reading resets the
// counters.  Synchronizes.
extern "C" int naiwa_stack_status(int* barrier_timeouts, int* missing_experts) {
    int rc = 0;
    bool fresh = false;
    uint8_t* sync = (uint8_t*)naiwa_scratch(NAIWA_SCRATCH_FUSED_STATUS, 4096, &rc, &fresh);
    if (!sync) return rc;
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return (int)e;
    int h[4] = {0, 0, 0, 0};
    if (!fresh && (e = hipMemcpy(h, sync + kStatusOff, sizeof(h), hipMemcpyDeviceToHost)) != hipSuccess) return (int)e;
    if (barrier_timeouts) *barrier_timeouts = h[0] + h[2];
    if (missing_experts) *missing_experts = h[1] + h[3];
    const int zero[4] = {0, 0, 0, 0};
    return naiwa_hip_rc(hipMemcpy(sync + kStatusOff, zero, sizeof(zero), hipMemcpyHostToDevice));
}

int naiwa_stack_fused(const naiwa_layer* layers, int n_layers, void* x, int rows, int H, int E, int k,
                      int mode, int act, uint32_t* ids_out, float* w_out, float* y_out, int64_t stream) {
    if (rows > kMaxRows || k > kMaxK || E > kMaxE || n_layers > kMaxLayers) return NAIWA_E_UNSUPPORTED;
    if (H % kChunk || (ids_out == nullptr) != (w_out == nullptr)) return NAIWA_E_INVALID;
    if (mode < 0 || mode > 2 || (act != NAIWA_ACT_SILU && act != NAIWA_ACT_GELU_PYTORCH_TANH))
        return NAIWA_E_UNSUPPORTED;
    if (((uintptr_t)x & 15) != 0) return NAIWA_E_INVALID;
    const naiwa_layer& L0 = layers[0];
    const int I = L0.gate.n;
    for (int l = 0; l < n_layers; ++l) {
        const naiwa_layer& L = layers[l];
        if (!L.router || !L.gate.base || !L.up.base || !L.down.base) return NAIWA_E_INVALID;
        if (L.gate.k != H || L.up.k != H || L.down.n != H || L.gate.n != I || L.up.n != I || L.down.k != I)
            return NAIWA_E_INVALID;
        if (L.gate.dtype != L0.gate.dtype || L.up.dtype != L0.gate.dtype || L.down.dtype != L0.down.dtype)
            return NAIWA_E_UNSUPPORTED;
        if (L.gate.slots != L.up.slots || L.gate.slots != L.down.slots) return NAIWA_E_INVALID;
        if (!L.slot_of_expert && L.gate.slots < E) return NAIWA_E_INVALID;
        const int64_t rg = naiwa_row_bytes(L.gate.dtype, H), rd = naiwa_row_bytes(L.down.dtype, I);
        if (rg < 0 || rd < 0 || L.gate.slot_stride < rg * I || L.up.slot_stride < rg * I ||
            L.down.slot_stride < rd * H)
            return NAIWA_E_INVALID;
        if (((uintptr_t)L.gate.base | (uintptr_t)L.up.base | (uintptr_t)L.down.base | L.gate.slot_stride |
             L.up.slot_stride | L.down.slot_stride) & 15)
            return NAIWA_E_INVALID;
        if (((uintptr_t)L.router & 15) || H % 32 || I % 32) return NAIWA_E_INVALID;
    }
    const int fg = naiwa_kernel_fmt(L0.gate.dtype, H), fd = naiwa_kernel_fmt(L0.down.dtype, I);
    if (fg == NAIWA_Q8_0_ODD) return NAIWA_E_UNSUPPORTED;
    if (fg == NAIWA_Q4_K && H > 8 * NAIWA_QK_K) return NAIWA_E_UNSUPPORTED; // one block per lane: H <= 2048
    const int sh = H == FixedShape<1>::H && I == FixedShape<1>::I && E == FixedShape<1>::E && k == FixedShape<1>::k;
    // Two tokens at the fixed shape run as two one-token launches, their routing and
    // outputs interleaved into the caller's layout afterwards: the one-token kernel's
    // paths make that faster than one two-token launch (~1.49 against 1.69 ms a step).
    const int launches = rows == 2 && sh && fg == NAIWA_Q4_K && fd == NAIWA_Q4_K ? 2 : 1;
    const int krows = rows / launches; // tokens per launch
    // dynamic LDS: activations | h staging
    constexpr size_t kMaxDynLds = 104 * 1024;   // 160 KB per CU minus the static LDS
    const size_t lds_x = (size_t)krows * fused_xstage(fg, H);
    const size_t lds_r = (size_t)E * kChunk * 4; // the next layer's router columns of the first chunk
    // activations | max(h staging, gate/up rounds) | prefetched down rows | router columns
    const size_t item = fg == NAIWA_Q4_K ? 4 * (size_t)naiwa_row_bytes(NAIWA_Q4_K, H) : 0;
    // h vectors per phase-C pass: as many as the pairs need, up to kCPairs, within the LDS
    int hpairs = std::min(kCPairs, krows * k);
    const size_t hstage = (size_t)naiwa_stage_bytes(fd, I);
    while (hpairs > 1 && lds_x + std::max((size_t)hpairs * hstage, item) + lds_r > kMaxDynLds) --hpairs;
    const size_t lds_h = (size_t)hpairs * hstage;
    if (lds_x + std::max(lds_h, item) + lds_r > kMaxDynLds) return NAIWA_E_UNSUPPORTED;
    // Q4_K down rows of the first phase-C pass, prefetched into LDS when phase C makes
    // a single pass (rows * k <= hpairs) and they fit beside one gate/up item
    int dpre = 0;
    size_t lds_pre = 0;
    if (fd == NAIWA_Q4_K && krows * k <= hpairs) {
        const size_t pre = (size_t)hpairs * kChunk * (size_t)naiwa_row_bytes(NAIWA_Q4_K, I);
        if (lds_x + std::max(lds_h, item) + pre + lds_r <= kMaxDynLds) {
            dpre = hpairs;
            lds_pre = pre;
        }
    }
    // Q4_K gate/up rounds: at most one item per 32-lane half-wave, at most what one
    // workgroup's share of a full step needs, within the LDS left over (the h staging
    // of phase C reuses the same bytes)
    int bitems = 0;
    if (fg == NAIWA_Q4_K) {
        const int share = (krows * k * (I / 2) + 255) / 256;
        bitems = (int)std::min<size_t>((size_t)std::min(kThreads / 32, share),
                                       (kMaxDynLds - lds_x - lds_pre - lds_r) / item);
        if (bitems < 1) return NAIWA_E_UNSUPPORTED;
    }
    const size_t hwb = (std::max(lds_h, (size_t)bitems * item) + 15) & ~size_t(15);
    size_t lds = lds_x + hwb + lds_pre + lds_r;
    if (lds > kMaxDynLds) return NAIWA_E_UNSUPPORTED;

    hipStream_t st = (hipStream_t)stream;
    int rc = 0, dev = 0, cus = 0, khz = 0;
    if ((rc = naiwa_hip_rc(hipGetDevice(&dev)))) return rc;
    if ((rc = naiwa_hip_rc(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)))) return rc;
    if ((rc = naiwa_hip_rc(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev)))) return rc;
    int per_cu = 0;
    const OccupancyOp occ{lds, &per_cu};
    const bool tr = g_trace_enabled;
    rc = krows == 1 ? with_kernel<1>(fg, fd, sh, tr, occ) : with_kernel<kMaxRows>(fg, fd, sh, tr, occ);
    if (rc) return rc;
    const int bpc = per_cu < g_fused_blocks_per_cu ? per_cu : g_fused_blocks_per_cu;
    if (bpc < 1) return NAIWA_E_UNSUPPORTED;
    const int blocks = cus * bpc;
    if (blocks < kLeaders || blocks > 4096) return NAIWA_E_UNSUPPORTED;

    const int nchunks = H / kChunk;
    if ((nchunks + blocks - 1) / blocks > kMaxChunks) return NAIWA_E_UNSUPPORTED;
    const int nprod = blocks < nchunks ? blocks : nchunks;
    if (dev < 0 || dev >= kMaxDev) return NAIWA_E_UNSUPPORTED;

    // tagged scratch: h [kMaxPairs][I] | partials [rows*E][nprod][2] | logits [rows*E] | x [2][rows][H/2] |
    // done [blocks]
    auto a256 = [](size_t b) { return (b + 255) & ~size_t(255); };
    const size_t h_bytes = a256((size_t)kMaxPairs * I * 8);
    const size_t part_bytes = a256((size_t)nprod * krows * E * 16);
    const size_t lg_bytes = a256((size_t)krows * E * 8);
    const size_t xt_bytes = a256((size_t)2 * krows * (H / 2) * 8);
    const size_t done_bytes = a256((size_t)blocks * 8);
    const size_t tag_bytes = h_bytes + part_bytes + lg_bytes + xt_bytes + done_bytes;
    bool fresh = false;
    uint8_t* ws = (uint8_t*)naiwa_scratch(NAIWA_SCRATCH_FUSED, tag_bytes, &rc, &fresh);
    if (!ws) return rc;
    bool sync_fresh = false;
    uint8_t* sync = (uint8_t*)naiwa_scratch(NAIWA_SCRATCH_FUSED_STATUS, 4096, &rc, &sync_fresh);
    if (!sync) return rc;
    // per-launch outputs of a two-launch step: ids, weights [2][layers][k], y [2][layers][H]
    const size_t tok_rk = (size_t)n_layers * k, tok_y = y_out ? (size_t)n_layers * H : 0;
    uint8_t* tout = nullptr;
    if (launches == 2 && (ids_out || y_out)) {
        tout = (uint8_t*)naiwa_scratch(NAIWA_SCRATCH_FUSED_TOKENS, 2 * (2 * tok_rk + tok_y) * 4, &rc);
        if (!tout) return rc;
    }
    uint32_t* const tids = tout ? (uint32_t*)tout : nullptr;
    float* const tw = tout ? (float*)tout + 2 * tok_rk : nullptr;
    float* const ty = tout ? (float*)tout + 4 * tok_rk : nullptr;
    // this launch's work on `st` (clearing the exchange words included) follows the previous
    // fused launch on this device, whatever its stream; the lock is held until this
    // launch's events are recorded
    FusedDev& fdev = g_fused[dev];
    std::lock_guard<std::mutex> flock(fdev.mu);
    if (!fdev.done && (rc = naiwa_hip_rc(hipEventCreateWithFlags(&fdev.done, hipEventDisableTiming)))) return rc;
    if (fdev.have_done && (rc = naiwa_hip_rc(hipStreamWaitEvent(st, fdev.done, 0)))) return rc;
    // a launch number for the tags of each launch (on clean exchange words)
    auto next_seq = [&]() -> uint32_t {
        std::lock_guard<std::mutex> lock(g_seq_mu);
        if (fresh) g_tag_clean[dev] = 0;
        fresh = false;
        if (++g_seq[dev] >= (1u << 24)) { // tags hold seq << 8: start over on clean memory
            g_seq[dev] = 1;
            g_tag_clean[dev] = 0;
        }
        if (g_tag_clean[dev] < tag_bytes) {
            const int n = (int)(tag_bytes / 4);
            zero_u32<<<(n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096, 256, 0, st>>>((unsigned int*)ws, n);
            g_tag_clean[dev] = tag_bytes;
        }
        return g_seq[dev];
    };

    // layer descriptors on the device (re-uploaded only when they change)
    std::vector<LayerDev> desc(n_layers);
    for (int l = 0; l < n_layers; ++l) {
        const naiwa_layer& L = layers[l];
        desc[l] = LayerDev{L.router, (const uint8_t*)L.gate.base, (const uint8_t*)L.up.base,
                           (const uint8_t*)L.down.base, L.gate.slot_stride, L.up.slot_stride,
                           L.down.slot_stride, L.slot_of_expert, L.gate.slots, 0};
    }
    DescSet* set = nullptr;
    if ((rc = desc_set(fdev, desc, st, &set))) return rc;
    LayerDev* dev_layers = set->dev;

    Params prm{};
    prm.layers = dev_layers;
    prm.n_layers = n_layers;
    prm.rows = krows;
    prm.H = H;
    prm.I = I;
    prm.E = E;
    prm.k = k;
    prm.mode = mode;
    prm.act = act;
    prm.x = (uint16_t*)x;
    prm.h = (u64*)ws;
    prm.part = (u64*)(ws + h_bytes);
    prm.logits = (u64*)(ws + h_bytes + part_bytes);
    prm.xt = (u64*)(ws + h_bytes + part_bytes + lg_bytes);
    prm.done = (u64*)(ws + h_bytes + part_bytes + lg_bytes + xt_bytes);
    prm.status = (int*)(sync + kStatusOff);
    prm.ids_out = ids_out;
    prm.w_out = w_out;
    prm.y_out = y_out;
    prm.spin_limit = (uint64_t)khz * 2000ull; // 2 s
    prm.bitems = bitems;
    prm.hpairs = hpairs;
    prm.dpre = dpre;
    prm.hwb_bytes = (int)hwb;
    prm.trace = g_trace_enabled ? (unsigned long long*)naiwa_scratch(
                                      NAIWA_SCRATCH_FUSED_TRACE, (size_t)blocks * (n_layers + 1) * kTraceSlots * 8, &rc)
                                : nullptr;
    if (g_trace_enabled && !prm.trace) return rc;
    g_trace_layers = n_layers;
    g_trace_blocks = blocks;
    if (sync_fresh) zero_u32<<<1, 64, 0, st>>>((unsigned int*)(sync + kStatusOff), 64);
    const LaunchOp go{&prm, blocks, lds, st};
    for (int t = 0; t < launches; ++t) {
        prm.seq = next_seq();
        prm.x = (uint16_t*)x + (size_t)t * krows * H;
        if (launches == 2) {
            prm.ids_out = ids_out ? tids + t * tok_rk : nullptr;
            prm.w_out = ids_out ? tw + t * tok_rk : nullptr;
            prm.y_out = y_out ? ty + t * tok_y : nullptr;
        }
        roll_status<<<1, 64, 0, st>>>((int*)(sync + kStatusOff));
        rc = krows == 1 ? with_kernel<1>(fg, fd, sh, tr, go) : with_kernel<kMaxRows>(fg, fd, sh, tr, go);
        if (rc) {
            // an earlier launch of this step is queued: later fused launches still follow it
            if (t > 0 && hipEventRecord(fdev.done, st) == hipSuccess) fdev.have_done = true;
            return rc;
        }
    }
    if (tout) {
        interleave_tokens<<<dim3((unsigned)n_layers, 2), 256, 0, st>>>(tids, tw, ty, n_layers, k, H, ids_out, w_out,
                                                                        y_out);
        if ((rc = naiwa_hip_rc(hipGetLastError()))) return rc;
    }
    // after the interleave: the next fused launch may reuse the per-launch outputs
    if ((rc = naiwa_hip_rc(hipEventRecord(fdev.done, st)))) return rc;
    fdev.have_done = true;
    return naiwa_hip_rc(hipEventRecord(set->used, st));
}
