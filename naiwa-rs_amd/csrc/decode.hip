// naiwa_moe_decode: the dequant-fused SwiGLU expert decode over a slot-indexed
// bank, replacing mistralrs_quant::indexed_moe_fused_decode as called at
// src/moe/stages/gpu.rs:27-66.
//
// Three launches, all stream-ordered:
//   1. segments: stable counting sort of the (token, slot) pairs by slot,
//      weight-0 pairs (the reference's padding, gpu.rs:117-129) left out;
//   2. gate+up: one block per (slot segment, tile of the intermediate); each
//      16-lane group owns one row of gate and the same row of up, streams their
//      codes with 16-byte loads and dots every code against up to 8 tokens of
//      the segment staged in LDS; h = act(g) * u;
//   3. down+combine: the output rows' (row, segment) items are spread over the
//      groups of each block; a row is streamed once per 8 tokens of its
//      segment and the weighted dots are added per (token, row) in ascending
//      slot order.  No atomics, so every run adds the same terms in the same
//      order.
// Calls of at most 512 pairs (16 per token) keep h in global memory in the down
// format's dot layout (written once by the gate/up blocks); the down rows are
// dotted in K parts of 2048 with the h slices in LDS, and a last launch adds the
// weighted parts per (token, row) in slot order.  Larger calls stage f32 h per
// block, 4 tokens per pass.
#include "decode.h"
#include "decode_mfma.h"
#include "rowdot.h"
#include "segments.h"
#include "workspace.h"

#include <algorithm>
#include <cstdlib>
#include <mutex>

namespace {

constexpr int kRowsPerBlock = 16;                    // 16 groups of 16 lanes
constexpr int kThreads = kRowsPerBlock * NAIWA_GROUP; // 256
constexpr int kTokMax = 4;                            // tokens staged per pass

struct BankArg {
    const uint8_t* base;
    int64_t stride;
    int64_t row_bytes;
};

__global__ void __launch_bounds__(NAIWA_SEG_THREADS)
segments_kernel(const uint32_t* slot_ids, const float* w, int n, int nslots, uint32_t* perm,
                int* seg_count, uint32_t* seg_key, uint32_t* seg_begin, int* bad) {
    __shared__ NaiwaSegSmem sm;
    naiwa_segment(sm, slot_ids, w, n, nslots, perm, nullptr, seg_count, seg_key, seg_begin, bad);
}

template <int DT>
__global__ void __launch_bounds__(kThreads)
gate_up_kernel(BankArg gate, BankArg up, const void* x, int x_bf16, int H, int I, int width,
               int tok_max, const int* seg_count, const uint32_t* seg_key,
               const uint32_t* seg_begin, const uint32_t* perm, int act, float* hbuf) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int s = blockIdx.x;
    if (s >= *seg_count) return;
    const int tid = threadIdx.x, grp = tid / NAIWA_GROUP, lr = tid % NAIWA_GROUP;
    const int r = blockIdx.y * kRowsPerBlock + grp;
    const uint32_t slot = seg_key[s];
    const int b = (int)seg_begin[s], e = (int)seg_begin[s + 1];
    const int stage = naiwa_stage_bytes(DT, H);
    const uint8_t* grow = gate.base + (int64_t)slot * gate.stride + (int64_t)r * gate.row_bytes;
    const uint8_t* urow = up.base + (int64_t)slot * up.stride + (int64_t)r * up.row_bytes;
    const int nu = Fmt<DT>::units(H);
    constexpr int UM = Umax<DT>::v;

    for (int c0 = b; c0 < e; c0 += tok_max) {
        const int nt = min(tok_max, e - c0);
        __syncthreads();
        for (int tt = 0; tt < nt; ++tt) {
            const int t = (int)perm[c0 + tt] / width;
            const void* src = x_bf16 ? (const void*)((const uint16_t*)x + (int64_t)t * H)
                                     : (const void*)((const float*)x + (int64_t)t * H);
            uint32_t* words = (uint32_t*)(smem + tt * stage);
            naiwa_stage<DT>(src, x_bf16 != 0, H, words, (float*)(words + H / 2), tid, kThreads);
        }
        __syncthreads();
        if (r >= I) continue;
        float ag[kTokMax], au[kTokMax];
#pragma unroll
        for (int tt = 0; tt < kTokMax; ++tt) ag[tt] = au[tt] = 0.0f;
        for (int base = lr; base < nu; base += NAIWA_GROUP * UM) {
            typename Fmt<DT>::Frag fg[UM], fu[UM];
#pragma unroll
            for (int i = 0; i < UM; ++i) {
                const int u = base + NAIWA_GROUP * i;
                if (u < nu) {
                    fg[i] = Fmt<DT>::load(grow, u);
                    fu[i] = Fmt<DT>::load(urow, u);
                }
            }
#pragma unroll
            for (int i = 0; i < UM; ++i) {
                const int u = base + NAIWA_GROUP * i;
                if (u >= nu) continue;
#pragma unroll
                for (int tt = 0; tt < kTokMax; ++tt) {
                    if (tt >= nt) break;
                    const uint32_t* words = (const uint32_t*)(smem + tt * stage);
                    const float* sums = (const float*)(words + H / 2);
                    ag[tt] += Fmt<DT>::dot(fg[i], u, words, sums);
                    au[tt] += Fmt<DT>::dot(fu[i], u, words, sums);
                }
            }
        }
#pragma unroll
        for (int tt = 0; tt < kTokMax; ++tt) {
            const float g = naiwa_group_sum<NAIWA_GROUP>(ag[tt]);
            const float u = naiwa_group_sum<NAIWA_GROUP>(au[tt]);
            if (tt < nt && lr == 0) hbuf[(int64_t)perm[c0 + tt] * I + r] = naiwa_act(act, g) * u;
        }
    }
}

template <int DT>
__global__ void __launch_bounds__(kThreads)
down_kernel(BankArg down, int H, int I, int rows, int width, int tok_max, const int* seg_count,
            const uint32_t* seg_key, const uint32_t* seg_begin, const uint32_t* perm,
            const float* w, const float* hbuf, int accumulate, float* out) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, grp = tid / NAIWA_GROUP, lr = tid % NAIWA_GROUP;
    const int r = blockIdx.x * kRowsPerBlock + grp;
    float* acc = (float*)smem; // [rows][kRowsPerBlock]
    const int acc_bytes = ((rows * kRowsPerBlock * 4) + 15) & ~15;
    uint8_t* stage_base = smem + acc_bytes;
    const int stage = naiwa_stage_bytes(DT, I);
    // the sum starts at 0, or at out's values (the same additions as one call over both sets)
    for (int i = tid; i < rows * kRowsPerBlock; i += kThreads) {
        const int rr = blockIdx.x * kRowsPerBlock + i % kRowsPerBlock;
        acc[i] = accumulate && rr < H ? out[(int64_t)(i / kRowsPerBlock) * H + rr] : 0.0f;
    }
    const int nseg = *seg_count;
    const int nu = Fmt<DT>::units(I);
    constexpr int UM = Umax<DT>::v;
    for (int s = 0; s < nseg; ++s) {
        const uint32_t slot = seg_key[s];
        const int b = (int)seg_begin[s], e = (int)seg_begin[s + 1];
        const uint8_t* drow = down.base + (int64_t)slot * down.stride + (int64_t)r * down.row_bytes;
        for (int c0 = b; c0 < e; c0 += tok_max) {
            const int nt = min(tok_max, e - c0);
            __syncthreads();
            for (int tt = 0; tt < nt; ++tt) {
                const float* src = hbuf + (int64_t)perm[c0 + tt] * I;
                uint32_t* words = (uint32_t*)(stage_base + tt * stage);
                naiwa_stage<DT>(src, false, I, words, (float*)(words + I / 2), tid, kThreads);
            }
            __syncthreads();
            if (r >= H) continue;
            float a[kTokMax];
#pragma unroll
            for (int tt = 0; tt < kTokMax; ++tt) a[tt] = 0.0f;
            for (int base = lr; base < nu; base += NAIWA_GROUP * UM) {
                typename Fmt<DT>::Frag f[UM];
#pragma unroll
                for (int i = 0; i < UM; ++i) {
                    const int u = base + NAIWA_GROUP * i;
                    if (u < nu) f[i] = Fmt<DT>::load(drow, u);
                }
#pragma unroll
                for (int i = 0; i < UM; ++i) {
                    const int u = base + NAIWA_GROUP * i;
                    if (u >= nu) continue;
#pragma unroll
                    for (int tt = 0; tt < kTokMax; ++tt) {
                        if (tt >= nt) break;
                        const uint32_t* words = (const uint32_t*)(stage_base + tt * stage);
                        a[tt] += Fmt<DT>::dot(f[i], u, words, (const float*)(words + I / 2));
                    }
                }
            }
#pragma unroll
            for (int tt = 0; tt < kTokMax; ++tt) {
                const float v = naiwa_group_sum<NAIWA_GROUP>(a[tt]);
                if (tt < nt && lr == 0) {
                    const uint32_t p = perm[c0 + tt];
                    acc[(p / width) * kRowsPerBlock + grp] += w[p] * v;
                }
            }
        }
    }
    __syncthreads();
    if (r < H && lr == 0)
        for (int t = 0; t < rows; ++t) out[(int64_t)t * H + r] = acc[t * kRowsPerBlock + grp];
}

// ---------------------------------------------------------------------------
// Decode with h staged once in global memory (calls of at most kPairsMax pairs)
// ---------------------------------------------------------------------------
// gate_up_staged: one block per (slot segment, span of I rows), span = the down
// format's sum span (16 rows for Q4_K down, 32 for Q8_0), one 16-lane group per
// row; up to kTokG tokens of the segment are staged in LDS per pass and every
// weight unit loaded is dotted with all of them.  The block then writes its
// rows of each token's h straight in the down format's dot layout (16-bit pair
// words + span sums, the same rounding and summation order as staging the f32
// h would give) to hst[pair].
// down_split + down_combine: the down rows' dots over K parts of I with the h
// slices staged in LDS (below), then the ordered per-(token, row) combine.
constexpr int kPairsMax = 512;
constexpr int kSmallSeg = 64; // calls of at most this many pairs are segmented inside gate/up

// The call's (slot, weight) pairs when gate/up segments them itself (slot_ids null:
// the segments launch has run).
struct SegIn {
    const uint32_t* slot_ids;
    const float* w;
    int n, nslots;
    int* bad;
};
// The folded wait of a call (flag null: none).  count: this waiter adds to *fail when
// it runs out (one waiter per call counts).
struct WaitArg {
    const uint32_t* flag;
    uint32_t target;
    uint64_t limit;
    uint32_t* fail;
};
__device__ inline void wait_flag(const WaitArg& a, bool count) {
    const uint64_t t0 = wall_clock64();
    // relaxed spin loads (an acquire load invalidates the L2 on every try), one acquire
    // after: the rows the other stream wrote are read only behind it
    while (__hip_atomic_load(a.flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) < a.target) {
        if (wall_clock64() - t0 > a.limit) {
            if (count) {
                const uint32_t n = __hip_atomic_load(a.fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                __hip_atomic_store(a.fail, n + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}
__global__ void __launch_bounds__(64) decode_wait_kernel(WaitArg a) {
    if (threadIdx.x == 0) wait_flag(a, true);
}

constexpr int kTokG = 8;
constexpr int kTokD = 8;
constexpr int kDownThreads = 256;
constexpr int kSplitK = 2048;     // I elements per K part of the down projection
constexpr int kCombineWidth = 16; // most pairs per token the combine orders
constexpr int kCombineParts = 8;  // K parts whose loads a combine lane issues at once
constexpr int kCombinePairs = 8;  // pairs whose loads a combine lane issues at once

// The staged-h path serves calls of at most kPairsMax pairs and kCombineWidth per token.
bool split_path(int n, int width) { return n <= kPairsMax && width <= kCombineWidth; }

// Calls of at least this many rows run their expert GEMMs on the matrix cores
// (NAIWA_DECODE_MFMA_ROWS; 0 switches the matrix-core decode off).
int mfma_rows() {
    static const int v = [] {
        const char* e = std::getenv("NAIWA_DECODE_MFMA_ROWS");
        return e && *e ? std::atoi(e) : 4;
    }();
    return v;
}
int split_ks(int I) { return I <= kSplitK ? I : kSplitK; }
int split_parts(int I) { return (I + split_ks(I) - 1) / split_ks(I); }

// TG: tokens staged per chunk at most (1, 4 or 8).  Calls of few tokens take a
// small TG: the accumulators of more tokens would hold registers, and with them the
// occupancy.  With TG <= 4 a Q4_K lane also loads 2 units of each row per round
// instead of 4; at 136-152 VGPRs a SIMD then keeps 3 waves instead of 2 (Mixtral
// bs1 367 -> 445 tok/s).
// one_row: the call has one token, whose activations are staged once, before the
// segments are known (by the waves other than wave 0 while it segments the pairs).
template <int DG, int DD, int TG>
__global__ void __launch_bounds__(512, TG == 1 || (TG <= 4 && DG != NAIWA_Q8_0) ? 3 : 1)
gate_up_staged_kernel(BankArg gate, BankArg up, const void* x, int x_bf16, int H, int I, int width, int tok_max,
                      const int* seg_count, const uint32_t* seg_key, const uint32_t* seg_begin,
                      const uint32_t* perm, int act, uint8_t* hst, int hst_stride, SegIn seg_in, int one_row,
                      WaitArg wt) {
    constexpr int SPAN = Fmt<DD>::kSumSpan;   // rows per block (one group of 16 lanes each)
    constexpr int GPG = SPAN / 4;             // 4-row groups per sum
    constexpr int NT = SPAN * NAIWA_GROUP;    // threads per block
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float hloc[TG][SPAN];
    __shared__ uint32_t l_perm[kSmallSeg], l_key[kSmallSeg], l_begin[kSmallSeg + 1];
    __shared__ int l_count, l_bad;
    const int wave = threadIdx.x >> 6;
    if (seg_in.slot_ids) {
        // the call's few pairs segmented by this block (wave 0) into LDS, meanwhile the one
        // token's activations staged by the other waves; block (0, 0)'s wave 1 then writes
        // the global copy of the segments the down launches read
        if (wave == 0)
            naiwa_segment_small(seg_in.slot_ids, seg_in.w, seg_in.n, seg_in.nslots, l_perm, &l_count, l_key, l_begin,
                                &l_bad);
        else if (one_row)
            naiwa_stage<DG>(x, x_bf16 != 0, H, (uint32_t*)smem, (float*)((uint32_t*)smem + H / 2), threadIdx.x - 64,
                            NT - 64);
        __syncthreads();
        if (wave == 1 && blockIdx.x == 0 && blockIdx.y == 0) {
            const int lane = threadIdx.x & 63, c = l_count;
            if (lane < seg_in.n) ((uint32_t*)perm)[lane] = l_perm[lane];
            if (lane < c) ((uint32_t*)seg_key)[lane] = l_key[lane];
            if (lane <= c) ((uint32_t*)seg_begin)[lane] = l_begin[lane];
            if (lane == 0) {
                *(int*)seg_count = c;
                *seg_in.bad = l_bad;
            }
        }
        seg_count = &l_count;
        seg_key = l_key;
        seg_begin = l_begin;
        perm = l_perm;
    } else if (one_row) {
        naiwa_stage<DG>(x, x_bf16 != 0, H, (uint32_t*)smem, (float*)((uint32_t*)smem + H / 2), threadIdx.x, NT);
    }
    const int s = blockIdx.x;
    if (s >= *seg_count) return;
    // the folded wait: every block's thread 0 waits (block (0, 0)'s counts a timeout)
    if (wt.flag) {
        if (threadIdx.x == 0) wait_flag(wt, blockIdx.x == 0 && blockIdx.y == 0);
        __syncthreads();
    }
    const int tid = threadIdx.x, grp = tid / NAIWA_GROUP, lr = tid % NAIWA_GROUP;
    const int r0 = blockIdx.y * SPAN, r = r0 + grp;
    const uint32_t slot = seg_key[s];
    const int b = (int)seg_begin[s], e = (int)seg_begin[s + 1];
    const int stage = naiwa_stage_bytes(DG, H);
    const uint8_t* grow = gate.base + (int64_t)slot * gate.stride + (int64_t)r * gate.row_bytes;
    const uint8_t* urow = up.base + (int64_t)slot * up.stride + (int64_t)r * up.row_bytes;
    const int nu = Fmt<DG>::units(H);
    constexpr int UM = TG <= 4 && DG == NAIWA_Q4_K ? 2 : Umax<DG>::v;
    for (int c0 = b; c0 < e; c0 += tok_max) {
        const int nt = min(tok_max, e - c0);
        __syncthreads();
        for (int tt = 0; tt < nt && !one_row; ++tt) {
            const int t = (int)perm[c0 + tt] / width;
            const void* src = x_bf16 ? (const void*)((const uint16_t*)x + (int64_t)t * H)
                                     : (const void*)((const float*)x + (int64_t)t * H);
            uint32_t* words = (uint32_t*)(smem + tt * stage);
            naiwa_stage<DG>(src, x_bf16 != 0, H, words, (float*)(words + H / 2), tid, NT);
        }
        __syncthreads();
        float ag[TG], au[TG];
#pragma unroll
        for (int tt = 0; tt < TG; ++tt) ag[tt] = au[tt] = 0.0f;
        if (r < I) {
            for (int base = lr; base < nu; base += NAIWA_GROUP * UM) {
                typename Fmt<DG>::Frag fg[UM], fu[UM];
#pragma unroll
                for (int i = 0; i < UM; ++i) {
                    const int u = base + NAIWA_GROUP * i;
                    if (u < nu) {
                        fg[i] = Fmt<DG>::load(grow, u);
                        fu[i] = Fmt<DG>::load(urow, u);
                    }
                }
#pragma unroll
                for (int i = 0; i < UM; ++i) {
                    const int u = base + NAIWA_GROUP * i;
                    if (u >= nu) continue;
#pragma unroll
                    for (int tt = 0; tt < TG; ++tt) {
                        if (tt >= nt) break;
                        const uint32_t* words = (const uint32_t*)(smem + (one_row ? 0 : tt) * stage);
                        const float* sums = (const float*)(words + H / 2);
                        ag[tt] += Fmt<DG>::dot(fg[i], u, words, sums);
                        au[tt] += Fmt<DG>::dot(fu[i], u, words, sums);
                    }
                }
            }
        }
#pragma unroll
        for (int tt = 0; tt < TG; ++tt) {
            const float g = naiwa_group_sum<NAIWA_GROUP>(ag[tt]);
            const float u = naiwa_group_sum<NAIWA_GROUP>(au[tt]);
            if (tt < nt && lr == 0) hloc[tt][grp] = r < I ? naiwa_act(act, g) * u : 0.0f;
        }
        __syncthreads();
        // the block's rows of each token's h in the down format's dot layout: thread
        // (tt, g4) writes the pair words of rows r0 + 4 g4 .. + 3, and the span's sum
        // (every lane of the first wave takes part in the group sums)
        if (tid < 64) {
            const bool in = tid < nt * GPG;
            const int tt = in ? tid / GPG : 0, g4 = tid % GPG;
            uint32_t h[4];
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h[i] = Fmt<DD>::to16(hloc[tt][4 * g4 + i]);
                v[i] = Fmt<DD>::from16(h[i]);
            }
            uint32_t* words = (uint32_t*)(hst + (size_t)perm[c0 + tt] * hst_stride);
            const int g = r0 / 4 + g4;
            if (in) {
                words[2 * g] = h[0] | (h[2] << 16);
                words[2 * g + 1] = h[1] | (h[3] << 16);
            }
            float part = (v[0] + v[1]) + (v[2] + v[3]);
            part = naiwa_group_sum<GPG>(part);
            if (in && g4 == 0) ((float*)(words + I / 2))[r0 / SPAN] = part;
        }
    }
}

// down_split: the down projection in K parts.  Block (row tile, K part, segment):
// up to tok_max tokens of the segment at a time have their h slice [k0, k0 + kn)
// copied from hst into LDS, and each 16-lane group streams its rows' slices,
// two rows at a time, dotting every unit with every staged token.  The unweighted
// partial dot of (K part, sorted position, row) goes to dpart.
// TD: tokens staged per chunk at most (1, 4 or 8), as TG of gate/up; one token of a
// Q4_K down projection loads 2 units per round and fits 4 waves a SIMD.
template <int DD, int TD>
__global__ void __launch_bounds__(kDownThreads, TD == 1 ? (DD == NAIWA_Q4_K ? 4 : 3) : (TD <= 4 ? 3 : 1))
down_split_kernel(BankArg down, int H, int I, int ks, int rpg, int tok_max, int n, const int* seg_count,
                  const uint32_t* seg_key, const uint32_t* seg_begin, const uint32_t* perm, const uint8_t* hst,
                  int hst_stride, float* dpart) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int SPAN = Fmt<DD>::kSumSpan;
    constexpr int UM = TD == 1 && DD == NAIWA_Q4_K ? 2 : Umax<DD>::v;
    const int sgi = blockIdx.z;
    if (sgi >= *seg_count) return;
    const int tid = threadIdx.x, grp = tid / NAIWA_GROUP, lr = tid % NAIWA_GROUP;
    const int kp = blockIdx.y, k0 = kp * ks, kn = min(ks, I - k0);
    const int u0 = Fmt<DD>::units(k0), nus = Fmt<DD>::units(kn);
    const int wb = kn * 2, nsum = kn / SPAN, nw4 = wb / 16;
    const int tstride = (wb + nsum * 4 + 15) & ~15;
    const uint32_t slot = seg_key[sgi];
    const int b = (int)seg_begin[sgi], e = (int)seg_begin[sgi + 1];
    const int rfirst = (blockIdx.x * (kDownThreads / NAIWA_GROUP) + grp) * rpg;
    const uint8_t* dslot = down.base + (int64_t)slot * down.stride;
    for (int c0 = b; c0 < e; c0 += tok_max) {
        const int nt = min(tok_max, e - c0);
        __syncthreads();
        // the h words and sums of the chunk's tokens: a thread's first word piece and first
        // sum are loaded together, the rest (more tokens) one round after another
        for (int i = tid; i < nt * max(nw4, nsum); i += kDownThreads) {
            const int tw = i / nw4, jw = i % nw4, ts = i / nsum, js = i % nsum;
            const bool w_in = i < nt * nw4, s_in = i < nt * nsum;
            uint4 wv = make_uint4(0u, 0u, 0u, 0u);
            float sv = 0.0f;
            if (w_in)
                wv = reinterpret_cast<const uint4*>(hst + (size_t)perm[c0 + tw] * hst_stride + (size_t)k0 * 2)[jw];
            if (s_in)
                sv = reinterpret_cast<const float*>(hst + (size_t)perm[c0 + ts] * hst_stride +
                                                    (size_t)I * 2)[k0 / SPAN + js];
            if (w_in) reinterpret_cast<uint4*>(smem + tw * tstride)[jw] = wv;
            if (s_in) reinterpret_cast<float*>(smem + ts * tstride + wb)[js] = sv;
        }
        __syncthreads();
        for (int i = 0; i < rpg; i += 2) {
            const int r = rfirst + i;
            if (r >= H) break;
            const bool two = i + 1 < rpg && r + 1 < H;
            const uint8_t* drow0 = dslot + (int64_t)r * down.row_bytes;
            const uint8_t* drow1 = drow0 + (two ? down.row_bytes : 0);
            float a0[TD], a1[TD];
#pragma unroll
            for (int tt = 0; tt < TD; ++tt) a0[tt] = a1[tt] = 0.0f;
            for (int base = lr; base < nus; base += NAIWA_GROUP * UM) {
                typename Fmt<DD>::Frag f0[UM], f1[UM];
#pragma unroll
                for (int q = 0; q < UM; ++q) {
                    const int u = base + NAIWA_GROUP * q;
                    if (u < nus) {
                        f0[q] = Fmt<DD>::load(drow0, u0 + u);
                        if (two) f1[q] = Fmt<DD>::load(drow1, u0 + u);
                    }
                }
#pragma unroll
                for (int q = 0; q < UM; ++q) {
                    const int u = base + NAIWA_GROUP * q;
                    if (u >= nus) continue;
#pragma unroll
                    for (int tt = 0; tt < TD; ++tt) {
                        if (tt >= nt) break;
                        const uint32_t* words = reinterpret_cast<const uint32_t*>(smem + tt * tstride);
                        const float* sums = reinterpret_cast<const float*>(smem + tt * tstride + wb);
                        a0[tt] += Fmt<DD>::dot(f0[q], u, words, sums);
                        if (two) a1[tt] += Fmt<DD>::dot(f1[q], u, words, sums);
                    }
                }
            }
#pragma unroll
            for (int tt = 0; tt < TD; ++tt) {
                const float v0 = naiwa_group_sum<NAIWA_GROUP>(a0[tt]);
                const float v1 = naiwa_group_sum<NAIWA_GROUP>(a1[tt]);
                if (tt < nt && lr == 0) {
                    float* dst = dpart + ((size_t)kp * n + c0 + tt) * H + r;
                    dst[0] = v0;
                    if (two) dst[1] = v1;
                }
            }
        }
    }
}

// down_combine: one wave per (64 output rows, token).  The token's sorted positions
// are listed (weight-0 pairs have none) with their routing weights, and ordered
// ascending; out(t, r) starts at 0, or at out's value, and adds w * (the pair's K
// parts summed in order) over those positions -- ascending slot, the order of one pass
// over all segments (and of one call over both halves of a split by slot).  Each load
// that does not depend on another is issued with the others, so a call costs a few
// memory round trips: the segment count, the position count, the permutation and
// weights, then every pair's parts (and the residual's x).
__global__ void __launch_bounds__(64)
down_combine_kernel(const float* dpart, int kparts, int n, int H, int rows, int width, const int* seg_count,
                    const uint32_t* seg_begin, const uint32_t* perm, const float* w, int accumulate, float* out,
                    uint16_t* res) {
    __shared__ int list[kCombineWidth];
    __shared__ float wl[kCombineWidth];
    __shared__ int cnt;
    const int lane = threadIdx.x;
    const int t = blockIdx.y;
    const int npos = (int)seg_begin[*seg_count];
    // the token's positions, compacted in ascending order as the scan meets them (a
    // ballot per 64 positions), with their routing weights
    int found = 0;
    for (int base = 0; base < npos; base += 64) {
        const int pos = base + lane;
        uint32_t p = 0;
        bool mine = false;
        if (pos < npos) {
            p = perm[pos];
            mine = (int)(p / (uint32_t)width) == t;
        }
        const unsigned long long m = __ballot(mine);
        if (mine) {
            const int idx = found + __popcll(m & ((1ull << lane) - 1ull));
            list[idx] = pos;
            wl[idx] = w[p];
        }
        found += __popcll(m);
    }
    if (lane == 0) cnt = found;
    __syncthreads();
    const int r = blockIdx.x * 64 + lane;
    if (r >= H) return;
    const int64_t o = (int64_t)t * H + r;
    const float x0 = res ? naiwa_bf16_to_f32(res[o]) : 0.0f;
    float acc = accumulate ? out[o] : 0.0f;
    const int c = cnt;
    for (int k0 = 0; k0 < c; k0 += kCombinePairs) {
        // the K-part dots of up to kCombinePairs pairs, their loads issued together;
        // each pair's parts added in part order, then the pairs in list order
        float v[kCombinePairs];
        for (int p0 = 0; p0 < kparts; p0 += kCombineParts) {
            float pv[kCombinePairs][kCombineParts];
#pragma unroll
            for (int q = 0; q < kCombinePairs; ++q)
#pragma unroll
                for (int i = 0; i < kCombineParts; ++i)
                    if (k0 + q < c && p0 + i < kparts)
                        pv[q][i] = dpart[((size_t)(p0 + i) * n + list[k0 + q]) * H + r];
#pragma unroll
            for (int q = 0; q < kCombinePairs; ++q)
#pragma unroll
                for (int i = 0; i < kCombineParts; ++i)
                    if (k0 + q < c && p0 + i < kparts) v[q] = (p0 + i == 0) ? pv[q][i] : v[q] + pv[q][i];
        }
#pragma unroll
        for (int q = 0; q < kCombinePairs; ++q)
            if (k0 + q < c) acc = __builtin_fmaf(wl[k0 + q], v[q], acc);
    }
    // with res (bf16 [rows, H]): the residual x = bf16(x + y) of the same y, in place
    if (res) res[o] = (uint16_t)naiwa_f32_to_bf16(x0 + acc);
    if (out) out[o] = acc;
}

// The combine of a one-token call (rows == 1, n pairs, n * kparts <= kOneLoads):
// every sorted position belongs to the token and the positions are already in slot
// order, so a lane issues the loads of every K-part dot of positions < n, its
// residual and its accumulator together with the permutation, before the position
// count is known; only the routing weights wait on the permutation.  The sums are
// those of down_combine_kernel in the same order (parts in part order, then pairs
// in position order), so the result is the same bit for bit.
constexpr int kOneLoads = 16;
__global__ void __launch_bounds__(64)
down_combine_one_kernel(const float* dpart, int kparts, int n, int H, const int* seg_count,
                        const uint32_t* seg_begin, const uint32_t* perm, const float* w, int accumulate, float* out,
                        uint16_t* res) {
    const int lane = threadIdx.x;
    const int r = blockIdx.x * 64 + lane;
    const bool in = r < H;
    const int rr = in ? r : 0;
    const int sc = *seg_count;
    const uint32_t p = lane < n ? perm[lane] : 0u;
    float pv[kOneLoads];
#pragma unroll
    for (int j = 0; j < kOneLoads; ++j) {
        const int q = j / kparts, i = j - q * kparts;
        pv[j] = q < n ? dpart[((size_t)i * n + q) * H + rr] : 0.0f;
    }
    const float x0 = res ? naiwa_bf16_to_f32(res[rr]) : 0.0f;
    float acc = accumulate ? out[rr] : 0.0f;
    const int npos = (int)seg_begin[sc];
    const float wv = lane < npos ? w[p] : 0.0f;
    float v = 0.0f;
#pragma unroll
    for (int j = 0; j < kOneLoads; ++j) {
        const int q = j / kparts, i = j - q * kparts;
        if (q >= npos) break;
        v = i == 0 ? pv[j] : v + pv[j];
        if (i == kparts - 1) {
            const float wq = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wv), q));
            acc = __builtin_fmaf(wq, v, acc);
        }
    }
    if (!in) return;
    if (res) res[r] = (uint16_t)naiwa_f32_to_bf16(x0 + acc);
    if (out) out[r] = acc;
}

// The down projection and the ordered combine of a one-token call in one launch
// (rows == 1, I in one K part, at most kOneMaxPos positions, a row's units in one
// round of down_split_kernel<DD, 1>): no partial dots go through global memory and
// no combine launch follows.  Block: kOneRows output rows x kOneHalves position
// groups, one 16-lane group each; a group dots its row against its positions
// (half, half + kOneHalves, ...) with down_split_kernel's unit assignment and
// summation order, and one thread per row then adds w * dot over the positions in
// ascending order from 0 or from out, as down_combine_one_kernel does: the same
// bits as the three-launch path.  The weight loads of a group's first positions go
// out before the h vectors are staged.
constexpr int kOneRows = 4;
constexpr int kOneHalves = kDownThreads / NAIWA_GROUP / kOneRows;
constexpr int kOneMaxPos = kCombineWidth;
constexpr int kOneChunk = 4; // positions whose weight loads a lane issues together

template <int DD>
__global__ void __launch_bounds__(kDownThreads)
down_one_kernel(BankArg down, int H, int I, int n, const int* seg_count, const uint32_t* seg_key,
                const uint32_t* seg_begin, const uint32_t* perm, const uint8_t* hst, int hst_stride, const float* w,
                int accumulate, float* out, uint16_t* res) {
    constexpr int UM = DD == NAIWA_Q4_K ? 2 : Umax<DD>::v; // as down_split_kernel<DD, 1>
    extern __shared__ __align__(16) uint8_t smem[];        // the positions' h vectors
    __shared__ uint32_t p_slot[kOneMaxPos], p_perm[kOneMaxPos];
    __shared__ float p_w[kOneMaxPos];
    __shared__ float vls[kOneMaxPos][kOneRows];
    __shared__ int s_npos;
    const int tid = threadIdx.x, grp = tid / NAIWA_GROUP, lr = tid % NAIWA_GROUP;
    const int row = grp % kOneRows, half = grp / kOneRows;
    const int r = blockIdx.x * kOneRows + row;
    // wave 0: every segment's slot over its positions, the permutation and the position
    // count, from one round of loads
    if (tid < 64) {
        const int sc = *seg_count;
        const bool in = tid < n;
        const uint32_t key = in ? seg_key[tid] : 0u, b0 = in ? seg_begin[tid] : 0u, b1 = in ? seg_begin[tid + 1] : 0u;
        const uint32_t pm = in ? perm[tid] : 0u;
        const int npos = sc > 0 ? __builtin_amdgcn_readlane((int)b1, sc - 1) : 0;
        if (tid < sc)
            for (uint32_t q = b0; q < b1; ++q) p_slot[q] = key;
        if (tid < npos) p_perm[tid] = pm;
        if (tid == 0) s_npos = npos;
    }
    __syncthreads();
    const int npos = s_npos;
    const int nus = Fmt<DD>::units(I);
    typename Fmt<DD>::Frag f[kOneChunk][UM];
    auto load_chunk = [&](int j0) {
#pragma unroll
        for (int c = 0; c < kOneChunk; ++c) {
            const int pos = half + kOneHalves * (j0 + c);
            if (pos >= npos || r >= H) continue;
            const uint8_t* drow = down.base + (int64_t)p_slot[pos] * down.stride + (int64_t)r * down.row_bytes;
#pragma unroll
            for (int q = 0; q < UM; ++q) {
                const int u = lr + NAIWA_GROUP * q;
                if (u < nus) f[c][q] = Fmt<DD>::load(drow, u);
            }
        }
    };
    load_chunk(0);
    // the h vectors of every position (and the routing weights) while the rows land
    {
        const int nv = hst_stride / 16;
        for (int i = tid; i < npos * nv; i += kDownThreads) {
            const int pos = i / nv, j = i % nv;
            reinterpret_cast<uint4*>(smem + (size_t)pos * hst_stride)[j] =
                reinterpret_cast<const uint4*>(hst + (size_t)p_perm[pos] * hst_stride)[j];
        }
        if (tid < npos) p_w[tid] = w[p_perm[tid]];
    }
    __syncthreads();
    for (int j0 = 0; half + kOneHalves * j0 < npos; j0 += kOneChunk) {
        if (j0 > 0) load_chunk(j0);
#pragma unroll
        for (int c = 0; c < kOneChunk; ++c) {
            const int pos = half + kOneHalves * (j0 + c);
            if (pos >= npos) break;
            const uint32_t* words = reinterpret_cast<const uint32_t*>(smem + (size_t)pos * hst_stride);
            const float* sums = reinterpret_cast<const float*>(smem + (size_t)pos * hst_stride + (size_t)I * 2);
            float a = 0.0f;
#pragma unroll
            for (int q = 0; q < UM; ++q) {
                const int u = lr + NAIWA_GROUP * q;
                if (u < nus && r < H) a += Fmt<DD>::dot(f[c][q], u, words, sums);
            }
            const float v = naiwa_group_sum<NAIWA_GROUP>(a);
            if (lr == 0) vls[pos][row] = v;
        }
    }
    __syncthreads();
    if (tid < kOneRows) {
        const int ro = blockIdx.x * kOneRows + tid;
        if (ro < H) {
            const float x0 = res ? naiwa_bf16_to_f32(res[ro]) : 0.0f;
            float acc = accumulate ? out[ro] : 0.0f;
            for (int q = 0; q < npos; ++q) acc = __builtin_fmaf(p_w[q], vls[q][tid], acc);
            if (res) res[ro] = (uint16_t)naiwa_f32_to_bf16(x0 + acc);
            if (out) out[ro] = acc;
        }
    }
}

bool bank_ok(const naiwa_bank* b) {
    if (!b || !b->base || b->slots <= 0 || b->n <= 0 || b->k <= 0) return false;
    if (b->dtype != NAIWA_Q4_K && b->dtype != NAIWA_Q8_0) return false;
    const int64_t rb = naiwa_row_bytes(b->dtype, b->k);
    if (rb < 0 || b->slot_stride < rb * b->n) return false;
    if (((uintptr_t)b->base & 15) != 0 || (b->slot_stride & 15) != 0) return false;
    return true;
}

int tok_cap(int dtype, int k) {
    const int per = naiwa_stage_bytes(dtype, k);
    int cap = (48 * 1024) / per;
    return cap < 1 ? 0 : (cap > kTokMax ? kTokMax : cap);
}

// Scratch of one decode call (n = rows * width pairs):
//   seg_count, bad | seg_key[n] | seg_begin[n+1] | perm[n] | h | dpart.
// Staged-h path: h = n vectors in the down format's dot layout (or, on the matrix
// cores, f16 x [rows, H] and h [n, I]), dpart = K parts x n x H f32.  Otherwise
// h = n x I f32 and no dpart.
struct DecodeScratch {
    size_t off_key, off_begin, off_perm, off_h, off_dpart, total;
    DecodeScratch(int rows, int width, int H, int I, int down_dtype) {
        const int n = rows * width;
        off_key = 256;
        off_begin = off_key + (((size_t)n * 4 + 255) & ~size_t(255));
        off_perm = off_begin + (((size_t)(n + 1) * 4 + 255) & ~size_t(255));
        off_h = off_perm + (((size_t)n * 4 + 255) & ~size_t(255));
        if (split_path(n, width)) {
            // h in the down format's dot layout, or the matrix-core path's f16 x and h
            const size_t hb =
                std::max((size_t)n * naiwa_stage_bytes(down_dtype, I), naiwa_decode_mfma_bytes(rows, n, H, I));
            off_dpart = off_h + ((hb + 255) & ~size_t(255));
            total = off_dpart + (size_t)split_parts(I) * n * H * 4;
        } else {
            off_dpart = 0;
            total = off_h + (size_t)n * I * 4;
        }
    }
};

__global__ void zero_f32_kernel(float* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0.0f;
}

// Argument checks shared by the entry points; 0 when the call is valid.
int check_args(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, const void* x, int x_dtype,
               const uint32_t* slot_ids, const float* w, int rows, int width, int act, float* out, int flags) {
    if (flags & ~NAIWA_DECODE_ACCUMULATE) return NAIWA_E_INVALID;
    if (!bank_ok(gate) || !bank_ok(up) || !bank_ok(down)) return NAIWA_E_INVALID;
    if (gate->dtype != up->dtype) return NAIWA_E_UNSUPPORTED;
    const int H = gate->k, I = gate->n;
    if (up->k != H || up->n != I || down->k != I || down->n != H) return NAIWA_E_INVALID;
    if (gate->slots != up->slots || gate->slots != down->slots) return NAIWA_E_INVALID;
    if (gate->slots > NAIWA_SEG_MAX_KEYS) return NAIWA_E_UNSUPPORTED;
    if (x_dtype != NAIWA_BF16 && x_dtype != NAIWA_F32) return NAIWA_E_UNSUPPORTED;
    if (act != NAIWA_ACT_SILU && act != NAIWA_ACT_GELU_PYTORCH_TANH) return NAIWA_E_UNSUPPORTED;
    if (rows < 0 || width < 0 || (int64_t)rows * width > 65536) return NAIWA_E_INVALID;
    if (H % 32 || I % 32) return NAIWA_E_INVALID;
    if (rows > 4096) return NAIWA_E_INVALID;
    if (rows > 0 && (!x || !out || (width > 0 && (!slot_ids || !w)))) return NAIWA_E_INVALID;
    const int tok_g = tok_cap(gate->dtype, H), tok_d = tok_cap(down->dtype, I);
    if (!tok_g || !tok_d) return NAIWA_E_UNSUPPORTED;
    const int acc_bytes = ((rows * kRowsPerBlock * 4) + 15) & ~15;
    const size_t lds_down = (size_t)acc_bytes + (size_t)tok_d * naiwa_stage_bytes(down->dtype, I);
    if (lds_down > 64 * 1024) return NAIWA_E_UNSUPPORTED;
    return NAIWA_OK;
}

// out (token, row) from the K parts' unweighted dots in dpart.
int combine_launch(const float* dpart, int kparts, int n, int H, int rows, int width, const int* seg_count,
                   const uint32_t* seg_begin, const uint32_t* perm, const float* w, int accumulate, float* out,
                   hipStream_t st, uint16_t* res = nullptr) {
    if (rows == 1 && n <= 64 && (int64_t)n * kparts <= kOneLoads) {
        down_combine_one_kernel<<<(H + 63) / 64, 64, 0, st>>>(dpart, kparts, n, H, seg_count, seg_begin, perm, w,
                                                              accumulate, out, res);
        return naiwa_hip_rc(hipGetLastError());
    }
    const dim3 cgrid((H + 63) / 64, rows);
    down_combine_kernel<<<cgrid, 64, 0, st>>>(dpart, kparts, n, H, rows, width, seg_count, seg_begin, perm, w,
                                               accumulate, out, res);
    return naiwa_hip_rc(hipGetLastError());
}

// The staged-h path: gate/up writes h in the down format's dot layout (one vector
// of naiwa_stage_bytes(DD, I) per pair, at most DecodeScratch's h bytes), then the
// item-parallel down + ordered combine.
template <int DG, int DD>
int staged_kernels(BankArg g, BankArg u, BankArg d, const void* x, int xb, int H, int I, int rows, int width,
                   int act, const float* w, float* out, int accumulate, int n, int slots, const int* seg_count,
                   const uint32_t* seg_key, const uint32_t* seg_begin, const uint32_t* perm, uint8_t* hst,
                   float* dpart, SegIn seg_in, hipStream_t st, uint16_t* res, WaitArg wt) {
    constexpr int SPAN = Fmt<DD>::kSumSpan;
    const int stage_g = naiwa_stage_bytes(DG, H);
    // tokens staged per chunk: a segment holds at most `rows` tokens unless a token repeats
    // a slot (the kernel then takes more chunks), and the LDS reservation sets how many
    // blocks fit on a CU (one token at H 4096 is 9 KB against 63 KB for seven)
    const int tok = std::max(1, std::min({kTokG, rows, (64 * 1024) / stage_g}));
    const int hst_stride = naiwa_stage_bytes(DD, I);
    // one column per possible segment: blocks past the segment count exit at once,
    // and each still costs a dispatch with its full LDS reservation
    const dim3 ggrid(std::max(1, std::min(n, slots)), I / SPAN);
    if (tok == 1)
        gate_up_staged_kernel<DG, DD, 1><<<ggrid, SPAN * NAIWA_GROUP, (size_t)stage_g, st>>>(
            g, u, x, xb, H, I, width, 1, seg_count, seg_key, seg_begin, perm, act, hst, hst_stride, seg_in, rows == 1, wt);
    else if (tok <= 4)
        gate_up_staged_kernel<DG, DD, 4><<<ggrid, SPAN * NAIWA_GROUP, (size_t)tok * stage_g, st>>>(
            g, u, x, xb, H, I, width, tok, seg_count, seg_key, seg_begin, perm, act, hst, hst_stride, seg_in, rows == 1, wt);
    else
        gate_up_staged_kernel<DG, DD, kTokG><<<ggrid, SPAN * NAIWA_GROUP, (size_t)tok * stage_g, st>>>(
            g, u, x, xb, H, I, width, tok, seg_count, seg_key, seg_begin, perm, act, hst, hst_stride, seg_in, rows == 1, wt);
    // down: rows per group doubled while the grid keeps at least 1024 blocks
    const int ks = split_ks(I), kparts = split_parts(I);
    const int segs = std::max(1, std::min(n, slots));
    const int groups = kDownThreads / NAIWA_GROUP;
    int rpg = 1;
    while (rpg < 8 && (int64_t)((H + groups * rpg * 2 - 1) / (groups * rpg * 2)) * kparts * segs >= 1024) rpg *= 2;
    const int stage_d = naiwa_stage_bytes(DD, ks);
    // one token whose down rows take one K part and one round of units: down and the
    // ordered combine in one launch
    constexpr int UM1 = DD == NAIWA_Q4_K ? 2 : Umax<DD>::v;
    if (rows == 1 && n <= kOneMaxPos && kparts == 1 && Fmt<DD>::units(I) <= NAIWA_GROUP * UM1 &&
        (size_t)n * hst_stride <= 64 * 1024) {
        down_one_kernel<DD><<<(H + kOneRows - 1) / kOneRows, kDownThreads, (size_t)n * hst_stride, st>>>(
            d, H, I, n, seg_count, seg_key, seg_begin, perm, hst, hst_stride, w, accumulate, out, res);
        return naiwa_hip_rc(hipGetLastError());
    }
    const int tok_d = std::max(1, std::min({kTokD, rows, (64 * 1024) / stage_d}));
    const dim3 dgrid((H + groups * rpg - 1) / (groups * rpg), kparts, segs);
    if (tok_d == 1)
        down_split_kernel<DD, 1><<<dgrid, kDownThreads, (size_t)stage_d, st>>>(
            d, H, I, ks, rpg, 1, n, seg_count, seg_key, seg_begin, perm, hst, hst_stride, dpart);
    else if (tok_d <= 4)
        down_split_kernel<DD, 4><<<dgrid, kDownThreads, (size_t)tok_d * stage_d, st>>>(
            d, H, I, ks, rpg, tok_d, n, seg_count, seg_key, seg_begin, perm, hst, hst_stride, dpart);
    else
        down_split_kernel<DD, kTokD><<<dgrid, kDownThreads, (size_t)tok_d * stage_d, st>>>(
            d, H, I, ks, rpg, tok_d, n, seg_count, seg_key, seg_begin, perm, hst, hst_stride, dpart);
    return combine_launch(dpart, kparts, n, H, rows, width, seg_count, seg_begin, perm, w, accumulate, out, st,
                          res);
}

int staged_launch(BankArg g, BankArg u, BankArg d, int gdt, int ddt, const void* x, int x_dtype, int H, int I,
                  int rows, int width, int act, const float* w, float* out, int accumulate, int n, int slots,
                  const int* seg_count, const uint32_t* seg_key, const uint32_t* seg_begin, const uint32_t* perm,
                  uint8_t* hst, float* dpart, SegIn seg_in, hipStream_t st, uint16_t* res, WaitArg wt) {
    const int xb = x_dtype == NAIWA_BF16;
    const int fg = naiwa_kernel_fmt(gdt, H), fd = naiwa_kernel_fmt(ddt, I);
#define NAIWA_STAGED(FG, FD)                                                                                       \
    if (fg == FG && fd == FD)                                                                                      \
        return staged_kernels<FG, FD>(g, u, d, x, xb, H, I, rows, width, act, w, out, accumulate, n, slots,         \
                                      seg_count, seg_key, seg_begin, perm, hst, dpart, seg_in, st, res, wt);
    NAIWA_STAGED(NAIWA_Q4_K, NAIWA_Q4_K)
    NAIWA_STAGED(NAIWA_Q4_K, NAIWA_Q8_0)
    NAIWA_STAGED(NAIWA_Q4_K, NAIWA_Q8_0_ODD)
    NAIWA_STAGED(NAIWA_Q8_0, NAIWA_Q4_K)
    NAIWA_STAGED(NAIWA_Q8_0, NAIWA_Q8_0)
    NAIWA_STAGED(NAIWA_Q8_0, NAIWA_Q8_0_ODD)
    NAIWA_STAGED(NAIWA_Q8_0_ODD, NAIWA_Q4_K)
    NAIWA_STAGED(NAIWA_Q8_0_ODD, NAIWA_Q8_0)
    NAIWA_STAGED(NAIWA_Q8_0_ODD, NAIWA_Q8_0_ODD)
#undef NAIWA_STAGED
    return NAIWA_E_UNSUPPORTED;
}

// The launches of one checked call over scratch ws (DecodeScratch(...).total bytes).
// res (bf16 x, staged calls only): the ordered combine also adds the result to it in
// place, x = bf16(x + y); out may then be null.
int decode_launch(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, const void* x, int x_dtype,
                  const uint32_t* slot_ids, const float* w, int rows, int width, int act, float* out, int flags,
                  uint8_t* ws, hipStream_t st, uint16_t* res = nullptr, const naiwa_decode_wait* wait = nullptr) {
    WaitArg wt{nullptr, 0u, 0ull, nullptr};
    if (wait) wt = WaitArg{wait->flag, wait->target, wait->limit_ticks, wait->fail};
    const int accumulate = (flags & NAIWA_DECODE_ACCUMULATE) ? 1 : 0;
    const int H = gate->k, I = gate->n;
    if (width == 0) {
        if (accumulate) return NAIWA_OK;
        const int64_t n = (int64_t)rows * H;
        zero_f32_kernel<<<(unsigned)std::min<int64_t>((n + 255) / 256, 1024), 256, 0, st>>>(out, n);
        return naiwa_hip_rc(hipGetLastError());
    }
    const int tok_g = tok_cap(gate->dtype, H), tok_d = tok_cap(down->dtype, I);
    const int acc_bytes = ((rows * kRowsPerBlock * 4) + 15) & ~15;
    const size_t lds_down = (size_t)acc_bytes + (size_t)tok_d * naiwa_stage_bytes(down->dtype, I);
    const int n = rows * width;
    const DecodeScratch L(rows, width, H, I, down->dtype);
    int* seg_count = (int*)ws;
    int* bad = (int*)(ws + 4);
    uint32_t* seg_key = (uint32_t*)(ws + L.off_key);
    uint32_t* seg_begin = (uint32_t*)(ws + L.off_begin);
    uint32_t* perm = (uint32_t*)(ws + L.off_perm);
    float* hbuf = (float*)(ws + L.off_h);

    BankArg g{(const uint8_t*)gate->base, gate->slot_stride, naiwa_row_bytes(gate->dtype, H)};
    BankArg u{(const uint8_t*)up->base, up->slot_stride, naiwa_row_bytes(up->dtype, H)};
    BankArg d{(const uint8_t*)down->base, down->slot_stride, naiwa_row_bytes(down->dtype, I)};
    const int mr = mfma_rows();
    const bool staged = split_path(n, width);
    const bool mfma = staged && mr > 0 && rows >= mr && naiwa_decode_mfma_ok(gate, up, down, x);
    // a staged call of few pairs is segmented by its gate/up blocks; every other call
    // by one segments launch first
    SegIn seg_in{nullptr, nullptr, 0, 0, nullptr};
    if (staged && !mfma && n <= kSmallSeg) {
        seg_in = SegIn{slot_ids, w, n, gate->slots, bad};
    } else if (wt.flag) {
        // the wait is not folded into gate/up blocks here: one wave waits first
        decode_wait_kernel<<<1, 64, 0, st>>>(wt);
        wt.flag = nullptr;
    }
    if (!seg_in.slot_ids)
        segments_kernel<<<1, NAIWA_SEG_THREADS, 0, st>>>(slot_ids, w, n, gate->slots, perm, seg_count, seg_key,
                                                         seg_begin, bad);
    if (staged) {
        float* dpart = (float*)(ws + L.off_dpart);
        if (mfma) {
            const int ks = split_ks(I), segs = std::max(1, std::min(n, gate->slots));
            int rc = naiwa_decode_mfma_experts(gate, up, down, x, x_dtype, rows, width, act, n, segs, ks, seg_count,
                                               seg_key, seg_begin, perm, (uint8_t*)hbuf, dpart, st);
            if (rc) return rc;
            return combine_launch(dpart, split_parts(I), n, H, rows, width, seg_count, seg_begin, perm, w,
                                  accumulate, out, st, res);
        }
        return staged_launch(g, u, d, gate->dtype, down->dtype, x, x_dtype, H, I, rows, width, act, w, out,
                             accumulate, n, gate->slots, seg_count, seg_key, seg_begin, perm, (uint8_t*)hbuf, dpart,
                             seg_in, st, res, wt);
    }
    const dim3 ggrid(n, (I + kRowsPerBlock - 1) / kRowsPerBlock);
    const size_t lds_g = (size_t)tok_g * naiwa_stage_bytes(gate->dtype, H);
    const int xb = x_dtype == NAIWA_BF16;
    switch (naiwa_kernel_fmt(gate->dtype, H)) {
    case NAIWA_Q4_K:
        gate_up_kernel<NAIWA_Q4_K><<<ggrid, kThreads, lds_g, st>>>(
            g, u, x, xb, H, I, width, tok_g, seg_count, seg_key, seg_begin, perm, act, hbuf);
        break;
    case NAIWA_Q8_0:
        gate_up_kernel<NAIWA_Q8_0><<<ggrid, kThreads, lds_g, st>>>(
            g, u, x, xb, H, I, width, tok_g, seg_count, seg_key, seg_begin, perm, act, hbuf);
        break;
    default:
        gate_up_kernel<NAIWA_Q8_0_ODD><<<ggrid, kThreads, lds_g, st>>>(
            g, u, x, xb, H, I, width, tok_g, seg_count, seg_key, seg_begin, perm, act, hbuf);
        break;
    }
    const dim3 dgrid((H + kRowsPerBlock - 1) / kRowsPerBlock);
    switch (naiwa_kernel_fmt(down->dtype, I)) {
    case NAIWA_Q4_K:
        down_kernel<NAIWA_Q4_K><<<dgrid, kThreads, lds_down, st>>>(
            d, H, I, rows, width, tok_d, seg_count, seg_key, seg_begin, perm, w, hbuf, accumulate, out);
        break;
    case NAIWA_Q8_0:
        down_kernel<NAIWA_Q8_0><<<dgrid, kThreads, lds_down, st>>>(
            d, H, I, rows, width, tok_d, seg_count, seg_key, seg_begin, perm, w, hbuf, accumulate, out);
        break;
    default:
        down_kernel<NAIWA_Q8_0_ODD><<<dgrid, kThreads, lds_down, st>>>(
            d, H, I, rows, width, tok_d, seg_count, seg_key, seg_begin, perm, w, hbuf, accumulate, out);
        break;
    }
    return naiwa_hip_rc(hipGetLastError());
}

// The allocation-free entry point's scratch: one array per device (each GPU the
// library runs on holds its own copy until the process ends).  Host code never
// uses the array's name as an address: the device address comes from
// hipGetSymbolAddress, once per device, with that device current.
constexpr size_t kNoAllocScratchBytes = NAIWA_DECODE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
uint8_t* g_noalloc_ptr[kMaxDevices];

// The current device's address of `scratch`, resolved on its first use.
int noalloc_scratch(uint8_t** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return NAIWA_E_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!ptr) return NAIWA_E_DEVICE;
        g_noalloc_ptr[dev] = (uint8_t*)ptr;
    }
    *out = g_noalloc_ptr[dev];
    return NAIWA_OK;
}

} // namespace

extern "C" int naiwa_moe_decode_ex(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down,
                                   const void* x, int x_dtype, const uint32_t* slot_ids, const float* w, int rows,
                                   int width, int act, float* out, int flags, int64_t stream) {
    int rc = check_args(gate, up, down, x, x_dtype, slot_ids, w, rows, width, act, out, flags);
    if (rc || rows == 0) return rc;
    uint8_t* ws = nullptr;
    if (width > 0) {
        const DecodeScratch L(rows, width, gate->k, gate->n, down->dtype);
        ws = (uint8_t*)naiwa_scratch(NAIWA_SCRATCH_DECODE, L.total, &rc);
        if (!ws) return rc;
    }
    return decode_launch(gate, up, down, x, x_dtype, slot_ids, w, rows, width, act, out, flags, ws,
                         (hipStream_t)stream);
}

extern "C" int naiwa_moe_decode_noalloc(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down,
                                        const void* x, int x_dtype, const uint32_t* slot_ids, const float* w,
                                        int rows, int width, int act, float* out, int flags, int64_t stream) {
    int rc = check_args(gate, up, down, x, x_dtype, slot_ids, w, rows, width, act, out, flags);
    if (rc || rows == 0) return rc;
    if (width > 0 && DecodeScratch(rows, width, gate->k, gate->n, down->dtype).total > kNoAllocScratchBytes)
        return NAIWA_E_TOO_LARGE;
    uint8_t* ws = nullptr;
    if ((rc = noalloc_scratch(&ws))) return rc;
    return decode_launch(gate, up, down, x, x_dtype, slot_ids, w, rows, width, act, out, flags, ws,
                         (hipStream_t)stream);
}

extern "C" int64_t naiwa_moe_decode_scratch_bytes(int rows, int width, int H, int I, int down_dtype) {
    if (rows < 0 || width < 0 || (int64_t)rows * width > 65536 || H <= 0 || I <= 0 || H % 32 || I % 32) return -1;
    if (down_dtype != NAIWA_Q4_K && down_dtype != NAIWA_Q8_0) return -1;
    if (rows == 0 || width == 0) return 0;
    return (int64_t)DecodeScratch(rows, width, H, I, down_dtype).total;
}

int naiwa_moe_decode_residual(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, void* x,
                              const uint32_t* slot_ids, const float* w, int rows, int width, int act, float* y,
                              int keep_y, int64_t stream, const naiwa_decode_wait* wait) {
    int rc = check_args(gate, up, down, x, NAIWA_BF16, slot_ids, w, rows, width, act, y, 0);
    if (rc || rows == 0 || width == 0) return rc;
    if (wait && (!wait->flag || !wait->fail)) return NAIWA_E_INVALID;
    const DecodeScratch L(rows, width, gate->k, gate->n, down->dtype);
    uint8_t* ws = (uint8_t*)naiwa_scratch(NAIWA_SCRATCH_DECODE, L.total, &rc);
    if (!ws) return rc;
    if (split_path(rows * width, width))
        return decode_launch(gate, up, down, x, NAIWA_BF16, slot_ids, w, rows, width, act, keep_y ? y : nullptr, 0,
                             ws, (hipStream_t)stream, (uint16_t*)x, wait);
    if ((rc = decode_launch(gate, up, down, x, NAIWA_BF16, slot_ids, w, rows, width, act, y, 0, ws,
                            (hipStream_t)stream, nullptr, wait)))
        return rc;
    return naiwa_residual_add_bf16(x, y, (int64_t)rows * gate->k, stream);
}

int naiwa_moe_decode_wait(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, const void* x,
                          int x_dtype, const uint32_t* slot_ids, const float* w, int rows, int width, int act,
                          float* out, int64_t stream, const naiwa_decode_wait* wait) {
    int rc = check_args(gate, up, down, x, x_dtype, slot_ids, w, rows, width, act, out, 0);
    if (rc || rows == 0) return rc;
    if (wait && (!wait->flag || !wait->fail)) return NAIWA_E_INVALID;
    uint8_t* ws = nullptr;
    if (width > 0) {
        const DecodeScratch L(rows, width, gate->k, gate->n, down->dtype);
        ws = (uint8_t*)naiwa_scratch(NAIWA_SCRATCH_DECODE, L.total, &rc);
        if (!ws) return rc;
    } else if (wait) {
        // nothing to compute: the wait still orders the stream
        decode_wait_kernel<<<1, 64, 0, (hipStream_t)stream>>>(
            WaitArg{wait->flag, wait->target, wait->limit_ticks, wait->fail});
        if ((rc = naiwa_hip_rc(hipGetLastError()))) return rc;
    }
    return decode_launch(gate, up, down, x, x_dtype, slot_ids, w, rows, width, act, out, 0, ws, (hipStream_t)stream,
                         nullptr, width > 0 ? wait : nullptr);
}

extern "C" int naiwa_moe_decode(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down,
                                const void* x, int x_dtype, const uint32_t* slot_ids, const float* w, int rows,
                                int width, int act, float* out, int64_t stream) {
    return naiwa_moe_decode_ex(gate, up, down, x, x_dtype, slot_ids, w, rows, width, act, out, 0, stream);
}
