// Router device functions shared by naiwa_router_topk and the fused stack
// kernel: the chunked fixed-point logit rule and the one-wave top-k.
#pragma once

#include "common.h"
#include "workspace.h"

#define NAIWA_ROUTER_CHUNK 8
#define NAIWA_ROUTER_MAX_E 1024
#define NAIWA_ROUTER_MAX_K 32

// 8 activations starting at element `off` (bf16 or f32 source).
__device__ __forceinline__ void naiwa_load_x8(const void* x, int x_bf16, int64_t off, float* xv) {
    if (x_bf16) {
        const uint4 r = *reinterpret_cast<const uint4*>((const uint16_t*)x + off);
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xv[2 * i] = naiwa_bf16_to_f32(w[i] & 0xffffu);
            xv[2 * i + 1] = naiwa_bf16_to_f32(w[i] >> 16);
        }
    } else {
        const float4 a = *reinterpret_cast<const float4*>((const float*)x + off);
        const float4 b = *reinterpret_cast<const float4*>((const float*)x + off + 4);
        xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
        xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
    }
}

// One chunk: f32 fma chain over 8 features, rounded half-to-even to int64
// with 32 fractional bits (scaling by 2^32 is exact).
template <int AS = 0>
__device__ __forceinline__ long long naiwa_router_chunk(const float* w8, const float* xv) {
    const float4 a = naiwa_ld<float4, AS>(w8);
    const float4 b = naiwa_ld<float4, AS>(w8 + 4);
    const float wv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) p = __builtin_fmaf(wv[i], xv[i], p);
    return (long long)__builtin_rintf(p * 4294967296.0f);
}

__device__ __forceinline__ float naiwa_router_fix_to_f32(long long s) {
    return (float)s * 0x1p-32f;
}

// Top-k of one token's logits (LDS, E <= NT * PER entries) by ranking: thread i
// computes the rank of expert e = i % E against the logits in its share of the
// comparison range, the shares are added in LDS, and the experts of rank < k
// write their slot of ids/w.  No step waits on another lane's result, so the
// cost is ~E/NT compares per thread instead of k serial wave reductions.
// rank_tmp: LDS scratch of E ints.  All NT threads of the block must call it.
template <int NT>
__device__ inline void naiwa_block_topk(const float* l, int E, int k, int mode, uint32_t* ids, float* w,
                                        int* rank_tmp, float* ex_tmp) {
    const int tid = threadIdx.x;
    const int shares = E > 0 && NT / E > 0 ? NT / E : 1;
    for (int i = tid; i < E; i += NT) rank_tmp[i] = 0;
    __syncthreads();
    for (int i = tid; i < E * shares; i += NT) {
        const int e = i % E, sh = i / E;
        const int lo = (int)((long long)E * sh / shares), hi = (int)((long long)E * (sh + 1) / shares);
        const float me = l[e];
        int r = 0;
#pragma unroll 8
        for (int o = lo; o < hi; ++o) {
            const float v = l[o];
            r += (v > me) | ((v == me) & (o < e));
        }
        atomicAdd(&rank_tmp[e], r);
    }
    __syncthreads();
    for (int e = tid; e < E; e += NT) {
        const int r = rank_tmp[e];
        if (r < k) {
            ids[r] = (uint32_t)e;
            ex_tmp[r] = l[e];
        }
    }
    __syncthreads();
    if (tid < 64) {
        // weights in rank order, the oracle's summation order
        const float mx = ex_tmp[0];
        float denom = 0.0f;
        if (mode == NAIWA_ROUTE_SOFTMAX_TOPK) {
            float part = 0.0f;
            for (int e = tid; e < E; e += 64) part += expf(l[e] - mx);
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) part += __shfl_xor(part, m, 64);
            denom = part;
        } else {
            for (int j = 0; j < k; ++j) denom += expf(ex_tmp[j] - mx);
        }
        if (tid < k) w[tid] = expf(ex_tmp[tid] - mx) / denom;
    }
    __syncthreads();
}

__device__ __forceinline__ long long naiwa_wave_sum_i64(long long v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// (value desc, id asc): is (va, ia) ranked before (vb, ib)?
__device__ __forceinline__ bool naiwa_rank_before(float va, int ia, float vb, int ib) {
    return va > vb || (va == vb && ia < ib);
}

// One wave (64 lanes) selects the top k of E <= 64 * PER logits and writes ids
// (rank order) and weights (mode).  Every lane must call it.
template <int PER = NAIWA_ROUTER_MAX_E / 64>
__device__ inline void naiwa_wave_topk(const float* l, int E, int k, int mode, uint32_t* ids,
                                       float* w) {
    const int lane = threadIdx.x & 63;
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = lane + 64 * i;
        v[i] = e < E ? l[e] : -__builtin_inff();
    }
    uint32_t taken = 0; // bit i: element lane + 64 i already selected
    float my_v = 0.0f;  // lane j < k keeps the rank-j selection
    int my_i = 0;
    float mx = 0.0f;
    for (int j = 0; j < k; ++j) {
        float bv = -__builtin_inff();
        int bi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = lane + 64 * i;
            if (e < E && !((taken >> i) & 1u) && naiwa_rank_before(v[i], e, bv, bi)) {
                bv = v[i];
                bi = e;
            }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = __shfl_xor(bv, m, 64);
            const int oi = __shfl_xor(bi, m, 64);
            if (naiwa_rank_before(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (lane == j) {
            my_v = bv;
            my_i = bi;
        }
        if (j == 0) mx = bv;
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    }
    // weights: exp(l - max) over the k, normalized by the k or by all E.  The
    // k-term sum runs in rank order in every lane (the oracle's order).
    float denom = 0.0f;
    if (mode == NAIWA_ROUTE_SOFTMAX_TOPK) {
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = lane + 64 * i;
            if (e < E) part += expf(v[i] - mx);
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) part += __shfl_xor(part, m, 64);
        denom = part;
    } else {
        for (int j = 0; j < k; ++j) denom += expf(__shfl(my_v, j, 64) - mx);
    }
    if (lane < k) {
        ids[lane] = (uint32_t)my_i;
        w[lane] = expf(my_v - mx) / denom;
    }
}

// One token's routing read-back in one launch: the logits of router 1 (and of router 2
// when W2 is given: the next layer's, for the lookahead's prediction), the top k of
// each into ids/w on the device, and tagged words (tag << 32 | value) in mapped host
// memory: ids1 at pay[0..k1), weights1 at pay[k1..2 k1), ids2 at pay[2 k1..2 k1 + k2).
// words: E1 + E2 device words for the tagged logits.  Launches that share words must
// not overlap, and tag must differ from the previous launch's.  limit_ticks bounds
// block 0's wait for the other blocks' logits.
int naiwa_route_one_publish(const void* x, int x_dtype, int H, const float* W1, const float* b1, int E1, int k1,
                            int mode1, uint32_t* ids1, float* w1, const float* W2, const float* b2, int E2, int k2,
                            int mode2, uint32_t* ids2, float* w2, uint32_t tag, uint64_t* words, uint64_t* pay,
                            uint64_t limit_ticks, int64_t stream);
