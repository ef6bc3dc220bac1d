// naiwa_router_topk: router logits, top-k and routing weights on the device,
// so the decode path never round-trips the routing through the host (the
// reference's host read costs 0.72-0.93 ms per layer,
// docs/worklogs/m28-routing-round-trip.md:225-235).
//
// Logits use the chunked fixed-point rule: each chunk of 8 features is an
// f32 fma chain, rounded to int64 with 32 fractional bits; chunk partials are
// added as integers.  Integer addition is associative, so any split of the
// chunks over threads (or over the blocks of the fused stack kernel) yields
// the same bits as the CPU oracle.  Top-k orders by (logit desc, id asc), the
// tie rule of top_k_ids (src/moe/cached_layer.rs:357-363).
#include <algorithm>

#include "common.h"
#include "router.h"

namespace {

constexpr int kLogitThreads = 256;
constexpr int kLogitPer = 4;      // chunk loads a thread issues before using any
constexpr int kLogitRows = 16;    // rows per block of the many-row kernel: 4 per wave
constexpr int kLogitFewRows = 32; // up to this many rows, one block per (expert, row)

// logits[t, e] for many rows: expert e = blockIdx.x and rows blockIdx.y * 16 + 0..15,
// one wave per row at a time; lane l takes the chunks l, l + 64, ...  CPL > 0: exactly
// CPL chunks per lane (H = 512 CPL); the expert's router chunks are loaded once and
// kept in registers, and a row's activation chunks are loaded together.  CPL = 0: any
// H, one chunk at a time.  Each chunk is the same f32 fma chain rounded to int64.
template <int CPL>
__global__ void __launch_bounds__(kLogitThreads)
router_logits_rows_kernel(const void* x, int x_bf16, const float* W, const float* bias, int rows, int H, int E,
                          float* logits) {
    const int e = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nchunks = H / NAIWA_ROUTER_CHUNK;
    const float* wr = W + (int64_t)e * H;
    const int t0 = blockIdx.y * kLogitRows;
    float wv[CPL > 0 ? CPL : 1][8];
    if constexpr (CPL > 0) {
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const float4* src = reinterpret_cast<const float4*>(wr + 8 * (lane + 64 * i));
            const float4 a = src[0], b = src[1];
            wv[i][0] = a.x; wv[i][1] = a.y; wv[i][2] = a.z; wv[i][3] = a.w;
            wv[i][4] = b.x; wv[i][5] = b.y; wv[i][6] = b.z; wv[i][7] = b.w;
        }
    }
    for (int t = t0 + wave; t < min(rows, t0 + kLogitRows); t += kLogitThreads / 64) {
        long long acc = 0;
        if constexpr (CPL > 0) {
            float xv[CPL][8];
#pragma unroll
            for (int i = 0; i < CPL; ++i) naiwa_load_x8(x, x_bf16, (int64_t)t * H + 8 * (lane + 64 * i), xv[i]);
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                float p = 0.0f;
#pragma unroll
                for (int q = 0; q < 8; ++q) p = __builtin_fmaf(wv[i][q], xv[i][q], p);
                acc += (long long)__builtin_rintf(p * 4294967296.0f);
            }
        } else {
            for (int c = lane; c < nchunks; c += 64) {
                float xv[8];
                naiwa_load_x8(x, x_bf16, (int64_t)t * H + 8 * c, xv);
                acc += naiwa_router_chunk(wr + 8 * c, xv);
            }
        }
        acc = naiwa_wave_sum_i64(acc);
        if (lane == 0) logits[(int64_t)t * E + e] = naiwa_router_fix_to_f32(acc) + (bias ? bias[e] : 0.0f);
    }
}

// logits[t, e] for few rows: expert e = blockIdx.x and rows t = blockIdx.y, + gridDim.y, ...: thread i takes the
// 8-feature chunks i, i + 256, ..., issuing up to kLogitPer chunks' loads at once;
// the waves' sums meet in LDS.  The chunk values are int64 fixed point, so their
// sum is the same in any order.
// logit[t, e] by the whole block, returned in thread 0 (part: kLogitThreads / 64
// words of LDS).
__device__ inline float logit_value(const void* x, int x_bf16, const float* W, const float* bias, int H, int e, int t,
                                    long long* part) {
    const int tid = threadIdx.x;
    const int nchunks = H / NAIWA_ROUTER_CHUNK;
    const float* wr = W + (int64_t)e * H;
    long long acc = 0;
    for (int c0 = tid; c0 < nchunks; c0 += kLogitThreads * kLogitPer) {
        float xv[kLogitPer][8];
#pragma unroll
        for (int i = 0; i < kLogitPer; ++i) {
            const int c = c0 + kLogitThreads * i;
            if (c < nchunks) naiwa_load_x8(x, x_bf16, (int64_t)t * H + 8 * c, xv[i]);
        }
#pragma unroll
        for (int i = 0; i < kLogitPer; ++i) {
            const int c = c0 + kLogitThreads * i;
            if (c < nchunks) acc += naiwa_router_chunk(wr + 8 * c, xv[i]);
        }
    }
    acc = naiwa_wave_sum_i64(acc);
    if ((tid & 63) == 0) part[tid >> 6] = acc;
    __syncthreads();
    float v = 0.0f;
    if (tid == 0) {
        long long sum = 0;
#pragma unroll
        for (int i = 0; i < kLogitThreads / 64; ++i) sum += part[i];
        v = naiwa_router_fix_to_f32(sum) + (bias ? bias[e] : 0.0f);
    }
    __syncthreads(); // part is reused by the next call
    return v;
}

__global__ void __launch_bounds__(kLogitThreads)
router_logits_kernel(const void* x, int x_bf16, const float* W, const float* bias, int rows, int H, int E,
                     float* logits) {
    __shared__ long long part[kLogitThreads / 64];
    for (int t = blockIdx.y; t < rows; t += gridDim.y) {
        const float v = logit_value(x, x_bf16, W, bias, H, blockIdx.x, t, part);
        if (threadIdx.x == 0) logits[(int64_t)t * E + blockIdx.x] = v;
    }
}

constexpr int kTopkThreads = 256;
static_assert(kTopkThreads == kLogitThreads, "the one-token routing kernel computes a logit per block");

__global__ void __launch_bounds__(kTopkThreads)
router_topk_kernel(const float* logits, int E, int k, int mode, uint32_t* ids, float* w, int ld) {
    __shared__ float l[NAIWA_ROUTER_MAX_E];
    __shared__ int rank_tmp[NAIWA_ROUTER_MAX_E];
    __shared__ float ex_tmp[NAIWA_ROUTER_MAX_E];
    __shared__ uint32_t ids_s[NAIWA_ROUTER_MAX_K];
    __shared__ float w_s[NAIWA_ROUTER_MAX_K];
    const int t = blockIdx.x;
    for (int e = threadIdx.x; e < E; e += kTopkThreads) l[e] = logits[(int64_t)t * E + e];
    __syncthreads();
    naiwa_block_topk<kTopkThreads>(l, E, k, mode, ids_s, w_s, rank_tmp, ex_tmp);
    if (threadIdx.x < k) {
        ids[(int64_t)t * ld + threadIdx.x] = ids_s[threadIdx.x];
        w[(int64_t)t * ld + threadIdx.x] = w_s[threadIdx.x];
    }
}

typedef __attribute__((address_space(1))) uint64_t gu64;
__device__ __forceinline__ uint64_t tagged_word(uint32_t tag, uint32_t v) { return ((uint64_t)tag << 32) | v; }

// One token's routing in one launch, under one router or two (a layer's, and the next
// layer's for the lookahead's prediction), published to the host without a fence.
// Block b computes logit b of the routers' concatenated experts and stores it as a
// tagged word (tag << 32 | f32 bits) in words[b]; block 0 then loads every logit,
// waiting (bounded) until each carries the tag, and ranks them (no arrival counter:
// 128 atomics on one word serialise at the L2).  The results go to
// the device outputs and, as tagged words, to the mapped payload: ids at pay[0..k0),
// weights at pay[k0..2 k0), the prediction's ids at pay[2 k0..2 k0 + k1).  Every
// word carries its own tag, so the host needs no ordering between them: it waits
// until all of them carry the step's tag.  A wait that runs out publishes nothing
// (the host's own bounded wait then reports the step).
struct RouteOne {
    const void* x;
    int x_bf16, H, nr;
    const float* W[2];
    const float* bias[2];
    int E[2], k[2], mode[2];
    uint32_t* ids[2];
    float* w[2];
    uint32_t tag;
    uint64_t* words;
    uint64_t* pay;
    uint64_t limit_ticks;
};

__global__ void __launch_bounds__(kTopkThreads) router_route_one_kernel(RouteOne a) {
    __shared__ long long part[kLogitThreads / 64];
    __shared__ float l[2 * NAIWA_ROUTER_MAX_E];
    __shared__ int rank_tmp[NAIWA_ROUTER_MAX_E];
    __shared__ float ex_tmp[NAIWA_ROUTER_MAX_E];
    __shared__ uint32_t ids_s[NAIWA_ROUTER_MAX_K];
    __shared__ float w_s[NAIWA_ROUTER_MAX_K];
    __shared__ int ok;
    const int b = blockIdx.x, tid = threadIdx.x, nb = (int)gridDim.x;
    const int r = b < a.E[0] ? 0 : 1, e = b - (r ? a.E[0] : 0);
    const float v = logit_value(a.x, a.x_bf16, a.W[r], a.bias[r], a.H, e, 0, part);
    if (tid == 0) {
        __hip_atomic_store((gu64*)(a.words + b), tagged_word(a.tag, __float_as_uint(v)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        ok = 1;
    }
    if (b != 0) return;
    __syncthreads();
    const uint64_t t0 = wall_clock64();
    for (int i = tid; i < nb; i += kTopkThreads) {
        uint64_t wd;
        while ((uint32_t)((wd = __hip_atomic_load((gu64*)(a.words + i), __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT)) >> 32) != a.tag) {
            if (wall_clock64() - t0 > a.limit_ticks) {
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        l[i] = __uint_as_float((uint32_t)wd);
    }
    __syncthreads();
    if (!ok) return;
    for (int q = 0; q < a.nr; ++q) {
        naiwa_block_topk<kTopkThreads>(l + (q ? a.E[0] : 0), a.E[q], a.k[q], a.mode[q], ids_s, w_s, rank_tmp, ex_tmp);
        if (tid < a.k[q]) {
            const uint32_t id = ids_s[tid];
            const float wv = w_s[tid];
            a.ids[q][tid] = id;
            a.w[q][tid] = wv;
            if (q == 0) {
                __hip_atomic_store((gu64*)(a.pay + tid), tagged_word(a.tag, id), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
                __hip_atomic_store((gu64*)(a.pay + a.k[0] + tid), tagged_word(a.tag, __float_as_uint(wv)),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            } else {
                __hip_atomic_store((gu64*)(a.pay + 2 * a.k[0] + tid), tagged_word(a.tag, id), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
        __syncthreads(); // ids_s, w_s and the ranking scratch are reused
    }
}

} // namespace

int naiwa_route_one_publish(const void* x, int x_dtype, int H, const float* W1, const float* b1, int E1, int k1,
                            int mode1, uint32_t* ids1, float* w1, const float* W2, const float* b2, int E2, int k2,
                            int mode2, uint32_t* ids2, float* w2, uint32_t tag, uint64_t* words, uint64_t* pay,
                            uint64_t limit_ticks, int64_t stream) {
    if (x_dtype != NAIWA_BF16 && x_dtype != NAIWA_F32) return NAIWA_E_UNSUPPORTED;
    const int nr = W2 ? 2 : 1;
    const int mode[2] = {mode1, mode2}, E[2] = {E1, E2}, k[2] = {k1, k2};
    for (int q = 0; q < nr; ++q) {
        if (mode[q] < NAIWA_ROUTE_SOFTMAX_TOPK_RENORM || mode[q] > NAIWA_ROUTE_SOFTMAX_TOPK)
            return NAIWA_E_UNSUPPORTED;
        if (E[q] <= 0 || E[q] > NAIWA_ROUTER_MAX_E || k[q] <= 0 || k[q] > E[q] || k[q] > NAIWA_ROUTER_MAX_K)
            return NAIWA_E_INVALID;
    }
    if (H <= 0 || H % NAIWA_ROUTER_CHUNK || !x || !W1 || !ids1 || !w1 || !words || !pay)
        return NAIWA_E_INVALID;
    if (nr == 2 && (!ids2 || !w2)) return NAIWA_E_INVALID;
    RouteOne a{};
    a.x = x;
    a.x_bf16 = x_dtype == NAIWA_BF16;
    a.H = H;
    a.nr = nr;
    a.W[0] = W1;
    a.W[1] = W2;
    a.bias[0] = b1;
    a.bias[1] = b2;
    a.ids[0] = ids1;
    a.ids[1] = ids2;
    a.w[0] = w1;
    a.w[1] = w2;
    for (int q = 0; q < 2; ++q) {
        a.E[q] = q < nr ? E[q] : 0;
        a.k[q] = q < nr ? k[q] : 0;
        a.mode[q] = q < nr ? mode[q] : 0;
    }
    a.tag = tag;
    a.words = words;
    a.pay = pay;
    a.limit_ticks = limit_ticks;
    router_route_one_kernel<<<(unsigned)(a.E[0] + a.E[1]), kTopkThreads, 0, (hipStream_t)stream>>>(a);
    return naiwa_hip_rc(hipGetLastError());
}

extern "C" int naiwa_router_topk_ld(const void* x, int x_dtype, const float* W, const float* bias, int rows, int H,
                                    int E, int k, int mode, uint32_t* ids_out, float* w_out, int ld,
                                    float* logits_out, int64_t stream) {
    if (x_dtype != NAIWA_BF16 && x_dtype != NAIWA_F32) return NAIWA_E_UNSUPPORTED;
    if (mode < NAIWA_ROUTE_SOFTMAX_TOPK_RENORM || mode > NAIWA_ROUTE_SOFTMAX_TOPK)
        return NAIWA_E_UNSUPPORTED;
    if (rows < 0 || H <= 0 || H % NAIWA_ROUTER_CHUNK || E <= 0 || E > NAIWA_ROUTER_MAX_E || k <= 0 ||
        k > E || k > NAIWA_ROUTER_MAX_K || ld < k)
        return NAIWA_E_INVALID;
    if (rows == 0) return NAIWA_OK;
    if (!x || !W || !ids_out || !w_out) return NAIWA_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    float* logits = logits_out;
    if (!logits) {
        int rc = 0;
        logits = (float*)naiwa_scratch(NAIWA_SCRATCH_ROUTER, (size_t)rows * E * 4, &rc);
        if (!logits) return rc;
    }
    // one block per (expert, row) for few rows, and whenever the 16-row blocks would not
    // fill the CUs (Mixtral at 64 rows: 32 of them); the same bits either way
    const int64_t row_blocks = (int64_t)E * ((rows + kLogitRows - 1) / kLogitRows);
    if (rows <= kLogitFewRows || row_blocks < 256) {
        router_logits_kernel<<<dim3((unsigned)E, (unsigned)std::min(rows, 65535)), kLogitThreads, 0, st>>>(
            x, x_dtype == NAIWA_BF16, W, bias, rows, H, E, logits);
    } else {
        const dim3 lg((unsigned)E, (unsigned)((rows + kLogitRows - 1) / kLogitRows));
        const int xb = x_dtype == NAIWA_BF16;
        if (H == 512 * 4)
            router_logits_rows_kernel<4><<<lg, kLogitThreads, 0, st>>>(x, xb, W, bias, rows, H, E, logits);
        else if (H == 512 * 8)
            router_logits_rows_kernel<8><<<lg, kLogitThreads, 0, st>>>(x, xb, W, bias, rows, H, E, logits);
        else
            router_logits_rows_kernel<0><<<lg, kLogitThreads, 0, st>>>(x, xb, W, bias, rows, H, E, logits);
    }
    router_topk_kernel<<<rows, kTopkThreads, 0, st>>>(logits, E, k, mode, ids_out, w_out, ld);
    return naiwa_hip_rc(hipGetLastError());
}

extern "C" int naiwa_router_topk_biased(const void* x, int x_dtype, const float* W, const float* bias, int rows,
                                        int H, int E, int k, int mode, uint32_t* ids_out, float* w_out,
                                        float* logits_out, int64_t stream) {
    return naiwa_router_topk_ld(x, x_dtype, W, bias, rows, H, E, k, mode, ids_out, w_out, k, logits_out, stream);
}

extern "C" int naiwa_router_topk(const void* x, int x_dtype, const float* W, int rows, int H, int E, int k,
                                 int mode, uint32_t* ids_out, float* w_out, float* logits_out, int64_t stream) {
    return naiwa_router_topk_biased(x, x_dtype, W, nullptr, rows, H, E, k, mode, ids_out, w_out, logits_out,
                                    stream);
}
