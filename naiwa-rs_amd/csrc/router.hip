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
// logit[t, e] by the whole block (part: kLogitThreads / 64 words of LDS).
__device__ inline void logit_block(const void* x, int x_bf16, const float* W, const float* bias, int H, int E, int e,
                                   int t, float* logits, long long* part) {
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
    if (tid == 0) {
        long long sum = 0;
#pragma unroll
        for (int i = 0; i < kLogitThreads / 64; ++i) sum += part[i];
        logits[(int64_t)t * E + e] = naiwa_router_fix_to_f32(sum) + (bias ? bias[e] : 0.0f);
    }
    __syncthreads(); // part is reused by the next call
}

__global__ void __launch_bounds__(kLogitThreads)
router_logits_kernel(const void* x, int x_bf16, const float* W, const float* bias, int rows, int H, int E,
                     float* logits) {
    __shared__ long long part[kLogitThreads / 64];
    for (int t = blockIdx.y; t < rows; t += gridDim.y)
        logit_block(x, x_bf16, W, bias, H, E, blockIdx.x, t, logits, part);
}

// One row under two routers (a layer's, and the next layer's for the lookahead's
// prediction): blocks [0, E1) take W1's experts, blocks [E1, E1 + E2) W2's.
__global__ void __launch_bounds__(kLogitThreads)
router_logits_pair_kernel(const void* x, int x_bf16, int H, const float* W1, const float* b1, int E1, float* l1,
                          const float* W2, const float* b2, int E2, float* l2) {
    __shared__ long long part[kLogitThreads / 64];
    const int b = blockIdx.x;
    if (b < E1)
        logit_block(x, x_bf16, W1, b1, H, E1, b, 0, l1, part);
    else
        logit_block(x, x_bf16, W2, b2, H, E2, b - E1, 0, l2, part);
}

constexpr int kTopkThreads = 256;

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

// router_topk_kernel for one row with the routing read-back published from the same
// block: ids and weights also go to the mapped payload (ids at pay[0..k), weights at
// pay[k..2k)), then the sequence word goes up by one with a system-scope release --
// the reference's TopkDoorbell publish (src/doorbell/d2h/topk.rs:20-125) without a
// launch of its own.
__global__ void __launch_bounds__(kTopkThreads)
router_topk_publish_kernel(const float* logits, int E, int k, int mode, uint32_t* ids, float* w, uint32_t* db_seq,
                           uint32_t* pay) {
    __shared__ float l[NAIWA_ROUTER_MAX_E];
    __shared__ int rank_tmp[NAIWA_ROUTER_MAX_E];
    __shared__ float ex_tmp[NAIWA_ROUTER_MAX_E];
    __shared__ uint32_t ids_s[NAIWA_ROUTER_MAX_K];
    __shared__ float w_s[NAIWA_ROUTER_MAX_K];
    for (int e = threadIdx.x; e < E; e += kTopkThreads) l[e] = logits[e];
    __syncthreads();
    naiwa_block_topk<kTopkThreads>(l, E, k, mode, ids_s, w_s, rank_tmp, ex_tmp);
    if (threadIdx.x < k) {
        const uint32_t id = ids_s[threadIdx.x];
        const float wv = w_s[threadIdx.x];
        ids[threadIdx.x] = id;
        w[threadIdx.x] = wv;
        volatile uint32_t* out = pay;
        out[threadIdx.x] = id;
        out[k + threadIdx.x] = __float_as_uint(wv);
    }
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t cur = __hip_atomic_load(db_seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(db_seq, cur + 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// The top k of both rows of router_logits_pair_kernel in one block, then one publish
// of the routing read-back: ids1 at pay[0..k1), weights1 at pay[k1..2k1), ids2 at
// pay[2k1..2k1+k2), and the sequence word up by one with a system-scope release.
__global__ void __launch_bounds__(kTopkThreads)
router_topk_pair_publish_kernel(const float* l1, int E1, int k1, int mode1, uint32_t* ids1, float* w1,
                                const float* l2, int E2, int k2, int mode2, uint32_t* ids2, float* w2,
                                uint32_t* db_seq, uint32_t* pay) {
    __shared__ float l[NAIWA_ROUTER_MAX_E];
    __shared__ int rank_tmp[NAIWA_ROUTER_MAX_E];
    __shared__ float ex_tmp[NAIWA_ROUTER_MAX_E];
    __shared__ uint32_t ids_s[NAIWA_ROUTER_MAX_K];
    __shared__ float w_s[NAIWA_ROUTER_MAX_K];
    volatile uint32_t* out = pay;
    for (int e = threadIdx.x; e < E1; e += kTopkThreads) l[e] = l1[e];
    __syncthreads();
    naiwa_block_topk<kTopkThreads>(l, E1, k1, mode1, ids_s, w_s, rank_tmp, ex_tmp);
    if (threadIdx.x < k1) {
        ids1[threadIdx.x] = ids_s[threadIdx.x];
        w1[threadIdx.x] = w_s[threadIdx.x];
        out[threadIdx.x] = ids_s[threadIdx.x];
        out[k1 + threadIdx.x] = __float_as_uint(w_s[threadIdx.x]);
    }
    __syncthreads(); // l, ids_s and w_s are reused
    for (int e = threadIdx.x; e < E2; e += kTopkThreads) l[e] = l2[e];
    __syncthreads();
    naiwa_block_topk<kTopkThreads>(l, E2, k2, mode2, ids_s, w_s, rank_tmp, ex_tmp);
    if (threadIdx.x < k2) {
        ids2[threadIdx.x] = ids_s[threadIdx.x];
        w2[threadIdx.x] = w_s[threadIdx.x];
        out[2 * k1 + threadIdx.x] = ids_s[threadIdx.x];
    }
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t cur = __hip_atomic_load(db_seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(db_seq, cur + 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

} // namespace

int naiwa_router_topk_publish(const void* x, int x_dtype, const float* W, const float* bias, int H, int E, int k,
                              int mode, uint32_t* ids_out, float* w_out, uint32_t* db_seq, uint32_t* pay,
                              int64_t stream) {
    if (x_dtype != NAIWA_BF16 && x_dtype != NAIWA_F32) return NAIWA_E_UNSUPPORTED;
    if (mode < NAIWA_ROUTE_SOFTMAX_TOPK_RENORM || mode > NAIWA_ROUTE_SOFTMAX_TOPK)
        return NAIWA_E_UNSUPPORTED;
    if (H <= 0 || H % NAIWA_ROUTER_CHUNK || E <= 0 || E > NAIWA_ROUTER_MAX_E || k <= 0 || k > E ||
        k > NAIWA_ROUTER_MAX_K)
        return NAIWA_E_INVALID;
    if (!x || !W || !ids_out || !w_out || !db_seq || !pay) return NAIWA_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    int rc = 0;
    float* logits = (float*)naiwa_scratch(NAIWA_SCRATCH_ROUTER, (size_t)E * 4, &rc);
    if (!logits) return rc;
    router_logits_kernel<<<dim3((unsigned)E, 1u), kLogitThreads, 0, st>>>(x, x_dtype == NAIWA_BF16, W, bias, 1, H, E,
                                                                         logits);
    router_topk_publish_kernel<<<1, kTopkThreads, 0, st>>>(logits, E, k, mode, ids_out, w_out, db_seq, pay);
    return naiwa_hip_rc(hipGetLastError());
}

int naiwa_router_topk_pair_publish(const void* x, int x_dtype, int H, const float* W1, const float* b1, int E1,
                                   int k1, int mode1, uint32_t* ids1, float* w1, const float* W2, const float* b2,
                                   int E2, int k2, int mode2, uint32_t* ids2, float* w2, uint32_t* db_seq,
                                   uint32_t* pay, int64_t stream) {
    if (x_dtype != NAIWA_BF16 && x_dtype != NAIWA_F32) return NAIWA_E_UNSUPPORTED;
    for (int m : {mode1, mode2})
        if (m < NAIWA_ROUTE_SOFTMAX_TOPK_RENORM || m > NAIWA_ROUTE_SOFTMAX_TOPK) return NAIWA_E_UNSUPPORTED;
    if (H <= 0 || H % NAIWA_ROUTER_CHUNK || E1 <= 0 || E1 > NAIWA_ROUTER_MAX_E || k1 <= 0 || k1 > E1 ||
        k1 > NAIWA_ROUTER_MAX_K || E2 <= 0 || E2 > NAIWA_ROUTER_MAX_E || k2 <= 0 || k2 > E2 ||
        k2 > NAIWA_ROUTER_MAX_K)
        return NAIWA_E_INVALID;
    if (!x || !W1 || !W2 || !ids1 || !w1 || !ids2 || !w2 || !db_seq || !pay) return NAIWA_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    int rc = 0;
    float* logits = (float*)naiwa_scratch(NAIWA_SCRATCH_ROUTER, (size_t)(E1 + E2) * 4, &rc);
    if (!logits) return rc;
    router_logits_pair_kernel<<<(unsigned)(E1 + E2), kLogitThreads, 0, st>>>(x, x_dtype == NAIWA_BF16, H, W1, b1, E1,
                                                                           logits, W2, b2, E2, logits + E1);
    router_topk_pair_publish_kernel<<<1, kTopkThreads, 0, st>>>(logits, E1, k1, mode1, ids1, w1, logits + E1, E2, k2,
                                                                mode2, ids2, w2, db_seq, pay);
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
