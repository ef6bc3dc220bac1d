/*
 * cpu_baseline.c -- the CPU expert path timed beside the GPU (bench.py's
 * cpu_baseline leg), at the speed class of the reference's own CPU kernels.
 *
 * TEST INFRASTRUCTURE ONLY: bench.py times it and tests/ check it; the product
 * library never calls it.  It is not the parity oracle (naiwa_oracle.c is):
 * like the reference's CPU path it quantizes the activations, so its results
 * differ from the oracle's f32 path by the activation rounding.
 *
 * What it restates (naiwa-rs paths):
 *   - the two-pass contract of fused_moe_decode as called at
 *     src/moe/stages/cpu_miss.rs:13-20, :45 -- pass 1: for every distinct
 *     (expert, row) pair with a nonzero weight, h = SiLU(gate . x) * (up . x);
 *     pass 2: out[row] = sum_j w_j * (down_j . h_j), in the pair order of the
 *     row, weight-0 pairs skipped;
 *   - its partition over threads: pass 1 over (pair, block of intermediate
 *     rows), pass 2 over (row, block of output features);
 *   - the kind of kernel the reference's CPU path runs (its dots reach
 *     2.45 GB/s of Q4_K weights per thread, docs/worklogs/m7.md:102-103):
 *     activations quantized per 256 values to int8 with one f32 scale and
 *     16-value sums (the public GGML Q8_K layout; per 32 values with one scale
 *     for Q8_0 weights), and integer dot products on AVX2
 *     (_mm256_maddubs_epi16 / _mm256_madd_epi16) with one float scale per
 *     block, as GGML's public q4_K x q8_K and q8_0 x q8_0 dots do.
 * The code is this build's own; the block formats are the public GGML ones.
 *
 * Threads: a persistent pool (created once, woken per pass), the calling
 * thread included.
 */
#define _GNU_SOURCE
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "cpu_baseline.h"

#define QK_K 256
#define Q4K_BYTES 144
#define QK8 32
#define Q80_BYTES 34

static float fp16_to_f32(uint16_t h) { return _cvtsh_ss(h); }

/* ---- activation quantization ------------------------------------------------ */

/* Q8_K-style block: 256 values -> d = amax / 127, q = round(x / d), sums of 16. */
typedef struct {
    float d;
    int8_t q[QK_K];
    int16_t bsums[QK_K / 16];
} q8k_block;

/* Q8_0-style activation block: 32 values, one f32 scale. */
typedef struct {
    float d;
    int8_t q[QK8];
} q8a_block;

static void quantize_q8k(const float* x, int64_t n, q8k_block* out) {
    for (int64_t b = 0; b < n / QK_K; ++b) {
        const float* xb = x + b * QK_K;
        float amax = 0.0f;
        for (int i = 0; i < QK_K; ++i) amax = fmaxf(amax, fabsf(xb[i]));
        q8k_block* o = out + b;
        if (amax == 0.0f) {
            memset(o, 0, sizeof(*o));
            continue;
        }
        const float d = amax / 127.0f, id = 127.0f / amax;
        o->d = d;
        for (int i = 0; i < QK_K; ++i) {
            int v = (int)lrintf(xb[i] * id);
            o->q[i] = (int8_t)(v > 127 ? 127 : (v < -127 ? -127 : v));
        }
        for (int g = 0; g < QK_K / 16; ++g) {
            int s = 0;
            for (int i = 0; i < 16; ++i) s += o->q[16 * g + i];
            o->bsums[g] = (int16_t)s;
        }
    }
}

static void quantize_q8a(const float* x, int64_t n, q8a_block* out) {
    for (int64_t b = 0; b < n / QK8; ++b) {
        const float* xb = x + b * QK8;
        float amax = 0.0f;
        for (int i = 0; i < QK8; ++i) amax = fmaxf(amax, fabsf(xb[i]));
        q8a_block* o = out + b;
        if (amax == 0.0f) {
            memset(o, 0, sizeof(*o));
            continue;
        }
        const float d = amax / 127.0f, id = 127.0f / amax;
        o->d = d;
        for (int i = 0; i < QK8; ++i) {
            int v = (int)lrintf(xb[i] * id);
            o->q[i] = (int8_t)(v > 127 ? 127 : (v < -127 ? -127 : v));
        }
    }
}

/* ---- dots --------------------------------------------------------------------- */

static inline float hsum_f32x8(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

/* 6-bit scale and min of sub-block j from a Q4_K header's 12 scale bytes. */
static inline void q4k_scale_min(const uint8_t* s, uint8_t* sc, uint8_t* m) {
    for (int j = 0; j < 4; ++j) {
        sc[j] = s[j] & 63;
        m[j] = s[j + 4] & 63;
    }
    for (int j = 4; j < 8; ++j) {
        sc[j] = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        m[j] = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* One Q4_K row (k values) with Q8_K activations. */
static float dot_q4k_q8k(const uint8_t* row, const q8k_block* x, int64_t k) {
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256 acc = _mm256_setzero_ps();
    float acc_min = 0.0f;
    for (int64_t b = 0; b < k / QK_K; ++b) {
        const uint8_t* blk = row + b * Q4K_BYTES;
        const q8k_block* xb = x + b;
        uint16_t hd, hm;
        memcpy(&hd, blk, 2);
        memcpy(&hm, blk + 2, 2);
        const float d = xb->d * fp16_to_f32(hd);
        const float dmin = xb->d * fp16_to_f32(hm);
        uint8_t sc[8], mn[8];
        q4k_scale_min(blk + 4, sc, mn);
        int summ = 0;
        for (int j = 0; j < 8; ++j) summ += mn[j] * (xb->bsums[2 * j] + xb->bsums[2 * j + 1]);
        acc_min += dmin * (float)summ;
        const uint8_t* qs = blk + 16;
        __m256i sumi = _mm256_setzero_si256();
        for (int c = 0; c < 4; ++c) {
            const __m256i q4 = _mm256_loadu_si256((const __m256i*)(qs + 32 * c));
            const __m256i lo = _mm256_and_si256(q4, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q4, 4), m4);
            const __m256i xl = _mm256_loadu_si256((const __m256i*)(xb->q + 64 * c));
            const __m256i xh = _mm256_loadu_si256((const __m256i*)(xb->q + 64 * c + 32));
            const __m256i pl = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, xl), _mm256_set1_epi16(sc[2 * c]));
            const __m256i ph = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, xh), _mm256_set1_epi16(sc[2 * c + 1]));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(pl, ph));
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum_f32x8(acc) - acc_min;
}

/* One Q8_0 row (k values) with Q8_0-style activations. */
static float dot_q80_q8a(const uint8_t* row, const q8a_block* x, int64_t k) {
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < k / QK8; ++b) {
        const uint8_t* blk = row + b * Q80_BYTES;
        uint16_t hd;
        memcpy(&hd, blk, 2);
        const __m256i w = _mm256_loadu_si256((const __m256i*)(blk + 2));
        const __m256i a = _mm256_loadu_si256((const __m256i*)x[b].q);
        /* |w| * (a with w's sign): unsigned x signed bytes, as maddubs needs */
        const __m256i p = _mm256_maddubs_epi16(_mm256_sign_epi8(w, w), _mm256_sign_epi8(a, w));
        const __m256i s = _mm256_madd_epi16(p, ones);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(fp16_to_f32(hd) * x[b].d), _mm256_cvtepi32_ps(s), acc);
    }
    return hsum_f32x8(acc);
}

/* ---- persistent thread pool ---------------------------------------------------- */

typedef void (*cb_task)(void* ctx, int unit);

struct cb_pool {
    int threads;
    pthread_t* tid;
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    uint64_t generation;
    int running;       /* workers still inside the current pass */
    int quit;
    cb_task fn;
    void* ctx;
    int units;
    atomic_int next;
};

static void run_units(cb_pool* p) {
    for (;;) {
        const int u = atomic_fetch_add(&p->next, 1);
        if (u >= p->units) return;
        p->fn(p->ctx, u);
    }
}

static void* worker(void* arg) {
    cb_pool* p = (cb_pool*)arg;
    uint64_t seen = 0;
    pthread_mutex_lock(&p->mu);
    for (;;) {
        while (!p->quit && p->generation == seen) pthread_cond_wait(&p->go, &p->mu);
        if (p->quit) break;
        seen = p->generation;
        pthread_mutex_unlock(&p->mu);
        run_units(p);
        pthread_mutex_lock(&p->mu);
        if (--p->running == 0) pthread_cond_signal(&p->done);
    }
    pthread_mutex_unlock(&p->mu);
    return NULL;
}

cb_pool* cb_pool_create(int threads) {
    if (threads < 1) threads = 1;
    cb_pool* p = (cb_pool*)calloc(1, sizeof(cb_pool));
    if (!p) return NULL;
    p->threads = threads;
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->go, NULL);
    pthread_cond_init(&p->done, NULL);
    p->tid = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
    for (int i = 1; i < threads; ++i) pthread_create(&p->tid[i], NULL, worker, p);
    return p;
}

void cb_pool_destroy(cb_pool* p) {
    if (!p) return;
    pthread_mutex_lock(&p->mu);
    p->quit = 1;
    pthread_cond_broadcast(&p->go);
    pthread_mutex_unlock(&p->mu);
    for (int i = 1; i < p->threads; ++i) pthread_join(p->tid[i], NULL);
    pthread_mutex_destroy(&p->mu);
    pthread_cond_destroy(&p->go);
    pthread_cond_destroy(&p->done);
    free(p->tid);
    free(p);
}

/* fn(ctx, u) for u in [0, units) on every pool thread, the caller included. */
static void pool_run(cb_pool* p, cb_task fn, void* ctx, int units) {
    pthread_mutex_lock(&p->mu);
    p->fn = fn;
    p->ctx = ctx;
    p->units = units;
    atomic_store(&p->next, 0);
    p->running = p->threads - 1;
    p->generation++;
    pthread_cond_broadcast(&p->go);
    pthread_mutex_unlock(&p->mu);
    run_units(p);
    pthread_mutex_lock(&p->mu);
    while (p->running > 0) pthread_cond_wait(&p->done, &p->mu);
    pthread_mutex_unlock(&p->mu);
}

/* ---- the two passes ------------------------------------------------------------- */

#define ROWS_PER_UNIT 32   /* intermediate rows (pass 1) / output features (pass 2) per unit */

typedef struct {
    const cb_stack *gate, *up, *down;
    int H, I;
    int npairs;
    const int* pair_expert;      /* distinct (expert, row) pairs of pass 1 */
    const int* pair_row;
    const void* xq;              /* per row: quantized x (Q8_K or Q8_0-style blocks) */
    size_t xq_stride;            /* bytes per row of xq */
    float* h;                    /* [npairs, I] */
    void* hq;                    /* per pair: quantized h */
    size_t hq_stride;
    int rows, width;
    const uint32_t* ids;
    const float* w;
    const int* pair_of;          /* [rows * width]: pass-1 pair of (row, j), -1 = skipped */
    float* out;
} passes;

static const uint8_t* expert_row(const cb_stack* s, int e, int r) {
    const int64_t rb = s->dtype == CB_Q4_K ? (s->k / QK_K) * Q4K_BYTES : (s->k / QK8) * Q80_BYTES;
    return s->base + ((int64_t)e * s->n + r) * rb;
}

static float row_dot(const cb_stack* s, int e, int r, const void* xq) {
    return s->dtype == CB_Q4_K ? dot_q4k_q8k(expert_row(s, e, r), (const q8k_block*)xq, s->k)
                               : dot_q80_q8a(expert_row(s, e, r), (const q8a_block*)xq, s->k);
}

static void pass1(void* ctx, int unit) {
    passes* P = (passes*)ctx;
    const int per = (P->I + ROWS_PER_UNIT - 1) / ROWS_PER_UNIT;
    const int q = unit / per, r0 = (unit % per) * ROWS_PER_UNIT;
    const int e = P->pair_expert[q], t = P->pair_row[q];
    const void* xq = (const uint8_t*)P->xq + (size_t)t * P->xq_stride;
    float* hq = P->h + (size_t)q * P->I;
    for (int r = r0; r < r0 + ROWS_PER_UNIT && r < P->I; ++r) {
        const float g = row_dot(P->gate, e, r, xq);
        const float u = row_dot(P->up, e, r, xq);
        hq[r] = g / (1.0f + expf(-g)) * u;
    }
}

static void quant_h(void* ctx, int q) {
    passes* P = (passes*)ctx;
    void* dst = (uint8_t*)P->hq + (size_t)q * P->hq_stride;
    if (P->down->dtype == CB_Q4_K)
        quantize_q8k(P->h + (size_t)q * P->I, P->I, (q8k_block*)dst);
    else
        quantize_q8a(P->h + (size_t)q * P->I, P->I, (q8a_block*)dst);
}

static void pass2(void* ctx, int unit) {
    passes* P = (passes*)ctx;
    const int per = (P->H + ROWS_PER_UNIT - 1) / ROWS_PER_UNIT;
    const int t = unit / per, f0 = (unit % per) * ROWS_PER_UNIT;
    const int f1 = f0 + ROWS_PER_UNIT < P->H ? f0 + ROWS_PER_UNIT : P->H;
    float* o = P->out + (size_t)t * P->H;
    for (int f = f0; f < f1; ++f) o[f] = 0.0f;
    for (int j = 0; j < P->width; ++j) {
        const int q = P->pair_of[t * P->width + j];
        if (q < 0) continue;
        const float wt = P->w[t * P->width + j];
        const void* hq = (const uint8_t*)P->hq + (size_t)q * P->hq_stride;
        const int e = (int)P->ids[t * P->width + j];
        for (int f = f0; f < f1; ++f) o[f] += wt * row_dot(P->down, e, f, hq);
    }
}

static size_t q8_bytes(int dtype, int k) {
    return dtype == CB_Q4_K ? (size_t)(k / QK_K) * sizeof(q8k_block) : (size_t)(k / QK8) * sizeof(q8a_block);
}

static int stack_ok(const cb_stack* s) {
    if (!s || !s->base || s->e <= 0 || s->n <= 0 || s->k <= 0) return 0;
    if (s->dtype == CB_Q4_K) return s->k % QK_K == 0;
    if (s->dtype == CB_Q8_0) return s->k % QK8 == 0;
    return 0;
}

int cb_fused_moe_decode(cb_pool* pool, const cb_stack* gate, const cb_stack* up, const cb_stack* down,
                        const float* xs, const uint32_t* ids, const float* w, int rows, int width, float* out) {
    if (!pool || !stack_ok(gate) || !stack_ok(up) || !stack_ok(down) || rows < 0 || width < 0) return -1;
    if (gate->dtype != up->dtype) return -1;
    const int H = gate->k, I = gate->n;
    if (up->k != H || up->n != I || down->k != I || down->n != H) return -1;
    const int n = rows * width;
    for (int i = 0; i < n; ++i)
        if (ids[i] >= (uint32_t)gate->e) return -1;
    int* pair_expert = (int*)malloc(sizeof(int) * (size_t)(n + 1));
    int* pair_row = (int*)malloc(sizeof(int) * (size_t)(n + 1));
    int* pair_of = (int*)malloc(sizeof(int) * (size_t)(n + 1));
    const size_t xq_stride = q8_bytes(gate->dtype, H), hq_stride = q8_bytes(down->dtype, I);
    void* xq = malloc(xq_stride * (size_t)(rows + 1));
    float* h = (float*)malloc(sizeof(float) * (size_t)I * (size_t)(n + 1));
    void* hq = malloc(hq_stride * (size_t)(n + 1));
    int rc = 0;
    if (!pair_expert || !pair_row || !pair_of || !xq || !h || !hq) {
        rc = -2;
        goto done;
    }
    /* distinct (expert, row) pairs with a nonzero weight, in row-major order */
    int np = 0;
    for (int t = 0; t < rows; ++t) {
        for (int j = 0; j < width; ++j) {
            const int i = t * width + j;
            pair_of[i] = -1;
            if (w[i] == 0.0f) continue;
            for (int jj = 0; jj < j; ++jj)
                if (ids[t * width + jj] == ids[i] && pair_of[t * width + jj] >= 0) pair_of[i] = pair_of[t * width + jj];
            if (pair_of[i] < 0) {
                pair_expert[np] = (int)ids[i];
                pair_row[np] = t;
                pair_of[i] = np++;
            }
        }
    }
    for (int t = 0; t < rows; ++t) {
        void* dst = (uint8_t*)xq + (size_t)t * xq_stride;
        if (gate->dtype == CB_Q4_K)
            quantize_q8k(xs + (size_t)t * H, H, (q8k_block*)dst);
        else
            quantize_q8a(xs + (size_t)t * H, H, (q8a_block*)dst);
    }
    passes P = {gate, up, down, H, I, np, pair_expert, pair_row, xq, xq_stride, h, hq, hq_stride,
                rows, width, ids, w, pair_of, out};
    const int per1 = (I + ROWS_PER_UNIT - 1) / ROWS_PER_UNIT, per2 = (H + ROWS_PER_UNIT - 1) / ROWS_PER_UNIT;
    if (np > 0) {
        pool_run(pool, pass1, &P, np * per1);
        pool_run(pool, quant_h, &P, np);
    }
    pool_run(pool, pass2, &P, rows * per2);
done:
    free(pair_expert);
    free(pair_row);
    free(pair_of);
    free(xq);
    free(h);
    free(hq);
    return rc;
}

int cb_threads(const cb_pool* pool) { return pool ? pool->threads : 0; }
