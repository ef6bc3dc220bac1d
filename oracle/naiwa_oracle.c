/*
 * naiwa_oracle.c -- CPU restatement of naiwa-rs's MoE expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity reference of the tests and the CPU baseline); the
 * product library never links or calls this file.  Build: oracle/Makefile
 * (-O2 -ffp-contract=off so every f32 operation is the one written here).
 */
#include "naiwa_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------- */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_fp16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ff;
    if (exp == 0) {
        /* zero or subnormal: mant * 2^-24, exact in f32 */
        float v = (float)mant * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (mant << 13));
    return u2f(sign | ((exp - 15 + 127) << 23) | (mant << 13));
}

uint16_t orc_f32_to_fp16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {
        /* below 2^-14: half subnormal, unit 2^-24; scaling by 2^24 is exact */
        float s = u2f(ax) * 16777216.0f;
        uint32_t m = (uint32_t)nearbyintf(s); /* round half to even */
        return (uint16_t)(sign | m);
    }
    uint32_t exp = (ax >> 23) - 127 + 15;
    uint32_t mant = ax & 0x7fffffu;
    uint32_t h = (exp << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t orc_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

void orc_f32_to_bf16_n(const float* x, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(x[i]);
}

void orc_bf16_to_f32_n(const uint16_t* x, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(x[i]);
}

/* ------------------------------------------------------------------------- */
/* block formats (public ggml layout)                                        */
/*   Q8_0: { fp16 d; int8 qs[32]; }                     34 B / 32 values      */
/*   Q4_K: { fp16 d; fp16 dmin; u8 scales[12]; u8 qs[128]; }  144 B / 256     */
/* ------------------------------------------------------------------------- */

#define QK8_0 32
#define QK_K 256
#define Q8_0_BYTES 34
#define Q4_K_BYTES 144

int orc_block_size(int dtype) {
    switch (dtype) {
    case ORC_Q8_0: return QK8_0;
    case ORC_Q4_K: return QK_K;
    case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
    default: return -1;
    }
}

int orc_type_size(int dtype) {
    switch (dtype) {
    case ORC_Q8_0: return Q8_0_BYTES;
    case ORC_Q4_K: return Q4_K_BYTES;
    case ORC_F32: return 4;
    case ORC_F16: case ORC_BF16: return 2;
    default: return -1;
    }
}

/* src/moe/slot.rs:84-95: bytes = N * (K / block_size) * type_size, K % block == 0 */
int64_t orc_row_bytes(int dtype, int64_t k) {
    int bs = orc_block_size(dtype), ts = orc_type_size(dtype);
    if (bs <= 0 || ts <= 0 || k % bs != 0) return -1;
    return (k / bs) * ts;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static void wr16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)(v & 0xff); p[1] = (uint8_t)(v >> 8); }

void orc_quantize_q8_0(const float* x, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / QK8_0; ++b) {
        const float* xb = x + b * QK8_0;
        uint8_t* ob = out + b * Q8_0_BYTES;
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; ++j) {
            float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr16(ob, orc_f32_to_fp16(d));
        for (int j = 0; j < QK8_0; ++j) {
            float v = roundf(xb[j] * id); /* half away from zero, as ggml */
            if (v > 127.0f) v = 127.0f;
            if (v < -128.0f) v = -128.0f;
            ob[2 + j] = (uint8_t)(int8_t)v;
        }
    }
}

void orc_dequantize_q8_0(const uint8_t* in, int64_t n, float* y) {
    for (int64_t b = 0; b < n / QK8_0; ++b) {
        const uint8_t* ib = in + b * Q8_0_BYTES;
        float d = orc_fp16_to_f32(rd16(ib));
        for (int j = 0; j < QK8_0; ++j) y[b * QK8_0 + j] = d * (float)(int8_t)ib[2 + j];
    }
}

/* 6-bit scale / min j of a Q4_K block (ggml get_scale_min_k4). */
static void scale_min_k4(int j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

static int nearest_int(float v) { return (int)lrintf(v); } /* round half to even */

/* The build's own Q4_K quantizer: per 32-value sub-block an affine range
 * [min(0, lo), hi] on 15 steps, 6-bit scales and mins relative to the
 * super-block's largest, then the nibble codes against the stored (fp16 and
 * 6-bit rounded) scale and min.  Simpler than ggml's iterative search; the
 * parity of the expert path never depends on it because the oracle and the
 * device read the same bytes. */
void orc_quantize_q4_k(const float* x, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / QK_K; ++b) {
        const float* xb = x + b * QK_K;
        uint8_t* ob = out + b * Q4_K_BYTES;
        float scales[8], mins[8];
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; ++j) {
            float lo = xb[32 * j], hi = xb[32 * j];
            for (int l = 1; l < 32; ++l) {
                float v = xb[32 * j + l];
                if (v < lo) lo = v;
                if (v > hi) hi = v;
            }
            if (lo > 0.0f) lo = 0.0f;
            scales[j] = (hi - lo) / 15.0f;
            mins[j] = -lo;
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        uint8_t ls[8], lm[8];
        for (int j = 0; j < 8; ++j) {
            int a = nearest_int(inv_scale * scales[j]);
            int c = nearest_int(inv_min * mins[j]);
            ls[j] = (uint8_t)(a > 63 ? 63 : (a < 0 ? 0 : a));
            lm[j] = (uint8_t)(c > 63 ? 63 : (c < 0 ? 0 : c));
        }
        uint8_t* sc = ob + 4;
        memset(sc, 0, 12);
        for (int j = 0; j < 8; ++j) {
            if (j < 4) {
                sc[j] = ls[j];
                sc[j + 4] = lm[j];
            } else {
                sc[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
                sc[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
                sc[j] |= (uint8_t)((lm[j] >> 4) << 6);
            }
        }
        uint16_t dh = orc_f32_to_fp16(max_scale / 63.0f);
        uint16_t mh = orc_f32_to_fp16(max_min / 63.0f);
        wr16(ob, dh);
        wr16(ob + 2, mh);
        float d = orc_fp16_to_f32(dh), dmin = orc_fp16_to_f32(mh);
        uint8_t q[QK_K];
        for (int j = 0; j < 8; ++j) {
            uint8_t s6, m6;
            scale_min_k4(j, sc, &s6, &m6);
            float dj = d * (float)s6;
            float mj = dmin * (float)m6;
            for (int l = 0; l < 32; ++l) {
                int v = 0;
                if (dj != 0.0f) v = nearest_int((xb[32 * j + l] + mj) / dj);
                q[32 * j + l] = (uint8_t)(v < 0 ? 0 : (v > 15 ? 15 : v));
            }
        }
        uint8_t* qs = ob + 16;
        for (int c = 0; c < 4; ++c)
            for (int l = 0; l < 32; ++l)
                qs[32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
    }
}

/* ggml dequantize_row_q4_K: chunk c of 64 values uses sub-blocks 2c (low
 * nibbles of qs[32c..32c+32]) and 2c+1 (high nibbles). */
void orc_dequantize_q4_k(const uint8_t* in, int64_t n, float* y) {
    for (int64_t b = 0; b < n / QK_K; ++b) {
        const uint8_t* ib = in + b * Q4_K_BYTES;
        float d = orc_fp16_to_f32(rd16(ib)), dmin = orc_fp16_to_f32(rd16(ib + 2));
        const uint8_t* sc = ib + 4;
        const uint8_t* qs = ib + 16;
        float* yb = y + b * QK_K;
        for (int c = 0; c < 4; ++c) {
            uint8_t s1, m1, s2, m2;
            scale_min_k4(2 * c, sc, &s1, &m1);
            scale_min_k4(2 * c + 1, sc, &s2, &m2);
            float d1 = d * (float)s1, mm1 = dmin * (float)m1;
            float d2 = d * (float)s2, mm2 = dmin * (float)m2;
            for (int l = 0; l < 32; ++l) yb[64 * c + l] = d1 * (float)(qs[32 * c + l] & 0xF) - mm1;
            for (int l = 0; l < 32; ++l) yb[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - mm2;
        }
    }
}

int orc_quantize(int dtype, const float* x, int64_t n, uint8_t* out) {
    if (orc_row_bytes(dtype, n) < 0) return -1;
    switch (dtype) {
    case ORC_Q8_0: orc_quantize_q8_0(x, n, out); return 0;
    case ORC_Q4_K: orc_quantize_q4_k(x, n, out); return 0;
    case ORC_F32: memcpy(out, x, (size_t)n * 4); return 0;
    case ORC_BF16: orc_f32_to_bf16_n(x, n, (uint16_t*)out); return 0;
    default: return -1;
    }
}

int orc_dequantize(int dtype, const uint8_t* in, int64_t n, float* y) {
    if (orc_row_bytes(dtype, n) < 0) return -1;
    switch (dtype) {
    case ORC_Q8_0: orc_dequantize_q8_0(in, n, y); return 0;
    case ORC_Q4_K: orc_dequantize_q4_k(in, n, y); return 0;
    case ORC_F32: memcpy(y, in, (size_t)n * 4); return 0;
    case ORC_BF16: orc_bf16_to_f32_n((const uint16_t*)in, n, y); return 0;
    default: return -1;
    }
}

int orc_dequantize_f64(int dtype, const uint8_t* in, int64_t n, double* y) {
    if (orc_row_bytes(dtype, n) < 0) return -1;
    if (dtype == ORC_Q8_0) {
        for (int64_t b = 0; b < n / QK8_0; ++b) {
            const uint8_t* ib = in + b * Q8_0_BYTES;
            double d = (double)orc_fp16_to_f32(rd16(ib));
            for (int j = 0; j < QK8_0; ++j) y[b * QK8_0 + j] = d * (double)(int8_t)ib[2 + j];
        }
        return 0;
    }
    if (dtype == ORC_Q4_K) {
        for (int64_t b = 0; b < n / QK_K; ++b) {
            const uint8_t* ib = in + b * Q4_K_BYTES;
            double d = orc_fp16_to_f32(rd16(ib)), dmin = orc_fp16_to_f32(rd16(ib + 2));
            const uint8_t* sc = ib + 4;
            const uint8_t* qs = ib + 16;
            for (int c = 0; c < 4; ++c) {
                uint8_t s1, m1, s2, m2;
                scale_min_k4(2 * c, sc, &s1, &m1);
                scale_min_k4(2 * c + 1, sc, &s2, &m2);
                for (int l = 0; l < 32; ++l) {
                    y[b * QK_K + 64 * c + l] = d * s1 * (double)(qs[32 * c + l] & 0xF) - dmin * m1;
                    y[b * QK_K + 64 * c + 32 + l] = d * s2 * (double)(qs[32 * c + l] >> 4) - dmin * m2;
                }
            }
        }
        return 0;
    }
    if (dtype == ORC_F32) {
        const float* f = (const float*)in;
        for (int64_t i = 0; i < n; ++i) y[i] = f[i];
        return 0;
    }
    if (dtype == ORC_BF16) {
        const uint16_t* h = (const uint16_t*)in;
        for (int64_t i = 0; i < n; ++i) y[i] = orc_bf16_to_f32(h[i]);
        return 0;
    }
    return -1;
}

/* ------------------------------------------------------------------------- */
/* deterministic synthetic data                                              */
/* ------------------------------------------------------------------------- */

static uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Box-Muller on a counter-based pair of uniforms: element i of the stream is
 * the cosine (even i) or sine (odd i) branch of pair i/2. */
void orc_fill_normal(uint64_t seed, uint64_t offset, int64_t n, float mean, float stdv, float* out) {
    const uint64_t key = mix64(seed ^ 0xD1B54A32D192ED03ull);
    for (int64_t i = 0; i < n; ++i) {
        uint64_t idx = offset + (uint64_t)i;
        uint64_t p = idx >> 1;
        uint64_t a = mix64(key ^ mix64(2 * p));
        uint64_t b = mix64(key ^ mix64(2 * p + 1));
        double u1 = ((double)(a >> 11) + 1.0) * 0x1p-53; /* (0, 1] */
        double u2 = (double)(b >> 11) * 0x1p-53;         /* [0, 1) */
        double r = sqrt(-2.0 * log(u1));
        double t = 6.283185307179586 * u2;
        double z = (idx & 1) ? r * sin(t) : r * cos(t);
        out[i] = (float)((double)mean + (double)stdv * z);
    }
}

/* ------------------------------------------------------------------------- */
/* expert math                                                               */
/* ------------------------------------------------------------------------- */

int64_t orc_expert_bytes(const orc_stack* s) {
    int64_t rb = orc_row_bytes(s->dtype, s->k);
    return rb < 0 ? -1 : rb * s->n;
}

static const uint8_t* expert_row(const orc_stack* s, int e, int r) {
    int64_t rb = orc_row_bytes(s->dtype, s->k);
    return s->base + (int64_t)e * s->n * rb + (int64_t)r * rb;
}

float orc_vec_dot(int dtype, const uint8_t* row, const float* x, int64_t k) {
    int bs = orc_block_size(dtype), ts = orc_type_size(dtype);
    float tmp[QK_K];
    float acc = 0.0f;
    if (bs == 1) {
        for (int64_t i = 0; i < k; ++i) {
            float v;
            if (dtype == ORC_F32) memcpy(&v, row + 4 * i, 4);
            else if (dtype == ORC_BF16) v = orc_bf16_to_f32(rd16(row + 2 * i));
            else v = orc_fp16_to_f32(rd16(row + 2 * i));
            acc += v * x[i];
        }
        return acc;
    }
    for (int64_t b = 0; b < k / bs; ++b) {
        orc_dequantize(dtype, row + b * ts, bs, tmp);
        for (int i = 0; i < bs; ++i) acc += tmp[i] * x[b * bs + i];
    }
    return acc;
}

static double vec_dot_f64(int dtype, const uint8_t* row, const double* x, int64_t k, double* scratch) {
    orc_dequantize_f64(dtype, row, k, scratch);
    double acc = 0.0;
    for (int64_t i = 0; i < k; ++i) acc += scratch[i] * x[i];
    return acc;
}

static int check_stacks(const orc_stack* g, const orc_stack* u, const orc_stack* d) {
    if (g->e != u->e || g->e != d->e) return -1;
    if (g->n != u->n || g->k != u->k) return -1;
    if (d->k != g->n || d->n != g->k) return -1;
    if (orc_row_bytes(g->dtype, g->k) < 0 || orc_row_bytes(u->dtype, u->k) < 0 ||
        orc_row_bytes(d->dtype, d->k) < 0)
        return -1;
    return 0;
}

/* src/moe/stages/cpu_miss.rs:13-20: pass 1 computes h = silu(gate.x) * (up.x)
 * once per distinct (expert, row) with a nonzero weight; pass 2 sums
 * w * (down.h) over the row's slots in ascending slot order; weight-0 slots
 * (the padding of cpu_miss.rs:90-100) contribute nothing. */
int orc_fused_moe_decode(const orc_stack* gate, const orc_stack* up, const orc_stack* down,
                         const float* xs, const uint32_t* ids, const float* w,
                         int rows, int width, float* out) {
    if (check_stacks(gate, up, down)) return -1;
    const int H = gate->k, I = gate->n, E = gate->e;
    for (int i = 0; i < rows * width; ++i)
        if (ids[i] >= (uint32_t)E) return -1;
    float* h = (float*)malloc(sizeof(float) * (size_t)width * (size_t)I);
    int* owner = (int*)malloc(sizeof(int) * (size_t)width);
    if (!h || !owner) { free(h); free(owner); return -2; }
    for (int t = 0; t < rows; ++t) {
        const float* x = xs + (int64_t)t * H;
        const uint32_t* id = ids + (int64_t)t * width;
        const float* wt = w + (int64_t)t * width;
        /* pass 1 */
        for (int j = 0; j < width; ++j) {
            owner[j] = -1;
            if (wt[j] == 0.0f) continue;
            for (int i = 0; i < j; ++i)
                if (owner[i] >= 0 && id[i] == id[j]) { owner[j] = owner[i]; break; }
            if (owner[j] >= 0) continue;
            owner[j] = j;
            for (int r = 0; r < I; ++r) {
                float g = orc_vec_dot(gate->dtype, expert_row(gate, (int)id[j], r), x, H);
                float u = orc_vec_dot(up->dtype, expert_row(up, (int)id[j], r), x, H);
                float s = g / (1.0f + expf(-g));
                h[(int64_t)j * I + r] = s * u;
            }
        }
        /* pass 2 */
        float* o = out + (int64_t)t * H;
        for (int r = 0; r < H; ++r) {
            float acc = 0.0f;
            for (int j = 0; j < width; ++j) {
                if (owner[j] < 0) continue;
                float y = orc_vec_dot(down->dtype, expert_row(down, (int)id[j], r),
                                      h + (int64_t)owner[j] * I, I);
                acc += wt[j] * y;
            }
            o[r] = acc;
        }
    }
    free(h);
    free(owner);
    return 0;
}

/* The same computation on `threads` host threads (the CPU baseline): pass 1's
 * (pair, row) values and pass 2's output features are split into contiguous
 * ranges, and each value is computed exactly as in orc_fused_moe_decode, so
 * the result is bit-identical to it. */
typedef struct {
    const orc_stack *gate, *up, *down;
    const float* x;
    const uint32_t* id;
    const float* wt;
    const int* owner;
    float* h;
    float* o;
    int width, pass, lo, hi; /* pass 1: flat (j * I + r) range; pass 2: feature range */
} mt_job;

static void* mt_run(void* arg) {
    const mt_job* jb = (const mt_job*)arg;
    const int H = jb->gate->k, I = jb->gate->n;
    if (jb->pass == 1) {
        for (int f = jb->lo; f < jb->hi; ++f) {
            const int j = f / I, r = f % I;
            if (jb->owner[j] != j) continue;
            float g = orc_vec_dot(jb->gate->dtype, expert_row(jb->gate, (int)jb->id[j], r), jb->x, H);
            float u = orc_vec_dot(jb->up->dtype, expert_row(jb->up, (int)jb->id[j], r), jb->x, H);
            float s = g / (1.0f + expf(-g));
            jb->h[(int64_t)j * I + r] = s * u;
        }
    } else {
        for (int r = jb->lo; r < jb->hi; ++r) {
            float acc = 0.0f;
            for (int j = 0; j < jb->width; ++j) {
                if (jb->owner[j] < 0) continue;
                float y = orc_vec_dot(jb->down->dtype, expert_row(jb->down, (int)jb->id[j], r),
                                      jb->h + (int64_t)jb->owner[j] * I, I);
                acc += jb->wt[j] * y;
            }
            jb->o[r] = acc;
        }
    }
    return NULL;
}

int orc_fused_moe_decode_mt(const orc_stack* gate, const orc_stack* up, const orc_stack* down,
                            const float* xs, const uint32_t* ids, const float* w,
                            int rows, int width, float* out, int threads) {
    if (check_stacks(gate, up, down)) return -1;
    if (threads < 1 || threads > 256) return -1;
    const int H = gate->k, I = gate->n, E = gate->e;
    for (int i = 0; i < rows * width; ++i)
        if (ids[i] >= (uint32_t)E) return -1;
    float* h = (float*)malloc(sizeof(float) * (size_t)width * (size_t)I);
    int* owner = (int*)malloc(sizeof(int) * (size_t)width);
    mt_job* jobs = (mt_job*)malloc(sizeof(mt_job) * (size_t)threads);
    pthread_t* tid = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    if (!h || !owner || !jobs || !tid) { free(h); free(owner); free(jobs); free(tid); return -2; }
    int rc = 0;
    for (int t = 0; t < rows && !rc; ++t) {
        const uint32_t* id = ids + (int64_t)t * width;
        const float* wt = w + (int64_t)t * width;
        for (int j = 0; j < width; ++j) { /* the same owners as the single-threaded pass 1 */
            owner[j] = -1;
            if (wt[j] == 0.0f) continue;
            for (int i = 0; i < j; ++i)
                if (owner[i] >= 0 && id[i] == id[j]) { owner[j] = owner[i]; break; }
            if (owner[j] < 0) owner[j] = j;
        }
        for (int pass = 1; pass <= 2 && !rc; ++pass) {
            const int n = pass == 1 ? width * I : H;
            int started = 0;
            for (int k = 0; k < threads; ++k) {
                jobs[k] = (mt_job){gate, up, down, xs + (int64_t)t * H, id, wt, owner, h, out + (int64_t)t * H,
                                   width, pass, (int)((int64_t)n * k / threads), (int)((int64_t)n * (k + 1) / threads)};
                if (pthread_create(&tid[k], NULL, mt_run, &jobs[k]) != 0) { rc = -2; break; }
                ++started;
            }
            for (int k = 0; k < started; ++k) pthread_join(tid[k], NULL);
        }
    }
    free(h);
    free(owner);
    free(jobs);
    free(tid);
    return rc;
}

int orc_fused_moe_decode_f64(const orc_stack* gate, const orc_stack* up, const orc_stack* down,
                             const float* xs, const uint32_t* ids, const float* w,
                             int rows, int width, double* out) {
    if (check_stacks(gate, up, down)) return -1;
    const int H = gate->k, I = gate->n, E = gate->e;
    for (int i = 0; i < rows * width; ++i)
        if (ids[i] >= (uint32_t)E) return -1;
    int64_t big = H > I ? H : I;
    double* x64 = (double*)malloc(sizeof(double) * (size_t)H);
    double* h = (double*)malloc(sizeof(double) * (size_t)I);
    double* scratch = (double*)malloc(sizeof(double) * (size_t)big);
    if (!x64 || !h || !scratch) { free(x64); free(h); free(scratch); return -2; }
    for (int t = 0; t < rows; ++t) {
        for (int i = 0; i < H; ++i) x64[i] = xs[(int64_t)t * H + i];
        double* o = out + (int64_t)t * H;
        for (int r = 0; r < H; ++r) o[r] = 0.0;
        for (int j = 0; j < width; ++j) {
            uint32_t e = ids[(int64_t)t * width + j];
            double wt = w[(int64_t)t * width + j];
            if (wt == 0.0) continue;
            for (int r = 0; r < I; ++r) {
                double g = vec_dot_f64(gate->dtype, expert_row(gate, (int)e, r), x64, H, scratch);
                double u = vec_dot_f64(up->dtype, expert_row(up, (int)e, r), x64, H, scratch);
                h[r] = g / (1.0 + exp(-g)) * u;
            }
            for (int r = 0; r < H; ++r)
                o[r] += wt * vec_dot_f64(down->dtype, expert_row(down, (int)e, r), h, I, scratch);
        }
    }
    free(x64);
    free(h);
    free(scratch);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* router                                                                    */
/* ------------------------------------------------------------------------- */

int orc_router_logits(const float* x, const float* W, int rows, int H, int E, float* logits) {
    if (H % ORC_ROUTER_CHUNK != 0) return -1;
    const float scale = 4294967296.0f; /* 2^32 */
    for (int t = 0; t < rows; ++t) {
        const float* xr = x + (int64_t)t * H;
        for (int e = 0; e < E; ++e) {
            const float* wr = W + (int64_t)e * H;
            int64_t acc = 0;
            for (int c = 0; c < H; c += ORC_ROUTER_CHUNK) {
                float p = 0.0f;
                for (int i = 0; i < ORC_ROUTER_CHUNK; ++i) p = fmaf(wr[c + i], xr[c + i], p);
                acc += (int64_t)llrintf(p * scale);
            }
            logits[(int64_t)t * E + e] = (float)acc * 0x1p-32f;
        }
    }
    return 0;
}

/* top_k_ids (src/moe/cached_layer.rs:357-363): logit desc, ties lowest id. */
int orc_topk(const float* logits, int rows, int E, int k, int mode, uint32_t* ids, float* w) {
    if (k <= 0 || k > E || k > 64) return -1;
    for (int t = 0; t < rows; ++t) {
        const float* l = logits + (int64_t)t * E;
        uint32_t* id = ids + (int64_t)t * k;
        float* wt = w + (int64_t)t * k;
        /* selection: k passes of arg-max with the (value desc, id asc) order */
        for (int j = 0; j < k; ++j) {
            int best = -1;
            for (int e = 0; e < E; ++e) {
                int taken = 0;
                for (int i = 0; i < j; ++i)
                    if (id[i] == (uint32_t)e) { taken = 1; break; }
                if (taken) continue;
                if (best < 0 || l[e] > l[best]) best = e;
            }
            id[j] = (uint32_t)best;
        }
        float mx = l[id[0]];
        float ex[64];
        float denom = 0.0f;
        for (int j = 0; j < k; ++j) {
            ex[j] = expf(l[id[j]] - mx);
            denom += ex[j];
        }
        if (mode == ORC_ROUTE_SOFTMAX_TOPK) {
            denom = 0.0f;
            for (int e = 0; e < E; ++e) denom += expf(l[e] - mx);
        } else if (mode != ORC_ROUTE_SOFTMAX_TOPK_RENORM && mode != ORC_ROUTE_TOPK_SOFTMAX) {
            return -1;
        }
        for (int j = 0; j < k; ++j) wt[j] = ex[j] / denom;
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* gather                                                                    */
/* ------------------------------------------------------------------------- */

int orc_gather(const uint32_t* ids, int n, int E, uint32_t* perm, uint32_t* offsets) {
    for (int i = 0; i < n; ++i)
        if (ids[i] >= (uint32_t)E) return -1;
    for (int e = 0; e <= E; ++e) offsets[e] = 0;
    for (int i = 0; i < n; ++i) offsets[ids[i] + 1]++;
    for (int e = 0; e < E; ++e) offsets[e + 1] += offsets[e];
    uint32_t* fill = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(E > 0 ? E : 1));
    if (!fill) return -2;
    for (int e = 0; e < E; ++e) fill[e] = offsets[e];
    for (int i = 0; i < n; ++i) perm[fill[ids[i]]++] = (uint32_t)i;
    free(fill);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* stack decode                                                              */
/* ------------------------------------------------------------------------- */

static int stack_decode_impl(const orc_layer* layers, int n_layers, uint16_t* x, int rows, int H,
                             int E, int k, int mode, uint32_t* ids_out, float* w_out, int threads) {
    float* xf = (float*)malloc(sizeof(float) * (size_t)rows * H);
    float* y = (float*)malloc(sizeof(float) * (size_t)rows * H);
    float* logits = (float*)malloc(sizeof(float) * (size_t)rows * E);
    uint32_t* ids = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)rows * k);
    float* w = (float*)malloc(sizeof(float) * (size_t)rows * k);
    int rc = 0;
    if (!xf || !y || !logits || !ids || !w) { rc = -2; goto done; }
    for (int l = 0; l < n_layers && rc == 0; ++l) {
        const orc_layer* L = &layers[l];
        orc_bf16_to_f32_n(x, (int64_t)rows * H, xf);
        if ((rc = orc_router_logits(xf, L->router, rows, H, E, logits))) break;
        if ((rc = orc_topk(logits, rows, E, k, mode, ids, w))) break;
        if (ids_out) memcpy(ids_out + (int64_t)l * rows * k, ids, sizeof(uint32_t) * (size_t)rows * k);
        if (w_out) memcpy(w_out + (int64_t)l * rows * k, w, sizeof(float) * (size_t)rows * k);
        rc = threads > 0 ? orc_fused_moe_decode_mt(&L->gate, &L->up, &L->down, xf, ids, w, rows, k, y, threads)
                         : orc_fused_moe_decode(&L->gate, &L->up, &L->down, xf, ids, w, rows, k, y);
        if (rc) break;
        for (int64_t i = 0; i < (int64_t)rows * H; ++i) x[i] = orc_f32_to_bf16(xf[i] + y[i]);
    }
done:
    free(xf);
    free(y);
    free(logits);
    free(ids);
    free(w);
    return rc;
}

int orc_stack_decode(const orc_layer* layers, int n_layers, uint16_t* x, int rows, int H,
                     int E, int k, int mode, uint32_t* ids_out, float* w_out) {
    return stack_decode_impl(layers, n_layers, x, rows, H, E, k, mode, ids_out, w_out, 0);
}

int orc_stack_decode_mt(const orc_layer* layers, int n_layers, uint16_t* x, int rows, int H,
                        int E, int k, int mode, uint32_t* ids_out, float* w_out, int threads) {
    if (threads < 1) return -1;
    return stack_decode_impl(layers, n_layers, x, rows, H, E, k, mode, ids_out, w_out, threads);
}
