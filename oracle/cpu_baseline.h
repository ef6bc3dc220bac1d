/*
 * cpu_baseline.h -- the CPU expert path timed beside the GPU (TEST
 * INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg and tests/ load it; the
 * product library never does).  The reference's CPU expert path
 * (fused_moe_decode, src/moe/stages/cpu_miss.rs:13-20, :45) with int8
 * activations and AVX2 integer dots, on a persistent thread pool.
 */
#ifndef NAIWA_CPU_BASELINE_H
#define NAIWA_CPU_BASELINE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CB_Q8_0 8
#define CB_Q4_K 12

/* A stacked [e, n, k] quantized tensor (expert x at base + x * n * row_bytes). */
typedef struct cb_stack {
    const uint8_t* base;
    int32_t e, n, k, dtype;
} cb_stack;

typedef struct cb_pool cb_pool;

cb_pool* cb_pool_create(int threads);
void cb_pool_destroy(cb_pool* pool);
int cb_threads(const cb_pool* pool);

/* out[rows, H] = sum_j w[t, j] * down_e(SiLU(gate_e x_t) * up_e x_t), e = ids[t, j],
 * xs [rows, H] f32.  Returns 0, -1 on a bad argument or id, -2 out of memory. */
int cb_fused_moe_decode(cb_pool* pool, const cb_stack* gate, const cb_stack* up, const cb_stack* down,
                        const float* xs, const uint32_t* ids, const float* w, int rows, int width, float* out);

#ifdef __cplusplus
}
#endif
#endif
