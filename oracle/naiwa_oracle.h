/*
 * naiwa_oracle.h -- CPU restatement of naiwa-rs's MoE expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity reference for the HIP
 * library under naiwa-rs_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the reference results
 * or as the timed CPU baseline.  The product path never calls into it.
 *
 * What it restates (reference files are naiwa-rs paths):
 *   - GGML block formats Q8_0 / Q4_K (public ggml layout; the byte stride rule
 *     of src/moe/expert.rs:123-145 and src/moe/slot.rs:84-95).
 *   - The CPU expert path contract of src/moe/stages/cpu_miss.rs:13-20
 *     (fused_moe_decode): pass 1 gate+up+SiLU per distinct (expert,row),
 *     pass 2 down with the router-weighted sum, weight-0 slots skipped,
 *     f32 activations (src/prefill_stream.rs:1961-1963).
 *   - Router top-k with ties to the lower id (src/moe/cached_layer.rs:357-363).
 *   - The token->expert gather as a stable counting sort
 *     (grouping rule of src/moe/stages/gpu.rs:100-133).
 *
 * Parity pinning (see tests/test_oracle.py): hand-built blocks with
 * hand-computed dequantization, quantizer round-trip bounds, an fp64
 * brute-force expert path, brute-force top-k / gather on tiny inputs, and the
 * known answers of the reference's unit tests (src/moe/tests.rs:113-186).
 */
#ifndef NAIWA_ORACLE_H
#define NAIWA_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (ggml.h enum ggml_type). */
#define ORC_F32  0
#define ORC_F16  1
#define ORC_Q8_0 8
#define ORC_Q4_K 12
#define ORC_BF16 30

/* Router weight modes (model-family routing rules, from public model configs). */
#define ORC_ROUTE_SOFTMAX_TOPK_RENORM 0 /* Qwen3 (norm_topk_prob): softmax, top-k, renormalize   */
#define ORC_ROUTE_TOPK_SOFTMAX        1 /* Mixtral: top-k on logits, softmax over the k          */
#define ORC_ROUTE_SOFTMAX_TOPK        2 /* DeepSeek-V2-Lite: softmax over all E, no renormalize  */

/* Router logit accumulation: chunks of ROUTER_CHUNK hidden dims are summed
 * sequentially in fp32 (fmaf chain), each chunk partial is rounded to a signed
 * 64-bit fixed-point value with ROUTER_FIX_BITS fractional bits, and the chunk
 * partials are summed exactly as integers.  The result is independent of how
 * the chunks are distributed over threads, which is what lets the device add
 * partials in any order (even with integer atomics) and still match bit for
 * bit. */
#define ORC_ROUTER_CHUNK    8
#define ORC_ROUTER_FIX_BITS 32

/* ---- scalar conversions ------------------------------------------------ */
float    orc_fp16_to_f32(uint16_t h);
uint16_t orc_f32_to_fp16(float f);      /* round to nearest even */
float    orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);      /* round to nearest even */
void     orc_f32_to_bf16_n(const float* x, int64_t n, uint16_t* out);
void     orc_bf16_to_f32_n(const uint16_t* x, int64_t n, float* out);

/* ---- block formats ------------------------------------------------------ */
int      orc_block_size(int dtype);     /* values per block  */
int      orc_type_size(int dtype);      /* bytes per block   */
int64_t  orc_row_bytes(int dtype, int64_t k);  /* -1 if k % block != 0 */
void     orc_quantize_q8_0(const float* x, int64_t n, uint8_t* out);
void     orc_dequantize_q8_0(const uint8_t* in, int64_t n, float* y);
void     orc_quantize_q4_k(const float* x, int64_t n, uint8_t* out);
void     orc_dequantize_q4_k(const uint8_t* in, int64_t n, float* y);
int      orc_quantize(int dtype, const float* x, int64_t n, uint8_t* out);
int      orc_dequantize(int dtype, const uint8_t* in, int64_t n, float* y);
/* fp64 dequantization (exact: every factor is a small integer or an fp16). */
int      orc_dequantize_f64(int dtype, const uint8_t* in, int64_t n, double* y);

/* ---- deterministic synthetic data -------------------------------------- */
/* Counter-based N(mean, std): value i depends only on (seed, offset + i). */
void     orc_fill_normal(uint64_t seed, uint64_t offset, int64_t n, float mean, float stdv, float* out);

/* ---- expert stacks ------------------------------------------------------- */
/* A stacked [E, N, K] quantized tensor: expert e starts at
 * base + e * N * row_bytes(dtype, K)   (src/moe/expert.rs:136). */
typedef struct orc_stack {
    const uint8_t* base;
    int32_t e, n, k, dtype;
} orc_stack;

int64_t  orc_expert_bytes(const orc_stack* s);  /* N * row_bytes(K) */

/* One quantized row dotted with f32 x: dequantize the row to f32 with the
 * ggml formula, then accumulate sequentially in f32. */
float    orc_vec_dot(int dtype, const uint8_t* row, const float* x, int64_t k);

/* fused_moe_decode restatement (src/moe/stages/cpu_miss.rs:13-20, :45).
 * xs [rows, H] f32, ids/w [rows, width] row-major, out [rows, H] f32.
 * Returns 0, or -1 on an id >= E or a shape mismatch. */
int      orc_fused_moe_decode(const orc_stack* gate, const orc_stack* up, const orc_stack* down,
                              const float* xs, const uint32_t* ids, const float* w,
                              int rows, int width, float* out);
/* The same computation in fp64 end to end (brute-force pin). */
/* The same on `threads` host threads, bit-identical (CPU baseline). */
int      orc_fused_moe_decode_mt(const orc_stack* gate, const orc_stack* up, const orc_stack* down,
                                 const float* xs, const uint32_t* ids, const float* w,
                                 int rows, int width, float* out, int threads);
int      orc_fused_moe_decode_f64(const orc_stack* gate, const orc_stack* up, const orc_stack* down,
                                  const float* xs, const uint32_t* ids, const float* w,
                                  int rows, int width, double* out);

/* ---- router ---------------------------------------------------------------- */
/* logits[rows, E] = W[E, H] . x[rows, H]  with the chunked fixed-point rule. */
int      orc_router_logits(const float* x, const float* W, int rows, int H, int E, float* logits);
/* top-k (value desc, id asc) of logits[rows, E] + weights per mode. */
int      orc_topk(const float* logits, int rows, int E, int k, int mode, uint32_t* ids, float* w);

/* ---- gather ---------------------------------------------------------------- */
/* Stable counting sort of the n = rows*k flattened ids by value:
 * perm[pos] = flat index, offsets[E+1] = segment starts.  -1 on id >= E. */
int      orc_gather(const uint32_t* ids, int n, int E, uint32_t* perm, uint32_t* offsets);

/* ---- a decode stack: x_{l+1} = bf16(x_l + MoE_l(x_l)) ---------------------- */
typedef struct orc_layer {
    const float* router;   /* [E, H] f32 */
    orc_stack gate, up, down;
} orc_layer;
/* x [rows, H] bf16 in/out.  Per layer: router logits, top-k (mode), fused
 * decode over all routed experts, residual add in f32, store bf16.  ids_out
 * (optional) receives [layers, rows, k] routed ids. */
int      orc_stack_decode(const orc_layer* layers, int n_layers, uint16_t* x, int rows, int H,
                          int E, int k, int mode, uint32_t* ids_out, float* w_out);
/* The same with the expert path on `threads` host threads (bit-identical). */
int      orc_stack_decode_mt(const orc_layer* layers, int n_layers, uint16_t* x, int rows, int H,
                             int E, int k, int mode, uint32_t* ids_out, float* w_out, int threads);

#ifdef __cplusplus
}
#endif
#endif
