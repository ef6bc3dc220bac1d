/*
 * naiwa_moe.h -- C ABI of the MI355X (gfx950) MoE expert hot path.
 *
 * Every entry point is `extern "C"`, takes plain pointers and sizes, returns
 * an int (0 = ok, > 0 a hipError_t, < 0 a NAIWA_E_* code) unless it keeps the
 * reference's own `void` signature, and never throws.  Device pointers are
 * caller-owned.  `stream` is a hipStream_t passed as int64_t (0 = the null
 * stream), as in the reference's doorbell FFI.  Launches are asynchronous and
 * stream-ordered.  One thread submits GPU work per device; the upload entry
 * points may be called from one other thread.  The decode, prefill, router
 * (when it keeps its logits internally) and layered-stack entry points reuse
 * one grow-only scratch buffer per device and entry point from call to call:
 * two such calls on different streams must be ordered by the caller (an event
 * between them).  The fused stack orders its launches itself, whatever their
 * streams.
 *
 * Reference interfaces each group replaces (naiwa-rs paths):
 *   doorbell_*            src/doorbell/mod.rs:31-69, src/doorbell/doorbell.cu:15-149
 *   naiwa_moe_decode      mistralrs_quant::indexed_moe_fused_decode, called at
 *                         src/moe/stages/gpu.rs:27-66
 *   naiwa_router_topk     the model-side router softmax/top-k consumed at
 *                         src/moe/decode.rs:33-39 (tie rule of
 *                         src/moe/cached_layer.rs:357-363)
 *   naiwa_moe_gather      the per-bank grouping of src/moe/stages/gpu.rs:100-133
 *   naiwa_moe_prefill     the fork's grouped MoEExperts::forward, called at
 *                         src/prefill_stream.rs:2080-2102
 *   naiwa_upload_expert   CopyStream::queue_async, src/copy_stream.rs:387-409
 *   naiwa_cache_* etc.    the slot policy of src/moe/cached_layer.rs and
 *                         src/moe/stages/{route,dma_miss}.rs, src/moe/staging.rs
 *                         (include/naiwa_policy.h)
 */
#ifndef NAIWA_MOE_H
#define NAIWA_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------- */
#define NAIWA_OK             0
#define NAIWA_E_INVALID     -1  /* bad argument, shape or alignment          */
#define NAIWA_E_UNSUPPORTED -2  /* dtype / activation / mode not served      */
#define NAIWA_E_TIMEOUT     -3  /* a bounded wait expired                    */
#define NAIWA_E_NOMEM       -4  /* allocation failed                         */
#define NAIWA_E_BAD_ID      -5  /* expert or slot id out of range            */
#define NAIWA_E_NOT_FOUND   -6  /* no such expert / slot / entry             */
#define NAIWA_E_DEVICE      -7  /* the device reported a failed condition    */
#define NAIWA_E_FORMAT      -8  /* malformed or unsupported file (GGUF)      */
#define NAIWA_E_IO          -9  /* a file cannot be opened or mapped         */
#define NAIWA_E_TOO_LARGE  -10  /* the call needs more than a fixed capacity */

/* ---- GGML type ids --------------------------------------------------------- */
#define NAIWA_F32  0
#define NAIWA_F16  1
#define NAIWA_Q8_0 8
#define NAIWA_Q4_K 12
#define NAIWA_BF16 30

/* ---- activations (src/moe/stages/gpu.rs:15-21) ------------------------------- */
#define NAIWA_ACT_SILU           0
#define NAIWA_ACT_GELU_PYTORCH_TANH 1

/* ---- router weight modes (public model configs) ------------------------------ */
#define NAIWA_ROUTE_SOFTMAX_TOPK_RENORM 0 /* Qwen3: softmax, top-k, renormalize  */
#define NAIWA_ROUTE_TOPK_SOFTMAX        1 /* Mixtral: softmax over the top-k     */
#define NAIWA_ROUTE_SOFTMAX_TOPK        2 /* DeepSeek-V2-Lite: no renormalize    */

const char* naiwa_status_string(int rc);

/* ======================================================================== */
/* Runtime plumbing (device memory, streams, events) so a host binding      */
/* needs nothing but this library.                                          */
/* ======================================================================== */
int naiwa_device_count(int* n);
int naiwa_set_device(int dev);
int naiwa_device_info(int dev, int* cu_count, int* wall_clock_khz, int64_t* hbm_bytes, char* name, int name_len);
int naiwa_malloc(void** p, size_t bytes);          /* 256-B aligned device memory */
int naiwa_free(void* p);
/* Free and total bytes of the current device (hipMemGetInfo). */
int naiwa_mem_info(uint64_t* free_bytes, uint64_t* total_bytes);
int naiwa_host_alloc(void** p, size_t bytes);      /* pinned, portable host memory */
int naiwa_host_free(void* p);
int naiwa_memcpy_h2d(void* dst, const void* src, size_t bytes, int64_t stream);
int naiwa_memcpy_d2h(void* dst, const void* src, size_t bytes, int64_t stream);
int naiwa_memcpy_d2d(void* dst, const void* src, size_t bytes, int64_t stream);
/* height rows of width bytes, device to device, rows dpitch / spitch bytes apart
 * (e.g. a [T, k] routing result into the first k columns of a [T, k + s] one). */
int naiwa_memcpy_2d_d2d(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width, size_t height,
                        int64_t stream);
/* The same in any direction (host or device pointers on either side, e.g. one
 * projection's [E] expert ranges into interleaved pinned host stacks). */
int naiwa_memcpy_2d(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width, size_t height,
                    int64_t stream);
int naiwa_memset(void* p, int value, size_t bytes, int64_t stream);
int naiwa_stream_create(int64_t* stream);
int naiwa_stream_destroy(int64_t stream);
int naiwa_stream_sync(int64_t stream);
int naiwa_stream_wait_event(int64_t stream, int64_t event);
int naiwa_event_create(int64_t* event, int timing);
int naiwa_event_destroy(int64_t event);
int naiwa_event_record(int64_t event, int64_t stream);
int naiwa_event_sync(int64_t event);
int naiwa_event_query(int64_t event);              /* 0 done, 1 pending, else error */
int naiwa_event_elapsed_ms(float* ms, int64_t start, int64_t end);
int naiwa_device_sync(void);
int naiwa_last_error(void);                        /* hipGetLastError as int */

/* ======================================================================== */
/* Doorbells -- same names and signatures as the reference FFI             */
/* (src/doorbell/mod.rs:31-69).  Mapped memory is fine-grained and host-    */
/* coherent (hipHostMallocMapped | hipHostMallocCoherent), zeroed here.     */
/* ======================================================================== */
/* cudaHostAlloc(Mapped) counterpart, src/doorbell/doorbell.cu:35-38. */
int  doorbell_alloc_mapped(void** out, size_t bytes);
/* src/doorbell/doorbell.cu:40-42. */
int  doorbell_free_host(void* p);
/* src/doorbell/doorbell.cu:44-46.  *dev = NULL on failure. */
void doorbell_get_device_ptr(void* host, void** dev);
/* Publish n u32 ids + n f32 weights, system fence, then *d_seq += 1
 * (src/doorbell/doorbell.cu:15-33, :48-61). */
void doorbell_ring(void* d_seq, void* d_ids, void* d_weights, const void* src_ids,
                   const void* src_weights, int n, int64_t stream);
/* Copy n f32 to a mapped slot, fence, *d_seq += 1 (doorbell.cu:70-96). */
void doorbell_copy_f32(void* d_seq, void* d_dst, const void* src, int n, int64_t stream);
/* Wait until *d_seq >= target, copy n f32 from d_payload + slot_off to dst,
 * fence, *d_consumed = target (doorbell.cu:105-149).  Unlike the reference the
 * wait is bounded (naiwa_doorbell_set_wait_limit_us): an expired wait copies
 * nothing, leaves d_consumed alone and counts a timeout. */
void doorbell_wait_copy_f32(void* d_seq, uint32_t target, void* d_payload, int64_t slot_off,
                            void* d_consumed, void* dst, int n, int64_t stream);
/* The persistent-wave variant of the device-side doorbell waits (the
 * reference launches one spinning kernel per wait, doorbell.cu:105-149):
 *  - doorbell_poll_serve: one wave answers `count` host rings in a row: for
 *    i = 0 .. count-1 it waits until *d_seq >= first + i, then stores first + i
 *    to *d_ack at system scope (the host's round trip is ring -> observe ack;
 *    the wave publishes nothing else, so no release fence goes with it);
 *  - doorbell_poll_wait: a stream-ordered wait for *d_flag >= target, polled by
 *    one wave (e.g. an "upload done" flag another stream raises) with relaxed
 *    loads and one acquire at the end: work queued after it on `stream` starts
 *    when it exits;
 *  - doorbell_poll_signal: store `value` to *d_flag (system scope) once the
 *    work queued before it on `stream` is done: that work has completed and its
 *    writes were released when it ended, so the store needs no fence.
 * Flags are u32 words in device memory or mapped memory (device pointers).
 * Every wait is bounded like doorbell_wait_copy_f32's; an expired wait counts a
 * timeout (naiwa_doorbell_timeouts) and the wave exits. */
int  doorbell_poll_serve(void* d_seq, void* d_ack, uint32_t first, uint32_t count, int64_t stream);
int  doorbell_poll_wait(const void* d_flag, uint32_t target, int64_t stream);
int  doorbell_poll_signal(void* d_flag, uint32_t value, int64_t stream);
/* Bound of every device-side doorbell wait (default 10 s; 0 restores it). */
int  naiwa_doorbell_set_wait_limit_us(uint64_t us);
/* Device waits that expired since the library was loaded. */
int  naiwa_doorbell_timeouts(uint32_t* count);
/* Host-side helpers of the doorbell protocol (src/doorbell/mapped.rs:99-141):
 * release-store a u32, acquire-load a u32, and wait (spin then sleep-poll)
 * for *word >= target with an optional timeout (timeout_us < 0: never).
 * naiwa_host_wait_ge returns 0 when reached, NAIWA_E_TIMEOUT otherwise. */
void naiwa_host_store_release_u32(void* word, uint32_t value);
uint32_t naiwa_host_load_acquire_u32(const void* word);
int  naiwa_host_wait_ge(const void* word, uint32_t target, int64_t timeout_us, int64_t poll_us);

/* ======================================================================== */
/* Expert banks: the slot-indexed GPU expert cache                           */
/* (src/moe/slot.rs:46-66).  One bank per projection: slot s of the bank    */
/* starts at base + s * slot_stride and holds one expert's [n, k] GGML       */
/* blocks verbatim.  base and slot_stride are 256-B aligned.                  */
/* ======================================================================== */
typedef struct naiwa_bank {
    const void* base;
    int64_t slot_stride;   /* bytes between slots (>= n * row_bytes(k))      */
    int32_t slots;         /* slots in the bank                                */
    int32_t n;             /* output rows                                      */
    int32_t k;             /* input features                                   */
    int32_t dtype;         /* NAIWA_Q4_K or NAIWA_Q8_0                         */
} naiwa_bank;

/* Bytes of one [n, k] projection in `dtype` (src/moe/slot.rs:84-95); -1 when
 * k is not a multiple of the block size. */
int64_t naiwa_projection_bytes(int dtype, int64_t n, int64_t k);

/* The replacement of indexed_moe_fused_decode (src/moe/stages/gpu.rs:27-66):
 *   out[t] = sum_j w[t,j] * down_s( act(gate_s x_t) * up_s x_t ),  s = slot_ids[t,j]
 * x [rows, H] bf16 or f32 (x_dtype), slot_ids/w [rows, width] device arrays,
 * out [rows, H] f32.  Weight-0 entries (the reference's padding) are skipped.
 * The combine is atomics-free: per output row, slots are added in ascending
 * slot order, the same on every run. */
int naiwa_moe_decode(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down,
                     const void* x, int x_dtype, const uint32_t* slot_ids, const float* w,
                     int rows, int width, int act, float* out, int64_t stream);
/* As naiwa_moe_decode; flags NAIWA_DECODE_ACCUMULATE continues each output
 * row's sum from out's values, so a call over the pairs of low slots and then
 * an accumulating call over the pairs of higher slots add exactly the terms,
 * in exactly the order, of one call over both (e.g. cache slots first, then
 * staging slots whose upload is still landing). */
#define NAIWA_DECODE_ACCUMULATE 1
int naiwa_moe_decode_ex(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down,
                        const void* x, int x_dtype, const uint32_t* slot_ids, const float* w,
                        int rows, int width, int act, float* out, int flags, int64_t stream);
/* No counterpart in the reference.  naiwa_moe_decode_ex for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the same kernels and the same results bit for bit, with
 * the scratch (segments, permutation, h) in a fixed device array of
 * NAIWA_DECODE_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends,
 * instead of the library's grow-only buffer.  No hipMalloc, hipFree or
 * allocating routine is called; nothing is cleared with a memset.  A call of
 * n = rows * width pairs (H the hidden size, I the intermediate size, a(v) = v
 * rounded up to a multiple of 256) needs
 *   S = 256 + 2 a(4 n) + a(4 (n + 1)) + T  bytes, where
 *   T = a(max(n D, a(2 rows H) + 2 n I)) + ceil(I / 2048) 4 n H
 *       when n <= 512 and width <= 16 (h staged once in the down format, D =
 *       its bytes per pair: 2 I + I / 4 for Q4_K, 2 I + I / 8 for Q8_0,
 *       rounded up to a multiple of 16; plus the f32 dots of each 2048-wide
 *       K part of down),
 *   T = 4 n I otherwise (h as f32),
 * which naiwa_moe_decode_scratch_bytes returns; the entry point returns
 * NAIWA_E_TOO_LARGE, before any device call, when S exceeds the array.  The
 * 8 MiB array holds 56 pairs (rows <= 28 at top-2) at H 4096, I 14336, Q4_K;
 * 2712 pairs (rows <= 339 at top-8) at H 2048, I 768.  S is not monotone in n:
 * the staged path's K-part dots cost more per pair than f32 h, so at H 5120,
 * I 1536, top-6, rows 1-55 and 86-227 fit and rows 56-85 do not.
 * Every call on one GPU uses that GPU's one array: calls that overlap
 * on the device (other streams, other host threads) race and must be ordered
 * by the caller. */
#define NAIWA_DECODE_NOALLOC_SCRATCH_BYTES (8u << 20)
int naiwa_moe_decode_noalloc(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down,
                             const void* x, int x_dtype, const uint32_t* slot_ids, const float* w,
                             int rows, int width, int act, float* out, int flags, int64_t stream);
/* No counterpart in the reference.  The scratch bytes S (above) that a decode
 * call of rows x width pairs needs at hidden size H, intermediate size I and
 * down format down_dtype; the no-alloc entry point accepts the call when S <=
 * NAIWA_DECODE_NOALLOC_SCRATCH_BYTES.  0 for an empty call, -1 for invalid
 * sizes.  No device call. */
int64_t naiwa_moe_decode_scratch_bytes(int rows, int width, int H, int I, int down_dtype);

/* Router: logits = W . x with the chunked fixed-point accumulation (chunks of 8
 * features summed as an f32 fma chain, each rounded to int64 with 32
 * fractional bits, chunk partials added exactly), top-k by (logit desc, id
 * asc), weights per mode.  x [rows, H] bf16/f32, W [E, H] f32; ids_out/w_out
 * [rows, k]; logits_out [rows, E] f32 or NULL.  H % 8 == 0, E <= 1024, k <= 32. */
int naiwa_router_topk(const void* x, int x_dtype, const float* W, int rows, int H, int E, int k,
                      int mode, uint32_t* ids_out, float* w_out, float* logits_out, int64_t stream);
/* As naiwa_router_topk with a per-expert f32 bias added to each logit after
 * the fixed-point sum (logit = sum * 2^-32 + bias[e], one f32 add); bias may
 * be null.  Routers with a bias term (and routing-skew studies) use it. */
int naiwa_router_topk_biased(const void* x, int x_dtype, const float* W, const float* bias, int rows, int H,
                             int E, int k, int mode, uint32_t* ids_out, float* w_out, float* logits_out,
                             int64_t stream);
/* As naiwa_router_topk_biased with ids_out / w_out rows ld >= k entries apart:
 * row t's k routed ids and weights go to [t * ld, t * ld + k) and the other
 * columns are left as they are.  No counterpart in the reference, which routes
 * one MoE layer's routed experts only: a caller that adds always-on experts
 * (DeepSeek-V2's shared experts, at weight 1 in columns k..ld-1 of the same
 * table for naiwa_moe_prefill) fills the table without a copy. */
int naiwa_router_topk_ld(const void* x, int x_dtype, const float* W, const float* bias, int rows, int H, int E,
                         int k, int mode, uint32_t* ids_out, float* w_out, int ld, float* logits_out,
                         int64_t stream);

/* Gather: stable counting sort of the n flattened ids by value.
 * perm_out[n] = flat (t*k + j) indices grouped by id, offsets_out[E+1] =
 * segment starts.  n <= 65536, E <= 4096.  Ids >= E are counted in
 * *bad_out (device int, may be NULL) and left out of every segment. */
int naiwa_moe_gather(const uint32_t* ids, int n, int E, uint32_t* perm_out, uint32_t* offsets_out,
                     int* bad_out, int64_t stream);

/* Prefill: the routed experts of a chunk of T tokens (many tokens per expert) as
 * grouped GEMMs on the matrix cores -- the counterpart of the fork's grouped
 * MoEExperts::forward (src/prefill_stream.rs:2080-2102).  Same banks, slot ids
 * and weights [T, k] as naiwa_moe_decode; x is bf16 [T, H]; out f32 [T, H].
 * Weights are dequantised in f32 in registers, rounded once to bf16 and
 * multiplied with v_mfma_f32_32x32x16_bf16 (f32 accumulation); x and h are
 * bf16.  Needs
 * H, I multiples of 128; gate/up Q4_K (H % 256 == 0) or Q8_0, down Q4_K (I %
 * 256 == 0) or Q8_0; T * k <= 65536; slots <= 4096.  Slot ids outside the
 * bank contribute nothing.  flags: NAIWA_PREFILL_ACCUMULATE adds to out
 * (e.g. shared experts on top of the routed ones) instead of overwriting. */
#define NAIWA_PREFILL_ACCUMULATE 1
/* NAIWA_PREFILL_RESIDUAL: also x = bf16(x + out) in place after out is formed, one
 * launch fewer than a separate residual add (the same bits); x must then be
 * writable and no other work may read it during the call. */
#define NAIWA_PREFILL_RESIDUAL 2
/* The matrix cores take x, the dequantised weights and h as bf16 (f32
 * accumulation): any finite activation is taken as it is, without clamping. */
int naiwa_moe_prefill(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, const void* x,
                      const uint32_t* slot_ids, const float* w, int T, int k, int act, float* out, int flags,
                      int64_t stream);

/* ======================================================================== */
/* A decode stack: per layer, x <- bf16(x + MoE_l(x)) with the router,      */
/* top-k, expert decode and combine all on the device.  The reference runs  */
/* one CachedExperts::forward per MoE layer (src/moe/cached_layer.rs:524)   */
/* after the model's router; this entry chains those calls for a whole      */
/* decode step so no routing decision leaves the GPU.                       */
/* ======================================================================== */
typedef struct naiwa_layer {
    const float* router;            /* [E, H] f32                                */
    naiwa_bank gate, up, down;      /* slot banks of this layer                  */
    const int32_t* slot_of_expert;  /* [E] device table (-1: not resident), or
                                       NULL when slot == expert id               */
} naiwa_layer;

#define NAIWA_STACK_LAYERED 0  /* router, decode and residual as separate launches */
#define NAIWA_STACK_FUSED   1  /* one persistent kernel for the whole stack        */

/* x: [rows, H] bf16 device buffer, updated in place.  ids_out / w_out:
 * [n_layers, rows, k] device buffers receiving the routing, or NULL. */
int naiwa_stack_decode(const naiwa_layer* layers, int n_layers, void* x, int rows, int H, int E,
                       int k, int mode, int act, uint32_t* ids_out, float* w_out, int flags,
                       int64_t stream);
/* As naiwa_stack_decode; y_out (may be NULL) is an f32 device buffer
 * [n_layers, rows, H] receiving each layer's MoE output MoE_l(x_l) before the
 * residual add and the bf16 store, so a caller can check every layer's expert
 * output on its own (x_{l+1} = bf16(f32(x_l) + y_l) exactly). */
int naiwa_stack_decode_y(const naiwa_layer* layers, int n_layers, void* x, int rows, int H, int E,
                         int k, int mode, int act, uint32_t* ids_out, float* w_out, float* y_out,
                         int flags, int64_t stream);

/* Blocks per CU of the fused kernel (1..8, capped by occupancy; default 1). */
int naiwa_stack_set_blocks_per_cu(int n);
/* Counters of every fused launch since the last call: waits for another
 * workgroup's data that gave up after their 2 s bound (the grid was not
 * co-resident, e.g. another tenant held CUs; that launch's output is invalid),
 * and routed experts with no resident slot (weight dropped).  Reading resets
 * them.  Synchronizes the device. */
int naiwa_stack_status(int* barrier_timeouts, int* missing_experts);

/* Diagnostic phase timestamps of the fused kernel: when enabled, every block
 * records s_memrealtime ticks at each phase boundary (at the Qwen3-30B-A3B
 * routing sizes a separate traced instantiation runs; the untraced one has no
 * marks compiled in).  naiwa_stack_trace_read copies
 * [blocks][n_layers + 1][24] ticks of the last launch (row n_layers is the
 * prologue) and synchronizes the device. */
int naiwa_stack_trace_enable(int on);
int naiwa_stack_trace_read(uint64_t* out, int capacity, int* n_layers, int* blocks);

/* x[i] <- bf16(f32(x[i]) + y[i]) for i < n (the residual of the stack). */
int naiwa_residual_add_bf16(void* x, const float* y, int64_t n, int64_t stream);

/* ======================================================================== */
/* Expert upload (CopyStream::queue_async + ReadFence, src/copy_stream.rs:   */
/* 387-409): on copy_stream, wait for read_fence (an event the compute      */
/* stream recorded after the last kernel that read the slot; 0 = none),     */
/* then copy the expert's gate/up/down bytes host -> device, then record    */
/* done_event (0 = none), which the compute stream waits on before reading  */
/* the slot.  src must be pinned (naiwa_host_alloc) for the copies to be    */
/* asynchronous DMA; it must stay valid until done_event completes.         */
/* ======================================================================== */
int naiwa_upload_expert(void* const dst[3], const void* const src[3], const size_t bytes[3],
                        int64_t copy_stream, int64_t read_fence, int64_t done_event);

/* Many host -> device ranges in one kernel on `stream` (the uploads of a     */
/* layer's staged experts, queued in the reference as one CopyStream copy    */
/* per projection, src/copy_stream.rs:387-409).  Every src must lie in      */
/* pinned host memory mapped for the device (naiwa_host_alloc), every dst   */
/* in device memory; src, dst and bytes 16-byte aligned.  Sources are        */
/* checked before the launch: NAIWA_E_UNSUPPORTED (nothing queued) when one  */
/* is not mapped pinned memory or not aligned, or a range exceeds 16 GiB,   */
/* and the caller copies those another way.  The ranges must not overlap.    */
#define NAIWA_COPY_BATCH_MAX 64
typedef struct naiwa_copy {
    void* dst;
    const void* src;
    uint64_t bytes;
} naiwa_copy;
int naiwa_copy_batch(const naiwa_copy* items, int n, int64_t stream);

/* ======================================================================== */
/* Synthetic data (benchmarks and tests): n values of the N(mean, std)       */
/* stream (seed, offset) -- value i depends only on (seed, offset + i) --    */
/* written as f32, bf16, Q8_0 or Q4_K bytes with the library's quantizers.   */
/* No counterpart in the reference, whose weights come from GGUF files.      */
/* ======================================================================== */
int naiwa_synth(int dtype, uint64_t seed, uint64_t offset, int64_t n, float mean, float stdv,
                void* out, int64_t stream);

#ifdef __cplusplus
}
#endif
#endif
