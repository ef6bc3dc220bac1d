/*
 * naiwa_doorbell.h -- the host<->device doorbell protocols and the CPU-task
 * executor of the MoE path, built on the reference-compatible doorbell kernels
 * of naiwa_moe.h (doorbell_ring / doorbell_copy_f32 / doorbell_wait_copy_f32).
 *
 *   naiwa_topk_doorbell_*   TopkDoorbell        src/doorbell/d2h/topk.rs:20-125
 *   naiwa_act_doorbell_*    ActivationDoorbell  src/doorbell/d2h/activation.rs:17-116
 *   naiwa_result_doorbell_* ResultDoorbell      src/doorbell/h2d/result.rs:27-123
 *                           over PayloadRing    src/doorbell/payload_ring.rs:14-81
 *   naiwa_pass_cell_*       PassCell            src/doorbell/handoff.rs:24-61
 *   naiwa_executor_*        Executor / Pending / SetFlag  src/executor.rs:28-392
 *
 * Layouts (fine-grained, coherent, mapped host memory):
 *   top-k:    [seq u32][pad u32][ids u32 x max_n][w f32 x max_n]
 *   payload:  [seq u32][consumed u32][DEPTH = 8 slots x max_n f32], slot = seq % 8
 * Host waits are bounded by the caller's timeout (the reference's top-k wait
 * has none; a zero timeout here means "no limit" only where stated).
 */
#ifndef NAIWA_DOORBELL_H
#define NAIWA_DOORBELL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NAIWA_PAYLOAD_DEPTH 8

/* ---- TopkDoorbell: device -> host top-k publication ---------------------- */
typedef struct naiwa_topk_doorbell naiwa_topk_doorbell;
int naiwa_topk_doorbell_create(int max_n, naiwa_topk_doorbell** out);
int naiwa_topk_doorbell_destroy(naiwa_topk_doorbell* db);
/* Queue the publish of n ids/weights (device pointers) on `stream`, then wait
 * (at most timeout_us; 0 = no limit) until the device has raised seq past its
 * value before the call, and read the payload into ids_out / w_out (host).
 * NAIWA_E_TIMEOUT when the wait gives up. */
int naiwa_topk_doorbell_publish_and_read(naiwa_topk_doorbell* db, const uint32_t* ids_dev, const float* w_dev, int n,
                                         int64_t stream, uint32_t* ids_out, float* w_out, int64_t timeout_us);

/* ---- ActivationDoorbell: device -> host activation ring ----------------- */
typedef struct naiwa_act_doorbell naiwa_act_doorbell;
int naiwa_act_doorbell_create(int max_n, naiwa_act_doorbell** out);
int naiwa_act_doorbell_destroy(naiwa_act_doorbell* db);
/* Copy n f32 (device src, ready once `main_stream` reaches this point) into
 * ring slot seq % 8 on the doorbell's side stream, then raise seq. */
int naiwa_act_doorbell_publish(naiwa_act_doorbell* db, const float* src_dev, int n, uint32_t seq, int64_t main_stream);
/* Wait (<= timeout_us) until seq has passed `seq`, then read slot seq % 8.
 * *found = 0 on timeout (the reference gives up after 250 ms). */
int naiwa_act_doorbell_wait_publish(naiwa_act_doorbell* db, uint32_t seq, int n, float* out, int64_t timeout_us,
                                    int* found);

/* ---- ResultDoorbell: host -> device result ring with backpressure ------- */
typedef struct naiwa_result_doorbell naiwa_result_doorbell;
int naiwa_result_doorbell_create(int max_n, naiwa_result_doorbell** out);
int naiwa_result_doorbell_destroy(naiwa_result_doorbell* db);
int naiwa_result_doorbell_max_n(const naiwa_result_doorbell* db);
/* Publish job `seq` (1-based): when values is non-null, reserve the slot (seq
 * <= 8, or the device has consumed seq - 8 within 2 ms), copy n values in;
 * then raise seq in every case, so the device never waits forever.
 * *written = 0 when the payload was dropped (a result stall). */
int naiwa_result_doorbell_publish(naiwa_result_doorbell* db, const float* values, int n, uint32_t seq, int* written);
/* On `stream`: wait for seq, copy len f32 of its slot to dst_dev, mark consumed. */
int naiwa_result_doorbell_wait_copy(naiwa_result_doorbell* db, uint32_t seq, int len, float* dst_dev, int64_t stream);
int naiwa_result_doorbell_consumed(const naiwa_result_doorbell* db, uint32_t* consumed);

/* ---- PassCell: copy-stream completion handed to a consumer -------------- */
typedef struct naiwa_pass_cell naiwa_pass_cell;
int naiwa_pass_cell_create(naiwa_pass_cell** out);
int naiwa_pass_cell_destroy(naiwa_pass_cell* c);
/* Record the completion event on copy_stream, then count the claim: returns
 * the claim number (1, 2, ...) in *claim. */
int naiwa_pass_cell_claim(naiwa_pass_cell* c, int64_t copy_stream, uint32_t* claim);
/* *latest = 0 when nothing was claimed (and no GPU work is queued); else the
 * latest claim, with `stream` made to wait for its event. */
int naiwa_pass_cell_wait_latest(naiwa_pass_cell* c, int64_t stream, uint32_t* latest);
int naiwa_pass_cell_claimed(const naiwa_pass_cell* c, uint32_t* claims);

/* ---- Executor: one FIFO worker thread for CPU tasks ----------------------- */
typedef struct naiwa_executor naiwa_executor;
typedef void (*naiwa_task_fn)(void* user);
/* Compute `len` f32 into out; return 0 on success, anything else = failure. */
typedef int (*naiwa_result_fn)(void* user, float* out, int len);
typedef struct naiwa_pending {
    uint32_t seq;
    int len;
    int chan; /* which result doorbell (the channel grows by replacement) */
} naiwa_pending;

int naiwa_executor_create(naiwa_executor** out);
/* Drains the queue, then stops and joins the worker. */
int naiwa_executor_destroy(naiwa_executor* ex);
int naiwa_executor_submit(naiwa_executor* ex, naiwa_task_fn fn, void* user);
int naiwa_executor_is_idle(const naiwa_executor* ex);
/* Block until the queue is empty and no task runs (<= timeout_us; 0 = no limit). */
int naiwa_executor_wait_idle(naiwa_executor* ex, int64_t timeout_us);
/* Run fn on the worker and publish its len values through the executor's
 * result doorbell (grown as needed).  A failing fn, or a wrong length,
 * publishes an empty payload (the device still advances) and records an
 * error that the next submit_result (or take_error) reports. */
int naiwa_executor_submit_result(naiwa_executor* ex, int len, naiwa_result_fn fn, void* user, naiwa_pending* out);
/* Pending::upload: queue the device-side wait + copy of the job's values into
 * dst_dev on `stream` (len f32). */
int naiwa_pending_upload(naiwa_executor* ex, const naiwa_pending* p, float* dst_dev, int64_t stream);
/* The first recorded task error (cleared): NAIWA_E_DEVICE and its message, or NAIWA_OK. */
int naiwa_executor_take_error(naiwa_executor* ex, char* msg, int cap);
/* Result payloads dropped because the device had not consumed the slot. */
int naiwa_executor_stalls(const naiwa_executor* ex, uint64_t* stalls);

#ifdef __cplusplus
}
#endif
#endif
