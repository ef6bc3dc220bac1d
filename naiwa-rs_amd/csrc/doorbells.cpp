// Doorbell protocols, PassCell and the CPU-task executor (include/naiwa_doorbell.h),
// over the reference-compatible doorbell kernels (csrc/doorbell.hip).
#include <hip/hip_runtime.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "../../include/naiwa_doorbell.h"
#include "common.h"

namespace {

constexpr size_t kHeader = 8; // [seq u32][pad or consumed u32]

// Mapped, zeroed host memory with its device alias.
struct Mapped {
    uint8_t* host = nullptr;
    uint8_t* dev = nullptr;
    size_t bytes = 0;
    int alloc(size_t n) {
        void* h = nullptr;
        int rc = doorbell_alloc_mapped(&h, n);
        if (rc) return rc;
        void* d = nullptr;
        doorbell_get_device_ptr(h, &d);
        if (!d) {
            doorbell_free_host(h);
            return NAIWA_E_DEVICE;
        }
        host = (uint8_t*)h;
        dev = (uint8_t*)d;
        bytes = n;
        return NAIWA_OK;
    }
    ~Mapped() {
        if (host) doorbell_free_host(host);
    }
    uint32_t* host_u32(size_t off) const { return (uint32_t*)(host + off); }
};

int64_t host_timeout(int64_t us) { return us == 0 ? -1 : us; }

// PayloadRing layout: [seq][consumed][8 slots of max_n f32].
struct PayloadRing {
    Mapped buf;
    int max_n = 0;
    int alloc(int n) {
        max_n = n;
        return buf.alloc(kHeader + (size_t)NAIWA_PAYLOAD_DEPTH * (size_t)n * 4);
    }
    size_t slot_off(uint32_t seq) const { return kHeader + (size_t)(seq % NAIWA_PAYLOAD_DEPTH) * max_n * 4; }
    float* slot_host(uint32_t seq) const { return (float*)(buf.host + slot_off(seq)); }
    void* slot_dev(uint32_t seq) const { return buf.dev + slot_off(seq); }
};

} // namespace

struct naiwa_topk_doorbell {
    Mapped buf;
    int max_n = 0;
};

struct naiwa_act_doorbell {
    PayloadRing ring;
    hipStream_t side = nullptr;
    hipEvent_t ready = nullptr;
};

struct naiwa_result_doorbell {
    PayloadRing ring;
};

struct naiwa_pass_cell {
    hipEvent_t done = nullptr;
    std::atomic<uint32_t> claims{0};
};

extern "C" {

// ---- TopkDoorbell ------------------------------------------------------------

int naiwa_topk_doorbell_create(int max_n, naiwa_topk_doorbell** out) {
    if (!out || max_n <= 0) return NAIWA_E_INVALID;
    auto* db = new (std::nothrow) naiwa_topk_doorbell;
    if (!db) return NAIWA_E_NOMEM;
    db->max_n = max_n;
    int rc = db->buf.alloc(kHeader + (size_t)max_n * 8);
    if (rc) {
        delete db;
        return rc;
    }
    *out = db;
    return NAIWA_OK;
}

int naiwa_topk_doorbell_destroy(naiwa_topk_doorbell* db) {
    delete db;
    return NAIWA_OK;
}

int naiwa_topk_doorbell_publish_and_read(naiwa_topk_doorbell* db, const uint32_t* ids_dev, const float* w_dev, int n,
                                         int64_t stream, uint32_t* ids_out, float* w_out, int64_t timeout_us) {
    if (!db || n < 0 || n > db->max_n || (n > 0 && (!ids_dev || !w_dev || !ids_out || !w_out)))
        return NAIWA_E_INVALID;
    const uint32_t last = naiwa_host_load_acquire_u32(db->buf.host_u32(0));
    doorbell_ring(db->buf.dev, db->buf.dev + kHeader, db->buf.dev + kHeader + (size_t)db->max_n * 4, ids_dev, w_dev, n,
                  stream);
    int rc = naiwa_hip_rc(hipGetLastError());
    if (rc) return rc;
    if ((rc = naiwa_host_wait_ge(db->buf.host_u32(0), last + 1, host_timeout(timeout_us), 50))) return rc;
    const volatile uint32_t* ids = (const volatile uint32_t*)(db->buf.host + kHeader);
    const volatile float* w = (const volatile float*)(db->buf.host + kHeader + (size_t)db->max_n * 4);
    for (int i = 0; i < n; ++i) {
        ids_out[i] = ids[i];
        w_out[i] = w[i];
    }
    return NAIWA_OK;
}

// ---- ActivationDoorbell ------------------------------------------------------------

int naiwa_act_doorbell_destroy(naiwa_act_doorbell* db) {
    if (!db) return NAIWA_OK;
    if (db->side) {
        (void)hipStreamSynchronize(db->side);
        (void)hipStreamDestroy(db->side);
    }
    if (db->ready) (void)hipEventDestroy(db->ready);
    delete db;
    return NAIWA_OK;
}

int naiwa_act_doorbell_create(int max_n, naiwa_act_doorbell** out) {
    if (!out || max_n <= 0) return NAIWA_E_INVALID;
    auto* db = new (std::nothrow) naiwa_act_doorbell;
    if (!db) return NAIWA_E_NOMEM;
    int rc = db->ring.alloc(max_n);
    if (!rc) rc = naiwa_hip_rc(hipStreamCreateWithFlags(&db->side, hipStreamNonBlocking));
    if (!rc) rc = naiwa_hip_rc(hipEventCreateWithFlags(&db->ready, hipEventDisableTiming));
    if (rc) {
        naiwa_act_doorbell_destroy(db);
        return rc;
    }
    *out = db;
    return NAIWA_OK;
}

int naiwa_act_doorbell_publish(naiwa_act_doorbell* db, const float* src_dev, int n, uint32_t seq, int64_t main_stream) {
    if (!db || n < 0 || n > db->ring.max_n || (n > 0 && !src_dev)) return NAIWA_E_INVALID;
    int rc = naiwa_hip_rc(hipEventRecord(db->ready, (hipStream_t)main_stream));
    if (!rc) rc = naiwa_hip_rc(hipStreamWaitEvent(db->side, db->ready, 0));
    if (rc) return rc;
    doorbell_copy_f32(db->ring.buf.dev, db->ring.slot_dev(seq), src_dev, n, (int64_t)db->side);
    return naiwa_hip_rc(hipGetLastError());
}

int naiwa_act_doorbell_wait_publish(naiwa_act_doorbell* db, uint32_t seq, int n, float* out, int64_t timeout_us,
                                    int* found) {
    if (!db || !found || n < 0 || n > db->ring.max_n || (n > 0 && !out)) return NAIWA_E_INVALID;
    *found = 0;
    const int rc = naiwa_host_wait_ge(db->ring.buf.host_u32(0), seq + 1, host_timeout(timeout_us), 100);
    if (rc == NAIWA_E_TIMEOUT) return NAIWA_OK;
    if (rc) return rc;
    const volatile float* p = db->ring.slot_host(seq);
    for (int i = 0; i < n; ++i) out[i] = p[i];
    *found = 1;
    return NAIWA_OK;
}

// ---- ResultDoorbell ------------------------------------------------------------

int naiwa_result_doorbell_create(int max_n, naiwa_result_doorbell** out) {
    if (!out || max_n <= 0) return NAIWA_E_INVALID;
    auto* db = new (std::nothrow) naiwa_result_doorbell;
    if (!db) return NAIWA_E_NOMEM;
    int rc = db->ring.alloc(max_n);
    if (rc) {
        delete db;
        return rc;
    }
    *out = db;
    return NAIWA_OK;
}

int naiwa_result_doorbell_destroy(naiwa_result_doorbell* db) {
    delete db;
    return NAIWA_OK;
}

int naiwa_result_doorbell_max_n(const naiwa_result_doorbell* db) { return db ? db->ring.max_n : 0; }

int naiwa_result_doorbell_publish(naiwa_result_doorbell* db, const float* values, int n, uint32_t seq, int* written) {
    if (!db || !written || n < 0 || n > db->ring.max_n) return NAIWA_E_INVALID;
    *written = 1;
    if (values) {
        // the slot's previous lap (seq - 8) must have been copied out by the device
        const bool free_slot = seq <= (uint32_t)NAIWA_PAYLOAD_DEPTH ||
                               naiwa_host_wait_ge(db->ring.buf.host_u32(4), seq - NAIWA_PAYLOAD_DEPTH, 2000, 50) ==
                                   NAIWA_OK;
        if (free_slot) std::memcpy(db->ring.slot_host(seq), values, (size_t)n * 4);
        else *written = 0;
    }
    naiwa_host_store_release_u32(db->ring.buf.host_u32(0), seq);
    return NAIWA_OK;
}

int naiwa_result_doorbell_wait_copy(naiwa_result_doorbell* db, uint32_t seq, int len, float* dst_dev, int64_t stream) {
    if (!db || len < 0 || len > db->ring.max_n || (len > 0 && !dst_dev)) return NAIWA_E_INVALID;
    doorbell_wait_copy_f32(db->ring.buf.dev, seq, db->ring.slot_dev(seq), 0, db->ring.buf.dev + 4, dst_dev, len,
                           stream);
    return naiwa_hip_rc(hipGetLastError());
}

int naiwa_result_doorbell_consumed(const naiwa_result_doorbell* db, uint32_t* consumed) {
    if (!db || !consumed) return NAIWA_E_INVALID;
    *consumed = naiwa_host_load_acquire_u32(db->ring.buf.host_u32(4));
    return NAIWA_OK;
}

// ---- PassCell ------------------------------------------------------------------------

int naiwa_pass_cell_create(naiwa_pass_cell** out) {
    if (!out) return NAIWA_E_INVALID;
    auto* c = new (std::nothrow) naiwa_pass_cell;
    if (!c) return NAIWA_E_NOMEM;
    int rc = naiwa_hip_rc(hipEventCreateWithFlags(&c->done, hipEventDisableTiming));
    if (rc) {
        delete c;
        return rc;
    }
    *out = c;
    return NAIWA_OK;
}

int naiwa_pass_cell_destroy(naiwa_pass_cell* c) {
    if (!c) return NAIWA_OK;
    if (c->done) (void)hipEventDestroy(c->done);
    delete c;
    return NAIWA_OK;
}

int naiwa_pass_cell_claim(naiwa_pass_cell* c, int64_t copy_stream, uint32_t* claim) {
    if (!c || !claim) return NAIWA_E_INVALID;
    int rc = naiwa_hip_rc(hipEventRecord(c->done, (hipStream_t)copy_stream));
    if (rc) return rc;
    *claim = c->claims.fetch_add(1, std::memory_order_acq_rel) + 1;
    return NAIWA_OK;
}

int naiwa_pass_cell_wait_latest(naiwa_pass_cell* c, int64_t stream, uint32_t* latest) {
    if (!c || !latest) return NAIWA_E_INVALID;
    const uint32_t claims = c->claims.load(std::memory_order_acquire);
    *latest = claims;
    if (claims == 0) return NAIWA_OK;
    return naiwa_hip_rc(hipStreamWaitEvent((hipStream_t)stream, c->done, 0));
}

int naiwa_pass_cell_claimed(const naiwa_pass_cell* c, uint32_t* claims) {
    if (!c || !claims) return NAIWA_E_INVALID;
    *claims = c->claims.load(std::memory_order_acquire);
    return NAIWA_OK;
}

} // extern "C"

// ---- Executor --------------------------------------------------------------------------

struct naiwa_executor {
    std::mutex mu;
    std::condition_variable work_cv, idle_cv;
    std::deque<std::function<void()>> jobs;
    bool running = false; // a task is executing
    bool stop = false;
    std::thread worker;
    // result channel: the current doorbell and the retired ones (kept alive for
    // pendings that still name them), job numbers per doorbell
    std::mutex chan_mu;
    std::vector<std::shared_ptr<naiwa_result_doorbell>> bells; // back() is current
    uint32_t next_seq = 0;
    std::mutex err_mu;
    std::string error;
    std::atomic<uint64_t> stalls{0};

    void run() {
        std::unique_lock<std::mutex> lock(mu);
        for (;;) {
            work_cv.wait(lock, [&] { return stop || !jobs.empty(); });
            if (jobs.empty() && stop) return;
            auto job = std::move(jobs.front());
            jobs.pop_front();
            running = true;
            lock.unlock();
            job();
            lock.lock();
            running = false;
            if (jobs.empty()) idle_cv.notify_all();
        }
    }
    void record_error(const std::string& msg) {
        std::lock_guard<std::mutex> lock(err_mu);
        if (error.empty()) error = msg;
    }
};

namespace {
void destroy_bell(naiwa_result_doorbell* b) { naiwa_result_doorbell_destroy(b); }

// SetFlag: publish exactly once -- values, or empty on failure / when dropped.
struct SetFlag {
    std::shared_ptr<naiwa_result_doorbell> bell;
    uint32_t seq;
    naiwa_executor* ex;
    bool published = false;
    SetFlag(std::shared_ptr<naiwa_result_doorbell> b, uint32_t s, naiwa_executor* e)
        : bell(std::move(b)), seq(s), ex(e) {}
    // one owner only: a copy's destructor would publish the job early
    SetFlag(const SetFlag&) = delete;
    SetFlag& operator=(const SetFlag&) = delete;
    void publish(const float* v, int n) {
        if (published) return;
        published = true;
        int written = 1;
        naiwa_result_doorbell_publish(bell.get(), v, n, seq, &written);
        if (v && !written) ex->stalls.fetch_add(1);
    }
    ~SetFlag() { publish(nullptr, 0); }
};
} // namespace

extern "C" {

int naiwa_executor_create(naiwa_executor** out) {
    if (!out) return NAIWA_E_INVALID;
    auto* ex = new (std::nothrow) naiwa_executor;
    if (!ex) return NAIWA_E_NOMEM;
    try {
        ex->worker = std::thread([ex] { ex->run(); });
    } catch (...) {
        delete ex;
        return NAIWA_E_NOMEM;
    }
    *out = ex;
    return NAIWA_OK;
}

int naiwa_executor_destroy(naiwa_executor* ex) {
    if (!ex) return NAIWA_OK;
    {
        std::lock_guard<std::mutex> lock(ex->mu);
        ex->stop = true;
    }
    ex->work_cv.notify_all();
    if (ex->worker.joinable()) ex->worker.join();
    delete ex;
    return NAIWA_OK;
}

int naiwa_executor_submit(naiwa_executor* ex, naiwa_task_fn fn, void* user) {
    if (!ex || !fn) return NAIWA_E_INVALID;
    {
        std::lock_guard<std::mutex> lock(ex->mu);
        if (ex->stop) return NAIWA_E_INVALID;
        ex->jobs.emplace_back([fn, user] { fn(user); });
    }
    ex->work_cv.notify_one();
    return NAIWA_OK;
}

int naiwa_executor_is_idle(const naiwa_executor* ex) {
    if (!ex) return NAIWA_E_INVALID;
    auto* e = const_cast<naiwa_executor*>(ex);
    std::lock_guard<std::mutex> lock(e->mu);
    return (e->jobs.empty() && !e->running) ? 1 : 0;
}

int naiwa_executor_wait_idle(naiwa_executor* ex, int64_t timeout_us) {
    if (!ex) return NAIWA_E_INVALID;
    std::unique_lock<std::mutex> lock(ex->mu);
    auto idle = [&] { return ex->jobs.empty() && !ex->running; };
    if (timeout_us <= 0) {
        ex->idle_cv.wait(lock, idle);
        return NAIWA_OK;
    }
    return ex->idle_cv.wait_for(lock, std::chrono::microseconds(timeout_us), idle) ? NAIWA_OK : NAIWA_E_TIMEOUT;
}

int naiwa_executor_submit_result(naiwa_executor* ex, int len, naiwa_result_fn fn, void* user, naiwa_pending* out) {
    if (!ex || !fn || !out || len <= 0) return NAIWA_E_INVALID;
    char msg[256];
    int rc = naiwa_executor_take_error(ex, msg, sizeof msg);
    if (rc) return rc; // a previous task failed: report it before queueing more
    std::shared_ptr<naiwa_result_doorbell> bell;
    uint32_t seq = 0;
    int chan = 0;
    {
        std::lock_guard<std::mutex> lock(ex->chan_mu);
        if (ex->bells.empty() || naiwa_result_doorbell_max_n(ex->bells.back().get()) < len) {
            const int old = ex->bells.empty() ? 0 : naiwa_result_doorbell_max_n(ex->bells.back().get());
            naiwa_result_doorbell* b = nullptr;
            if ((rc = naiwa_result_doorbell_create(len > 2 * old ? len : 2 * old, &b))) return rc;
            ex->bells.emplace_back(b, destroy_bell);
            ex->next_seq = 0;
        }
        bell = ex->bells.back();
        chan = (int)ex->bells.size() - 1;
        seq = ++ex->next_seq;
    }
    auto flag = std::make_shared<SetFlag>(bell, seq, ex);
    {
        std::lock_guard<std::mutex> lock(ex->mu);
        if (ex->stop) return NAIWA_E_INVALID;
        ex->jobs.emplace_back([ex, flag, fn, user, len] {
            std::vector<float> v((size_t)len);
            const int r = fn(user, v.data(), len);
            if (r == 0) {
                flag->publish(v.data(), len);
            } else {
                ex->record_error("a CPU result task failed with status " + std::to_string(r));
                flag->publish(nullptr, 0);
            }
        });
    }
    ex->work_cv.notify_one();
    out->seq = seq;
    out->len = len;
    out->chan = chan;
    return NAIWA_OK;
}

int naiwa_pending_upload(naiwa_executor* ex, const naiwa_pending* p, float* dst_dev, int64_t stream) {
    if (!ex || !p || !dst_dev) return NAIWA_E_INVALID;
    std::shared_ptr<naiwa_result_doorbell> bell;
    {
        std::lock_guard<std::mutex> lock(ex->chan_mu);
        if (p->chan < 0 || p->chan >= (int)ex->bells.size()) return NAIWA_E_INVALID;
        bell = ex->bells[(size_t)p->chan];
    }
    return naiwa_result_doorbell_wait_copy(bell.get(), p->seq, p->len, dst_dev, stream);
}

int naiwa_executor_take_error(naiwa_executor* ex, char* msg, int cap) {
    if (!ex) return NAIWA_E_INVALID;
    std::lock_guard<std::mutex> lock(ex->err_mu);
    if (ex->error.empty()) return NAIWA_OK;
    if (msg && cap > 0) {
        std::strncpy(msg, ex->error.c_str(), (size_t)cap - 1);
        msg[cap - 1] = 0;
    }
    ex->error.clear();
    return NAIWA_E_DEVICE;
}

int naiwa_executor_stalls(const naiwa_executor* ex, uint64_t* stalls) {
    if (!ex || !stalls) return NAIWA_E_INVALID;
    *stalls = ex->stalls.load();
    return NAIWA_OK;
}

} // extern "C"
