// One MoE layer's decode step over a partial expert cache (include/naiwa_cached.h):
// device routing, host policy, PCIe staging into ring slots, the expert kernel
// over resident + staged slots, and promotion -- the stage order of the
// reference's decode path (src/moe/decode.rs:241-381) -- plus the lookahead
// that loads the next layer's predicted experts while this layer computes
// (src/moe/cached_layer.rs:1236-1300, src/moe/stages/preload.rs:18-111).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <memory>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

#include "../../include/naiwa_cached.h"
#include "../../include/naiwa_doorbell.h"
#include "common.h"
#include "decode.h"
#include "router.h"
#include "upload.h"

namespace {

bool bank_ok(const naiwa_bank& b, int n, int k, int min_slots) {
    return b.base && b.n == n && b.k == k && b.slots >= min_slots &&
           naiwa_projection_bytes(b.dtype, n, k) > 0 && b.slot_stride >= naiwa_projection_bytes(b.dtype, n, k);
}

// Doorbell layout of a layer's routing read-back (fine-grained mapped host memory):
// [16 u32 header words: word 1 counts the staged-upload waits that ran out]
// [tagged u64 words: ids n | weights n | predicted ids n].  Each payload word is
// tag << 32 | value with the step's tag: the host waits until every word it needs
// carries the tag, so the words need no ordering among themselves and the device
// publishes them without a system-scope fence (which writes back the L2 and cost
// ~2.5 us a publish).
constexpr int kDbHead = 16;
// Device words of the one-token routing kernel: tagged logits of two routers.
constexpr int kRouteWords = 2 * NAIWA_ROUTER_MAX_E;

typedef __attribute__((address_space(1))) uint64_t gu64;

// The routing of one step (several tokens) into the mapped doorbell as tagged words
// (the reference's TopkDoorbell publish, src/doorbell/d2h/topk.rs:20-125).
__global__ void __launch_bounds__(256) routing_publish_kernel(uint64_t* pay, uint32_t tag, const uint32_t* ids,
                                                              const float* w, int n, const uint32_t* pred, int npred) {
    const uint64_t t = (uint64_t)tag << 32;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        __hip_atomic_store((gu64*)(pay + i), t | ids[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store((gu64*)(pay + n + i), t | __float_as_uint(w[i]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
    for (int i = threadIdx.x; i < npred; i += blockDim.x)
        __hip_atomic_store((gu64*)(pay + 2 * n + i), t | pred[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The step's inputs (slot ids and split weights, nwords words) from mapped host memory
// into device memory, by one wave: a few reads over PCIe here instead of in every block
// of the expert kernels.
__global__ void __launch_bounds__(64) pull_inputs_kernel(uint32_t* dst, const uint32_t* src, int nwords) {
    for (int i = threadIdx.x; i < nwords; i += 64) dst[i] = src[i];
}

// The staged-upload wait of the poll mode: one wave spins (bounded) until the copy
// stream's flag reaches target.  A wait that runs out adds one to *fail (a word of the
// layer's mapped routing doorbell, read by the host before its next step), so the
// step's output is known to be invalid instead of silently wrong.
__global__ void __launch_bounds__(64)
staged_wait_kernel(const uint32_t* flag, uint32_t target, uint64_t limit_ticks, uint32_t* fail) {
    if (threadIdx.x != 0) return;
    const uint64_t t0 = wall_clock64();
    // relaxed spin loads (an acquire load invalidates the L2 on every try); the kernels
    // queued behind this one acquire at their start
    while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) < target) {
        if (wall_clock64() - t0 > limit_ticks) {
            const uint32_t n = __hip_atomic_load(fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(fail, n + 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// The step's activations for the CPU job: bf16 x [n] as f32 into mapped host memory
// behind a sequence word (the reference's ActivationDoorbell publish,
// src/doorbell/d2h/activation.rs:17-116): payload, system fence, then seq + 1.
constexpr int kXHead = 64; // words before the payload
__global__ void __launch_bounds__(256) x_publish_kernel(uint32_t* db, const uint16_t* x, int n) {
    volatile float* out = reinterpret_cast<volatile float*>(db + kXHead);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = __uint_as_float((uint32_t)x[i] << 16);
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t cur = __hip_atomic_load(db, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(db, cur + 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// out += cpu (the CPU pairs' sum, added after the resident and staged pairs).
__global__ void add_f32_kernel(float* out, const float* cpu, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) out[i] += cpu[i];
}

// The CPU misses run on one process-wide executor worker (the reference's
// executor::cpu(), src/executor.rs:116-166), created on first use.
naiwa_executor* cpu_executor(int* rc) {
    static naiwa_executor* ex = nullptr;
    static int create_rc = NAIWA_OK;
    static std::once_flag once;
    std::call_once(once, [] { create_rc = naiwa_executor_create(&ex); });
    *rc = create_rc;
    return ex;
}

// One CPU job: wait for the published activations (bounded, the reference's 250 ms),
// copy them out of the mapped page, run the CPU pairs.
constexpr int64_t kXWaitUs = 250 * 1000;
struct CpuJob {
    naiwa_host_experts hx;
    const uint32_t* seq;   // host view of the publish page
    uint32_t target;
    int rows, width, act;
    std::vector<uint32_t> ids;
    std::vector<float> w;  // 0 for the pairs served on the device
};
int cpu_job_run(void* user, float* out, int len) {
    std::unique_ptr<CpuJob> j(static_cast<CpuJob*>(user));
    const int H = j->hx.hidden;
    if (len != j->rows * H) return NAIWA_E_INVALID;
    if (naiwa_host_wait_ge(j->seq, j->target, kXWaitUs, 20) != NAIWA_OK) return NAIWA_E_TIMEOUT;
    const float* src = reinterpret_cast<const float*>(j->seq + kXHead);
    std::vector<float> x(src, src + (size_t)len);
    return naiwa_cpu_moe_decode(&j->hx, x.data(), j->ids.data(), j->w.data(), j->rows, j->width, j->act, out);
}

// Bound of the host's wait for a routing doorbell.
constexpr int64_t kRouteWaitUs = 10 * 1000 * 1000;
// How long that wait spins before it sleep-polls.  The routing doorbell rings within
// tens of microseconds of the call (the device first finishes the previous layer), and
// a sleep costs the OS timer slack, ~50 us or more, on every layer of every token.
constexpr int64_t kRouteSpinUs = 2000;

// Every one of the nw tagged words carries tag: spin (pause) for up to kRouteSpinUs,
// then sleep-poll every 20 us, until kRouteWaitUs have passed (NAIWA_E_TIMEOUT).  The
// words' values (low halves) then go to out.
int wait_routing(const uint64_t* words, int nw, uint32_t tag, uint32_t* out) {
    using clock = std::chrono::steady_clock;
    const auto t0 = clock::now();
    const auto spin_end = t0 + std::chrono::microseconds(kRouteSpinUs);
    const auto deadline = t0 + std::chrono::microseconds(kRouteWaitUs);
    int have = 0; // words[0..have) carry the tag
    for (uint32_t i = 0;; ++i) {
        while (have < nw) {
            const uint64_t v = __atomic_load_n(words + have, __ATOMIC_ACQUIRE);
            if ((uint32_t)(v >> 32) != tag) break;
            out[have++] = (uint32_t)v;
        }
        if (have == nw) return NAIWA_OK;
        if ((i & 63) == 0) {
            const auto now = clock::now();
            if (now >= deadline) return NAIWA_E_TIMEOUT;
            if (now >= spin_end) std::this_thread::sleep_for(std::chrono::microseconds(20));
        }
#if defined(__x86_64__)
        __builtin_ia32_pause();
#endif
    }
}

} // namespace

struct naiwa_cached_layer {
    naiwa_cached_layer_desc d{};
    naiwa_ring* ring = nullptr;
    int ring_len = 0;
    naiwa_cache* cache = nullptr;
    hipStream_t copy = nullptr;
    size_t bytes[3] = {0, 0, 0};   // one expert's bytes per projection
    // routing buffers: device results, pinned host copies
    int cap_rows = 0;
    // one allocation each for the routing read-back [ids | weights] and for the step's
    // inputs [slot ids | weights of the cache pairs | of the staged pairs], so that each
    // crosses the link in one copy; the views below are set per step (n = rows * k)
    uint32_t* route_dev_base = nullptr;
    uint32_t* in_dev_base = nullptr; // device copy of the step's inputs, read by the kernels
    uint32_t* in_map_base = nullptr; // device view of in_h_base (mapped, coherent host memory)
    uint32_t* in_h_base = nullptr;
    uint32_t* ids_dev = nullptr;
    float* w_dev = nullptr;
    uint32_t* slots_dev = nullptr;
    uint32_t* ids_h = nullptr;
    float* w_h = nullptr;
    int32_t* slots_h = nullptr;
    uint32_t* slots_up = nullptr;  // host view of the step's slot ids, read by the kernels
    float* wsplit_h = nullptr;     // host view: weights of the cache pairs | of the staged pairs
    float* wsplit_dev = nullptr;
    int last_rows = 0;
    // routing read-back doorbell: host view, device view, publishes so far (the tag of
    // the latest); the values read back (ids | weights | predicted ids); the one-token
    // routing kernel's tagged logits and arrival counter
    uint32_t* db_host = nullptr;
    uint32_t* db_dev = nullptr;
    uint32_t db_seq = 0;
    std::vector<uint32_t> route_h;
    uint64_t* rwords_dev = nullptr;
    // the stream of the previous step: a step on another stream waits for read_done first
    hipStream_t last_stream = nullptr;
    bool have_last_stream = false;
    // staged-upload completion: an event the stream waits for, or (poll mode) a device
    // flag the copy stream raises and one wave polls; the flag and its epoch
    int upload_sync = NAIWA_UPLOAD_SYNC_POLL; // measured faster on cache25 (165.6 vs 159.9 tok/s)
    uint32_t* upload_flag = nullptr;
    uint32_t upload_epoch = 0;
    uint32_t upload_fail_seen = 0;       // poll waits that ran out, as already reported
    // misses left to the CPU: the host stacks, the activation publish page
    // [seq][pad][rows * H f32] (mapped), its publishes so far, and the CPU sum on the device
    bool cpu_misses = true;
    naiwa_host_experts hx{};
    uint32_t* xpub_host = nullptr;
    uint32_t* xpub_dev = nullptr;
    uint32_t xpub_seq = 0;
    float* cpu_out = nullptr;
    hipEvent_t staged_done = nullptr;
    bool batch_uploads = false;          // staged uploads as one batched copy kernel, reading
    const void* host_dev[3] = {nullptr, nullptr, nullptr}; // the host stacks' device views
    size_t host_stride[3] = {0, 0, 0};   // bytes between experts in each host stack
    // an expert's gate | up | down are adjacent both in the host stacks and in a slot:
    // one expert is one range (one DMA copy, or one range of the batched copy kernel)
    bool contiguous = false;
    size_t expert_bytes = 0;
    bool dma_uploads = false;            // staged uploads as DMA copies even from mapped stacks
    // lookahead: this layer's prediction (its router on the previous layer's
    // activation), the fence after the last step that read its cache slots,
    // and the claim a forward waits for before its expert kernel
    uint32_t* pred_ids_dev = nullptr;
    float* pred_w_dev = nullptr;
    uint32_t* pred_ids_h = nullptr;
    int pred_rows = 0;
    std::vector<uint32_t> predicted;
    hipEvent_t read_done = nullptr;
    bool read_recorded = false;
    // read_done is recorded when something needs it (a step on another stream, a
    // lookahead upload into this layer's slots): recording it on last_stream then covers
    // every read queued there so far.  Once a lookahead targets the layer it is recorded
    // at the end of every step, so that its uploads need not wait for later work.
    bool read_pending = false;
    bool lookahead_target = false;
    int record_reads() {
        if (!read_pending) return NAIWA_OK;
        const int rc = naiwa_hip_rc(hipEventRecord(read_done, last_stream));
        if (rc) return rc;
        read_pending = false;
        read_recorded = true;
        return NAIWA_OK;
    }
    hipEvent_t ahead_done = nullptr;
    bool ahead_claimed = false;

    void release_buffers() {
        if (route_dev_base) (void)hipFree(route_dev_base);
        if (rwords_dev) (void)hipFree(rwords_dev);
        rwords_dev = nullptr;
        if (in_dev_base) (void)hipFree(in_dev_base);
        in_map_base = nullptr;
        if (db_host) (void)doorbell_free_host(db_host);
        db_host = db_dev = nullptr;
        db_seq = 0;
        if (in_h_base) (void)doorbell_free_host(in_h_base);
        if (slots_h) (void)hipHostFree(slots_h);
        route_dev_base = in_dev_base = in_h_base = nullptr;
        route_h.clear();
        views(0);
        if (pred_ids_dev) (void)hipFree(pred_ids_dev);
        if (pred_w_dev) (void)hipFree(pred_w_dev);
        if (pred_ids_h) (void)hipHostFree(pred_ids_h);
        if (xpub_host) (void)doorbell_free_host(xpub_host);
        if (cpu_out) (void)hipFree(cpu_out);
        xpub_host = xpub_dev = nullptr;
        xpub_seq = 0;
        cpu_out = nullptr;
        pred_ids_dev = nullptr;
        pred_w_dev = nullptr;
        pred_ids_h = nullptr;
        slots_h = nullptr;
        cap_rows = 0;
        last_rows = 0;
        pred_rows = 0;
    }

    int ensure_rows(int rows) {
        if (rows <= cap_rows) return NAIWA_OK;
        hipError_t e = hipDeviceSynchronize(); // earlier steps may still read the old buffers
        if (e != hipSuccess) return (int)e;
        release_buffers();
        const size_t n = (size_t)rows * d.top_k;
        void* db = nullptr;
        void* in = nullptr;
        void* xp = nullptr;
        const size_t xn = (size_t)rows * d.hidden;
        if (hipMalloc(&route_dev_base, 2 * n * 4) != hipSuccess || hipMalloc(&in_dev_base, 3 * n * 4) != hipSuccess ||
            hipMalloc(&rwords_dev, kRouteWords * 8) != hipSuccess ||
            hipMemset(rwords_dev, 0, kRouteWords * 8) != hipSuccess ||
            doorbell_alloc_mapped(&db, kDbHead * 4 + 3 * n * 8) != NAIWA_OK ||
            doorbell_alloc_mapped(&in, 3 * n * 4) != NAIWA_OK || hipHostMalloc(&slots_h, n * 4, 0) != hipSuccess ||
            hipMalloc(&pred_ids_dev, n * 4) != hipSuccess || hipMalloc(&pred_w_dev, n * 4) != hipSuccess ||
            hipHostMalloc(&pred_ids_h, n * 4, 0) != hipSuccess ||
            doorbell_alloc_mapped(&xp, (kXHead + xn) * 4) != NAIWA_OK || hipMalloc(&cpu_out, xn * 4) != hipSuccess) {
            if (db) db_host = (uint32_t*)db;
            if (in) in_h_base = (uint32_t*)in;
            if (xp) xpub_host = (uint32_t*)xp;
            release_buffers();
            return NAIWA_E_NOMEM;
        }
        db_host = (uint32_t*)db;
        in_h_base = (uint32_t*)in;
        xpub_host = (uint32_t*)xp;
        void* dv = nullptr;
        void* iv = nullptr;
        void* xv = nullptr;
        doorbell_get_device_ptr(db, &dv);
        doorbell_get_device_ptr(in, &iv);
        doorbell_get_device_ptr(xp, &xv);
        if (!dv || !iv || !xv) {
            release_buffers();
            return NAIWA_E_DEVICE;
        }
        db_dev = (uint32_t*)dv;
        in_map_base = (uint32_t*)iv;
        xpub_dev = (uint32_t*)xv;
        db_seq = 0;
        upload_fail_seen = 0;
        xpub_seq = 0;
        route_h.assign(3 * n, 0u);
        cap_rows = rows;
        return NAIWA_OK;
    }

    // the step's views of the combined buffers for n = rows * k pairs (0: none)
    void views(int n) {
        ids_dev = route_dev_base;
        w_dev = route_dev_base ? (float*)(route_dev_base + n) : nullptr;
        ids_h = route_h.empty() ? nullptr : route_h.data();
        w_h = route_h.empty() ? nullptr : (float*)(route_h.data() + n);
        slots_dev = in_dev_base;
        wsplit_dev = in_dev_base ? (float*)(in_dev_base + n) : nullptr;
        slots_up = in_h_base;
        wsplit_h = in_h_base ? (float*)(in_h_base + n) : nullptr;
    }

    void slot_ptrs(int slot, void* dst[3]) const {
        dst[0] = (uint8_t*)d.gate.base + (int64_t)slot * d.gate.slot_stride;
        dst[1] = (uint8_t*)d.up.base + (int64_t)slot * d.up.slot_stride;
        dst[2] = (uint8_t*)d.down.base + (int64_t)slot * d.down.slot_stride;
    }
    void host_ptrs(int expert, const void* src[3]) const {
        src[0] = (const uint8_t*)d.host_gate + (size_t)expert * host_stride[0];
        src[1] = (const uint8_t*)d.host_up + (size_t)expert * host_stride[1];
        src[2] = (const uint8_t*)d.host_down + (size_t)expert * host_stride[2];
    }

    // Queue the upload of `expert` into `slot` on the copy stream after `fence` (0 = none):
    // one DMA copy when the expert is contiguous, else one per projection.
    int upload(int expert, int slot, int64_t fence) const {
        void* dst[3];
        const void* src[3];
        slot_ptrs(slot, dst);
        host_ptrs(expert, src);
        if (!contiguous) return naiwa_upload_expert(dst, src, bytes, (int64_t)copy, fence, 0);
        int rc = 0;
        if (fence && (rc = naiwa_hip_rc(hipStreamWaitEvent(copy, (hipEvent_t)fence, 0)))) return rc;
        return naiwa_hip_rc(hipMemcpyAsync(dst[0], src[0], expert_bytes, hipMemcpyHostToDevice, copy));
    }

    // predict (src/moe/cached_layer.rs:1245-1259): this layer's router on the
    // previous layer's activation, ranked by its logits (the bias term included,
    // as in this layer's own routing; without one these are the reference's raw
    // logits), read back with the caller's next synchronisation of `stream`
    int predict_launch(const void* x, int rows, int64_t stream) {
        int rc = naiwa_router_topk_biased(x, NAIWA_BF16, d.router, d.router_bias, rows, d.hidden, d.num_experts,
                                          d.top_k, NAIWA_ROUTE_TOPK_SOFTMAX, pred_ids_dev, pred_w_dev, nullptr,
                                          stream);
        if (rc) return rc;
        pred_rows = rows;
        return NAIWA_OK;
    }

    // prefetch_predicted (src/moe/cached_layer.rs:1268-1300) once the prediction
    // is on the host: the union of the rows' top-k by votes; each predicted
    // expert is admitted into an empty slot, else, while swaps < swaps_per_row *
    // rows, replaces the LRU resident outside the prediction.  Uploads go on
    // the copy stream behind the last step that read this layer's slots; the
    // slots are published at once, because the only reader, this layer's next
    // expert kernel, waits for the claim (ahead_done) recorded after them.
    int prefetch_apply(const uint32_t* pred_ids, int swaps_per_row, naiwa_lookahead_step* info) {
        naiwa_lookahead_step a{};
        const int rows = pred_rows, k = d.top_k;
        std::vector<int> lens((size_t)rows, k);
        predicted.assign((size_t)rows * k, 0u);
        int np = 0;
        int rc = naiwa_union_by_votes(pred_ids, lens.data(), rows, predicted.data(), (int)predicted.size(), &np);
        if (rc) return rc;
        predicted.resize((size_t)np);
        a.predicted = np;
        std::vector<int32_t> table((size_t)d.num_experts), protect(predicted.begin(), predicted.end());
        if ((rc = naiwa_cache_slot_table(cache, table.data()))) return rc;
        for (uint32_t e : predicted)
            if (e < (uint32_t)d.num_experts && table[e] >= 0) ++a.resident;
        const int max_swaps = swaps_per_row * rows;
        lookahead_target = true;
        if ((rc = record_reads())) return rc;
        const int64_t fence = read_recorded ? (int64_t)read_done : 0;
        for (uint32_t e : predicted) {
            if (e >= (uint32_t)d.num_experts) continue;
            int slot = -1;
            bool swap = false;
            if ((rc = naiwa_cache_admit(cache, (int)e, &slot))) return rc;
            if (slot < 0 && a.swaps < max_swaps) {
                if ((rc = naiwa_cache_replace(cache, (int)e, protect.data(), (int)protect.size(), &slot))) return rc;
                swap = slot >= 0;
            }
            if (slot < 0) continue;
            if ((rc = upload((int)e, slot, fence))) {
                naiwa_cache_unreserve(cache, slot);
                return rc;
            }
            if ((rc = naiwa_cache_publish(cache, slot))) return rc;
            ++(swap ? a.swaps : a.loads);
            a.pcie_bytes += (int64_t)(bytes[0] + bytes[1] + bytes[2]);
        }
        // the claim: recorded after the batch, before a reader can see it
        if ((rc = naiwa_hip_rc(hipEventRecord(ahead_done, copy)))) return rc;
        ahead_claimed = true;
        naiwa_cache_stats s{};
        s.lookahead_loads = (uint64_t)a.loads;
        s.swaps = (uint64_t)a.swaps;
        naiwa_stats_add(&s);
        if (info) *info = a;
        return NAIWA_OK;
    }
};

namespace {

// One decode step of L; with `next`, also the next layer's lookahead on the same
// activation: its router runs beside L's before the one routing read-back, and
// its uploads are queued after L's expert kernel, so they overlap L's compute.
// res_x (the stack driver's x, or null): when the step runs one expert pass, that pass
// also adds its output to res_x in place (x = bf16(x + out)) and *folded is set.
int forward_impl(naiwa_cached_layer* L, naiwa_cached_layer* next, int swaps_per_row, const void* x, int rows,
                 float* out, float pcie_frac, int promote_cap, uint64_t min_hits, int64_t stream,
                 naiwa_cached_step* info, naiwa_lookahead_step* ahead, void* res_x = nullptr,
                 bool* folded = nullptr) {
    if (!L || !x || !out || rows <= 0 || swaps_per_row < 0) return NAIWA_E_INVALID;
    // the lookahead publishes the next layer's prediction in this layer's routing
    // doorbell, sized for this layer's top_k
    if (next && (next == L || next->d.hidden != L->d.hidden || next->d.top_k != L->d.top_k)) return NAIWA_E_INVALID;
    const naiwa_cached_layer_desc& d = L->d;
    const int k = d.top_k, n = rows * k;
    hipStream_t st = (hipStream_t)stream;
    // a CPU job of an earlier step that failed (its result was not computed): report it
    // before this step touches anything
    int rc = NAIWA_OK;
    naiwa_executor* ex = L->cpu_misses ? cpu_executor(&rc) : nullptr;
    if (rc) return rc;
    if (ex && (rc = naiwa_executor_take_error(ex, nullptr, 0))) return rc;
    rc = L->ensure_rows(rows);
    if (!rc && next) rc = next->ensure_rows(rows);
    if (rc) return rc;
    L->views(n);
    naiwa_cached_step step{};

    // one layer's steps run in order whatever stream each is queued on: the routing
    // buffers, the step inputs and the ring slots of the previous step are then free
    for (naiwa_cached_layer* o : {L, next}) {
        if (!o || !o->have_last_stream || o->last_stream == st) continue;
        if ((rc = o->record_reads())) return rc;
        if (o->read_recorded && (rc = naiwa_hip_rc(hipStreamWaitEvent(st, o->read_done, 0)))) return rc;
    }

    // route on the device, then read the top-k back through the mapped doorbell: the
    // router's results (and the lookahead's prediction) are published as words tagged
    // with the step's sequence number and the host spins on the tags, with no stream
    // synchronisation (the routing round trip)
    const uint32_t tag = ++L->db_seq;
    uint64_t* pay_dev = reinterpret_cast<uint64_t*>(L->db_dev + kDbHead);
    const int nwords = 2 * n + (next ? n : 0);
    if (rows == 1 && (!next || next->d.top_k == k)) {
        // one token: both routers' logits (the layer's, and the next layer's for the
        // prediction), the top ks and the publish in one launch
        rc = naiwa_route_one_publish(x, NAIWA_BF16, d.hidden, d.router, d.router_bias, d.num_experts, k, d.mode,
                                     L->ids_dev, L->w_dev, next ? next->d.router : nullptr,
                                     next ? next->d.router_bias : nullptr, next ? next->d.num_experts : 0, k,
                                     NAIWA_ROUTE_TOPK_SOFTMAX, next ? next->pred_ids_dev : nullptr,
                                     next ? next->pred_w_dev : nullptr, tag, L->rwords_dev, pay_dev,
                                     naiwa_wall_ticks_ms(2000), stream);
        if (rc) return rc;
        if (next) next->pred_rows = rows;
    } else {
        rc = naiwa_router_topk_biased(x, NAIWA_BF16, d.router, d.router_bias, rows, d.hidden, d.num_experts, k,
                                      d.mode, L->ids_dev, L->w_dev, nullptr, stream);
        if (!rc && next) rc = next->predict_launch(x, rows, stream);
        if (rc) return rc;
        routing_publish_kernel<<<1, 256, 0, st>>>(pay_dev, tag, L->ids_dev, L->w_dev, n,
                                                  next ? next->pred_ids_dev : nullptr, next ? n : 0);
        if ((rc = naiwa_hip_rc(hipGetLastError()))) return rc;
    }
    if ((rc = wait_routing(reinterpret_cast<const uint64_t*>(L->db_host + kDbHead), nwords, tag, L->route_h.data())))
        return rc;
    L->last_rows = rows;

    // the previous step's staged-upload wait ran out (poll mode; its kernels ran before
    // this step's routing): that step's output was invalid.  Reported before any policy
    // state changes.
    {
        const uint32_t fails = naiwa_host_load_acquire_u32(L->db_host + 1);
        if (fails != L->upload_fail_seen) {
            L->upload_fail_seen = fails;
            return NAIWA_E_TIMEOUT;
        }
    }
    // without the CPU path, a step that would leave a miss unstaged is refused before
    // the policy is touched (no tick, hit count or ring position moves)
    if (!L->cpu_misses) {
        naiwa_step_plan plan{};
        if ((rc = naiwa_cache_plan(L->cache, L->ring_len, L->ids_h, L->w_h, rows, k, pcie_frac, &plan))) return rc;
        if (plan.cpu > 0) return NAIWA_E_UNSUPPORTED;
    }

    // hit/miss split, then the misses to stream into the ring; the rest go to the CPU
    if ((rc = naiwa_cache_route(L->cache, L->ids_h, rows, k, L->slots_h))) return rc;
    std::vector<uint32_t> chosen((size_t)L->ring_len);
    std::vector<int32_t> pos((size_t)L->ring_len);
    int nc = 0;
    if ((rc = naiwa_cache_stage(L->ring, L->ids_h, L->w_h, rows, k, pcie_frac, L->slots_h, chosen.data(), pos.data(),
                                &nc)))
        return rc;
    std::vector<char> on_cpu((size_t)n, 0);
    for (int i = 0; i < n; ++i) {
        if (L->slots_h[i] < 0) { // a CPU pair: slot 0 with weight 0 on the device
            ++step.cpu;
            on_cpu[(size_t)i] = 1;
            L->slots_up[i] = 0u;
        } else if (L->slots_h[i] >= NAIWA_STAGING_RING_FIRST) {
            ++step.staged;
            L->slots_up[i] = (uint32_t)(d.usable + (L->slots_h[i] - NAIWA_STAGING_RING_FIRST));
        } else {
            ++step.hits;
            L->slots_up[i] = (uint32_t)L->slots_h[i];
        }
    }
    const bool cpu = step.cpu > 0;

    // Staged uploads by the batched copy kernel hold up kernels that run beside them (its
    // PCIe reads stall the memory pipeline they share), so a cache-pair pass queued ahead
    // of the upload wait would end with the upload anyway: with that kernel, one expert
    // pass over every pair runs after the upload.  With DMA uploads the cache pairs go
    // first, during the upload, and the staged pairs after it.
    const bool batch = L->batch_uploads && !L->dma_uploads && 3 * nc <= NAIWA_COPY_BATCH_MAX;
    const bool split = nc && !batch;

    // the step's inputs: slot ids and, for split passes, the weights of the cache pairs
    // and of the staged pairs, written into mapped coherent host memory.  The previous
    // step of this layer has finished reading them: its kernels precede this step's
    // routing, whose doorbell the host waited for above.  Split passes run the cache
    // pairs during the uploads, so their inputs are pulled into device memory by one wave
    // first (its few PCIe reads would otherwise queue behind megabytes of upload reads).
    // One pass after the uploads (or with none) reads the slot ids from the mapped memory
    // itself, in the gate/up segmentation: one launch and its gap fewer per layer.
    // With CPU pairs, one pass reads the weights there too, the CPU pairs' set to 0.
    if (split || cpu) {
        float* w_res = L->wsplit_h;
        float* w_stg = L->wsplit_h + n;
        for (int i = 0; i < n; ++i) {
            const bool staged_pair = !on_cpu[(size_t)i] && L->slots_up[i] >= (uint32_t)d.usable;
            w_res[i] = on_cpu[(size_t)i] || (split && staged_pair) ? 0.0f : L->w_h[i];
            w_stg[i] = staged_pair ? L->w_h[i] : 0.0f;
        }
    }
    std::atomic_thread_fence(std::memory_order_release);
    if (split) {
        pull_inputs_kernel<<<1, 64, 0, st>>>(L->in_dev_base, L->in_map_base, n * 3);
        if ((rc = naiwa_hip_rc(hipGetLastError()))) return rc;
    }
    const uint32_t* slot_ids = split ? L->slots_dev : L->in_map_base;
    const float* w_one = cpu ? (const float*)(L->in_map_base + n) : L->w_dev; // one pass: its weights

    // the CPU pairs: x goes out through the publish page, and the job (the pairs' ids,
    // weights 0 except on the CPU pairs) is queued on the executor now, so it runs while
    // the device takes the resident and staged pairs (src/moe/stages/cpu_miss.rs:73-162)
    naiwa_pending pend{};
    if (cpu) {
        x_publish_kernel<<<1, 256, 0, st>>>(L->xpub_dev, (const uint16_t*)x, rows * d.hidden);
        if ((rc = naiwa_hip_rc(hipGetLastError()))) return rc;
        CpuJob* job = new (std::nothrow) CpuJob;
        if (!job) return NAIWA_E_NOMEM;
        job->hx = L->hx;
        job->seq = L->xpub_host;
        job->target = ++L->xpub_seq;
        job->rows = rows;
        job->width = k;
        job->act = d.act;
        job->ids.assign(L->ids_h, L->ids_h + n);
        job->w.resize((size_t)n);
        for (int i = 0; i < n; ++i) job->w[(size_t)i] = on_cpu[(size_t)i] ? L->w_h[i] : 0.0f;
        if ((rc = naiwa_executor_submit_result(ex, rows * d.hidden, cpu_job_run, job, &pend))) {
            delete job;
            return rc;
        }
    }

    // uploads on the copy stream: one kernel for all of them when the host stacks are
    // mapped pinned memory (one range per expert when its projections are adjacent, else
    // one per projection), else DMA copies (one per expert when adjacent, else one per
    // projection).  They need no fence of their own: every earlier read of this layer's
    // ring slots (expert passes, promotion copies) precedes the previous step's read_done,
    // which precedes this step's routing on the device, and the host has seen that
    // routing complete (its doorbell) before it queues these uploads.
    {
        naiwa_copy items[NAIWA_COPY_BATCH_MAX];
        int ni = 0;
        for (int i = 0; i < nc; ++i) {
            if (batch) {
                void* dst[3];
                L->slot_ptrs(d.usable + pos[i], dst);
                if (L->contiguous)
                    items[ni++] = naiwa_copy{dst[0], (const uint8_t*)L->host_dev[0] + (size_t)chosen[i] * L->host_stride[0],
                                             (uint64_t)L->expert_bytes};
                else
                    for (int p = 0; p < 3; ++p)
                        items[ni++] = naiwa_copy{dst[p],
                                                 (const uint8_t*)L->host_dev[p] + (size_t)chosen[i] * L->host_stride[p],
                                                 (uint64_t)L->bytes[p]};
            } else if ((rc = L->upload((int)chosen[i], d.usable + pos[i], 0))) {
                return rc;
            }
        }
        if (batch && (rc = naiwa_copy_batch_mapped(items, ni, (int64_t)L->copy))) return rc;
        step.pcie_bytes += (int64_t)nc * (int64_t)(L->bytes[0] + L->bytes[1] + L->bytes[2]);
    }
    step.staged_experts = nc;
    const bool poll = L->upload_sync == NAIWA_UPLOAD_SYNC_POLL;
    if (nc && poll && (rc = doorbell_poll_signal(L->upload_flag, ++L->upload_epoch, (int64_t)L->copy))) return rc;
    if (nc && !poll && (rc = naiwa_hip_rc(hipEventRecord(L->staged_done, L->copy)))) return rc;
    // the stream's wait for the staged uploads
    auto wait_staged = [&]() -> int {
        if (!poll) return naiwa_hip_rc(hipStreamWaitEvent(st, L->staged_done, 0));
        staged_wait_kernel<<<1, 64, 0, st>>>(L->upload_flag, L->upload_epoch, naiwa_doorbell_wait_limit_ticks(),
                                             L->db_dev + 1);
        return naiwa_hip_rc(hipGetLastError());
    };

    // the expert kernel after the latest lookahead claim (src/moe/cached_layer.rs:808-819):
    // a slot it published may still be in flight
    if (L->ahead_claimed) {
        if ((rc = naiwa_hip_rc(hipStreamWaitEvent(st, L->ahead_done, 0)))) return rc;
        ++step.preload_waits;
    }
    if (!split) {
        // poll mode: the wait rides in the expert kernels (a one-token call's gate/up
        // blocks segment the pairs and stage x while the uploads land, then wait)
        const naiwa_decode_wait wt{L->upload_flag, L->upload_epoch, naiwa_doorbell_wait_limit_ticks(), L->db_dev + 1};
        const naiwa_decode_wait* wp = nc && poll ? &wt : nullptr;
        if (nc && !poll && (rc = wait_staged())) return rc;
        if (res_x && !cpu) {
            // out keeps the layer's output; the residual rides in the ordered combine
            if ((rc = naiwa_moe_decode_residual(&d.gate, &d.up, &d.down, res_x, slot_ids, w_one, rows, k,
                                                d.act, out, 1, stream, wp)))
                return rc;
            if (folded) *folded = true;
        } else if ((rc = naiwa_moe_decode_wait(&d.gate, &d.up, &d.down, x, NAIWA_BF16, slot_ids, w_one, rows, k,
                                               d.act, out, stream, wp))) {
            return rc;
        }
    } else {
        // the cache pairs first, while the staged experts are still on the wire, then the
        // staged pairs added on top: ring slots sort after cache slots, so the two calls
        // add the terms of one call in its order (src/moe/decode.rs:226-233 runs the
        // resident experts before the staging wait for the same reason)
        if ((rc = naiwa_moe_decode_ex(&d.gate, &d.up, &d.down, x, NAIWA_BF16, L->slots_dev, L->wsplit_dev, rows, k,
                                      d.act, out, 0, stream)))
            return rc;
        if ((rc = wait_staged())) return rc;
        if ((rc = naiwa_moe_decode_ex(&d.gate, &d.up, &d.down, x, NAIWA_BF16, L->slots_dev, L->wsplit_dev + n, rows,
                                      k, d.act, out, NAIWA_DECODE_ACCUMULATE, stream)))
            return rc;
    }
    // promotion: staged -> cache slot copies, ordered after the kernel by the stream
    if (promote_cap > 0 && nc > 0) {
        std::vector<int32_t> pe((size_t)promote_cap), ps((size_t)promote_cap);
        int np = 0;
        if ((rc = naiwa_cache_promote_pick(L->cache, chosen.data(), nc, promote_cap, min_hits, pe.data(), ps.data(),
                                           &np)))
            return rc;
        for (int i = 0; i < np; ++i) {
            int from = -1;
            for (int j = 0; j < nc; ++j)
                if ((int)chosen[j] == pe[i]) from = d.usable + pos[j];
            void* dst[3];
            void* src[3];
            L->slot_ptrs(ps[i], dst);
            L->slot_ptrs(from, src);
            // the three projections in one kernel (device to device), one range when adjacent
            naiwa_copy items[3];
            int nitems = 1;
            if (L->contiguous) {
                items[0] = naiwa_copy{dst[0], src[0], (uint64_t)L->expert_bytes};
            } else {
                nitems = 3;
                for (int p = 0; p < 3; ++p) items[p] = naiwa_copy{dst[p], src[p], (uint64_t)L->bytes[p]};
            }
            rc = naiwa_copy_batch_mapped(items, nitems, (int64_t)st);
            if (rc == NAIWA_E_UNSUPPORTED) { // not 16-byte aligned: runtime copies
                rc = NAIWA_OK;
                for (int p = 0; p < nitems && !rc; ++p)
                    rc = naiwa_hip_rc(hipMemcpyAsync(items[p].dst, items[p].src, items[p].bytes, hipMemcpyDeviceToDevice,
                                                     st));
            }
            if (rc) {
                naiwa_cache_unreserve(L->cache, ps[i]);
                return rc;
            }
            if ((rc = naiwa_cache_publish(L->cache, ps[i]))) return rc;
            ++step.promoted;
        }
    }

    // the CPU pairs' sum, added last: the device waits for the job's result doorbell,
    // copies it and adds it to the resident and staged sum (src/moe/decode.rs:371-381)
    if (cpu) {
        if ((rc = naiwa_pending_upload(ex, &pend, L->cpu_out, stream))) return rc;
        const int nx = rows * d.hidden;
        add_f32_kernel<<<(nx + 255) / 256 < 1024 ? (nx + 255) / 256 : 1024, 256, 0, st>>>(out, L->cpu_out, nx);
        if ((rc = naiwa_hip_rc(hipGetLastError()))) return rc;
    }
    // every read of this layer's cache slots and of its publish page is before this
    // point on `stream` (the CPU job has finished reading x once its result arrived):
    // read_done is recorded here, or later on this stream when first needed
    L->last_stream = st;
    L->have_last_stream = true;
    L->read_pending = true;
    if (L->lookahead_target && (rc = L->record_reads())) return rc;

    naiwa_cache_stats s{};
    s.hits = (uint64_t)step.hits;
    s.misses = (uint64_t)step.cpu;
    s.staged = (uint64_t)step.staged;
    s.pcie_misses = (uint64_t)nc;
    s.pcie_bytes = (uint64_t)step.pcie_bytes;
    s.promotions = (uint64_t)step.promoted;
    s.sync_waits = (uint64_t)((nc ? 1 : 0) + step.preload_waits);
    naiwa_stats_add(&s);
    if (info) *info = step;
    if (next) return next->prefetch_apply(L->route_h.data() + 2 * n, swaps_per_row, ahead);
    return NAIWA_OK;
}

} // namespace

extern "C" {

int naiwa_cached_layer_create(const naiwa_cached_layer_desc* d, naiwa_ring* ring, int ring_len,
                              int64_t copy_stream, naiwa_cached_layer** out) {
    if (!d || !ring || !out || ring_len <= 0 || d->num_experts <= 0 || d->top_k <= 0 || d->usable < 0 ||
        !d->router || !d->host_gate || !d->host_up || !d->host_down)
        return NAIWA_E_INVALID;
    const int need = d->usable + ring_len;
    if (!bank_ok(d->gate, d->inter, d->hidden, need) || !bank_ok(d->up, d->inter, d->hidden, need) ||
        !bank_ok(d->down, d->hidden, d->inter, need))
        return NAIWA_E_INVALID;
    naiwa_cached_layer* L = new (std::nothrow) naiwa_cached_layer;
    if (!L) return NAIWA_E_NOMEM;
    L->d = *d;
    L->ring = ring;
    L->ring_len = ring_len;
    L->copy = (hipStream_t)copy_stream;
    L->bytes[0] = (size_t)naiwa_projection_bytes(d->gate.dtype, d->inter, d->hidden);
    L->bytes[1] = (size_t)naiwa_projection_bytes(d->up.dtype, d->inter, d->hidden);
    L->bytes[2] = (size_t)naiwa_projection_bytes(d->down.dtype, d->hidden, d->inter);
    // a positive stride shorter than a projection would make experts overlap in the stacks
    if (d->host_expert_stride < 0 ||
        (d->host_expert_stride > 0 &&
         (size_t)d->host_expert_stride < std::max(L->bytes[0], std::max(L->bytes[1], L->bytes[2])))) {
        delete L;
        return NAIWA_E_INVALID;
    }
    // host stacks: each projection stacked on its own (stride = its bytes), or experts
    // interleaved with a common stride (host_expert_stride)
    for (int p = 0; p < 3; ++p) L->host_stride[p] = d->host_expert_stride > 0 ? (size_t)d->host_expert_stride : L->bytes[p];
    L->expert_bytes = L->bytes[0] + L->bytes[1] + L->bytes[2];
    L->hx = naiwa_host_experts{d->host_gate, d->host_up, d->host_down,
                               (int64_t)L->host_stride[0], (int64_t)L->host_stride[1], (int64_t)L->host_stride[2],
                               d->gate.dtype, d->up.dtype, d->down.dtype, d->num_experts, d->hidden, d->inter};
    {
        const uint8_t* hg = (const uint8_t*)d->host_gate;
        const uint8_t* g = (const uint8_t*)d->gate.base;
        L->contiguous = d->host_expert_stride >= (int64_t)L->expert_bytes &&
                        (const uint8_t*)d->host_up == hg + L->bytes[0] &&
                        (const uint8_t*)d->host_down == hg + L->bytes[0] + L->bytes[1] &&
                        (const uint8_t*)d->up.base == g + L->bytes[0] &&
                        (const uint8_t*)d->down.base == g + L->bytes[0] + L->bytes[1] &&
                        d->gate.slot_stride == d->up.slot_stride && d->gate.slot_stride == d->down.slot_stride &&
                        d->gate.slot_stride >= (int64_t)L->expert_bytes;
    }
    // staged uploads read the host stacks through their device mapping when all three
    // are mapped pinned memory and every expert range is 16-byte aligned
    {
        const void* hs[3] = {d->host_gate, d->host_up, d->host_down};
        bool ok = true;
        for (int p = 0; p < 3 && ok; ++p) {
            const size_t span = L->host_stride[p] * (size_t)(d->num_experts - 1) + L->bytes[p];
            L->host_dev[p] = naiwa_device_view(hs[p], span);
            ok = L->host_dev[p] && !(((uintptr_t)L->host_dev[p] | L->bytes[p] | L->host_stride[p]) & 15);
        }
        L->batch_uploads = ok;
    }
    int rc = naiwa_cache_create(d->num_experts, d->usable, d->usable, &L->cache);
    if (rc) {
        delete L;
        return rc;
    }
    for (hipEvent_t* ev : {&L->staged_done, &L->read_done, &L->ahead_done})
        if (hipEventCreateWithFlags(ev, hipEventDisableTiming) != hipSuccess) rc = NAIWA_E_DEVICE;
    if (!rc && (hipMalloc(&L->upload_flag, 256) != hipSuccess || hipMemset(L->upload_flag, 0, 256) != hipSuccess))
        rc = NAIWA_E_NOMEM;
    if (!rc) rc = L->ensure_rows(8);
    if (rc) {
        naiwa_cached_layer_destroy(L);
        return rc;
    }
    *out = L;
    return NAIWA_OK;
}

int naiwa_cached_layer_destroy(naiwa_cached_layer* L) {
    if (!L) return NAIWA_OK;
    (void)hipDeviceSynchronize();
    L->release_buffers();
    for (hipEvent_t ev : {L->staged_done, L->read_done, L->ahead_done})
        if (ev) (void)hipEventDestroy(ev);
    if (L->upload_flag) (void)hipFree(L->upload_flag);
    naiwa_cache_destroy(L->cache);
    delete L;
    return NAIWA_OK;
}

int naiwa_cached_layer_set_upload_sync(naiwa_cached_layer* L, int mode) {
    if (!L || (mode != NAIWA_UPLOAD_SYNC_EVENT && mode != NAIWA_UPLOAD_SYNC_POLL)) return NAIWA_E_INVALID;
    L->upload_sync = mode;
    return NAIWA_OK;
}

int naiwa_cached_layer_set_upload_path(naiwa_cached_layer* L, int path) {
    if (!L || (path != NAIWA_UPLOAD_PATH_KERNEL && path != NAIWA_UPLOAD_PATH_DMA)) return NAIWA_E_INVALID;
    L->dma_uploads = path == NAIWA_UPLOAD_PATH_DMA;
    return NAIWA_OK;
}

int naiwa_cached_layer_set_cpu_misses(naiwa_cached_layer* L, int on) {
    if (!L) return NAIWA_E_INVALID;
    L->cpu_misses = on != 0;
    return NAIWA_OK;
}

int naiwa_cached_layer_upload_timeouts(const naiwa_cached_layer* L, uint32_t* count) {
    if (!L || !count) return NAIWA_E_INVALID;
    *count = L->db_host ? naiwa_host_load_acquire_u32(L->db_host + 1) : 0u;
    return NAIWA_OK;
}

int naiwa_cached_layer_cache(naiwa_cached_layer* L, naiwa_cache** out) {
    if (!L || !out) return NAIWA_E_INVALID;
    *out = L->cache;
    return NAIWA_OK;
}

int naiwa_cached_layer_fill(naiwa_cached_layer* L, int expert, int* slot_out) {
    if (!L || !slot_out) return NAIWA_E_INVALID;
    int rc = naiwa_cache_admit(L->cache, expert, slot_out);
    if (rc || *slot_out < 0) return rc;
    rc = L->upload(expert, *slot_out, 0);
    if (!rc) rc = naiwa_hip_rc(hipStreamSynchronize(L->copy));
    if (rc) {
        naiwa_cache_unreserve(L->cache, *slot_out);
        *slot_out = -1;
        return rc;
    }
    return naiwa_cache_publish(L->cache, *slot_out);
}

int naiwa_cached_layer_seed(naiwa_cached_layer* L, const uint32_t* experts, int n, float fill_share, int* filled) {
    if (!L || !filled || n < 0 || (n > 0 && !experts) || !(fill_share >= 0.0f && fill_share <= 1.0f))
        return NAIWA_E_INVALID;
    *filled = 0;
    const int budget = (int)std::llround((double)L->d.usable * (double)fill_share);
    std::vector<int> slots;
    int rc = NAIWA_OK;
    for (int i = 0; i < n && i < budget && !rc; ++i) {
        if (experts[i] >= (uint32_t)L->d.num_experts) continue; // not in this model: skipped
        int slot = -1;
        if ((rc = naiwa_cache_admit(L->cache, (int)experts[i], &slot)) || slot < 0) continue;
        rc = L->upload((int)experts[i], slot, 0);
        slots.push_back(slot);
    }
    if (!rc) rc = naiwa_hip_rc(hipStreamSynchronize(L->copy));
    for (int slot : slots) {
        if (rc) {
            naiwa_cache_unreserve(L->cache, slot);
        } else {
            if ((rc = naiwa_cache_publish(L->cache, slot))) return rc;
            ++*filled;
        }
    }
    return rc;
}

int naiwa_cached_layer_forward(naiwa_cached_layer* L, const void* x, int rows, float* out, float pcie_frac,
                               int promote_cap, uint64_t min_hits, int64_t stream, naiwa_cached_step* info) {
    return forward_impl(L, nullptr, 0, x, rows, out, pcie_frac, promote_cap, min_hits, stream, info, nullptr);
}

int naiwa_cached_layer_forward_ahead(naiwa_cached_layer* L, naiwa_cached_layer* next, int lookahead_swaps,
                                     const void* x, int rows, float* out, float pcie_frac, int promote_cap,
                                     uint64_t min_hits, int64_t stream, naiwa_cached_step* info,
                                     naiwa_lookahead_step* ahead) {
    if (!next) return NAIWA_E_INVALID;
    return forward_impl(L, next, lookahead_swaps, x, rows, out, pcie_frac, promote_cap, min_hits, stream, info,
                        ahead);
}

int naiwa_cached_layer_prefetch(naiwa_cached_layer* next, const void* x, int rows, int lookahead_swaps,
                                int64_t stream, naiwa_lookahead_step* info) {
    if (!next || !x || rows <= 0 || lookahead_swaps < 0) return NAIWA_E_INVALID;
    int rc = next->ensure_rows(rows);
    if (!rc) rc = next->predict_launch(x, rows, stream);
    if (!rc)
        rc = naiwa_hip_rc(hipMemcpyAsync(next->pred_ids_h, next->pred_ids_dev, (size_t)rows * next->d.top_k * 4,
                                         hipMemcpyDeviceToHost, (hipStream_t)stream));
    if (!rc) rc = naiwa_hip_rc(hipStreamSynchronize((hipStream_t)stream));
    if (rc) return rc;
    return next->prefetch_apply(next->pred_ids_h, lookahead_swaps, info);
}

int naiwa_cached_stack_forward(naiwa_cached_layer* const* layers, int n_layers, void* x, int rows, float* y,
                               float pcie_frac, int promote_cap, uint64_t min_hits, int lookahead_swaps,
                               int64_t stream, naiwa_cached_step* total, naiwa_lookahead_step* ahead_total) {
    if (!layers || n_layers <= 0 || !x || !y || rows <= 0) return NAIWA_E_INVALID;
    const int H = layers[0] ? layers[0]->d.hidden : 0;
    for (int l = 0; l < n_layers; ++l)
        if (!layers[l] || layers[l]->d.hidden != H) return NAIWA_E_INVALID;
    if (total) *total = naiwa_cached_step{};
    if (ahead_total) *ahead_total = naiwa_lookahead_step{};
    for (int l = 0; l < n_layers; ++l) {
        naiwa_cached_step s{};
        naiwa_lookahead_step a{};
        const bool ahead = lookahead_swaps >= 0 && l + 1 < n_layers;
        bool folded = false;
        int rc = forward_impl(layers[l], ahead ? layers[l + 1] : nullptr, ahead ? lookahead_swaps : 0, x, rows, y,
                              pcie_frac, promote_cap, min_hits, stream, &s, ahead ? &a : nullptr, x, &folded);
        if (!rc && !folded) rc = naiwa_residual_add_bf16(x, y, (int64_t)rows * H, stream);
        if (rc) return rc;
        if (total) {
            total->hits += s.hits;
            total->staged += s.staged;
            total->staged_experts += s.staged_experts;
            total->promoted += s.promoted;
            total->pcie_bytes += s.pcie_bytes;
            total->preload_waits += s.preload_waits;
            total->cpu += s.cpu;
        }
        if (ahead_total && ahead) {
            ahead_total->predicted += a.predicted;
            ahead_total->resident += a.resident;
            ahead_total->loads += a.loads;
            ahead_total->swaps += a.swaps;
            ahead_total->pcie_bytes += a.pcie_bytes;
        }
    }
    return NAIWA_OK;
}

int naiwa_cached_layer_predicted(const naiwa_cached_layer* L, uint32_t* ids, int capacity, int* n_out) {
    if (!L || !n_out || (capacity > 0 && !ids)) return NAIWA_E_INVALID;
    const int n = (int)L->predicted.size();
    if (capacity < n) return NAIWA_E_INVALID;
    for (int i = 0; i < n; ++i) ids[i] = L->predicted[(size_t)i];
    *n_out = n;
    return NAIWA_OK;
}

int naiwa_cached_layer_routing(const naiwa_cached_layer* L, uint32_t* ids, float* w, int capacity) {
    if (!L || !ids || !w) return NAIWA_E_INVALID;
    const int n = L->last_rows * L->d.top_k;
    if (capacity < n) return NAIWA_E_INVALID;
    for (int i = 0; i < n; ++i) {
        ids[i] = L->ids_h[i];
        w[i] = L->w_h[i];
    }
    return NAIWA_OK;
}

} // extern "C"
