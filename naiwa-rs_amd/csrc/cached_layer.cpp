// One MoE layer's decode step over a partial expert cache (include/naiwa_cached.h):
// device routing, host policy, PCIe staging into ring slots, the expert kernel
// over resident + staged slots, and promotion -- the stage order of the
// reference's decode path (src/moe/decode.rs:241-381).
#include <hip/hip_runtime.h>

#include <new>
#include <vector>

#include "../../include/naiwa_cached.h"
#include "common.h"

namespace {

bool bank_ok(const naiwa_bank& b, int n, int k, int min_slots) {
    return b.base && b.n == n && b.k == k && b.slots >= min_slots &&
           naiwa_projection_bytes(b.dtype, n, k) > 0 && b.slot_stride >= naiwa_projection_bytes(b.dtype, n, k);
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
    uint32_t* ids_dev = nullptr;
    float* w_dev = nullptr;
    uint32_t* slots_dev = nullptr;
    uint32_t* ids_h = nullptr;
    float* w_h = nullptr;
    int32_t* slots_h = nullptr;
    uint32_t* slots_up = nullptr;  // pinned source of the slot-id upload
    int last_rows = 0;
    std::vector<hipEvent_t> ring_fence;  // per ring position: recorded after the step that read it
    std::vector<char> ring_fenced;
    hipEvent_t staged_done = nullptr;

    void release_buffers() {
        if (ids_dev) (void)hipFree(ids_dev);
        if (w_dev) (void)hipFree(w_dev);
        if (slots_dev) (void)hipFree(slots_dev);
        if (ids_h) (void)hipHostFree(ids_h);
        if (w_h) (void)hipHostFree(w_h);
        if (slots_h) (void)hipHostFree(slots_h);
        if (slots_up) (void)hipHostFree(slots_up);
        ids_dev = nullptr;
        w_dev = nullptr;
        slots_dev = nullptr;
        ids_h = nullptr;
        w_h = nullptr;
        slots_h = nullptr;
        slots_up = nullptr;
        cap_rows = 0;
    }

    int ensure_rows(int rows) {
        if (rows <= cap_rows) return NAIWA_OK;
        hipError_t e = hipDeviceSynchronize(); // earlier steps may still read the old buffers
        if (e != hipSuccess) return (int)e;
        release_buffers();
        const size_t n = (size_t)rows * d.top_k;
        if (hipMalloc(&ids_dev, n * 4) != hipSuccess || hipMalloc(&w_dev, n * 4) != hipSuccess ||
            hipMalloc(&slots_dev, n * 4) != hipSuccess || hipHostMalloc(&ids_h, n * 4, 0) != hipSuccess ||
            hipHostMalloc(&w_h, n * 4, 0) != hipSuccess || hipHostMalloc(&slots_h, n * 4, 0) != hipSuccess ||
            hipHostMalloc(&slots_up, n * 4, 0) != hipSuccess) {
            release_buffers();
            return NAIWA_E_NOMEM;
        }
        cap_rows = rows;
        return NAIWA_OK;
    }

    void slot_ptrs(int slot, void* dst[3]) const {
        dst[0] = (uint8_t*)d.gate.base + (int64_t)slot * d.gate.slot_stride;
        dst[1] = (uint8_t*)d.up.base + (int64_t)slot * d.up.slot_stride;
        dst[2] = (uint8_t*)d.down.base + (int64_t)slot * d.down.slot_stride;
    }
    void host_ptrs(int expert, const void* src[3]) const {
        src[0] = (const uint8_t*)d.host_gate + (size_t)expert * bytes[0];
        src[1] = (const uint8_t*)d.host_up + (size_t)expert * bytes[1];
        src[2] = (const uint8_t*)d.host_down + (size_t)expert * bytes[2];
    }
};

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
    int rc = naiwa_cache_create(d->num_experts, d->usable, d->usable, &L->cache);
    if (rc) {
        delete L;
        return rc;
    }
    L->ring_fence.assign((size_t)ring_len, nullptr);
    L->ring_fenced.assign((size_t)ring_len, 0);
    for (auto& ev : L->ring_fence)
        if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) rc = NAIWA_E_DEVICE;
    if (hipEventCreateWithFlags(&L->staged_done, hipEventDisableTiming) != hipSuccess) rc = NAIWA_E_DEVICE;
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
    for (auto ev : L->ring_fence)
        if (ev) (void)hipEventDestroy(ev);
    if (L->staged_done) (void)hipEventDestroy(L->staged_done);
    naiwa_cache_destroy(L->cache);
    delete L;
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
    void* dst[3];
    const void* src[3];
    L->slot_ptrs(*slot_out, dst);
    L->host_ptrs(expert, src);
    rc = naiwa_upload_expert(dst, src, L->bytes, (int64_t)L->copy, 0, 0);
    if (!rc) rc = naiwa_hip_rc(hipStreamSynchronize(L->copy));
    if (rc) {
        naiwa_cache_unreserve(L->cache, *slot_out);
        *slot_out = -1;
        return rc;
    }
    return naiwa_cache_publish(L->cache, *slot_out);
}

int naiwa_cached_layer_forward(naiwa_cached_layer* L, const void* x, int rows, float* out, float pcie_frac,
                               int promote_cap, uint64_t min_hits, int64_t stream, naiwa_cached_step* info) {
    if (!L || !x || !out || rows <= 0) return NAIWA_E_INVALID;
    const naiwa_cached_layer_desc& d = L->d;
    const int k = d.top_k, n = rows * k;
    hipStream_t st = (hipStream_t)stream;
    int rc = L->ensure_rows(rows);
    if (rc) return rc;
    naiwa_cached_step step{};

    // route on the device, then read the top-k back (the routing round trip)
    rc = naiwa_router_topk_biased(x, NAIWA_BF16, d.router, d.router_bias, rows, d.hidden, d.num_experts, k, d.mode,
                                  L->ids_dev, L->w_dev, nullptr, stream);
    if (rc) return rc;
    if ((rc = naiwa_hip_rc(hipMemcpyAsync(L->ids_h, L->ids_dev, (size_t)n * 4, hipMemcpyDeviceToHost, st))) ||
        (rc = naiwa_hip_rc(hipMemcpyAsync(L->w_h, L->w_dev, (size_t)n * 4, hipMemcpyDeviceToHost, st))) ||
        (rc = naiwa_hip_rc(hipStreamSynchronize(st))))
        return rc;
    L->last_rows = rows;

    // hit/miss split, then the misses to stream into the ring
    if ((rc = naiwa_cache_route(L->cache, L->ids_h, rows, k, L->slots_h))) return rc;
    std::vector<uint32_t> chosen((size_t)L->ring_len);
    std::vector<int32_t> pos((size_t)L->ring_len);
    int nc = 0;
    if ((rc = naiwa_cache_stage(L->ring, L->ids_h, L->w_h, rows, k, pcie_frac, L->slots_h, chosen.data(), pos.data(),
                                &nc)))
        return rc;
    for (int i = 0; i < n; ++i) {
        if (L->slots_h[i] < 0) return NAIWA_E_UNSUPPORTED; // a CPU miss: no product CPU path here
        if (L->slots_h[i] >= NAIWA_STAGING_RING_FIRST) {
            ++step.staged;
            L->slots_up[i] = (uint32_t)(d.usable + (L->slots_h[i] - NAIWA_STAGING_RING_FIRST));
        } else {
            ++step.hits;
            L->slots_up[i] = (uint32_t)L->slots_h[i];
        }
    }

    // uploads on the copy stream, each after the last step that read its ring slot
    for (int i = 0; i < nc; ++i) {
        void* dst[3];
        const void* src[3];
        L->slot_ptrs(d.usable + pos[i], dst);
        L->host_ptrs((int)chosen[i], src);
        const int64_t fence = L->ring_fenced[pos[i]] ? (int64_t)L->ring_fence[pos[i]] : 0;
        if ((rc = naiwa_upload_expert(dst, src, L->bytes, (int64_t)L->copy, fence, 0))) return rc;
        step.pcie_bytes += (int64_t)(L->bytes[0] + L->bytes[1] + L->bytes[2]);
    }
    step.staged_experts = nc;
    if (nc) {
        if ((rc = naiwa_hip_rc(hipEventRecord(L->staged_done, L->copy))) ||
            (rc = naiwa_hip_rc(hipStreamWaitEvent(st, L->staged_done, 0))))
            return rc;
    }

    // the expert kernel over cache + ring slots
    if ((rc = naiwa_hip_rc(hipMemcpyAsync(L->slots_dev, L->slots_up, (size_t)n * 4, hipMemcpyHostToDevice, st))))
        return rc;
    if ((rc = naiwa_moe_decode(&d.gate, &d.up, &d.down, x, NAIWA_BF16, L->slots_dev, L->w_dev, rows, k, d.act, out,
                               stream)))
        return rc;
    for (int i = 0; i < nc; ++i) {
        if ((rc = naiwa_hip_rc(hipEventRecord(L->ring_fence[pos[i]], st)))) return rc;
        L->ring_fenced[pos[i]] = 1;
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
            for (int p = 0; p < 3 && !rc; ++p)
                rc = naiwa_hip_rc(hipMemcpyAsync(dst[p], src[p], L->bytes[p], hipMemcpyDeviceToDevice, st));
            if (rc) {
                naiwa_cache_unreserve(L->cache, ps[i]);
                return rc;
            }
            if ((rc = naiwa_cache_publish(L->cache, ps[i]))) return rc;
            ++step.promoted;
        }
    }

    naiwa_cache_stats s{};
    s.hits = (uint64_t)step.hits;
    s.staged = (uint64_t)step.staged;
    s.pcie_misses = (uint64_t)nc;
    s.pcie_bytes = (uint64_t)step.pcie_bytes;
    s.promotions = (uint64_t)step.promoted;
    s.sync_waits = nc ? 1 : 0;
    naiwa_stats_add(&s);
    if (info) *info = step;
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
