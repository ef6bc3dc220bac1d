// The whole-layer prefill stream and its memory plan (include/naiwa_prefill.h):
// the reference's PrefillStream (src/prefill_stream.rs:342-1693) and
// plan_with_lend_depth (src/prefill_stream.rs:122-310), over a ring of device
// layer buffers filled from pinned host stacks on a copy stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <new>
#include <vector>

#include "../../include/naiwa_prefill.h"
#include "common.h"

namespace {

constexpr uint64_t kMiB = 1ull << 20;
constexpr uint64_t kKiB = 1ull << 10;
constexpr uint64_t kMaxHeadroom = 512 * kMiB; // MAX_HEADROOM
constexpr uint64_t kChunkHead = 256 * kMiB;   // CHUNK_HEAD
constexpr int kPlanGrid = 256;                // PLAN_GRID
constexpr int kSubRows = 256;                 // SUB_ROWS
constexpr int kMaxDepth = 4;                  // MAX_DEPTH

// An unsigned integer environment override, as the reference's probes read them.
bool env_u64(const char* name, uint64_t* v) {
    const char* s = std::getenv(name);
    if (!s || !*s) return false;
    char* end = nullptr;
    const unsigned long long x = std::strtoull(s, &end, 10);
    if (!end || *end) return false;
    *v = (uint64_t)x;
    return true;
}

uint64_t sat_sub(uint64_t a, uint64_t b) { return a > b ? a - b : 0; }

} // namespace

struct naiwa_prefill_stream {
    naiwa_prefill_stream_desc d{};
    std::vector<const void*> hg, hu, hd; // host stacks per layer
    hipStream_t copy = nullptr;
    size_t eb[3] = {0, 0, 0};       // one expert's bytes per projection
    int64_t stride[3] = {0, 0, 0};  // device slot stride per projection (16-byte multiple)
    struct Buf {
        void* mem[3] = {nullptr, nullptr, nullptr};
        int loaded = -1;            // the layer whose upload was queued last
        hipEvent_t ready = nullptr; // recorded on the copy stream after that upload
        hipEvent_t released = nullptr; // recorded on the compute stream after the last read
        bool read = false;
    };
    std::vector<Buf> bufs;
    naiwa_prefill_stream_stats stats{};

    int load(int layer) {
        Buf& b = bufs[(size_t)(layer % d.depth)];
        if (b.loaded == layer) return NAIWA_OK;
        hipError_t e = hipSuccess;
        // the last kernel that read this buffer goes first (the reference's ReadFence)
        if (b.read) e = hipStreamWaitEvent(copy, b.released, 0);
        const void* src[3] = {hg[(size_t)layer], hu[(size_t)layer], hd[(size_t)layer]};
        for (int p = 0; p < 3 && e == hipSuccess; ++p)
            e = hipMemcpy2DAsync(b.mem[p], (size_t)stride[p], src[p], eb[p], eb[p], (size_t)d.num_experts,
                                 hipMemcpyHostToDevice, copy);
        if (e == hipSuccess) e = hipEventRecord(b.ready, copy);
        if (e != hipSuccess) {
            b.loaded = -1;
            return naiwa_hip_rc(e);
        }
        b.loaded = layer;
        ++stats.uploads;
        stats.upload_bytes += (uint64_t)d.num_experts * (eb[0] + eb[1] + eb[2]);
        return NAIWA_OK;
    }

    void banks(int layer, naiwa_bank out[3]) const {
        const Buf& b = bufs[(size_t)(layer % d.depth)];
        const int n[3] = {d.inter, d.inter, d.hidden}, k[3] = {d.hidden, d.hidden, d.inter};
        const int dt[3] = {d.dtype_gate, d.dtype_up, d.dtype_down};
        for (int p = 0; p < 3; ++p) {
            out[p].base = b.mem[p];
            out[p].slot_stride = stride[p];
            out[p].slots = d.num_experts;
            out[p].n = n[p];
            out[p].k = k[p];
            out[p].dtype = dt[p];
        }
    }

    void release() {
        for (auto& b : bufs) {
            for (auto& m : b.mem)
                if (m) (void)hipFree(m);
            if (b.ready) (void)hipEventDestroy(b.ready);
            if (b.released) (void)hipEventDestroy(b.released);
        }
        bufs.clear();
    }
};

extern "C" {

uint64_t naiwa_prefill_chunk_scratch(int rows) {
    uint64_t fixed = 32 * kMiB, per_row = 354 * kKiB, v = 0;
    if (env_u64("NAIWA_CHUNK_FIXED_MIB", &v)) fixed = v * kMiB;
    if (env_u64("NAIWA_CHUNK_PER_ROW_KIB", &v)) per_row = v * kKiB;
    return fixed + per_row * (uint64_t)std::max(rows, 0);
}

uint64_t naiwa_prefill_activation_bytes(int chunk) {
    const uint64_t c = (uint64_t)std::max(chunk, 0);
    const uint64_t moe = 160 * kMiB + 680 * kMiB * std::min<uint64_t>(c, kSubRows) / 1024;
    return moe + c * 24 * kKiB;
}

int naiwa_prefill_plan(uint64_t free_bytes, uint64_t layer_bytes, int ceiling, int borrowing, uint64_t kv_reserve,
                       uint64_t lend_bytes, int max_depth, int* stride_out, int* chunk_out) {
    if (!stride_out || !chunk_out || ceiling < 0) return NAIWA_E_INVALID;
    *stride_out = 0;
    *chunk_out = 0;
    const uint64_t free = sat_sub(free_bytes, kv_reserve);
    uint64_t slack = 0;
    const bool slack_set = env_u64("NAIWA_PREFILL_SLACK_MIB", &slack);
    auto fits = [&](int chunk, int stride) {
        const uint64_t head = slack_set ? slack * kMiB : std::max(kMaxHeadroom, free / 8);
        if (borrowing) return free >= naiwa_prefill_chunk_scratch(chunk) + std::min(head, kChunkHead);
        return free >= (uint64_t)stride * layer_bytes + naiwa_prefill_chunk_scratch(chunk) + head;
    };
    // the largest chunk with one buffer: fits is monotone in the chunk, so bisect the grid
    int lo = 1, hi = std::max(std::min(ceiling, 8192) / kPlanGrid, 1), best = 0;
    while (lo <= hi) {
        const int mid = lo + (hi - lo) / 2;
        if (fits(mid * kPlanGrid, 1)) {
            best = mid * kPlanGrid;
            lo = mid + 1;
        } else {
            hi = mid - 1;
        }
    }
    if (best == 0) return NAIWA_OK;
    uint64_t reserve = 700 * kMiB, v = 0;
    if (env_u64("NAIWA_DECODE_RESERVE_MIB", &v)) reserve = v * kMiB;
    const int depth_max = std::min(std::max(max_depth, 1), kMaxDepth);
    int stride = 1;
    if (borrowing) {
        uint64_t cap = 2;
        if (env_u64("NAIWA_DEPTH_CAP", &v)) cap = v;
        const uint64_t ranges = lend_bytes / std::max<uint64_t>(layer_bytes, 1);
        const uint64_t top = std::min<uint64_t>((uint64_t)depth_max, cap);
        stride = (int)std::max<uint64_t>(1, std::min<uint64_t>(ranges, std::max<uint64_t>(top, 1)));
    } else {
        for (int dd = depth_max; dd >= 2; --dd) {
            const bool owns = fits(best, dd) &&
                              sat_sub(free, (uint64_t)dd * layer_bytes + naiwa_prefill_chunk_scratch(best) +
                                                kMaxHeadroom) >= reserve;
            if (owns) {
                stride = dd;
                break;
            }
        }
    }
    *stride_out = stride;
    *chunk_out = best;
    return NAIWA_OK;
}

int naiwa_prefill_stream_create(const naiwa_prefill_stream_desc* d, int64_t copy_stream, naiwa_prefill_stream** out) {
    if (!d || !out || d->n_layers <= 0 || d->num_experts <= 0 || d->hidden <= 0 || d->inter <= 0 || d->depth < 1 ||
        d->depth > kMaxDepth || !d->host_gate || !d->host_up || !d->host_down)
        return NAIWA_E_INVALID;
    *out = nullptr;
    const int64_t eb[3] = {naiwa_projection_bytes(d->dtype_gate, d->inter, d->hidden),
                           naiwa_projection_bytes(d->dtype_up, d->inter, d->hidden),
                           naiwa_projection_bytes(d->dtype_down, d->hidden, d->inter)};
    if (eb[0] <= 0 || eb[1] <= 0 || eb[2] <= 0) return NAIWA_E_UNSUPPORTED;
    for (int l = 0; l < d->n_layers; ++l)
        if (!d->host_gate[l] || !d->host_up[l] || !d->host_down[l]) return NAIWA_E_INVALID;
    naiwa_prefill_stream* ps = new (std::nothrow) naiwa_prefill_stream;
    if (!ps) return NAIWA_E_NOMEM;
    ps->d = *d;
    ps->hg.assign(d->host_gate, d->host_gate + d->n_layers);
    ps->hu.assign(d->host_up, d->host_up + d->n_layers);
    ps->hd.assign(d->host_down, d->host_down + d->n_layers);
    ps->copy = (hipStream_t)copy_stream;
    for (int p = 0; p < 3; ++p) {
        ps->eb[p] = (size_t)eb[p];
        ps->stride[p] = (eb[p] + 255) & ~int64_t(255);
    }
    int rc = NAIWA_OK;
    try {
        ps->bufs.resize((size_t)d->depth);
    } catch (...) {
        delete ps;
        return NAIWA_E_NOMEM;
    }
    for (auto& b : ps->bufs) {
        for (int p = 0; p < 3 && !rc; ++p)
            if (hipMalloc(&b.mem[p], (size_t)ps->stride[p] * (size_t)d->num_experts) != hipSuccess) rc = NAIWA_E_NOMEM;
        if (!rc && (hipEventCreateWithFlags(&b.ready, hipEventDisableTiming) != hipSuccess ||
                    hipEventCreateWithFlags(&b.released, hipEventDisableTiming) != hipSuccess))
            rc = NAIWA_E_DEVICE;
    }
    if (rc) {
        ps->release();
        delete ps;
        return rc;
    }
    *out = ps;
    return NAIWA_OK;
}

int naiwa_prefill_stream_destroy(naiwa_prefill_stream* ps) {
    if (!ps) return NAIWA_OK;
    (void)hipDeviceSynchronize(); // uploads in flight read the host stacks and write the buffers
    ps->release();
    delete ps;
    return NAIWA_OK;
}

int naiwa_prefill_stream_forward(naiwa_prefill_stream* ps, int layer, const void* x, const uint32_t* expert_ids,
                                 const float* w, int T, int k, int act, float* out, int flags, int64_t stream) {
    if (!ps || layer < 0 || layer >= ps->d.n_layers) return NAIWA_E_INVALID;
    int rc = ps->load(layer);
    // the next layers' uploads go out now, behind this one, each into its own buffer
    for (int ahead = 1; !rc && ahead < ps->d.depth && layer + ahead < ps->d.n_layers; ++ahead)
        rc = ps->load(layer + ahead);
    if (rc) return rc;
    naiwa_prefill_stream::Buf& b = ps->bufs[(size_t)(layer % ps->d.depth)];
    hipStream_t st = (hipStream_t)stream;
    if ((rc = naiwa_hip_rc(hipStreamWaitEvent(st, b.ready, 0)))) return rc;
    naiwa_bank bk[3];
    ps->banks(layer, bk);
    if ((rc = naiwa_moe_prefill(&bk[0], &bk[1], &bk[2], x, expert_ids, w, T, k, act, out, flags, stream))) return rc;
    if ((rc = naiwa_hip_rc(hipEventRecord(b.released, st)))) return rc;
    b.read = true;
    ++ps->stats.forwards;
    return NAIWA_OK;
}

int naiwa_prefill_stream_banks(const naiwa_prefill_stream* ps, int layer, naiwa_bank* gate, naiwa_bank* up,
                               naiwa_bank* down) {
    if (!ps || !gate || !up || !down || layer < 0 || layer >= ps->d.n_layers) return NAIWA_E_INVALID;
    if (ps->bufs[(size_t)(layer % ps->d.depth)].loaded != layer) return NAIWA_E_NOT_FOUND;
    naiwa_bank bk[3];
    ps->banks(layer, bk);
    *gate = bk[0];
    *up = bk[1];
    *down = bk[2];
    return NAIWA_OK;
}

int naiwa_prefill_stream_stats_read(const naiwa_prefill_stream* ps, naiwa_prefill_stream_stats* out) {
    if (!ps || !out) return NAIWA_E_INVALID;
    *out = ps->stats;
    return NAIWA_OK;
}

} // extern "C"
