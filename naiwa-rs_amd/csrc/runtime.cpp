// Runtime plumbing of the C ABI: device memory, pinned host memory, streams,
// events and the per-device scratch buffers.  A host binding (ctypes, a Rust
// build.rs FFI, ...) needs nothing but this library to drive the kernels.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string.h>

#include "common.h"
#include "workspace.h"

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
NaiwaScratch g_scratch[kMaxDevices][NAIWA_SCRATCH_TAGS];
} // namespace

void* naiwa_scratch(int tag, size_t bytes, int* rc) { return naiwa_scratch(tag, bytes, rc, nullptr); }

void* naiwa_scratch(int tag, size_t bytes, int* rc, bool* fresh) {
    if (fresh) *fresh = false;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices || tag < 0 || tag >= NAIWA_SCRATCH_TAGS) {
        *rc = e != hipSuccess ? (int)e : NAIWA_E_INVALID;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    NaiwaScratch& s = g_scratch[dev][tag];
    if (s.bytes < bytes) {
        size_t want = bytes < 4096 ? 4096 : bytes;
        want = (want + 255) & ~size_t(255);
        if (s.ptr) {
            // A queued kernel may still read the old buffer.
            e = hipDeviceSynchronize();
            if (e != hipSuccess) { *rc = (int)e; return nullptr; }
            (void)hipFree(s.ptr);
            s.ptr = nullptr;
            s.bytes = 0;
        }
        e = hipMalloc(&s.ptr, want);
        if (e != hipSuccess) {
            s.ptr = nullptr;
            *rc = NAIWA_E_NOMEM;
            return nullptr;
        }
        s.bytes = want;
        if (fresh) *fresh = true;
    }
    *rc = NAIWA_OK;
    return s.ptr;
}

extern "C" {

const char* naiwa_status_string(int rc) {
    switch (rc) {
    case NAIWA_OK: return "ok";
    case NAIWA_E_INVALID: return "invalid argument";
    case NAIWA_E_UNSUPPORTED: return "unsupported dtype, activation or mode";
    case NAIWA_E_TIMEOUT: return "wait timed out";
    case NAIWA_E_NOMEM: return "out of memory";
    case NAIWA_E_BAD_ID: return "expert or slot id out of range";
    case NAIWA_E_NOT_FOUND: return "not found";
    case NAIWA_E_DEVICE: return "device reported failure";
    case NAIWA_E_FORMAT: return "malformed or unsupported file";
    case NAIWA_E_IO: return "file cannot be opened or mapped";
    case NAIWA_E_TOO_LARGE: return "request exceeds a fixed capacity";
    default: return rc > 0 ? hipGetErrorString((hipError_t)rc) : "unknown status";
    }
}

int naiwa_device_count(int* n) { return naiwa_hip_rc(hipGetDeviceCount(n)); }
int naiwa_set_device(int dev) { return naiwa_hip_rc(hipSetDevice(dev)); }

int naiwa_device_info(int dev, int* cu_count, int* wall_clock_khz, int64_t* hbm_bytes, char* name,
                      int name_len) {
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return (int)e;
    if (cu_count) *cu_count = p.multiProcessorCount;
    if (wall_clock_khz) {
        int khz = 0;
        e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
        if (e != hipSuccess) return (int)e;
        *wall_clock_khz = khz;
    }
    if (hbm_bytes) *hbm_bytes = (int64_t)p.totalGlobalMem;
    if (name && name_len > 0) {
        strncpy(name, p.gcnArchName, (size_t)name_len - 1);
        name[name_len - 1] = 0;
    }
    return NAIWA_OK;
}

int naiwa_malloc(void** p, size_t bytes) {
    if (!p) return NAIWA_E_INVALID;
    *p = nullptr;
    return hipMalloc(p, bytes ? bytes : 1) == hipSuccess ? NAIWA_OK : NAIWA_E_NOMEM;
}

int naiwa_free(void* p) { return naiwa_hip_rc(hipFree(p)); }

int naiwa_mem_info(uint64_t* free_bytes, uint64_t* total_bytes) {
    if (!free_bytes || !total_bytes) return NAIWA_E_INVALID;
    size_t f = 0, t = 0;
    const int rc = naiwa_hip_rc(hipMemGetInfo(&f, &t));
    *free_bytes = f;
    *total_bytes = t;
    return rc;
}

int naiwa_host_alloc(void** p, size_t bytes) {
    if (!p) return NAIWA_E_INVALID;
    *p = nullptr;
    return hipHostMalloc(p, bytes ? bytes : 1, hipHostMallocPortable) == hipSuccess ? NAIWA_OK
                                                                                     : NAIWA_E_NOMEM;
}

int naiwa_host_free(void* p) { return naiwa_hip_rc(hipHostFree(p)); }

int naiwa_memcpy_h2d(void* dst, const void* src, size_t bytes, int64_t stream) {
    return naiwa_hip_rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
}

int naiwa_memcpy_d2h(void* dst, const void* src, size_t bytes, int64_t stream) {
    return naiwa_hip_rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
}

int naiwa_memcpy_d2d(void* dst, const void* src, size_t bytes, int64_t stream) {
    return naiwa_hip_rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
}

int naiwa_memcpy_2d_d2d(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width, size_t height,
                        int64_t stream) {
    if (!height || !width) return NAIWA_OK;
    if (!dst || !src || width > dpitch || width > spitch) return NAIWA_E_INVALID;
    return naiwa_hip_rc(
        hipMemcpy2DAsync(dst, dpitch, src, spitch, width, height, hipMemcpyDeviceToDevice, (hipStream_t)stream));
}

int naiwa_memcpy_2d(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width, size_t height,
                    int64_t stream) {
    if (!height || !width) return NAIWA_OK;
    if (!dst || !src || width > dpitch || width > spitch) return NAIWA_E_INVALID;
    return naiwa_hip_rc(
        hipMemcpy2DAsync(dst, dpitch, src, spitch, width, height, hipMemcpyDefault, (hipStream_t)stream));
}

int naiwa_upload_expert(void* const dst[3], const void* const src[3], const size_t bytes[3],
                        int64_t copy_stream, int64_t read_fence, int64_t done_event) {
    if (!dst || !src || !bytes) return NAIWA_E_INVALID;
    for (int i = 0; i < 3; ++i)
        if (bytes[i] && (!dst[i] || !src[i])) return NAIWA_E_INVALID;
    hipStream_t st = (hipStream_t)copy_stream;
    int rc = 0;
    if (read_fence && (rc = naiwa_hip_rc(hipStreamWaitEvent(st, (hipEvent_t)read_fence, 0)))) return rc;
    for (int i = 0; i < 3; ++i)
        if (bytes[i] && (rc = naiwa_hip_rc(hipMemcpyAsync(dst[i], src[i], bytes[i], hipMemcpyHostToDevice, st))))
            return rc;
    if (done_event) return naiwa_hip_rc(hipEventRecord((hipEvent_t)done_event, st));
    return NAIWA_OK;
}

int naiwa_memset(void* p, int value, size_t bytes, int64_t stream) {
    return naiwa_hip_rc(hipMemsetAsync(p, value, bytes, (hipStream_t)stream));
}

int naiwa_stream_create(int64_t* stream) {
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    *stream = (int64_t)s;
    return naiwa_hip_rc(e);
}

int naiwa_stream_destroy(int64_t stream) { return naiwa_hip_rc(hipStreamDestroy((hipStream_t)stream)); }
int naiwa_stream_sync(int64_t stream) { return naiwa_hip_rc(hipStreamSynchronize((hipStream_t)stream)); }

int naiwa_stream_wait_event(int64_t stream, int64_t event) {
    return naiwa_hip_rc(hipStreamWaitEvent((hipStream_t)stream, (hipEvent_t)event, 0));
}

int naiwa_event_create(int64_t* event, int timing) {
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreateWithFlags(&ev, timing ? hipEventDefault : hipEventDisableTiming);
    *event = (int64_t)ev;
    return naiwa_hip_rc(e);
}

int naiwa_event_destroy(int64_t event) { return naiwa_hip_rc(hipEventDestroy((hipEvent_t)event)); }

int naiwa_event_record(int64_t event, int64_t stream) {
    return naiwa_hip_rc(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
}

int naiwa_event_sync(int64_t event) { return naiwa_hip_rc(hipEventSynchronize((hipEvent_t)event)); }

int naiwa_event_query(int64_t event) {
    hipError_t e = hipEventQuery((hipEvent_t)event);
    if (e == hipSuccess) return 0;
    if (e == hipErrorNotReady) return 1;
    return (int)e;
}

int naiwa_event_elapsed_ms(float* ms, int64_t start, int64_t end) {
    return naiwa_hip_rc(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
}

int naiwa_device_sync(void) { return naiwa_hip_rc(hipDeviceSynchronize()); }

int naiwa_last_error(void) { return (int)hipGetLastError(); }

int64_t naiwa_projection_bytes(int dtype, int64_t n, int64_t k) {
    const int64_t rb = naiwa_row_bytes(dtype, k);
    return rb < 0 || n < 0 ? -1 : rb * n;
}

} // extern "C"
