// Doorbells: fine-grained, host-coherent mapped memory through which the host
// and the GPU hand each other payloads and progress counters without stream
// syncs (the protocol of src/doorbell/mod.rs:1-27):
//
//   payload stores -> system-scope fence -> release-store of a mapped counter;
//   the consumer acquire-loads the counter, then reads the payload behind it.
//
// The six `doorbell_*` entry points keep the reference's names and
// signatures (src/doorbell/mod.rs:31-69).  One deliberate difference: every
// device-side wait is bounded by a wall-clock limit (s_memrealtime ticks), so
// a producer that never publishes ends the kernel with a counted timeout
// instead of a hung GPU.
#include <atomic>
#include <cstring>
#include <chrono>
#include <mutex>
#include <thread>

#include "common.h"

namespace {

__device__ uint32_t g_doorbell_timeouts = 0;

std::atomic<uint64_t> g_wait_limit_us{10ull * 1000 * 1000};

int wall_clock_khz_current() {
    static std::mutex mu;
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 100000;
    std::lock_guard<std::mutex> lock(mu);
    if (!cached[dev]) {
        int khz = 0;
        if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0)
            khz = 100000;
        cached[dev] = khz;
    }
    return cached[dev];
}

uint64_t wait_limit_ticks() {
    const uint64_t us = g_wait_limit_us.load(std::memory_order_relaxed);
    return us * (uint64_t)wall_clock_khz_current() / 1000ull;
}

__device__ __forceinline__ void store_release_sys(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Spin loads are relaxed (an acquire load invalidates the L2 on every try); the
// wait ends with one acquire fence.
__device__ __forceinline__ uint32_t load_relaxed_sys(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void acquire_sys() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, ""); }

// Every thread fences its own payload stores at system scope before the
// block barrier, then one thread bumps the counter with a release store.
__device__ __forceinline__ void publish_bump(uint32_t* d_seq) {
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t cur = __hip_atomic_load(d_seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        store_release_sys(d_seq, cur + 1u);
    }
}

__global__ void __launch_bounds__(128)
doorbell_ring_kernel(uint32_t* d_seq, volatile uint32_t* d_ids, volatile float* d_w,
                     const uint32_t* src_ids, const float* src_w, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        d_ids[i] = src_ids[i];
        d_w[i] = src_w[i];
    }
    publish_bump(d_seq);
}

__global__ void __launch_bounds__(128)
doorbell_copy_f32_kernel(uint32_t* d_seq, volatile float* d_dst, const float* src, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) d_dst[i] = src[i];
    publish_bump(d_seq);
}

__global__ void __launch_bounds__(128)
doorbell_wait_copy_f32_kernel(const uint32_t* d_seq, uint32_t target, const volatile float* d_payload,
                              int64_t slot_off, uint32_t* d_consumed, float* dst, int n,
                              uint64_t limit_ticks) {
    __shared__ int ok;
    if (threadIdx.x == 0) {
        const uint64_t t0 = wall_clock64();
        int reached = 1;
        while (load_relaxed_sys(d_seq) < target) {
            if (wall_clock64() - t0 > limit_ticks) {
                reached = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (!reached) atomicAdd(&g_doorbell_timeouts, 1u);
        ok = reached;
    }
    __syncthreads();
    if (!ok) return;
    __threadfence_system();
    for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] = d_payload[slot_off + i];
    __threadfence_system();
    __syncthreads();
    // Every read of the slot has retired; the host may overwrite it.
    if (threadIdx.x == 0) store_release_sys(d_consumed, target);
}

// The persistent-wave doorbell: one wave answers `count` host rings in a row.
// For ring i it waits (bounded) until *d_seq >= first + i, then stores first + i
// to *d_ack (system scope; the wave writes nothing else, so the store needs no
// release fence, which would write back the L2 on every ring).  A wait that runs
// past its limit counts a timeout and ends the kernel, so the wave always exits.
__global__ void __launch_bounds__(64)
doorbell_poll_serve_kernel(const uint32_t* d_seq, uint32_t* d_ack, uint32_t first, uint32_t count,
                           uint64_t limit_ticks) {
    if (threadIdx.x != 0) return;
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t target = first + i;
        const uint64_t t0 = wall_clock64();
        while (load_relaxed_sys(d_seq) < target) {
            if (wall_clock64() - t0 > limit_ticks) {
                atomicAdd(&g_doorbell_timeouts, 1u);
                return;
            }
        }
        acquire_sys();
        __hip_atomic_store(d_ack, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// A stream-ordered wait on a flag another stream (or the host) raises: one
// wave spins (bounded) until *d_flag >= target; the kernels queued after it on
// the stream start once it exits.
__global__ void __launch_bounds__(64)
doorbell_poll_wait_kernel(const uint32_t* d_flag, uint32_t target, uint64_t limit_ticks) {
    if (threadIdx.x != 0) return;
    const uint64_t t0 = wall_clock64();
    while (load_relaxed_sys(d_flag) < target) {
        if (wall_clock64() - t0 > limit_ticks) {
            atomicAdd(&g_doorbell_timeouts, 1u);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    acquire_sys();
}

// Raise *d_flag to value once the work queued before it on the stream is done.
// Stream order starts this kernel after that work has completed, and each kernel's
// writes are released when it ends, so the store needs no fence of its own (a
// system-scope fence writes back the L2: ~2.5 us).
__global__ void __launch_bounds__(64) doorbell_poll_signal_kernel(uint32_t* d_flag, uint32_t value) {
    if (threadIdx.x != 0) return;
    __hip_atomic_store(d_flag, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

} // namespace

// The bound of the device-side doorbell waits, in wall-clock ticks (for other
// kernels of the library that wait on a doorbell word).
uint64_t naiwa_doorbell_wait_limit_ticks() { return wait_limit_ticks(); }
uint64_t naiwa_wall_ticks_ms(uint64_t ms) { return ms * (uint64_t)wall_clock_khz_current(); }

extern "C" {

int doorbell_poll_serve(void* d_seq, void* d_ack, uint32_t first, uint32_t count, int64_t stream) {
    if (!d_seq || !d_ack) return NAIWA_E_INVALID;
    if (count == 0) return NAIWA_OK;
    doorbell_poll_serve_kernel<<<1, 64, 0, (hipStream_t)stream>>>((const uint32_t*)d_seq, (uint32_t*)d_ack,
                                                                   first, count, wait_limit_ticks());
    return naiwa_hip_rc(hipGetLastError());
}

int doorbell_poll_wait(const void* d_flag, uint32_t target, int64_t stream) {
    if (!d_flag) return NAIWA_E_INVALID;
    doorbell_poll_wait_kernel<<<1, 64, 0, (hipStream_t)stream>>>((const uint32_t*)d_flag, target,
                                                                  wait_limit_ticks());
    return naiwa_hip_rc(hipGetLastError());
}

int doorbell_poll_signal(void* d_flag, uint32_t value, int64_t stream) {
    if (!d_flag) return NAIWA_E_INVALID;
    doorbell_poll_signal_kernel<<<1, 64, 0, (hipStream_t)stream>>>((uint32_t*)d_flag, value);
    return naiwa_hip_rc(hipGetLastError());
}

int doorbell_alloc_mapped(void** out, size_t bytes) {
    if (!out) return NAIWA_E_INVALID;
    *out = nullptr;
    hipError_t e = hipHostMalloc(out, bytes ? bytes : 1,
                                 hipHostMallocMapped | hipHostMallocCoherent | hipHostMallocPortable);
    if (e != hipSuccess) {
        *out = nullptr;
        return (int)e;
    }
    std::memset(*out, 0, bytes);
    return NAIWA_OK;
}

int doorbell_free_host(void* p) { return naiwa_hip_rc(hipHostFree(p)); }

void doorbell_get_device_ptr(void* host, void** dev) {
    if (!dev) return;
    *dev = nullptr;
    void* d = nullptr;
    if (hipHostGetDevicePointer(&d, host, 0) == hipSuccess) *dev = d;
}

void doorbell_ring(void* d_seq, void* d_ids, void* d_weights, const void* src_ids,
                   const void* src_weights, int n, int64_t stream) {
    doorbell_ring_kernel<<<1, 128, 0, (hipStream_t)stream>>>(
        (uint32_t*)d_seq, (volatile uint32_t*)d_ids, (volatile float*)d_weights,
        (const uint32_t*)src_ids, (const float*)src_weights, n > 0 ? n : 0);
}

void doorbell_copy_f32(void* d_seq, void* d_dst, const void* src, int n, int64_t stream) {
    doorbell_copy_f32_kernel<<<1, 128, 0, (hipStream_t)stream>>>(
        (uint32_t*)d_seq, (volatile float*)d_dst, (const float*)src, n > 0 ? n : 0);
}

void doorbell_wait_copy_f32(void* d_seq, uint32_t target, void* d_payload, int64_t slot_off,
                            void* d_consumed, void* dst, int n, int64_t stream) {
    doorbell_wait_copy_f32_kernel<<<1, 128, 0, (hipStream_t)stream>>>(
        (const uint32_t*)d_seq, target, (const volatile float*)d_payload, slot_off,
        (uint32_t*)d_consumed, (float*)dst, n > 0 ? n : 0, wait_limit_ticks());
}

int naiwa_doorbell_set_wait_limit_us(uint64_t us) {
    g_wait_limit_us.store(us ? us : 10ull * 1000 * 1000, std::memory_order_relaxed);
    return NAIWA_OK;
}

int naiwa_doorbell_timeouts(uint32_t* count) {
    if (!count) return NAIWA_E_INVALID;
    return naiwa_hip_rc(hipMemcpyFromSymbol(count, HIP_SYMBOL(g_doorbell_timeouts), sizeof(uint32_t), 0,
                                            hipMemcpyDeviceToHost));
}

void naiwa_host_store_release_u32(void* word, uint32_t value) {
    std::atomic_thread_fence(std::memory_order_release);
    *(volatile uint32_t*)word = value;
}

uint32_t naiwa_host_load_acquire_u32(const void* word) {
    const uint32_t v = *(const volatile uint32_t*)word;
    std::atomic_thread_fence(std::memory_order_acquire);
    return v;
}

// src/doorbell/mapped.rs:116-141: spin briefly, then sleep-poll.
int naiwa_host_wait_ge(const void* word, uint32_t target, int64_t timeout_us, int64_t poll_us) {
    using clock = std::chrono::steady_clock;
    const auto deadline = clock::now() + std::chrono::microseconds(timeout_us < 0 ? 0 : timeout_us);
    uint32_t spins = 0;
    for (;;) {
        if (naiwa_host_load_acquire_u32(word) >= target) return NAIWA_OK;
        if (timeout_us >= 0 && clock::now() >= deadline) return NAIWA_E_TIMEOUT;
        if (spins < 2000) {
            ++spins;
#if defined(__x86_64__)
            __builtin_ia32_pause();
#endif
        } else {
            std::this_thread::sleep_for(std::chrono::microseconds(poll_us > 0 ? poll_us : 50));
        }
    }
}

} // extern "C"
