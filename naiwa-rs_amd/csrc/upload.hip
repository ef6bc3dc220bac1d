// Batched host -> device uploads: every range of a layer's staged experts in
// one kernel launch that reads the pinned host stacks through their device
// mapping, instead of one DMA copy per projection (each with its own
// submission and completion on the copy stream).  The reference queues one
// copy per projection on its CopyStream (src/copy_stream.rs:387-409); the
// ranges, their order on the stream and the fences around them are the same.
#include "common.h"
#include "upload.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 4;     // 16-byte loads in flight per thread
constexpr int kBlocksPerRange = 16; // more loads in flight measured slower over PCIe
constexpr uint64_t kMaxRangeBytes = uint64_t(1) << 34; // 16 GiB: unit indices stay far below 2^32

// The ranges travel as kernel arguments, sized to the batch: a launch's host cost grows
// with its argument bytes (~3.1 us with a few, ~4.4 us with all 64 ranges' 1.5 KB).
template <int CAP> struct CopyArgs {
    naiwa_copy c[CAP];
    int n;
};

// blockIdx.y = range; the blocks of a range stride over its 16-byte units,
// each thread with kCopyUnroll loads issued before its stores.
template <int CAP>
__global__ void __launch_bounds__(kCopyThreads) copy_batch_kernel(CopyArgs<CAP> a) {
    const int r = blockIdx.y;
    if (r >= a.n) return;
    const u32x4* src = reinterpret_cast<const u32x4*>(a.c[r].src);
    u32x4* dst = reinterpret_cast<u32x4*>(a.c[r].dst);
    // 32-bit unit indices (ranges are at most kMaxRangeBytes): 26 VGPRs instead of 36, so
    // that a wave fits on a SIMD beside three waves of the staged gate/up kernels that
    // wait for this copy (up to 160 VGPRs each)
    const uint32_t n16 = (uint32_t)(a.c[r].bytes / 16);
    const uint32_t step = gridDim.x * kCopyThreads;
    for (uint32_t i0 = blockIdx.x * kCopyThreads + threadIdx.x; i0 < n16; i0 += step * kCopyUnroll) {
        u32x4 v[kCopyUnroll];
#pragma unroll
        for (int u = 0; u < kCopyUnroll; ++u)
            if (i0 + u * step < n16) v[u] = src[i0 + u * step];
#pragma unroll
        for (int u = 0; u < kCopyUnroll; ++u)
            if (i0 + u * step < n16) dst[i0 + u * step] = v[u];
    }
}

// Attributes of p; a pointer the runtime does not know (pageable memory) is
// an error there, which is cleared so that it does not surface at a later call.
bool pointer_attributes(hipPointerAttribute_t* a, const void* p) {
    if (hipPointerGetAttributes(a, p) == hipSuccess) return true;
    (void)hipGetLastError();
    return false;
}

} // namespace

// The device address of [p, p + bytes) when it lies in pinned host memory
// mapped for the device (checked at both ends), else null.
const void* naiwa_device_view(const void* p, size_t bytes) {
    if (!p || !bytes) return nullptr;
    hipPointerAttribute_t a{}, b{};
    if (!pointer_attributes(&a, p) || a.type != hipMemoryTypeHost || !a.devicePointer || !a.hostPointer)
        return nullptr;
    const uint8_t* last = (const uint8_t*)p + bytes - 1;
    if (!pointer_attributes(&b, last) || b.type != hipMemoryTypeHost || !b.devicePointer || !b.hostPointer)
        return nullptr;
    const ptrdiff_t off = (const uint8_t*)p - (const uint8_t*)a.hostPointer;
    const ptrdiff_t offb = last - (const uint8_t*)b.hostPointer;
    const uint8_t* dp = (const uint8_t*)a.devicePointer + off;
    // both ends in one mapping: the device view of the last byte follows from the first
    if ((const uint8_t*)b.devicePointer + offb != dp + bytes - 1) return nullptr;
    return dp;
}

namespace {
template <int CAP> int copy_launch(const naiwa_copy* c, int m, hipStream_t st) {
    CopyArgs<CAP> a{};
    for (int i = 0; i < m; ++i) a.c[i] = c[i];
    a.n = m;
    copy_batch_kernel<CAP><<<dim3(kBlocksPerRange, m), kCopyThreads, 0, st>>>(a);
    return naiwa_hip_rc(hipGetLastError());
}
} // namespace

int naiwa_copy_batch_mapped(const naiwa_copy* items, int n, int64_t stream) {
    if (n < 0 || n > NAIWA_COPY_BATCH_MAX || (n > 0 && !items)) return NAIWA_E_INVALID;
    naiwa_copy c[NAIWA_COPY_BATCH_MAX];
    int m = 0;
    for (int i = 0; i < n; ++i) {
        const naiwa_copy& it = items[i];
        if (!it.bytes) continue;
        if (!it.dst || !it.src) return NAIWA_E_INVALID;
        if (((uintptr_t)it.dst | (uintptr_t)it.src | (uintptr_t)it.bytes) & 15) return NAIWA_E_UNSUPPORTED;
        if ((uint64_t)it.bytes > kMaxRangeBytes) return NAIWA_E_UNSUPPORTED;
        c[m++] = it;
    }
    if (!m) return NAIWA_OK;
    const hipStream_t st = (hipStream_t)stream;
    if (m <= 4) return copy_launch<4>(c, m, st);
    if (m <= 16) return copy_launch<16>(c, m, st);
    return copy_launch<NAIWA_COPY_BATCH_MAX>(c, m, st);
}

int naiwa_copy_batch(const naiwa_copy* items, int n, int64_t stream) {
    if (n < 0 || n > NAIWA_COPY_BATCH_MAX || (n > 0 && !items)) return NAIWA_E_INVALID;
    naiwa_copy mapped[NAIWA_COPY_BATCH_MAX];
    for (int i = 0; i < n; ++i) {
        mapped[i] = items[i];
        if (!items[i].bytes) continue;
        if (!items[i].dst || !items[i].src) return NAIWA_E_INVALID;
        const void* dv = naiwa_device_view(items[i].src, (size_t)items[i].bytes);
        if (!dv) return NAIWA_E_UNSUPPORTED; // not pinned and mapped: the caller copies another way
        mapped[i].src = dv;
    }
    return naiwa_copy_batch_mapped(mapped, n, stream);
}
