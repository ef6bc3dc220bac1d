// Per-device grow-only scratch memory of the library's own entry points.
//
// The reference's fork allocates its decode workspace per call
// (docs/worklogs/m1.md:21-33); here each device keeps one buffer that only
// grows, so steady-state decode steps allocate nothing.  One GPU-submitting
// thread per device is assumed (the reference's token-thread rule,
// src/moe/decode.rs:17-19); calls from several threads on one device are
// serialized by the mutex only around the allocation, not the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <mutex>
#include <stddef.h>

struct NaiwaScratch {
    void* ptr = nullptr;
    size_t bytes = 0;
};

// Returns a device pointer of at least `bytes` for (device, tag), growing the
// buffer (with a device sync, since a kernel may still read the old one).
void* naiwa_scratch(int tag, size_t bytes, int* rc);
// As above; *fresh tells whether this call (re)allocated the buffer, whose
// contents are then undefined.
void* naiwa_scratch(int tag, size_t bytes, int* rc, bool* fresh);

// One buffer per user: a buffer shared by two entry points would let one overwrite what
// the other keeps there between calls (the fused kernel's tagged exchange words are only
// cleared when they are known to be dirty).
enum {
    NAIWA_SCRATCH_DECODE = 0,
    NAIWA_SCRATCH_ROUTER = 1,
    NAIWA_SCRATCH_STACK = 2,        // layered stack: per-layer routing and outputs
    NAIWA_SCRATCH_FUSED = 3,        // fused stack: tagged exchange words
    NAIWA_SCRATCH_FUSED_STATUS = 4, // fused stack: status counters
    NAIWA_SCRATCH_FUSED_TRACE = 5,  // fused stack: phase timestamps
    NAIWA_SCRATCH_FUSED_TOKENS = 6, // fused stack: per-launch outputs of two-launch steps
    NAIWA_SCRATCH_PREFILL = 7,
    NAIWA_SCRATCH_TAGS = 8
};
