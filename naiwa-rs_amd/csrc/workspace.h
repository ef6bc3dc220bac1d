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

enum { NAIWA_SCRATCH_DECODE = 0, NAIWA_SCRATCH_ROUTER = 1, NAIWA_SCRATCH_STACK = 2, NAIWA_SCRATCH_TAGS = 6 };
