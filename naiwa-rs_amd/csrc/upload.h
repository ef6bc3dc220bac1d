// Internal: the pieces of naiwa_copy_batch for callers that map their host
// ranges once (the cached layer's pinned expert stacks) and then queue
// batches of device views without per-call pointer lookups.
#pragma once

#include "../../include/naiwa_moe.h"

// The device address of [p, p + bytes) when it lies in pinned host memory
// mapped for the device (both ends checked), else null.
const void* naiwa_device_view(const void* p, size_t bytes);
// naiwa_copy_batch over sources that are already device views.
int naiwa_copy_batch_mapped(const naiwa_copy* items, int n, int64_t stream);
