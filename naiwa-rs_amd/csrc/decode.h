// Internal entry points of the decode kernels for the library's own drivers.
#pragma once

#include "../../include/naiwa_moe.h"

// naiwa_moe_decode of bf16 x [rows, H] followed by x = bf16(x + y), x updated in place:
// the residual is folded into the ordered combine when the call takes the staged paths
// (y, f32 [rows, H], is then written only with keep_y), else it goes through y and a
// residual launch.  The same bits either way.
// wait: see naiwa_decode_wait.
struct naiwa_decode_wait;
int naiwa_moe_decode_residual(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, void* x,
                              const uint32_t* slot_ids, const float* w, int rows, int width, int act, float* y,
                              int keep_y, int64_t stream, const naiwa_decode_wait* wait = nullptr);

// A wait on a word that another stream raises (the staged uploads' flag), folded into a
// decode call: no kernel of the call reads expert rows before *flag >= target.  The
// one-token gate/up blocks wait themselves, after their segmentation and activation
// staging (work that overlaps the uploads), else one wave waits before the call's
// kernels.  A wait that runs past limit_ticks adds one to *fail (mapped host memory,
// read by the host) and the call goes on: its output is then invalid, and known to be.
struct naiwa_decode_wait {
    const uint32_t* flag;
    uint32_t target;
    uint64_t limit_ticks;
    uint32_t* fail;
};

// naiwa_moe_decode with a folded wait (see naiwa_decode_wait).
int naiwa_moe_decode_wait(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, const void* x,
                          int x_dtype, const uint32_t* slot_ids, const float* w, int rows, int width, int act,
                          float* out, int64_t stream, const naiwa_decode_wait* wait);
