// Internal entry points of the decode kernels for the library's own drivers.
#pragma once

#include "../../include/naiwa_moe.h"

// naiwa_moe_decode of bf16 x [rows, H] followed by x = bf16(x + y), x updated in place:
// the residual is folded into the ordered combine when the call takes the staged paths
// (y, f32 [rows, H], is then written only with keep_y), else it goes through y and a
// residual launch.  The same bits either way.
int naiwa_moe_decode_residual(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, void* x,
                              const uint32_t* slot_ids, const float* w, int rows, int width, int act, float* y,
                              int keep_y, int64_t stream);
