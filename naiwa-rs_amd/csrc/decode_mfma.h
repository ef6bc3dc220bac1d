// The expert GEMMs of naiwa_moe_decode calls with several tokens per expert, on
// the matrix cores (prefill.hip): x -> bf16 in the 16x16x32 K order, gate/up per
// (64 features, slot segment), down per (64 rows, K part, slot segment) into
// unweighted partial dots that the decode's ordered combine adds up.
#pragma once

#include "common.h"

// Whether the call's formats and shapes fit the matrix-core decode.
bool naiwa_decode_mfma_ok(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, const void* x);

// Scratch bytes of its bf16 x [rows, H] and h [n, I].
size_t naiwa_decode_mfma_bytes(int rows, int n, int H, int I);

// The launches: ws holds naiwa_decode_mfma_bytes bytes; dpart receives K parts of
// ks values of I: dpart[(part * n + sorted position) * H + row].
int naiwa_decode_mfma_experts(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, const void* x,
                              int x_dtype, int rows, int width, int act, int n, int seg_bound, int ks,
                              const int* seg_count, const uint32_t* seg_key, const uint32_t* seg_begin,
                              const uint32_t* perm, uint8_t* ws, float* dpart, hipStream_t st);
