// naiwa_stack_decode: a whole decode step through every MoE layer of a model,
// x <- bf16(x + MoE_l(x)), with routing kept on the device.
//
// NAIWA_STACK_LAYERED chains the standalone entry points (router top-k,
// slot lookup, naiwa_moe_decode, residual) per layer.
#include "decode.h"
#include "router.h"
#include "rowdot.h"
#include "workspace.h"

namespace {

__global__ void residual_kernel(uint16_t* x, const float* y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = (uint16_t)naiwa_f32_to_bf16(naiwa_bf16_to_f32(x[i]) + y[i]);
}

// ids [n] expert ids -> slots via the layer's table; a missing expert (-1)
// gets weight 0 so the decode skips it.
__global__ void slot_map_kernel(const uint32_t* ids, const float* w, const int32_t* slot_of, int E,
                                int n, uint32_t* slots, float* wout) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t e = ids[i];
    const int32_t s = e < (uint32_t)E ? slot_of[e] : -1;
    slots[i] = s < 0 ? 0u : (uint32_t)s;
    wout[i] = s < 0 ? 0.0f : w[i];
}

} // namespace

extern "C" int naiwa_residual_add_bf16(void* x, const float* y, int64_t n, int64_t stream) {
    if (n < 0 || (n > 0 && (!x || !y))) return NAIWA_E_INVALID;
    if (n == 0) return NAIWA_OK;
    residual_kernel<<<dim3((unsigned)((n + 255) / 256)), 256, 0, (hipStream_t)stream>>>(
        (uint16_t*)x, y, n);
    return naiwa_hip_rc(hipGetLastError());
}

int naiwa_stack_fused(const naiwa_layer* layers, int n_layers, void* x, int rows, int H, int E, int k,
                      int mode, int act, uint32_t* ids_out, float* w_out, float* y_out, int64_t stream);

extern "C" int naiwa_stack_decode(const naiwa_layer* layers, int n_layers, void* x, int rows, int H,
                                  int E, int k, int mode, int act, uint32_t* ids_out, float* w_out,
                                  int flags, int64_t stream) {
    return naiwa_stack_decode_y(layers, n_layers, x, rows, H, E, k, mode, act, ids_out, w_out, nullptr, flags,
                                stream);
}

extern "C" int naiwa_stack_decode_y(const naiwa_layer* layers, int n_layers, void* x, int rows, int H,
                                    int E, int k, int mode, int act, uint32_t* ids_out, float* w_out,
                                    float* y_out, int flags, int64_t stream) {
    if (!layers || n_layers < 0 || !x || rows < 0 || H <= 0 || E <= 0 || k <= 0 || k > E)
        return NAIWA_E_INVALID;
    if (rows == 0 || n_layers == 0) return NAIWA_OK;
    if (flags == NAIWA_STACK_FUSED)
        return naiwa_stack_fused(layers, n_layers, x, rows, H, E, k, mode, act, ids_out, w_out, y_out, stream);
    if (flags != NAIWA_STACK_LAYERED) return NAIWA_E_UNSUPPORTED;
    hipStream_t st = (hipStream_t)stream;
    const int n = rows * k;
    // scratch: ids, w, slots, w_mapped (n each) | y [rows * H] f32
    const size_t seg = ((size_t)n * 4 + 255) & ~size_t(255);
    int rc = 0;
    uint8_t* ws = (uint8_t*)naiwa_scratch(NAIWA_SCRATCH_STACK, 4 * seg + (size_t)rows * H * 4, &rc);
    if (!ws) return rc;
    uint32_t* ids_tmp = (uint32_t*)ws;
    float* w_tmp = (float*)(ws + seg);
    uint32_t* slots = (uint32_t*)(ws + 2 * seg);
    float* w_mapped = (float*)(ws + 3 * seg);
    float* y = (float*)(ws + 4 * seg);
    for (int l = 0; l < n_layers; ++l) {
        const naiwa_layer& L = layers[l];
        uint32_t* ids = ids_out ? ids_out + (size_t)l * n : ids_tmp;
        float* w = w_out ? w_out + (size_t)l * n : w_tmp;
        if ((rc = naiwa_router_topk(x, NAIWA_BF16, L.router, rows, H, E, k, mode, ids, w, nullptr, stream)))
            return rc;
        const uint32_t* dec_ids = ids;
        const float* dec_w = w;
        if (L.slot_of_expert) {
            slot_map_kernel<<<(n + 255) / 256, 256, 0, st>>>(ids, w, L.slot_of_expert, E, n, slots, w_mapped);
            dec_ids = slots;
            dec_w = w_mapped;
        }
        if (!y_out) {
            // the residual in the decode's ordered combine where it can be (one launch fewer)
            if ((rc = naiwa_moe_decode_residual(&L.gate, &L.up, &L.down, x, dec_ids, dec_w, rows, k, act, y, 0,
                                                stream)))
                return rc;
            continue;
        }
        if ((rc = naiwa_moe_decode(&L.gate, &L.up, &L.down, x, NAIWA_BF16, dec_ids, dec_w, rows, k, act, y,
                                   stream)))
            return rc;
        if ((rc = naiwa_hip_rc(hipMemcpyAsync(y_out + (size_t)l * rows * H, y, (size_t)rows * H * 4,
                                              hipMemcpyDeviceToDevice, st))))
            return rc;
        if ((rc = naiwa_residual_add_bf16(x, y, (int64_t)rows * H, stream))) return rc;
    }
    return naiwa_hip_rc(hipGetLastError());
}
