// Synthetic expert weights and activations generated on the device.
//
// A Qwen3-30B-A3B-shaped stack is 16 GB of Q4_K bytes; generating and
// quantizing it on the host would take minutes, so the benchmark draws its
// N(mean, std) values with a counter-based generator here and quantizes them
// in place.  Value i of a stream depends only on (seed, offset + i): a
// SplitMix64-mixed counter pair feeds Box-Muller in f64 (cosine branch for
// even i, sine for odd).  The quantizers are the library's own: Q8_0 as ggml
// (amax / 127, round half away from zero), Q4_K with an affine [min(0, lo),
// hi] range on 15 steps per 32-value sub-block and 6-bit scales and mins
// relative to the super-block maximum.
#include "common.h"

namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// The two values of counter pair p (even index = cosine, odd = sine).
__device__ __forceinline__ void normal_pair(uint64_t key, uint64_t p, float mean, float stdv, float* v0,
                                            float* v1) {
    const uint64_t a = mix64(key ^ mix64(2 * p));
    const uint64_t b = mix64(key ^ mix64(2 * p + 1));
    const double u1 = ((double)(a >> 11) + 1.0) * 0x1p-53;
    const double u2 = (double)(b >> 11) * 0x1p-53;
    const double r = sqrt(-2.0 * log(u1));
    const double t = 6.283185307179586 * u2;
    *v0 = (float)((double)mean + (double)stdv * (r * cos(t)));
    *v1 = (float)((double)mean + (double)stdv * (r * sin(t)));
}

__device__ __forceinline__ float normal_at(uint64_t key, uint64_t idx, float mean, float stdv) {
    float a, b;
    normal_pair(key, idx >> 1, mean, stdv, &a, &b);
    return (idx & 1) ? b : a;
}

__global__ void synth_f32_kernel(uint64_t key, uint64_t offset, int64_t n, float mean, float stdv,
                                 float* out, int to_bf16) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = normal_at(key, offset + (uint64_t)i, mean, stdv);
    if (to_bf16)
        reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)naiwa_f32_to_bf16(v);
    else
        out[i] = v;
}

// One thread per Q8_0 block.
__global__ void synth_q8_0_kernel(uint64_t key, uint64_t offset, int64_t nblocks, float mean,
                                  float stdv, uint8_t* out) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    float x[32];
    const uint64_t base = offset + (uint64_t)b * 32;
    for (int j = 0; j < 32; ++j) x[j] = normal_at(key, base + j, mean, stdv);
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t* ob = out + b * NAIWA_Q8_0_BYTES;
    const uint32_t dh = naiwa_f32_to_f16(d);
    ob[0] = (uint8_t)(dh & 0xff);
    ob[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 32; ++j) {
        float v = roundf(x[j] * id);
        v = fminf(127.0f, fmaxf(-128.0f, v));
        ob[2 + j] = (uint8_t)(int8_t)v;
    }
}

// One wave per Q4_K block: lane l holds values 4l..4l+3 (sub-block l/8).
__global__ void __launch_bounds__(64)
synth_q4_k_kernel(uint64_t key, uint64_t offset, int64_t nblocks, float mean, float stdv,
                  uint8_t* out) {
    const int64_t b = blockIdx.x;
    if (b >= nblocks) return;
    const int lane = threadIdx.x;
    const uint64_t base = offset + (uint64_t)b * 256 + 4 * lane;
    float x[4];
    normal_pair(key, base >> 1, mean, stdv, &x[0], &x[1]);
    normal_pair(key, (base >> 1) + 1, mean, stdv, &x[2], &x[3]);
    // sub-block range over 8 lanes
    float lo = fminf(fminf(x[0], x[1]), fminf(x[2], x[3]));
    float hi = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    for (int m = 1; m < 8; m <<= 1) {
        lo = fminf(lo, __shfl_xor(lo, m, 64));
        hi = fmaxf(hi, __shfl_xor(hi, m, 64));
    }
    if (lo > 0.0f) lo = 0.0f;
    const float scale = (hi - lo) / 15.0f;
    const float minv = -lo;
    float max_scale = scale, max_min = minv;
    for (int m = 8; m < 64; m <<= 1) {
        max_scale = fmaxf(max_scale, __shfl_xor(max_scale, m, 64));
        max_min = fmaxf(max_min, __shfl_xor(max_min, m, 64));
    }
    const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    const int ls = min(63, max(0, (int)__builtin_rintf(inv_scale * scale)));
    const int lm = min(63, max(0, (int)__builtin_rintf(inv_min * minv)));
    const uint32_t dh = naiwa_f32_to_f16(max_scale / 63.0f);
    const uint32_t mh = naiwa_f32_to_f16(max_min / 63.0f);
    const float d = naiwa_f16_to_f32(dh), dmin = naiwa_f16_to_f32(mh);
    const float dj = d * (float)ls;
    const float mj = dmin * (float)lm;
    int q[4];
    for (int i = 0; i < 4; ++i) {
        int v = 0;
        if (dj != 0.0f) v = (int)__builtin_rintf((x[i] + mj) / dj);
        q[i] = v < 0 ? 0 : (v > 15 ? 15 : v);
    }
    uint8_t* ob = out + b * NAIWA_Q4_K_BYTES;
    // scales: lane 8j carries (ls, lm) of sub-block j
    int sc[8], mm[8];
    for (int s = 0; s < 8; ++s) {
        sc[s] = __shfl(ls, 8 * s, 64);
        mm[s] = __shfl(lm, 8 * s, 64);
    }
    if (lane == 0) {
        uint8_t s12[12] = {0};
        for (int s = 0; s < 8; ++s) {
            if (s < 4) {
                s12[s] = (uint8_t)sc[s];
                s12[s + 4] = (uint8_t)mm[s];
            } else {
                s12[s + 4] = (uint8_t)((sc[s] & 0xF) | ((mm[s] & 0xF) << 4));
                s12[s - 4] |= (uint8_t)((sc[s] >> 4) << 6);
                s12[s] |= (uint8_t)((mm[s] >> 4) << 6);
            }
        }
        ob[0] = (uint8_t)(dh & 0xff);
        ob[1] = (uint8_t)(dh >> 8);
        ob[2] = (uint8_t)(mh & 0xff);
        ob[3] = (uint8_t)(mh >> 8);
        for (int s = 0; s < 12; ++s) ob[4 + s] = s12[s];
    }
    // nibbles: values 64c + l (l < 32) pair with 64c + 32 + l, held 8 lanes up
    int partner[4];
    for (int i = 0; i < 4; ++i) partner[i] = __shfl(q[i], (lane + 8) & 63, 64);
    const int c = lane >> 4, lin = lane & 15;
    if (lin < 8) {
        for (int i = 0; i < 4; ++i)
            ob[16 + 32 * c + 4 * lin + i] = (uint8_t)(q[i] | (partner[i] << 4));
    }
}

uint64_t host_mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

} // namespace

// Fill `out` with n values of the N(mean, std) stream (seed, offset), as f32,
// bf16, Q8_0 or Q4_K bytes.  n must be a multiple of the block size.
extern "C" int naiwa_synth(int dtype, uint64_t seed, uint64_t offset, int64_t n, float mean,
                           float stdv, void* out, int64_t stream) {
    if (n < 0 || !out) return NAIWA_E_INVALID;
    if (n == 0) return NAIWA_OK;
    const uint64_t key = host_mix64(seed ^ 0xD1B54A32D192ED03ull);
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
    case NAIWA_F32:
    case NAIWA_BF16: {
        const int64_t grid = (n + 255) / 256;
        synth_f32_kernel<<<dim3((unsigned)grid), 256, 0, st>>>(key, offset, n, mean, stdv, (float*)out,
                                                               dtype == NAIWA_BF16);
        break;
    }
    case NAIWA_Q8_0: {
        if (n % NAIWA_QK8_0) return NAIWA_E_INVALID;
        const int64_t nb = n / NAIWA_QK8_0;
        synth_q8_0_kernel<<<dim3((unsigned)((nb + 255) / 256)), 256, 0, st>>>(key, offset, nb, mean, stdv,
                                                                             (uint8_t*)out);
        break;
    }
    case NAIWA_Q4_K: {
        if (n % NAIWA_QK_K || (offset & 1)) return NAIWA_E_INVALID;
        const int64_t nb = n / NAIWA_QK_K;
        if (nb > 0x7fffffff) return NAIWA_E_INVALID;
        synth_q4_k_kernel<<<dim3((unsigned)nb), 64, 0, st>>>(key, offset, nb, mean, stdv, (uint8_t*)out);
        break;
    }
    default:
        return NAIWA_E_UNSUPPORTED;
    }
    return naiwa_hip_rc(hipGetLastError());
}
