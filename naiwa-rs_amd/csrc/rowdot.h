// Row-dot building blocks shared by the decode kernels and the fused stack
// kernel: per-format unit loads, activation staging into LDS, and the dot of
// one quantized row against one staged activation vector by a group of 16
// lanes.
#pragma once

#include "common.h"

#define NAIWA_GROUP 16 // lanes cooperating on one weight row

// A staged activation vector in LDS: perm words [K/2] followed by sums.
// Q4_K: bf16 words, one sum per 16 values.  Q8_0: fp16 words, one per 32.
template <int DT> struct Fmt;

template <> struct Fmt<NAIWA_Q4_K> {
    static constexpr int kSumSpan = 16;
    struct Frag {
        uint4 q, hd;
    };
    __host__ __device__ static int units(int k) { return (k / NAIWA_QK_K) * 8; }
    template <int AS = 0>
    __device__ __forceinline__ static Frag load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (u >> 3) * NAIWA_Q4_K_BYTES;
        Frag f;
        f.hd = naiwa_ld<uint4, AS>(blk);
        f.q = naiwa_ld<uint4, AS>(blk + 16 + 16 * (u & 7));
        return f;
    }
    // words: perm words of the vector (K/2), sums: K/16 sums
    __device__ __forceinline__ static float dot(const Frag& f, int u, const uint32_t* words, const float* sums) {
        const int j = u & 7, c = j >> 1;
        const int elo = (u >> 3) * NAIWA_QK_K + 64 * c + 16 * (j & 1);
        const uint4* xl = reinterpret_cast<const uint4*>(words + elo / 2);
        const uint4* xh = reinterpret_cast<const uint4*>(words + elo / 2 + 16);
        uint32_t lo[8], hi[8];
        const uint4 l0 = xl[0], l1 = xl[1], h0 = xh[0], h1 = xh[1];
        lo[0] = l0.x; lo[1] = l0.y; lo[2] = l0.z; lo[3] = l0.w;
        lo[4] = l1.x; lo[5] = l1.y; lo[6] = l1.z; lo[7] = l1.w;
        hi[0] = h0.x; hi[1] = h0.y; hi[2] = h0.z; hi[3] = h0.w;
        hi[4] = h1.x; hi[5] = h1.y; hi[6] = h1.z; hi[7] = h1.w;
        return naiwa_q4k_unit(f.q, f.hd, c, lo, hi, sums[elo / 16], sums[elo / 16 + 2]);
    }
    __device__ static uint32_t to16(float v) { return naiwa_f32_to_bf16(v); }
    __device__ static float from16(uint32_t h) { return naiwa_bf16_to_f32(h); }
};

template <> struct Fmt<NAIWA_Q8_0> {
    static constexpr int kSumSpan = 32;
    struct Frag {
        uint32_t d[17];
    };
    __host__ __device__ static int units(int k) { return k / (2 * NAIWA_QK8_0); }
    template <int AS = 0>
    __device__ __forceinline__ static Frag load(const uint8_t* row, int u) {
        const uint8_t* p = row + 68 * u;
        Frag f;
#pragma unroll
        for (int i = 0; i < 17; ++i) f.d[i] = naiwa_ld<uint32_t, AS>(p + 4 * i);
        return f;
    }
    __device__ __forceinline__ static float dot(const Frag& f, int u, const uint32_t* words, const float* sums) {
        uint32_t xw[32];
        const uint4* xv = reinterpret_cast<const uint4*>(words + 32 * u);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint4 v = xv[i];
            xw[4 * i] = v.x; xw[4 * i + 1] = v.y; xw[4 * i + 2] = v.z; xw[4 * i + 3] = v.w;
        }
        return naiwa_q8_0_pair(f.d, xw, sums[2 * u], sums[2 * u + 1]);
    }
    __device__ static uint32_t to16(float v) { return naiwa_f32_to_f16(v); }
    __device__ static float from16(uint32_t h) { return naiwa_f16_to_f32(h); }
};

// Q8_0 rows with an odd number of blocks are only 2-byte aligned: one block per
// unit, its 34 bytes read as 17 halfwords.  Internal format tag.
#define NAIWA_Q8_0_ODD 1008

template <> struct Fmt<NAIWA_Q8_0_ODD> {
    static constexpr int kSumSpan = 32;
    struct Frag {
        uint32_t d;
        uint32_t q[8];
    };
    __host__ __device__ static int units(int k) { return k / NAIWA_QK8_0; }
    template <int AS = 0>
    __device__ __forceinline__ static Frag load(const uint8_t* row, int u) {
        const uint8_t* p = row + NAIWA_Q8_0_BYTES * u;
        Frag f;
        f.d = naiwa_ld<uint16_t, AS>(p);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            f.q[i] = (uint32_t)naiwa_ld<uint16_t, AS>(p + 2 + 4 * i) |
                     ((uint32_t)naiwa_ld<uint16_t, AS>(p + 4 + 4 * i) << 16);
        return f;
    }
    __device__ __forceinline__ static float dot(const Frag& f, int u, const uint32_t* words, const float* sums) {
        // the final multiply never fuses into the caller's add (the same bits in every kernel)
#pragma clang fp contract(off)
        const uint4* xv = reinterpret_cast<const uint4*>(words + 16 * u);
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 v = xv[i];
            const uint32_t xw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t w = f.q[2 * i + h] ^ 0x80808080u;
                a = naiwa_dot2_f16((w & 0x00FF00FFu) | 0x64006400u, xw[2 * h], a);
                a = naiwa_dot2_f16(((w >> 8) & 0x00FF00FFu) | 0x64006400u, xw[2 * h + 1], a);
            }
        }
        return naiwa_f16_to_f32(f.d) * __builtin_fmaf(-1152.0f, sums[u], a);
    }
    __device__ static uint32_t to16(float v) { return naiwa_f32_to_f16(v); }
    __device__ static float from16(uint32_t h) { return naiwa_f16_to_f32(h); }
};

// LDS bytes of one staged vector of length k, rounded up to 16 so that
// consecutive vectors keep 16-byte aligned words.
__host__ __device__ inline int naiwa_stage_bytes(int dtype, int k) {
    const int span = dtype == NAIWA_Q4_K ? 16 : 32; // Q8_0 (either variant): 32
    return (k * 2 + (k / span) * 4 + 15) & ~15;
}

// 8 bytes of activations; device-coherent (bypassing the non-coherent caches)
// when COH, for vectors other blocks of a persistent kernel have just written.
template <bool COH>
__device__ __forceinline__ uint2 naiwa_ld8(const void* p) {
    if (COH) {
        const unsigned long long v =
            __hip_atomic_load((const unsigned long long*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
    }
    return *reinterpret_cast<const uint2*>(p);
}

// Stage `k` activations (f32 source, or bf16 when src_bf16) into the perm
// layout + sums of format DT.  All `nthr` threads of the block take part;
// k % 32 == 0.  The caller synchronizes afterwards.  A thread issues the loads of
// up to kStageRounds of its rounds before converting any, so staging costs one
// memory round trip per kStageRounds rounds instead of one per round.
constexpr int kStageRounds = 4;
template <int DT, bool COH = false>
__device__ inline void naiwa_stage(const void* src, bool src_bf16, int k, uint32_t* words,
                                   float* sums, int tid, int nthr) {
    constexpr int span = Fmt<DT>::kSumSpan;
    constexpr int gpg = span / 4; // 4-element groups per sum
    // Thread handles groups g = tid, tid + nthr, ...; nthr is a multiple of gpg
    // so the lanes summing one span sit in one aligned run of the wave.
    for (int g00 = 0; g00 < k / 4; g00 += kStageRounds * nthr) {
        uint2 raw[kStageRounds][2];
#pragma unroll
        for (int i = 0; i < kStageRounds; ++i) {
            const int g = g00 + i * nthr + tid;
            if (g < k / 4) {
                if (src_bf16) {
                    raw[i][0] = naiwa_ld8<COH>((const uint16_t*)src + 4 * g);
                } else {
                    raw[i][0] = naiwa_ld8<COH>((const float*)src + 4 * g);
                    raw[i][1] = naiwa_ld8<COH>((const float*)src + 4 * g + 2);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < kStageRounds; ++i) {
            if (g00 + i * nthr >= k / 4) break; // uniform: every lane takes the group sums
            const int g = g00 + i * nthr + tid;
            float part = 0.0f;
            if (g < k / 4) {
                float v[4];
                if (src_bf16) {
                    v[0] = naiwa_bf16_to_f32(raw[i][0].x & 0xffffu);
                    v[1] = naiwa_bf16_to_f32(raw[i][0].x >> 16);
                    v[2] = naiwa_bf16_to_f32(raw[i][0].y & 0xffffu);
                    v[3] = naiwa_bf16_to_f32(raw[i][0].y >> 16);
                } else {
                    v[0] = __uint_as_float(raw[i][0].x); v[1] = __uint_as_float(raw[i][0].y);
                    v[2] = __uint_as_float(raw[i][1].x); v[3] = __uint_as_float(raw[i][1].y);
                }
                uint32_t h[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    h[j] = Fmt<DT>::to16(v[j]);
                    v[j] = Fmt<DT>::from16(h[j]);
                }
                words[2 * g] = h[0] | (h[2] << 16);
                words[2 * g + 1] = h[1] | (h[3] << 16);
                part = (v[0] + v[1]) + (v[2] + v[3]);
            }
            part = naiwa_group_sum<gpg>(part);
            if (g < k / 4 && (g % gpg) == 0) sums[g / gpg] = part;
        }
    }
}

// Loads in flight per lane per pass, by format (about 32 VGPRs of codes).
template <int DT> struct Umax { static constexpr int v = 4; };
template <> struct Umax<NAIWA_Q8_0> { static constexpr int v = 2; };
template <> struct Umax<NAIWA_Q8_0_ODD> { static constexpr int v = 4; };

// Kernel format tag of a bank: Q8_0 rows with an odd block count use the
// halfword-loading variant.
__host__ __device__ inline int naiwa_kernel_fmt(int dtype, int k) {
    return dtype == NAIWA_Q8_0 && (k / NAIWA_QK8_0) % 2 ? NAIWA_Q8_0_ODD : dtype;
}
