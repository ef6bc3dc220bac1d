// Shared device/host helpers of the gfx950 MoE expert path.
//
// Block formats are the public GGML layouts:
//   Q8_0: { fp16 d; int8 qs[32]; }                               34 B / 32 values
//   Q4_K: { fp16 d; fp16 dmin; u8 scales[12]; u8 qs[128]; }     144 B / 256 values
// Q4_K chunk c (64 values) takes its low nibbles from qs[32c..32c+32) with
// sub-block 2c and its high nibbles from the same bytes with sub-block 2c+1.
//
// Dot products never dequantize to f32.  A 4-bit code q becomes the bf16
// number 128 + q by OR-ing 0x4300 into its 16-bit lane, an int8 code q becomes
// the fp16 number 1152 + q by flipping its sign bit and OR-ing 0x6400, and
// v_dot2_f32_{bf16,f16} multiplies two such codes by two activations and
// accumulates in f32.  The constant offset times the activation sum is
// subtracted once per sub-block, so a 16-byte load of codes costs ~1.5 VALU
// operations per weight instead of ~4 for an f32 dequantize + fma.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/naiwa_moe.h"

// Loads through an explicit address space: AS 1 = global, 3 = LDS, 0 =
// generic.  Pointers that come out of LDS-resident descriptors are generic to
// the compiler, and generic (flat) accesses wait on both memory counters.
#define NAIWA_AS_GLOBAL 1
#define NAIWA_AS_LDS 3
// 16-byte types (uint4, float4: class types whose copy constructor would take
// a generic reference) are loaded as a native 4 x u32 vector.
template <class T, int AS>
__device__ __forceinline__ T naiwa_ld(const void* p) {
    if constexpr (sizeof(T) == 16) {
        typedef unsigned int v4u __attribute__((ext_vector_type(4)));
        v4u v;
        if constexpr (AS == NAIWA_AS_GLOBAL) v = *(const __attribute__((address_space(1))) v4u*)p;
        else if constexpr (AS == NAIWA_AS_LDS) v = *(const __attribute__((address_space(3))) v4u*)p;
        else v = *(const v4u*)p;
        T out;
        __builtin_memcpy(&out, &v, 16);
        return out;
    } else {
        if constexpr (AS == NAIWA_AS_GLOBAL) return *(const __attribute__((address_space(1))) T*)p;
        else if constexpr (AS == NAIWA_AS_LDS) return *(const __attribute__((address_space(3))) T*)p;
        else return *(const T*)p;
    }
}

#define NAIWA_QK8_0 32
#define NAIWA_QK_K 256
#define NAIWA_Q8_0_BYTES 34
#define NAIWA_Q4_K_BYTES 144

typedef __bf16 naiwa_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 naiwa_f16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------
static inline int naiwa_hip_rc(hipError_t e) { return e == hipSuccess ? NAIWA_OK : (int)e; }

__host__ __device__ static inline int64_t naiwa_row_bytes(int dtype, int64_t k) {
    switch (dtype) {
    case NAIWA_Q8_0: return k % NAIWA_QK8_0 ? -1 : (k / NAIWA_QK8_0) * NAIWA_Q8_0_BYTES;
    case NAIWA_Q4_K: return k % NAIWA_QK_K ? -1 : (k / NAIWA_QK_K) * NAIWA_Q4_K_BYTES;
    case NAIWA_F32: return k * 4;
    case NAIWA_F16: case NAIWA_BF16: return k * 2;
    default: return -1;
    }
}

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float naiwa_bf16_to_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }

__device__ __forceinline__ uint32_t naiwa_f32_to_bf16(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (x >> 16) | 0x40u;
    x += 0x7fffu + ((x >> 16) & 1u);
    return x >> 16;
}

__device__ __forceinline__ float naiwa_f16_to_f32(uint32_t h16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)h16);
    return (float)h;
}

__device__ __forceinline__ uint32_t naiwa_f32_to_f16(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float naiwa_dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(naiwa_bf16x2, a),
                                           __builtin_bit_cast(naiwa_bf16x2, b), c, false);
}

__device__ __forceinline__ float naiwa_dot2_f16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(naiwa_f16x2, a),
                                  __builtin_bit_cast(naiwa_f16x2, b), c, false);
}

// One DPP lane move (no LDS round trip): quad permutations and the 8/16-lane
// mirrors.
template <int CTRL>
__device__ __forceinline__ float naiwa_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of W lanes (a power of two <= 64), result in every
// lane of the group.  Up to 16 lanes the steps are DPP moves within a row
// (xor 1, xor 2, then the 8- and 16-lane mirrors); every lane ends with the
// same bits because each step adds the same two values in either order.
template <int W>
__device__ __forceinline__ float naiwa_group_sum(float v) {
    if (W >= 2) v += naiwa_dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    if (W >= 4) v += naiwa_dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    if (W >= 8) v += naiwa_dpp<0x141>(v);  // row_half_mirror
    if (W >= 16) v += naiwa_dpp<0x140>(v); // row_mirror
#pragma unroll
    for (int m = 16; m < W; m <<= 1) v += __shfl_xor(v, m, W);
    return v;
}

template <int CTRL>
__device__ __forceinline__ long long naiwa_dpp_i64(long long v) {
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(v & 0xffffffffll), CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(v >> 32), CTRL, 0xF, 0xF, false);
    return (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

// Exact int64 sum over aligned groups of 16 lanes (DPP), result in every lane.
__device__ __forceinline__ long long naiwa_group_sum16_i64(long long v) {
    v += naiwa_dpp_i64<0xB1>(v);
    v += naiwa_dpp_i64<0x4E>(v);
    v += naiwa_dpp_i64<0x141>(v);
    v += naiwa_dpp_i64<0x140>(v);
    return v;
}

__device__ __forceinline__ float naiwa_silu(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ float naiwa_gelu_tanh(float g) {
    const float k0 = 0.7978845608028654f, k1 = 0.044715f;
    return 0.5f * g * (1.0f + tanhf(k0 * (g + k1 * g * g * g)));
}

__device__ __forceinline__ float naiwa_act(int act, float g) {
    return act == NAIWA_ACT_GELU_PYTORCH_TANH ? naiwa_gelu_tanh(g) : naiwa_silu(g);
}

// ---------------------------------------------------------------------------
// Activation layouts for the dot kernels.
//
// "perm" words: activation pairs in the order the code unpacking produces
// them: word 2i = (x[4i], x[4i+2]), word 2i+1 = (x[4i+1], x[4i+3]), low half
// first.  Q4_K rows use bf16 pairs and sums over 16 values; Q8_0 rows use
// fp16 pairs and sums over 32 values.  Each sum is the sum of the rounded
// values that the dot products see.
// ---------------------------------------------------------------------------

// Q4_K: one 16-byte slice of codes (unit j = 0..7 of a block) against its 32
// activations.  `q` holds qs[16j..16j+16), `hd` the block's first 16 bytes
// (d, dmin, scales).  The unit covers elements 64c + 16h + [0,16) with
// sub-block 2c and the same +32 with sub-block 2c+1 (c = j/2, h = j%2).
// xlo/xhi are the 8 perm words of those two 16-element runs, slo/shi their sums.
// Two Q4_K nibbles (bits 0-3 and 16-19 of q) as the bf16 pair (128 + n0, 128 + n1):
// (q & 0x000F000F) | 0x43004300 in one v_and_or_b32, with the mask held in a
// VGPR and the exponent bits in an SGPR (a gfx9 VOP3 takes no literal and reads
// at most one SGPR; with both as literals it takes two instructions).
struct NaiwaNib {
    uint32_t mask, magic;
};
__device__ __forceinline__ NaiwaNib naiwa_nib_consts() {
    uint32_t m = 0x000F000Fu, g = 0x43004300u;
    asm volatile("" : "+v"(m));
    asm volatile("" : "+s"(g));
    return {m, g};
}
__device__ __forceinline__ uint32_t naiwa_nib(uint32_t q, const NaiwaNib& c) { return (q & c.mask) | c.magic; }

__device__ __forceinline__ float naiwa_q4k_unit(uint4 q, uint4 hd, int c, const uint32_t* xlo,
                                                const uint32_t* xhi, float slo, float shi) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    const NaiwaNib nc = naiwa_nib_consts();
    float alo = 0.0f, ahi = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a0 = naiwa_nib(w[i], nc);
        const uint32_t a1 = naiwa_nib(w[i] >> 8, nc);
        const uint32_t b0 = naiwa_nib(w[i] >> 4, nc);
        const uint32_t b1 = naiwa_nib(w[i] >> 12, nc);
        alo = naiwa_dot2_bf16(a0, xlo[2 * i], alo);
        alo = naiwa_dot2_bf16(a1, xlo[2 * i + 1], alo);
        ahi = naiwa_dot2_bf16(b0, xhi[2 * i], ahi);
        ahi = naiwa_dot2_bf16(b1, xhi[2 * i + 1], ahi);
    }
    // 6-bit scales / mins of sub-blocks 2c and 2c+1 (ggml get_scale_min_k4).
    const int sh = (c & 1) * 16;
    const uint32_t A = hd.y >> sh;  // s[2c'], s[2c'+1]      (c' = c mod 2)
    const uint32_t B = hd.z >> sh;  // s[4+2c'], s[5+2c']
    const uint32_t Cw = hd.w >> sh; // s[8+2c'], s[9+2c']
    uint32_t sc0, sc1, m0, m1;
    if (c < 2) {
        sc0 = A & 63u;
        sc1 = (A >> 8) & 63u;
        m0 = B & 63u;
        m1 = (B >> 8) & 63u;
    } else {
        sc0 = (Cw & 0xFu) | (((A >> 6) & 3u) << 4);
        sc1 = ((Cw >> 8) & 0xFu) | (((A >> 14) & 3u) << 4);
        m0 = ((Cw >> 4) & 0xFu) | (((B >> 6) & 3u) << 4);
        m1 = ((Cw >> 12) & 0xFu) | (((B >> 14) & 3u) << 4);
    }
    const float d = naiwa_f16_to_f32(hd.x & 0xffffu);
    const float dmin = naiwa_f16_to_f32(hd.x >> 16);
    // every multiply-add is an explicit fma or stays apart, so no kernel that inlines
    // this gets a different contraction (and different bits) than another
    const float qlo = __builtin_fmaf(-128.0f, slo, alo); // sum q * x over the low run
    const float qhi = __builtin_fmaf(-128.0f, shi, ahi);
    const float sq = __builtin_fmaf((float)sc0, qlo, (float)sc1 * qhi);
    const float mm = __builtin_fmaf((float)m0, slo, (float)m1 * shi);
    return __builtin_fmaf(d, sq, -(dmin * mm));
}

// Q8_0: a pair of blocks (68 bytes = 17 dwords, 4-byte aligned because every
// row holds an even number of blocks) against its 64 activations.
// xw: 32 fp16 perm words; s0/s1: sums of the two 32-element halves.
__device__ __forceinline__ float naiwa_q8_0_pair(const uint32_t* D, const uint32_t* xw, float s0,
                                                 float s1) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // block 0 codes start at byte 2: realign two dwords
        const uint32_t w = __builtin_amdgcn_alignbyte(D[i + 1], D[i], 2) ^ 0x80808080u;
        const uint32_t p0 = (w & 0x00FF00FFu) | 0x64006400u;
        const uint32_t p1 = ((w >> 8) & 0x00FF00FFu) | 0x64006400u;
        a0 = naiwa_dot2_f16(p0, xw[2 * i], a0);
        a0 = naiwa_dot2_f16(p1, xw[2 * i + 1], a0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t w = D[9 + i] ^ 0x80808080u;
        const uint32_t p0 = (w & 0x00FF00FFu) | 0x64006400u;
        const uint32_t p1 = ((w >> 8) & 0x00FF00FFu) | 0x64006400u;
        a1 = naiwa_dot2_f16(p0, xw[16 + 2 * i], a1);
        a1 = naiwa_dot2_f16(p1, xw[16 + 2 * i + 1], a1);
    }
    const float d0 = naiwa_f16_to_f32(D[0] & 0xffffu);
    const float d1 = naiwa_f16_to_f32(D[8] >> 16);
    // explicit fmas: the same bits in every kernel that inlines this
    const float t0 = __builtin_fmaf(-1152.0f, s0, a0), t1 = __builtin_fmaf(-1152.0f, s1, a1);
    return __builtin_fmaf(d0, t0, d1 * t1);
}

// The bound of the device-side doorbell waits in wall-clock ticks (doorbell.hip;
// naiwa_doorbell_set_wait_limit_us sets it).
uint64_t naiwa_doorbell_wait_limit_ticks();
// Wall-clock ticks (s_memrealtime) in `ms` milliseconds on the current device, for
// bounds on waits between the workgroups of one launch (not the doorbell bound).
uint64_t naiwa_wall_ticks_ms(uint64_t ms);
