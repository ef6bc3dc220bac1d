// naiwa_moe_prefill: the routed experts of a prefill chunk (many tokens per
// expert) as grouped GEMMs on the matrix cores -- the counterpart of the fork's
// MoEExperts::forward called from src/prefill_stream.rs:2080-2102.
//
//   1. gather:   (token, k) pairs sorted by slot (stable), offsets per slot;
//   2. tiles:    the sorted pairs cut into tiles of 32 pairs of one slot;
//   3. gate/up:  per (tile, 128 intermediate features): x rows [32, H] times the
//                slot's gate and up rows, K-steps of 128 dequantised to bf16 in
//                LDS, v_mfma_f32_32x32x16_bf16 with f32 accumulation; the
//                epilogue writes h = act(gate) * up as bf16;
//   4. down:     per (tile, 128 output features): h rows [32, I] times the down
//                rows, the epilogue scales by the pair's routing weight and
//                writes the pair's f32 output row;
//   5. combine:  out[t] = sum over j ascending of the pair outputs (no atomics).
//
// MFMA 32x32x16 bf16 operand layout: lane l holds A[l % 32][8 (l / 32) + 0..7]
// and B[8 (l / 32) + 0..7][l % 32]; accumulator v of lane l is D[8 (v / 4) +
// 4 (l / 32) + v % 4][l % 32].
#include "common.h"
#include "workspace.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kTM = 32;          // pairs per tile
constexpr int kTN = 128;         // output features per block (4 waves x 32)
constexpr int kKS = 128;         // K per step
constexpr int kLdsRow = kKS + 8; // bf16 per LDS row (16 bytes of padding)
constexpr int NAIWA_SCRATCH_PREFILL = 5;

struct Tiles {
    int* start; // first sorted position of the tile
    int* count; // pairs in the tile (<= 32)
    int* slot;  // the tile's slot
    int* n;     // number of tiles
};

// Cut the sorted pairs into tiles of <= 32 pairs of one slot.  One block.
__global__ void __launch_bounds__(kThreads) tiles_kernel(const uint32_t* offsets, int slots, Tiles t) {
    __shared__ int part[kThreads + 1];
    const int tid = threadIdx.x;
    const int per = (slots + kThreads - 1) / kThreads;
    const int s0 = min(slots, tid * per), s1 = min(slots, s0 + per);
    int mine = 0;
    for (int s = s0; s < s1; ++s) mine += (int)((offsets[s + 1] - offsets[s] + kTM - 1) / kTM);
    part[tid] = mine;
    __syncthreads();
    if (tid == 0) {
        int acc = 0;
        for (int i = 0; i < kThreads; ++i) {
            const int v = part[i];
            part[i] = acc;
            acc += v;
        }
        part[kThreads] = acc;
        *t.n = acc;
    }
    __syncthreads();
    int at = part[tid];
    for (int s = s0; s < s1; ++s) {
        const int b = (int)offsets[s], n = (int)(offsets[s + 1] - offsets[s]);
        for (int m = 0; m < n; m += kTM, ++at) {
            t.start[at] = b + m;
            t.count[at] = min(kTM, n - m);
            t.slot[at] = s;
        }
    }
}

// Dequantise K-step [k0, k0 + 128) of one weight row into 128 bf16 at dst (LDS).
template <int DT>
__device__ inline void dequant_step(const uint8_t* row, int k0, __bf16* dst);

template <>
__device__ inline void dequant_step<NAIWA_Q4_K>(const uint8_t* row, int k0, __bf16* dst) {
    const uint8_t* blk = row + (k0 / NAIWA_QK_K) * NAIWA_Q4_K_BYTES;
    const uint4 hd = *reinterpret_cast<const uint4*>(blk);
    const float d = naiwa_f16_to_f32(hd.x & 0xffffu), dmin = naiwa_f16_to_f32(hd.x >> 16);
    auto sc = [&](int j) -> int { // scale byte j (0..11): bytes 4..15 of the header
        const uint32_t wd = j < 4 ? hd.y : (j < 8 ? hd.z : hd.w);
        return (int)((wd >> (8 * (j & 3))) & 0xFFu);
    };
    const int c0 = ((k0 / 128) & 1) * 2;                             // first 64-value chunk of the step
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
        const int c = c0 + cc;
        // sub-blocks 2c (low nibbles) and 2c + 1 (high nibbles): ggml get_scale_min_k4
        float scale[2], mn[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int j = 2 * c + h;
            int s, m;
            if (j < 4) {
                s = sc(j) & 63;
                m = sc(j + 4) & 63;
            } else {
                s = (sc(j + 4) & 0xF) | ((sc(j - 4) >> 6) << 4);
                m = (sc(j + 4) >> 4) | ((sc(j) >> 6) << 4);
            }
            scale[h] = d * (float)s;
            mn[h] = dmin * (float)m;
        }
        const uint4* q = reinterpret_cast<const uint4*>(blk + 16 + 32 * c);
        const uint4 qa = q[0], qb = q[1];
        const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        __bf16 lo[32], hi[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const uint32_t byte = (w[i / 4] >> (8 * (i % 4))) & 0xFFu;
            lo[i] = (__bf16)(scale[0] * (float)(byte & 0xF) - mn[0]);
            hi[i] = (__bf16)(scale[1] * (float)(byte >> 4) - mn[1]);
        }
        __bf16* o = dst + 64 * cc;
#pragma unroll
        for (int i = 0; i < 32; i += 8) {
            *reinterpret_cast<bf16x8*>(o + i) = *reinterpret_cast<const bf16x8*>(lo + i);
            *reinterpret_cast<bf16x8*>(o + 32 + i) = *reinterpret_cast<const bf16x8*>(hi + i);
        }
    }
}

template <>
__device__ inline void dequant_step<NAIWA_Q8_0>(const uint8_t* row, int k0, __bf16* dst) {
    // 4 blocks of {fp16 d, int8 q[32]}, 136 bytes, 4-byte aligned (k0 is a multiple of 128)
    const uint32_t* p = reinterpret_cast<const uint32_t*>(row + (k0 / NAIWA_QK8_0) * NAIWA_Q8_0_BYTES);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        // block b is bytes [34 b, 34 b + 34): halfword-aligned, covered by the 9 aligned
        // words from 34 b / 4 (never past the 136 bytes of the step)
        uint32_t wds[9];
        const int w0 = (34 * b) / 4, sh = ((34 * b) % 4) * 8;
#pragma unroll
        for (int i = 0; i < 9; ++i) wds[i] = p[w0 + i];
        auto byte_at = [&](int i) -> uint32_t { // byte i of the block (0..33)
            const int bit = sh + 8 * i;
            return (wds[bit / 32] >> (bit % 32)) & 0xFFu;
        };
        const float d = naiwa_f16_to_f32(byte_at(0) | (byte_at(1) << 8));
        __bf16 v[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = (__bf16)(d * (float)(int8_t)byte_at(2 + i));
#pragma unroll
        for (int i = 0; i < 32; i += 8)
            *reinterpret_cast<bf16x8*>(dst + 32 * b + i) = *reinterpret_cast<const bf16x8*>(v + i);
    }
}

struct Bank {
    const uint8_t* base;
    int64_t stride;
    int64_t row_bytes;
};

// gate/up: one tile of <= 32 pairs x 128 intermediate features.
template <int DG>
__global__ void __launch_bounds__(kThreads)
gateup_kernel(Bank gate, Bank up, const uint16_t* x, int H, int I, int k, const uint32_t* perm, Tiles tl,
              int act, uint16_t* hbuf) {
    __shared__ __align__(16) __bf16 xs[kTM][kLdsRow];
    __shared__ __align__(16) __bf16 wg[kTN][kLdsRow];
    __shared__ __align__(16) __bf16 wu[kTN][kLdsRow];
    const int tile = blockIdx.y;
    if (tile >= *tl.n) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int start = tl.start[tile], cnt = tl.count[tile], slot = tl.slot[tile];
    const int n0 = blockIdx.x * kTN;
    const uint8_t* grow0 = gate.base + (int64_t)slot * gate.stride + (int64_t)n0 * gate.row_bytes;
    const uint8_t* urow0 = up.base + (int64_t)slot * up.stride + (int64_t)n0 * up.row_bytes;
    floatx16 accg = {}, accu = {};
    for (int k0 = 0; k0 < H; k0 += kKS) {
        __syncthreads(); // the previous step's MFMAs read the tiles
        // activations: 32 rows x 128 bf16, 16 bytes per thread per pass (2 passes)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int v = tid + kThreads * i, r = v / 16, c = (v % 16) * 8;
            uint4 val = make_uint4(0u, 0u, 0u, 0u);
            if (r < cnt) {
                const int t = (int)perm[start + r] / k;
                val = *reinterpret_cast<const uint4*>(x + (size_t)t * H + k0 + c);
            }
            *reinterpret_cast<uint4*>(&xs[r][c]) = val;
        }
        // weights: thread < 128 dequantises gate row n0 + tid, the others up row n0 + tid - 128
        if (tid < kTN) dequant_step<DG>(grow0 + (int64_t)tid * gate.row_bytes, k0, &wg[tid][0]);
        else dequant_step<DG>(urow0 + (int64_t)(tid - kTN) * up.row_bytes, k0, &wu[tid - kTN][0]);
        __syncthreads();
        const int r = lane % 32, kh = 8 * (lane / 32), n = 32 * wave + lane % 32;
#pragma unroll
        for (int kk = 0; kk < kKS; kk += 16) {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(&xs[r][kk + kh]);
            const bf16x8 bg = *reinterpret_cast<const bf16x8*>(&wg[n][kk + kh]);
            const bf16x8 bu = *reinterpret_cast<const bf16x8*>(&wu[n][kk + kh]);
            accg = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bg, accg, 0, 0, 0);
            accu = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bu, accu, 0, 0, 0);
        }
    }
    // epilogue: h = act(g) * u as bf16, rows of the tile's sorted positions
    const int col = n0 + 32 * wave + lane % 32;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int m = 8 * (v / 4) + 4 * (lane / 32) + v % 4;
        if (m < cnt) hbuf[(size_t)(start + m) * I + col] = (uint16_t)naiwa_f32_to_bf16(naiwa_act(act, accg[v]) * accu[v]);
    }
}

// down: one tile of <= 32 pairs x 128 output features; pair rows scaled by their weight.
template <int DD>
__global__ void __launch_bounds__(kThreads)
down_kernel(Bank down, const uint16_t* hbuf, int H, int I, const uint32_t* perm, const float* w, Tiles tl,
            float* ypair) {
    __shared__ __align__(16) __bf16 hs[kTM][kLdsRow];
    __shared__ __align__(16) __bf16 wd[kTN][kLdsRow];
    const int tile = blockIdx.y;
    if (tile >= *tl.n) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int start = tl.start[tile], cnt = tl.count[tile], slot = tl.slot[tile];
    const int n0 = blockIdx.x * kTN;
    const uint8_t* drow0 = down.base + (int64_t)slot * down.stride + (int64_t)n0 * down.row_bytes;
    floatx16 acc = {};
    for (int k0 = 0; k0 < I; k0 += kKS) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int v = tid + kThreads * i, r = v / 16, c = (v % 16) * 8;
            uint4 val = make_uint4(0u, 0u, 0u, 0u);
            if (r < cnt) val = *reinterpret_cast<const uint4*>(hbuf + (size_t)(start + r) * I + k0 + c);
            *reinterpret_cast<uint4*>(&hs[r][c]) = val;
        }
        if (tid < kTN) dequant_step<DD>(drow0 + (int64_t)tid * down.row_bytes, k0, &wd[tid][0]);
        __syncthreads();
        const int r = lane % 32, kh = 8 * (lane / 32), n = 32 * wave + lane % 32;
#pragma unroll
        for (int kk = 0; kk < kKS; kk += 16) {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(&hs[r][kk + kh]);
            const bf16x8 b = *reinterpret_cast<const bf16x8*>(&wd[n][kk + kh]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
        }
    }
    const int col = n0 + 32 * wave + lane % 32;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int m = 8 * (v / 4) + 4 * (lane / 32) + v % 4;
        if (m < cnt) {
            const uint32_t p = perm[start + m];
            ypair[(size_t)p * H + col] = acc[v] * w[p];
        }
    }
}

// out[t] = sum over j = 0..k-1 of the pair rows whose slot id is valid.
__global__ void __launch_bounds__(kThreads)
combine_kernel(const float* ypair, const uint32_t* ids, int k, int H, int slots, int accumulate, float* out) {
    const int t = blockIdx.x;
    for (int c = threadIdx.x; c < H; c += kThreads) {
        float y = accumulate ? out[(size_t)t * H + c] : 0.0f;
        for (int j = 0; j < k; ++j)
            if (ids[(size_t)t * k + j] < (uint32_t)slots) y += ypair[((size_t)t * k + j) * H + c];
        out[(size_t)t * H + c] = y;
    }
}

bool fmt_ok(int dtype, int kdim) {
    return (dtype == NAIWA_Q4_K && kdim % NAIWA_QK_K == 0) || (dtype == NAIWA_Q8_0 && kdim % kKS == 0);
}

} // namespace

extern "C" int naiwa_moe_prefill(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, const void* x,
                                 const uint32_t* slot_ids, const float* w, int T, int k, int act, float* out,
                                 int flags, int64_t stream) {
    if (!gate || !up || !down || T < 0 || k <= 0 || (flags & ~NAIWA_PREFILL_ACCUMULATE)) return NAIWA_E_INVALID;
    if (T == 0) return NAIWA_OK;
    if (!x || !slot_ids || !w || !out) return NAIWA_E_INVALID;
    const int H = gate->k, I = gate->n, slots = gate->slots;
    if (up->k != H || up->n != I || down->n != H || down->k != I || up->slots != slots || down->slots != slots)
        return NAIWA_E_INVALID;
    if (gate->dtype != up->dtype || !fmt_ok(gate->dtype, H) || !fmt_ok(down->dtype, I)) return NAIWA_E_UNSUPPORTED;
    if (H % kTN || I % kTN || H % kKS || I % kKS) return NAIWA_E_UNSUPPORTED;
    if (act != NAIWA_ACT_SILU && act != NAIWA_ACT_GELU_PYTORCH_TANH) return NAIWA_E_UNSUPPORTED;
    const int64_t n = (int64_t)T * k;
    if (n > 65536 || slots <= 0 || slots > 4096) return NAIWA_E_UNSUPPORTED;
    const int64_t rbg = naiwa_row_bytes(gate->dtype, H), rbd = naiwa_row_bytes(down->dtype, I);
    if (gate->slot_stride < rbg * I || up->slot_stride < rbg * I || down->slot_stride < rbd * H) return NAIWA_E_INVALID;
    if (((uintptr_t)gate->base | (uintptr_t)up->base | (uintptr_t)down->base | gate->slot_stride | up->slot_stride |
         down->slot_stride | (uintptr_t)x) & 15)
        return NAIWA_E_INVALID;
    if (gate->dtype == NAIWA_Q4_K && (rbg % 16)) return NAIWA_E_INVALID;

    // scratch: perm [n] | offsets [slots + 1] | bad | tiles 3 x max + n | h bf16 [n, I] | ypair f32 [n, H]
    const int64_t max_tiles = (n + kTM - 1) / kTM + slots;
    auto a256 = [](size_t b) { return (b + 255) & ~size_t(255); };
    const size_t o_perm = 0, o_off = a256(o_perm + (size_t)n * 4), o_bad = a256(o_off + (size_t)(slots + 1) * 4);
    const size_t o_tiles = a256(o_bad + 4), o_h = a256(o_tiles + (size_t)(3 * max_tiles + 1) * 4);
    const size_t o_y = a256(o_h + (size_t)n * I * 2), total = a256(o_y + (size_t)n * H * 4);
    int rc = 0;
    uint8_t* ws = (uint8_t*)naiwa_scratch(NAIWA_SCRATCH_PREFILL, total, &rc);
    if (!ws) return rc;
    uint32_t* perm = (uint32_t*)(ws + o_perm);
    uint32_t* offsets = (uint32_t*)(ws + o_off);
    Tiles tl;
    tl.start = (int*)(ws + o_tiles);
    tl.count = tl.start + max_tiles;
    tl.slot = tl.count + max_tiles;
    tl.n = tl.slot + max_tiles;
    uint16_t* hbuf = (uint16_t*)(ws + o_h);
    float* ypair = (float*)(ws + o_y);
    hipStream_t st = (hipStream_t)stream;

    if ((rc = naiwa_moe_gather(slot_ids, (int)n, slots, perm, offsets, (int*)(ws + o_bad), stream))) return rc;
    tiles_kernel<<<1, kThreads, 0, st>>>(offsets, slots, tl);
    const Bank bg{(const uint8_t*)gate->base, gate->slot_stride, rbg}, bu{(const uint8_t*)up->base, up->slot_stride, rbg};
    const Bank bd{(const uint8_t*)down->base, down->slot_stride, rbd};
    const dim3 g1(I / kTN, (unsigned)max_tiles), g2(H / kTN, (unsigned)max_tiles);
    if (gate->dtype == NAIWA_Q4_K)
        gateup_kernel<NAIWA_Q4_K><<<g1, kThreads, 0, st>>>(bg, bu, (const uint16_t*)x, H, I, k, perm, tl, act, hbuf);
    else
        gateup_kernel<NAIWA_Q8_0><<<g1, kThreads, 0, st>>>(bg, bu, (const uint16_t*)x, H, I, k, perm, tl, act, hbuf);
    if (down->dtype == NAIWA_Q4_K)
        down_kernel<NAIWA_Q4_K><<<g2, kThreads, 0, st>>>(bd, hbuf, H, I, perm, w, tl, ypair);
    else
        down_kernel<NAIWA_Q8_0><<<g2, kThreads, 0, st>>>(bd, hbuf, H, I, perm, w, tl, ypair);
    combine_kernel<<<T, kThreads, 0, st>>>(ypair, slot_ids, k, H, slots, (flags & NAIWA_PREFILL_ACCUMULATE) ? 1 : 0,
                                           out);
    return naiwa_hip_rc(hipGetLastError());
}
