// naiwa_moe_prefill: the routed experts of a prefill chunk (many tokens per
// expert) as grouped GEMMs on the matrix cores -- the counterpart of the fork's
// MoEExperts::forward called from src/prefill_stream.rs:2080-2102.
//
//   1. gather:   (token, k) pairs sorted by slot (stable), offsets per slot;
//   2. tiles:    the sorted pairs cut into tiles of 64 pairs of one slot;
//   3. prep:     x (bf16) laid out once in the K order of the gate/up weight
//                format (below);
//   4. gate/up:  per (tile, 128 intermediate features): 64 x rows times the
//                slot's gate and up rows with v_mfma_f32_32x32x16_bf16; every
//                lane dequantises its own weight values in f32 and rounds them
//                once to bf16, straight into the MFMA B operand; the epilogue
//                writes h = act(gate) * up as bf16 in the K order of the down
//                format;
//   5. down:     per (tile, 128 output features): h rows times the down rows,
//                scaled by the pair's routing weight into the pair's f32 row;
//   6. combine:  out[t] = sum over j ascending of the pair rows (no atomics).
//
// MFMA 32x32x16 operand layout: lane l holds A[l % 32][8 (l / 32) + 0..7] and
// B[8 (l / 32) + 0..7][l % 32]; accumulator v of lane l is D[8 (v / 4) +
// 4 (l / 32) + v % 4][l % 32].
//
// K order.  A dot product may visit K in any order as long as A and B agree,
// so each format fixes the order its blocks unpack fastest in.  The K dimension
// is cut into K-blocks (Q4_K: one 256-value block; Q8_0: four 32-value blocks,
// 128 values); MFMA step s of a K-block takes 8 values from each lane half h
// (lanes 0-31: h = 0, lanes 32-63: h = 1), a "run" of 8 consecutive values of
// the row, in the order the lane's unpacking yields them:
//   Q4_K: step s = 4c + t reads, in 64-value chunk c, the bytes 16h + 8 (t % 2)
//         + 0..7 of the chunk's 32 quant bytes, low nibbles for t < 2 and high
//         ones for t >= 2: run r = 8c + 4 (t / 2) + 2h + t % 2, elements in
//         byte order 0 2 1 3 4 6 5 7 (one mask-and-or unpacks bytes 0 and 2);
//   Q8_0: step s = 4j + u reads block b = 2j + h, its values 8u + 0..7:
//         run r = 4b + u, elements in order.
// The activations (x for gate/up, h for down) are stored as groups g = 2s + h
// of 8 bf16 in that order, so the A operand of a step is one 16-byte read.
// bf16 operands carry the f32 exponent range: any finite activation goes in
// without clamping or scaling.
#include "common.h"
#include "decode_mfma.h"
#include "workspace.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // gather helpers, prep, combine
constexpr int kGemm = 512;     // GEMM blocks: 8 waves, one 32-feature weight strip each
constexpr int kTM = 64;        // pairs per tile: two 32-row MFMA subtiles
constexpr int kTNG = 128;      // gate/up features per block (waves 0-3 gate, 4-7 up)
constexpr int kTND = 256;      // down output features per block

// Two f32 values rounded to nearest-even bf16 (v_cvt_pk_bf16_f32), as one word.
__device__ __forceinline__ uint32_t bf16x2_bits(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{a, b}, bf16x2));
}
// Eight f32 values as the bf16 MFMA operand.
__device__ __forceinline__ bf16x8 to_bf16x8(const float (&f)[8]) {
    const u32x4 w = {bf16x2_bits(f[0], f[1]), bf16x2_bits(f[2], f[3]), bf16x2_bits(f[4], f[5]),
                     bf16x2_bits(f[6], f[7])};
    return __builtin_bit_cast(bf16x8, w);
}

template <int DT> struct KBlock;
template <> struct KBlock<NAIWA_Q4_K> {
    static constexpr int kVals = 256, kSteps = 16;
};
template <> struct KBlock<NAIWA_Q8_0> {
    static constexpr int kVals = 128, kSteps = 8;
};

// Element i of a laid-out Q4_K run holds byte q4_elem(i) of the run (an involution).
__host__ __device__ constexpr int q4_elem(int i) { return (i == 1 || i == 2 || i == 5 || i == 6) ? (i ^ 3) : i; }

// The group (2s + h) that holds run r of a K-block.
template <int DT>
__host__ __device__ inline int group_of_run(int r) {
    if (DT == NAIWA_Q4_K) {
        const int c = r / 8, q = r % 8;
        const int t = 2 * (q / 4) + (q % 2), h = (q / 2) % 2;
        return 2 * (4 * c + t) + h;
    } else {
        const int b = r / 4, u = r % 4;
        return 2 * (4 * (b / 2) + u) + (b % 2);
    }
}

// Position, in the laid-out row, of value f of the original row.
template <int DT>
__host__ __device__ inline int laid_pos(int f) {
    constexpr int KV = KBlock<DT>::kVals;
    const int kb = f / KV, r = (f % KV) / 8, e = f % 8;
    return kb * KV + 8 * group_of_run<DT>(r) + (DT == NAIWA_Q4_K ? q4_elem(e) : e);
}

struct Tiles {
    int* start; // first sorted position of the tile
    int* count; // pairs in the tile (<= kTM)
    int* slot;  // the tile's slot
    int* n;     // number of tiles
};

// The (tile, column block) of GEMM block b; false for a block with none.  The grid
// holds ncol * (max tiles rounded up to 8) blocks.
//  - plain order (xcd = 0): block b is column b % ncol of tile b / ncol;
//  - XCD order (xcd = 1): workgroups are dealt to the 8 XCDs round-robin (block b
//    runs on XCD b % 8), and each XCD takes a contiguous range of the tiles (sorted by
//    slot, so an expert's tiles are neighbours), all column blocks of a tile one after
//    the other: the blocks that read a tile's activation rows share one L2, and so do
//    those that read the weight strips of an expert with few tiles.
// Either mapping covers every (tile, column) once, wherever blocks actually run.
__device__ __forceinline__ bool tile_col(int b, int ntiles, int ncol, int xcd, int* tile, int* col) {
    if (!xcd) {
        *tile = b / ncol;
        *col = b % ncol;
        return *tile < ntiles;
    }
    const int x = b & 7, r = b >> 3;
    const int t0 = ntiles * x / 8, t1 = ntiles * (x + 1) / 8;
    if (r >= (t1 - t0) * ncol) return false;
    *tile = t0 + r / ncol;
    *col = r % ncol;
    return true;
}

// Cut the sorted pairs into tiles of <= kTM pairs of one slot.  One block.
__device__ inline void tiles_block(const uint32_t* offsets, int slots, Tiles t) {
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

// One word of two 16-bit values: element e0 (low half) and element e1 (high half)
// of the 8 values held in w (two a word, low half first).
__device__ __forceinline__ uint32_t pick16(const uint32_t (&w)[4], int e0, int e1) {
    const uint32_t a = (w[e0 >> 1] >> (16 * (e0 & 1))) & 0xffffu;
    const uint32_t b = (w[e1 >> 1] >> (16 * (e1 & 1))) & 0xffffu;
    return a | (b << 16);
}

// x bf16 [T, H] -> xp bf16 [T, H] in the K order of DT (the values unchanged, only
// placed).  One thread per run of 8 values.
template <int DT>
__device__ inline void prep_block(const uint16_t* x, int T, int H, uint16_t* xp, int block) {
    const int runs = H / 8;
    const int64_t i = (int64_t)block * kThreads + threadIdx.x;
    if (i >= (int64_t)T * runs) return;
    const int t = (int)(i / runs), run = (int)(i % runs);
    const uint4 v = *reinterpret_cast<const uint4*>(x + (size_t)t * H + 8 * run);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    auto el = [](int e) { return DT == NAIWA_Q4_K ? q4_elem(e) : e; };
    const int dst = laid_pos<DT>(8 * run); // the run's group (its element 0 is byte 0)
    uint4 o;
    o.x = pick16(w, el(0), el(1));
    o.y = pick16(w, el(2), el(3));
    o.z = pick16(w, el(4), el(5));
    o.w = pick16(w, el(6), el(7));
    *reinterpret_cast<uint4*>(xp + (size_t)t * H + dst) = o;
}

// The placed activations (every block but the last) and the tile list (the last block)
// in one launch: the two do not depend on each other.
template <int DT>
__global__ void __launch_bounds__(kThreads) prep_tiles_kernel(const uint16_t* x, int T, int H, uint16_t* xp,
                                                              const uint32_t* offsets, int slots, Tiles t) {
    if (blockIdx.x == gridDim.x - 1)
        tiles_block(offsets, slots, t);
    else
        prep_block<DT>(x, T, H, xp, blockIdx.x);
}

// (d * scale, -dmin * min) of 32-value sub-block j of a Q4_K block whose first 16
// bytes are hd (ggml's get_scale_min_k4), exact in f32 (an f16 times a 6-bit integer).
__device__ __forceinline__ void q4k_scale_min(const u32x4& hd, int j, float& sc, float& mn) {
    const uint32_t s3[3] = {hd.y, hd.z, hd.w};
    auto sb = [&](int i) -> int { return (int)((s3[i >> 2] >> (8 * (i & 3))) & 0xFFu); };
    int s, m;
    if (j < 4) {
        s = sb(j) & 63;
        m = sb(j + 4) & 63;
    } else {
        s = (sb(j + 4) & 0xF) | ((sb(j - 4) >> 6) << 4);
        m = (sb(j + 4) >> 4) | ((sb(j) >> 6) << 4);
    }
    sc = naiwa_f16_to_f32(hd.x & 0xffffu) * (float)s;
    mn = -(naiwa_f16_to_f32(hd.x >> 16) * (float)m);
}

// Nibble masks held in registers.  A nibble masked into the mantissa of an f16 magic
// number reads as magic + q exactly: a low nibble (bits 0-3) in 1024.0 (0x6400), a
// high one left at bits 4-7 in 64.0 (0x5400).  With the mask in a VGPR,
// (w & mask) | magic is one v_and_or_b32 (a VOP3 here takes at most one literal or
// SGPR, so two immediates would cost a separate and and or).
struct NibMask {
    uint32_t m[2]; // low nibbles 0x000F000F, high nibbles 0x00F000F0
};
__device__ __forceinline__ NibMask nib_mask() {
    NibMask n{{0x000F000Fu, 0x00F000F0u}};
    asm("" : "+v"(n.m[0]));
    asm("" : "+v"(n.m[1]));
    return n;
}

// The 8 weights q * sc + mn of quant words da, db (bytes 0-7 of a run), the low
// nibbles when hi = 0 and the high ones when hi = 1, in byte order 0 2 1 3 4 6 5 7,
// rounded once to bf16.  Each pair of nibbles becomes two f16 magic + q (one
// v_and_or_b32), and each weight one v_fma_mix_f32: (magic + q) * sc + (mn - magic
// * sc) in f32.  The folded offset is rounded once in f32 (an error below 2^-14 sc,
// far under the bf16 rounding of the weight).
__device__ __forceinline__ bf16x8 q4k_unpack(uint32_t da, uint32_t db, int hi, const NibMask& nm, float sc,
                                             float mn) {
    const uint32_t mk = nm.m[hi], magic = hi ? 0x54005400u : 0x64006400u;
    const float m2 = __builtin_fmaf(hi ? -64.0f : -1024.0f, sc, mn);
    const uint32_t p[4] = {(da & mk) | magic, ((da >> 8) & mk) | magic, (db & mk) | magic,
                           ((db >> 8) & mk) | magic};
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2v v = __builtin_bit_cast(half2v, p[i]);
        f[2 * i] = __builtin_fmaf((float)v[0], sc, m2);
        f[2 * i + 1] = __builtin_fmaf((float)v[1], sc, m2);
    }
    return to_bf16x8(f);
}

// The 8 weights d * q of the signed bytes of words d0, d1 (values in order): the
// product is exact in f32 and rounded once to bf16.
__device__ __forceinline__ bf16x8 q8_unpack(uint32_t d0, uint32_t d1, float d) {
    float f[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        f[k] = (float)(int8_t)(d0 >> (8 * k)) * d;
        f[4 + k] = (float)(int8_t)(d1 >> (8 * k)) * d;
    }
    return to_bf16x8(f);
}

// One lane's share of a weight row for one K-block: raw words, then unpacked
// step by step into the MFMA B operand (8 bf16).
template <int DT> struct BRow;

template <> struct BRow<NAIWA_Q4_K> {
    u32x4 hd;   // d, dmin, 12 scale bytes
    u32x4 q[4]; // per 64-value chunk: bytes 16h .. 16h + 15 of its 32 quant bytes

    __device__ __forceinline__ void load(const uint8_t* row, int kb, int h) {
        const uint8_t* blk = row + (size_t)kb * NAIWA_Q4_K_BYTES;
        hd = *reinterpret_cast<const u32x4*>(blk);
#pragma unroll
        for (int c = 0; c < 4; ++c) q[c] = *reinterpret_cast<const u32x4*>(blk + 16 + 32 * c + 16 * h);
    }
    __device__ __forceinline__ bf16x8 step(int s) const {
        const int c = s / 4, t = s % 4;
        const uint32_t da = (t % 2) ? q[c].z : q[c].x, db = (t % 2) ? q[c].w : q[c].y;
        float a, b;
        q4k_scale_min(hd, 2 * c + t / 2, a, b);
        return q4k_unpack(da, db, t / 2, nib_mask(), a, b);
    }
};

template <> struct BRow<NAIWA_Q8_0> {
    uint32_t w[2][9]; // blocks 2j + h (j = 0, 1): 9 words from the block's aligned start
    int sh[2];        // byte offset of each block within its first word (0 or 2)

    __device__ __forceinline__ void load(const uint8_t* row, int kb, int h) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int off = (4 * kb + 2 * j + h) * NAIWA_Q8_0_BYTES;
            sh[j] = off & 3;
            const uint32_t* p = reinterpret_cast<const uint32_t*>(row + (off & ~3));
#pragma unroll
            for (int i = 0; i < 9; ++i) w[j][i] = p[i];
        }
    }
    __device__ __forceinline__ bf16x8 step(int s) const {
        const int j = s / 4, u = s % 4;
        // values 8u .. 8u + 7 are bytes sh + 2 + 8u .. of the window: words 2u + 1 and
        // 2u + 2 when the block starts at byte 2 of its first word, else shifted by 2
        const uint32_t d0 = sh[j] ? w[j][2 * u + 1] : __builtin_amdgcn_alignbyte(w[j][2 * u + 1], w[j][2 * u], 2);
        const uint32_t d1 =
            sh[j] ? w[j][2 * u + 2] : __builtin_amdgcn_alignbyte(w[j][2 * u + 2], w[j][2 * u + 1], 2);
        const uint32_t dbits = sh[j] ? (w[j][0] >> 16) : (w[j][0] & 0xffffu);
        return q8_unpack(d0, d1, naiwa_f16_to_f32(dbits));
    }
};

// LDS A tile of one K-block: group g of tile row m at [g][m] (16 bytes each), rows of
// groups padded to kTM + 1 slots.  A step's read of 32 rows of one group covers 32
// consecutive slots at an offset fixed at compile time from the lane's own base; a
// staging store of consecutive groups of one row steps 1040 bytes (16 mod 256) from
// lane to lane, so it spreads over the banks.
template <int DT> struct ATile {
    static constexpr int kGroups = 2 * KBlock<DT>::kSteps;
    u32x4 v[kGroups][kTM + 1];
    __device__ __forceinline__ u32x4& at(int g, int m) { return v[g][m]; }
    __device__ __forceinline__ const u32x4& at(int g, int m) const { return v[g][m]; }
};

// Each thread's share of staging one K-block of the A tile: global -> registers
// (issued early) -> LDS (after the previous step's reads).
template <int DT> struct AStage {
    static constexpr int kPer = ATile<DT>::kGroups * kTM / kGemm; // 16-byte pieces per thread
    u32x4 r[kPer];
    // base: the activation matrix (a kernel argument, so the loads are global ones);
    // rows[m]: element offset of tile row m
    // piece p: row p / G, group p % G, so the lanes of a load cover whole rows
    // pieces i0 .. i1 - 1 only, when given (staging in parts holds fewer registers)
    __device__ __forceinline__ void load(const uint16_t* base, const int* rows, int kb, int tid, int i0 = 0,
                                         int i1 = kPer) {
        constexpr int G = ATile<DT>::kGroups;
#pragma unroll
        for (int i = i0; i < i1; ++i) {
            const int p = tid + kGemm * i, m = p / G, g = p % G;
            r[i] = *reinterpret_cast<const u32x4*>(base + rows[m] + kb * KBlock<DT>::kVals + 8 * g);
        }
    }
    __device__ __forceinline__ void store(ATile<DT>& a, int tid, int i0 = 0, int i1 = kPer) const {
        constexpr int G = ATile<DT>::kGroups;
#pragma unroll
        for (int i = i0; i < i1; ++i) {
            const int p = tid + kGemm * i;
            a.at(p % G, p / G) = r[i];
        }
    }
};

// Workgroup barrier for an LDS hand-off: waits for this wave's LDS operations only.
// (__syncthreads also waits for every global load in flight, which would make each
// K-block wait out the latency of the next K-block's weight loads.)
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

struct Bank {
    const uint8_t* base;
    int64_t stride;
    int64_t row_bytes;
};

// The K loop of one tile: acc[ms] += A (64 rows staged through the LDS double buffer
// `as`) x B (this lane's share of weight row `wrow`), K-blocks 0 .. nkb - 1.  The next
// K-block's loads are issued before the current one is used; the last K-block reloads
// itself, so the loads are unconditional and the compiler waits only for the registers
// each step uses.
template <int DT>
__device__ __forceinline__ void tile_k_loop(const uint16_t* abase, const int* rows, const uint8_t* wrow, int nkb,
                                            ATile<DT>* as, int tid, int lane, int h, floatx16* acc) {
    AStage<DT> st;
    if constexpr (DT == NAIWA_Q4_K) {
        // Rolling prefetch: chunk c of the next K-block replaces chunk c of the current one
        // as soon as its four steps are done, and the next header replaces the current one
        // once the last chunk's scales are taken, so a lane holds one K-block of weights
        // instead of two.  At most 128 VGPRs then, two 8-wave blocks fit on a CU.
        BRow<DT> b;
        const NibMask nm = nib_mask();
        // this lane's A operand slot in buffer 0: step s, subtile ms reads
        // alane[buffer + 2 s (kTM + 1) + 32 ms] (one base register, offsets fixed)
        const u32x4* alane = &as[0].v[h][lane & 31];
        constexpr int kBuf = sizeof(ATile<DT>) / sizeof(u32x4);
        st.load(abase, rows, 0, tid);
        b.load(wrow, 0, h);
        st.store(as[0], tid);
        __syncthreads();
        for (int kb = 0; kb < nkb; ++kb) {
            const int kn = min(kb + 1, nkb - 1);
            const uint8_t* nblk = wrow + (size_t)kn * NAIWA_Q4_K_BYTES;
            // the next A tile's loads go out now and land in the other buffer (its last
            // reads were before the previous barrier) after this block's last chunk: a
            // whole K-block of MFMA work hides their latency
            st.load(abase, rows, kn, tid);
            __builtin_amdgcn_sched_barrier(0); // keep the prefetches where they are issued
            const u32x4* ab = alane + (kb & 1) * kBuf;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float sc[2], mn[2];
                q4k_scale_min(b.hd, 2 * c, sc[0], mn[0]);
                q4k_scale_min(b.hd, 2 * c + 1, sc[1], mn[1]);
                // the last chunk's scales are taken: the next header can replace this one
                if (c == 3) b.hd = *reinterpret_cast<const u32x4*>(nblk);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int s = 4 * c + t;
                    const uint32_t da = (t % 2) ? b.q[c].z : b.q[c].x, db = (t % 2) ? b.q[c].w : b.q[c].y;
                    const bf16x8 wv = q4k_unpack(da, db, t / 2, nm, sc[t / 2], mn[t / 2]);
#pragma unroll
                    for (int ms = 0; ms < 2; ++ms) {
                        const bf16x8 x8 = __builtin_bit_cast(bf16x8, ab[2 * s * (kTM + 1) + 32 * ms]);
                        acc[ms] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x8, wv, acc[ms], 0, 0, 0);
                    }
                }
                b.q[c] = *reinterpret_cast<const u32x4*>(nblk + 16 + 32 * c + 16 * h);
                __builtin_amdgcn_sched_barrier(0);
                if (c == 3) st.store(as[(kb + 1) & 1], tid);
            }
            lds_barrier();
        }
    } else {
        BRow<DT> b0, b1; // this K-block's row share and the next one's, alternating
        st.load(abase, rows, 0, tid);
        b0.load(wrow, 0, h);
        st.store(as[0], tid);
        __syncthreads();
        auto block = [&](int kb, const BRow<DT>& bw, BRow<DT>& nw) {
            const int kn = min(kb + 1, nkb - 1);
            st.load(abase, rows, kn, tid);
            nw.load(wrow, kn, h);
            const ATile<DT>& a = as[kb & 1];
#pragma unroll
            for (int s = 0; s < KBlock<DT>::kSteps; ++s) {
                const bf16x8 wv = bw.step(s);
#pragma unroll
                for (int ms = 0; ms < 2; ++ms) {
                    const bf16x8 x8 = __builtin_bit_cast(bf16x8, a.at(2 * s + h, 32 * ms + (lane & 31)));
                    acc[ms] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x8, wv, acc[ms], 0, 0, 0);
                }
            }
            st.store(as[(kb + 1) & 1], tid);
            lds_barrier();
        };
        int kb = 0;
        for (; kb + 2 <= nkb; kb += 2) {
            block(kb, b0, b1);
            block(kb + 1, b1, b0);
        }
        if (kb < nkb) block(kb, b0, b1);
    }
}

// gate/up: one tile of <= 64 pairs x 128 intermediate features; waves 0-3 the
// gate rows, waves 4-7 the up rows of the same 4 x 32 features.  xp: x in the K
// order of DG; hp (out): h in the K order of DD, bf16 [pairs, I].
template <int DG, int DD>
__global__ void __launch_bounds__(kGemm, 4)
gateup_kernel(Bank gate, Bank up, const uint16_t* xp, int H, int I, int k, const uint32_t* perm, Tiles tl,
              int act, uint16_t* hp, int xcd) {
    __shared__ ATile<DG> as[2];
    __shared__ int rows[kTM];
    int tile = 0, colb = 0;
    if (!tile_col(blockIdx.x, *tl.n, I / kTNG, xcd, &tile, &colb)) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5;
    const int is_up = wave >> 2, strip = wave & 3;
    const int start = tl.start[tile], cnt = tl.count[tile], slot = tl.slot[tile];
    if (tid < kTM) rows[tid] = (int)(perm[start + min(tid, cnt - 1)] / k) * H;
    const int n = colb * kTNG + 32 * strip + (lane & 31); // this lane's weight row
    const Bank& bank = is_up ? up : gate;
    const uint8_t* wrow = bank.base + (int64_t)slot * bank.stride + (int64_t)n * bank.row_bytes;
    const int nkb = H / KBlock<DG>::kVals;
    __syncthreads();

    floatx16 acc[2] = {}; // [m subtile]
    tile_k_loop<DG>(xp, rows, wrow, nkb, as, tid, lane, h, acc);
    // epilogue: the gate waves hand act(g) to the up waves of the same strip through
    // LDS (the A tiles are no longer read); h = act(g) * u as bf16 at its laid-out
    // position for the down format
    float* xch = reinterpret_cast<float*>(&as[0]);
    const int xbase = (strip * 32) * 64 + lane;
    if (!is_up) {
#pragma unroll
        for (int ms = 0; ms < 2; ++ms)
#pragma unroll
            for (int v = 0; v < 16; ++v) xch[xbase + (16 * ms + v) * 64] = naiwa_act(act, acc[ms][v]);
    }
    __syncthreads();
    if (is_up) {
        const int col = laid_pos<DD>(n);
#pragma unroll
        for (int ms = 0; ms < 2; ++ms)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = 32 * ms + 8 * (v / 4) + 4 * h + v % 4;
                if (m < cnt) {
                    const float g = xch[xbase + (16 * ms + v) * 64];
                    hp[(size_t)(start + m) * I + col] = (uint16_t)bf16x2_bits(g * acc[ms][v], 0.0f);
                }
            }
    }
}

// down: one tile of <= 64 pairs x 256 output features (32 per wave); pair rows
// scaled by their weight.
template <int DD>
__global__ void __launch_bounds__(kGemm, 4)
down_kernel(Bank down, const uint16_t* hp, int H, int I, const uint32_t* perm, const float* w, Tiles tl,
            float* ypair, int xcd) {
    __shared__ ATile<DD> as[2];
    __shared__ int rows[kTM];
    int tile = 0, col = 0;
    if (!tile_col(blockIdx.x, *tl.n, H / kTND, xcd, &tile, &col)) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5;
    const int start = tl.start[tile], cnt = tl.count[tile], slot = tl.slot[tile];
    if (tid < kTM) rows[tid] = (start + min(tid, cnt - 1)) * I;
    const int n = col * kTND + 32 * wave + (lane & 31);
    const uint8_t* drow = down.base + (int64_t)slot * down.stride + (int64_t)n * down.row_bytes;
    const int nkb = I / KBlock<DD>::kVals;
    __syncthreads();

    floatx16 acc[2] = {};
    tile_k_loop<DD>(hp, rows, drow, nkb, as, tid, lane, h, acc);
#pragma unroll
    for (int ms = 0; ms < 2; ++ms)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = 32 * ms + 8 * (v / 4) + 4 * h + v % 4;
            if (m < cnt) {
                const uint32_t p = perm[start + m];
                ypair[(size_t)p * H + n] = acc[ms][v] * w[p];
            }
        }
}

// out[t] = sum over j = 0..k-1 of the pair rows whose slot id is valid, in j order.
// V = 4: 16 bytes per thread (H % 4 == 0, out 16-byte aligned), the loads of up to
// 8 pair rows issued before their sums; the same additions in the same order as V = 1.
// res (bf16 [T, H], or null): also res = bf16(res + out), the residual add.
template <int V>
__global__ void __launch_bounds__(kThreads)
combine_kernel(const float* ypair, const uint32_t* ids, int k, int H, int slots, int accumulate, float* out,
               uint16_t* res) {
    typedef float vec __attribute__((ext_vector_type(V)));
    constexpr int kJ = 8;
    const int t = blockIdx.x, HV = H / V;
    const vec* yp = reinterpret_cast<const vec*>(ypair + (size_t)t * k * H);
    vec* o = reinterpret_cast<vec*>(out + (size_t)t * H);
    // blockIdx.y: a slice of kThreads vectors of the token's row, so that every load of
    // the call is in flight at once rather than in rounds per block
    for (int c = blockIdx.y * kThreads + threadIdx.x; c < HV; c += kThreads * gridDim.y) {
        vec y = accumulate ? o[c] : vec(0.0f);
        uint16_t xr[V];
        if (res) {
#pragma unroll
            for (int i = 0; i < V; ++i) xr[i] = res[(size_t)t * H + (size_t)c * V + i];
        }
        for (int j0 = 0; j0 < k; j0 += kJ) {
            // every pair row of the token is in the buffer: its load does not wait for the
            // slot id, which only decides whether the row is added
            vec v[kJ];
            uint32_t id[kJ];
#pragma unroll
            for (int u = 0; u < kJ; ++u) {
                const int j = j0 + u;
                if (j < k) {
                    id[u] = ids[(size_t)t * k + j];
                    v[u] = yp[(size_t)j * HV + c];
                }
            }
#pragma unroll
            for (int u = 0; u < kJ; ++u)
                if (j0 + u < k && id[u] < (uint32_t)slots) y += v[u];
        }
        o[c] = y;
        if (res) {
#pragma unroll
            for (int i = 0; i < V; ++i)
                res[(size_t)t * H + (size_t)c * V + i] = (uint16_t)naiwa_f32_to_bf16(naiwa_bf16_to_f32(xr[i]) + y[i]);
        }
    }
}

// ---------------------------------------------------------------------------
// Multi-token decode on the matrix cores
// ---------------------------------------------------------------------------
// naiwa_moe_decode calls with several tokens per expert run their expert GEMMs
// here.  A block of 4 waves takes one slot segment (the sorted pairs of one
// slot) and 64 features; chunks of up to 16 of the segment's tokens are the A
// operand of v_mfma_f32_16x16x32_bf16 and each lane dequantises its own weight
// values once into the B operand, so a weight costs the same whatever the
// token count.  Lane l = 16 g + m holds A[m][8 g + 0..7] (token m of the
// chunk), B[8 g + 0..7][m] (feature m of the wave's 16) and D[4 g + i][m].
// Gate and up accumulate in the same wave, so h = act(g) * u is formed in
// registers.
//
// K order of the 16x16x32 steps.  In every K-block lane group g reads:
//   Q4_K (256 values): 64-value chunk g; step s = 2 p + t takes its quant bytes
//        8 p + 0..7, low nibbles for t = 0 and high ones for t = 1: values
//        64 g + 32 t + 8 p + (0 2 1 3 4 6 5 7);
//   Q8_0 (128 values, 4 blocks): block g; step s takes its values 8 s + 0..7.
// The activations (x for gate/up, h for down) are stored as groups G = 4 s + g
// of 8 f16 in that order.
constexpr int kDecM = 16;        // tokens per MFMA tile
constexpr int kDecThreads = 256; // 4 waves of 16 features
constexpr int kDecF = 64;        // features (gate/up) or output rows (down) per block

template <int DT> struct K16;
template <> struct K16<NAIWA_Q4_K> {
    static constexpr int kVals = 256, kSteps = 8;
};
template <> struct K16<NAIWA_Q8_0> {
    static constexpr int kVals = 128, kSteps = 4;
};

// Position, in the laid-out row, of value f of the original row.
template <int DT>
__host__ __device__ inline int laid16(int f) {
    constexpr int KV = K16<DT>::kVals;
    const int kb = f / KV, r = f % KV;
    if (DT == NAIWA_Q4_K) {
        const int g = r / 64, t = (r % 64) / 32, p = (r % 32) / 8;
        return kb * KV + 8 * (4 * (2 * p + t) + g) + q4_elem(r % 8);
    }
    const int g = r / 32, st = (r % 32) / 8;
    return kb * KV + 8 * (4 * st + g) + r % 8;
}

// Per-K-block scale state of one lane (Q4_K: its two sub-blocks 2 g and 2 g + 1).
struct Scl {
    float sc[2], mn[2];
};

// One lane's weights of one K-block (row `row`, lane group g).
template <int DT> struct W16;

template <> struct W16<NAIWA_Q4_K> {
    u32x4 hd, q0, q1; // header; quant bytes 0-15 and 16-31 of chunk g
    __device__ __forceinline__ void load(const uint8_t* row, int kb, int g) {
        const uint8_t* blk = row + (size_t)kb * NAIWA_Q4_K_BYTES;
        hd = *reinterpret_cast<const u32x4*>(blk);
        q0 = *reinterpret_cast<const u32x4*>(blk + 16 + 32 * g);
        q1 = *reinterpret_cast<const u32x4*>(blk + 32 + 32 * g);
    }
    __device__ __forceinline__ void prep(int g, Scl& c) const {
        q4k_scale_min(hd, 2 * g, c.sc[0], c.mn[0]);
        q4k_scale_min(hd, 2 * g + 1, c.sc[1], c.mn[1]);
    }
    __device__ __forceinline__ bf16x8 step(int s, const Scl& c, const NibMask& nm) const {
        const int p = s >> 1, t = s & 1;
        const u32x4& q = p < 2 ? q0 : q1;
        const uint32_t da = (p & 1) ? q.z : q.x, db = (p & 1) ? q.w : q.y;
        return q4k_unpack(da, db, t, nm, c.sc[t], c.mn[t]);
    }
};

template <> struct W16<NAIWA_Q8_0> {
    uint32_t w[9]; // block 4 kb + g: 9 words from its aligned start
    int sh;        // its byte offset within the first word (0 or 2)
    __device__ __forceinline__ void load(const uint8_t* row, int kb, int g) {
        const int off = (4 * kb + g) * NAIWA_Q8_0_BYTES;
        sh = off & 3;
        const uint32_t* p = reinterpret_cast<const uint32_t*>(row + (off & ~3));
#pragma unroll
        for (int i = 0; i < 9; ++i) w[i] = p[i];
    }
    __device__ __forceinline__ void prep(int, Scl&) const {}
    __device__ __forceinline__ bf16x8 step(int s, const Scl&, const NibMask&) const {
        const uint32_t d0 = sh ? w[2 * s + 1] : __builtin_amdgcn_alignbyte(w[2 * s + 1], w[2 * s], 2);
        const uint32_t d1 = sh ? w[2 * s + 2] : __builtin_amdgcn_alignbyte(w[2 * s + 2], w[2 * s + 1], 2);
        const uint32_t dbits = sh ? (w[0] >> 16) : (w[0] & 0xffffu);
        return q8_unpack(d0, d1, naiwa_f16_to_f32(dbits));
    }
};

// LDS A tile of one K-block: group G of token row m at [G][m ^ (G % 16)].
// MT subtiles of 16 token rows (a chunk of 16 MT tokens); the XOR keeps a row in its subtile.
template <int DT, int MT> struct ATile16 {
    static constexpr int kGroups = 4 * K16<DT>::kSteps;
    u32x4 v[kGroups][kDecM * MT];
    __device__ __forceinline__ u32x4& at(int G, int m) { return v[G][m ^ (G & 15)]; }
    __device__ __forceinline__ const u32x4& at(int G, int m) const { return v[G][m ^ (G & 15)]; }
};

// Thread tid's pieces of one K-block of the A tile: piece p = tid + kDecThreads * i is
// row p / G, group p % G (the lanes of a load cover whole rows); rows[m] < 0 is a zero row.
template <int DT, int MT> struct AStage16 {
    static constexpr int G = ATile16<DT, MT>::kGroups;
    static constexpr int kRows = kDecM * MT;
    static constexpr int kPer = (G * kRows + kDecThreads - 1) / kDecThreads;
    u32x4 r[kPer];
    __device__ __forceinline__ void load(const uint16_t* base, const int* rows, int kb, int tid) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int p = tid + kDecThreads * i;
            r[i] = u32x4{0u, 0u, 0u, 0u};
            if (p < G * kRows) {
                const int ro = rows[p / G];
                if (ro >= 0) r[i] = *reinterpret_cast<const u32x4*>(base + ro + kb * K16<DT>::kVals + 8 * (p % G));
            }
        }
    }
    __device__ __forceinline__ void store(ATile16<DT, MT>& a, int tid) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int p = tid + kDecThreads * i;
            if (p < G * kRows) a.at(p % G, p / G) = r[i];
        }
    }
};

// x (bf16 or f32) [T, H] -> xl bf16 [T, H] in the 16x16x32 K order of DT, one thread
// per run of 8 values (bf16 input unchanged, f32 rounded to nearest-even bf16).
template <int DT>
__global__ void __launch_bounds__(kThreads) dec_prep_kernel(const void* x, int x_bf16, int T, int H, uint16_t* xl) {
    const int runs = H / 8;
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const bool in = i < (int64_t)T * runs;
    const int t = in ? (int)(i / runs) : 0, run = in ? (int)(i % runs) : 0;
    float f[8] = {};
    if (in) {
        if (x_bf16) {
            const uint4 v = *reinterpret_cast<const uint4*>((const uint16_t*)x + (size_t)t * H + 8 * run);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f[2 * j] = __uint_as_float(w[j] << 16);
                f[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
            }
        } else {
            const float4* src = reinterpret_cast<const float4*>((const float*)x + (size_t)t * H + 8 * run);
            const float4 a = src[0], b = src[1];
            f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
            f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
        }
    }
    if (!in) return;
    float g[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) g[e] = f[DT == NAIWA_Q4_K ? q4_elem(e) : e];
    uint4 o;
    o.x = bf16x2_bits(g[0], g[1]);
    o.y = bf16x2_bits(g[2], g[3]);
    o.z = bf16x2_bits(g[4], g[5]);
    o.w = bf16x2_bits(g[6], g[7]);
    *reinterpret_cast<uint4*>(xl + (size_t)t * H + laid16<DT>(8 * run)) = o;
}

// The K-block loop of one chunk of 16 MT tokens: NP weight rows (gate and up, or down)
// against the A rows listed in `rows`, K-blocks kb0 .. kb0 + nkb - 1; each step's
// dequantised B operand serves the MT subtiles.
template <int DT, int NP, int MT>
__device__ __forceinline__ void dec_chunk(const uint16_t* abase, const int* rows, const uint8_t* const* wrow,
                                          int kb0, int nkb, ATile16<DT, MT>* as, int tid, int g, int m,
                                          floatx4 (&acc)[NP][MT]) {
    AStage16<DT, MT> st;
    W16<DT> cur[NP], nxt[NP];
    const NibMask nm = nib_mask();
    st.load(abase, rows, kb0, tid);
#pragma unroll
    for (int q = 0; q < NP; ++q) cur[q].load(wrow[q], kb0, g);
    st.store(as[0], tid);
    __syncthreads();
    // one K-block; the next one's loads are unconditional (the last block reloads
    // itself) so the compiler waits only for this block's registers
    auto block = [&](int j, const W16<DT>* bw, W16<DT>* nw) {
        const int kn = kb0 + min(j + 1, nkb - 1);
        st.load(abase, rows, kn, tid);
#pragma unroll
        for (int q = 0; q < NP; ++q) nw[q].load(wrow[q], kn, g);
        Scl c[NP];
#pragma unroll
        for (int q = 0; q < NP; ++q) bw[q].prep(g, c[q]);
        const ATile16<DT, MT>& a = as[j & 1];
#pragma unroll
        for (int s = 0; s < K16<DT>::kSteps; ++s) {
            bf16x8 x8[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) x8[mt] = __builtin_bit_cast(bf16x8, a.at(4 * s + g, kDecM * mt + m));
#pragma unroll
            for (int q = 0; q < NP; ++q) {
                const bf16x8 b = bw[q].step(s, c[q], nm);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[q][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x8[mt], b, acc[q][mt], 0, 0, 0);
            }
        }
        st.store(as[(j + 1) & 1], tid);
        lds_barrier();
    };
    int j = 0;
    for (; j + 2 <= nkb; j += 2) {
        block(j, cur, nxt);
        block(j + 1, nxt, cur);
    }
    if (j < nkb) block(j, cur, nxt);
}

// gate/up: block (64 features, slot segment); h = act(gate) * up as bf16 at the
// pair's sorted position, in the 16x16x32 K order of DD.
template <int DG, int DD, int MT>
__global__ void __launch_bounds__(kDecThreads, 2)
dec_gateup_kernel(Bank gate, Bank up, const uint16_t* xl, int H, int I, int width, const int* seg_count,
                  const uint32_t* seg_key, const uint32_t* seg_begin, const uint32_t* perm, int act, uint16_t* hl) {
    constexpr int CM = kDecM * MT; // tokens per chunk
    __shared__ ATile16<DG, MT> as[2];
    __shared__ int rows[CM];
    const int sg = blockIdx.y;
    if (sg >= *seg_count) return;
    const int tid = threadIdx.x, lane = tid & 63, m = lane & 15, g = lane >> 4;
    const uint32_t slot = seg_key[sg];
    const int b = (int)seg_begin[sg], e = (int)seg_begin[sg + 1];
    const int n = blockIdx.x * kDecF + 16 * (tid >> 6) + m;
    const uint8_t* wrow[2] = {gate.base + (int64_t)slot * gate.stride + (int64_t)n * gate.row_bytes,
                              up.base + (int64_t)slot * up.stride + (int64_t)n * up.row_bytes};
    const int col = laid16<DD>(n);
    for (int c0 = b; c0 < e; c0 += CM) {
        const int cnt = min(CM, e - c0);
        __syncthreads(); // the previous chunk is done with rows and the A tiles
        if (tid < CM) rows[tid] = tid < cnt ? (int)(perm[c0 + tid] / (uint32_t)width) * H : -1;
        __syncthreads();
        floatx4 acc[2][MT] = {};
        dec_chunk<DG, 2, MT>(xl, rows, wrow, 0, H / K16<DG>::kVals, as, tid, g, m, acc);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int mm = kDecM * mt + 4 * g + i;
                if (mm < cnt)
                    hl[(size_t)(c0 + mm) * I + col] =
                        (uint16_t)bf16x2_bits(naiwa_act(act, acc[0][mt][i]) * acc[1][mt][i], 0.0f);
            }
    }
}

// down: block (64 output rows, K part, slot segment); the unweighted partial dot of
// (K part, sorted position, row) into dpart.
template <int DD, int MT>
__global__ void __launch_bounds__(kDecThreads, 2)
dec_down_kernel(Bank down, const uint16_t* hl, int H, int I, int ks, int npairs, const int* seg_count,
                const uint32_t* seg_key, const uint32_t* seg_begin, float* dpart) {
    constexpr int CM = kDecM * MT;
    __shared__ ATile16<DD, MT> as[2];
    __shared__ int rows[CM];
    const int sg = blockIdx.z;
    if (sg >= *seg_count) return;
    const int tid = threadIdx.x, lane = tid & 63, m = lane & 15, g = lane >> 4;
    const uint32_t slot = seg_key[sg];
    const int b = (int)seg_begin[sg], e = (int)seg_begin[sg + 1];
    const int kp = blockIdx.y, k0 = kp * ks;
    const int r = blockIdx.x * kDecF + 16 * (tid >> 6) + m;
    const uint8_t* wrow[1] = {down.base + (int64_t)slot * down.stride + (int64_t)r * down.row_bytes};
    for (int c0 = b; c0 < e; c0 += CM) {
        const int cnt = min(CM, e - c0);
        __syncthreads();
        if (tid < CM) rows[tid] = tid < cnt ? (c0 + tid) * I : -1;
        __syncthreads();
        floatx4 acc[1][MT] = {};
        dec_chunk<DD, 1, MT>(hl, rows, wrow, k0 / K16<DD>::kVals, min(ks, I - k0) / K16<DD>::kVals, as, tid, g, m,
                             acc);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int mm = kDecM * mt + 4 * g + i;
                if (mm < cnt) dpart[((size_t)kp * npairs + c0 + mm) * H + r] = acc[0][mt][i];
            }
    }
}

// K of a projection in this format: whole K-blocks.
bool fmt_ok(int dtype, int kdim) {
    return (dtype == NAIWA_Q4_K && kdim % KBlock<NAIWA_Q4_K>::kVals == 0) ||
           (dtype == NAIWA_Q8_0 && kdim % KBlock<NAIWA_Q8_0>::kVals == 0);
}

template <int DG, int DD>
void launch_gateup(dim3 g, hipStream_t st, Bank bg, Bank bu, const uint16_t* xp, int H, int I, int k,
                   const uint32_t* perm, Tiles tl, int act, uint16_t* hp, int xcd) {
    gateup_kernel<DG, DD><<<g, kGemm, 0, st>>>(bg, bu, xp, H, I, k, perm, tl, act, hp, xcd);
}

template <int MT>
void dec_experts(bool g4, bool d4, dim3 g1, dim3 g2, Bank bg, Bank bu, Bank bd, const uint16_t* xl, uint16_t* hl,
                 int H, int I, int width, int ks, int n, const int* seg_count, const uint32_t* seg_key,
                 const uint32_t* seg_begin, const uint32_t* perm, int act, float* dpart, hipStream_t st) {
    if (g4 && d4)
        dec_gateup_kernel<NAIWA_Q4_K, NAIWA_Q4_K, MT><<<g1, kDecThreads, 0, st>>>(bg, bu, xl, H, I, width, seg_count,
                                                                                  seg_key, seg_begin, perm, act, hl);
    else if (g4)
        dec_gateup_kernel<NAIWA_Q4_K, NAIWA_Q8_0, MT><<<g1, kDecThreads, 0, st>>>(bg, bu, xl, H, I, width, seg_count,
                                                                                  seg_key, seg_begin, perm, act, hl);
    else if (d4)
        dec_gateup_kernel<NAIWA_Q8_0, NAIWA_Q4_K, MT><<<g1, kDecThreads, 0, st>>>(bg, bu, xl, H, I, width, seg_count,
                                                                                  seg_key, seg_begin, perm, act, hl);
    else
        dec_gateup_kernel<NAIWA_Q8_0, NAIWA_Q8_0, MT><<<g1, kDecThreads, 0, st>>>(bg, bu, xl, H, I, width, seg_count,
                                                                                  seg_key, seg_begin, perm, act, hl);
    if (d4)
        dec_down_kernel<NAIWA_Q4_K, MT><<<g2, kDecThreads, 0, st>>>(bd, hl, H, I, ks, n, seg_count, seg_key, seg_begin,
                                                                     dpart);
    else
        dec_down_kernel<NAIWA_Q8_0, MT><<<g2, kDecThreads, 0, st>>>(bd, hl, H, I, ks, n, seg_count, seg_key, seg_begin,
                                                                     dpart);
}

} // namespace

bool naiwa_decode_mfma_ok(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, const void* x) {
    const int H = gate->k, I = gate->n;
    auto fmt = [](int dt, int k) {
        return (dt == NAIWA_Q4_K && k % K16<NAIWA_Q4_K>::kVals == 0) ||
               (dt == NAIWA_Q8_0 && k % K16<NAIWA_Q8_0>::kVals == 0);
    };
    if (gate->dtype != up->dtype || !fmt(gate->dtype, H) || !fmt(down->dtype, I)) return false;
    if (H % kDecF || I % kDecF) return false;
    return ((uintptr_t)x & 15) == 0; // 16-byte loads of x
}

size_t naiwa_decode_mfma_bytes(int rows, int n, int H, int I) {
    return (((size_t)rows * H * 2 + 255) & ~size_t(255)) + (size_t)n * I * 2;
}

int naiwa_decode_mfma_experts(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, const void* x,
                              int x_dtype, int rows, int width, int act, int n, int seg_bound, int ks,
                              const int* seg_count, const uint32_t* seg_key, const uint32_t* seg_begin,
                              const uint32_t* perm, uint8_t* ws, float* dpart, hipStream_t st) {
    const int H = gate->k, I = gate->n;
    uint16_t* xl = (uint16_t*)ws;
    uint16_t* hl = (uint16_t*)(ws + (((size_t)rows * H * 2 + 255) & ~size_t(255)));
    const Bank bg{(const uint8_t*)gate->base, gate->slot_stride, naiwa_row_bytes(gate->dtype, H)};
    const Bank bu{(const uint8_t*)up->base, up->slot_stride, naiwa_row_bytes(up->dtype, H)};
    const Bank bd{(const uint8_t*)down->base, down->slot_stride, naiwa_row_bytes(down->dtype, I)};
    const int xb = x_dtype == NAIWA_BF16;
    const unsigned pb = (unsigned)(((int64_t)rows * (H / 8) + kThreads - 1) / kThreads);
    const bool g4 = gate->dtype == NAIWA_Q4_K, d4 = down->dtype == NAIWA_Q4_K;
    if (g4)
        dec_prep_kernel<NAIWA_Q4_K><<<pb, kThreads, 0, st>>>(x, xb, rows, H, xl);
    else
        dec_prep_kernel<NAIWA_Q8_0><<<pb, kThreads, 0, st>>>(x, xb, rows, H, xl);
    const dim3 g1(I / kDecF, seg_bound), g2(H / kDecF, (I + ks - 1) / ks, seg_bound);
    // two 16-token subtiles per chunk when the segments average more than 8 tokens:
    // each weight is then dequantised once per 32 tokens instead of 16
    if (n > 8 * seg_bound)
        dec_experts<2>(g4, d4, g1, g2, bg, bu, bd, xl, hl, H, I, width, ks, n, seg_count, seg_key, seg_begin, perm,
                       act, dpart, st);
    else
        dec_experts<1>(g4, d4, g1, g2, bg, bu, bd, xl, hl, H, I, width, ks, n, seg_count, seg_key, seg_begin, perm,
                       act, dpart, st);
    return naiwa_hip_rc(hipGetLastError());
}

extern "C" int naiwa_moe_prefill(const naiwa_bank* gate, const naiwa_bank* up, const naiwa_bank* down, const void* x,
                                 const uint32_t* slot_ids, const float* w, int T, int k, int act, float* out,
                                 int flags, int64_t stream) {
    if (!gate || !up || !down || T < 0 || k <= 0 || (flags & ~(NAIWA_PREFILL_ACCUMULATE | NAIWA_PREFILL_RESIDUAL)))
        return NAIWA_E_INVALID;
    if (T == 0) return NAIWA_OK;
    if (!x || !slot_ids || !w || !out) return NAIWA_E_INVALID;
    const int H = gate->k, I = gate->n, slots = gate->slots;
    if (up->k != H || up->n != I || down->n != H || down->k != I || up->slots != slots || down->slots != slots)
        return NAIWA_E_INVALID;
    if (gate->dtype != up->dtype || !fmt_ok(gate->dtype, H) || !fmt_ok(down->dtype, I)) return NAIWA_E_UNSUPPORTED;
    if (H % kTND || I % kTNG) return NAIWA_E_UNSUPPORTED;
    if (act != NAIWA_ACT_SILU && act != NAIWA_ACT_GELU_PYTORCH_TANH) return NAIWA_E_UNSUPPORTED;
    const int64_t n = (int64_t)T * k;
    if (n > 65536 || slots <= 0 || slots > 4096) return NAIWA_E_UNSUPPORTED;
    if ((int64_t)T * H > INT32_MAX || n * I > INT32_MAX) return NAIWA_E_UNSUPPORTED; // 32-bit row offsets
    const int64_t rbg = naiwa_row_bytes(gate->dtype, H), rbd = naiwa_row_bytes(down->dtype, I);
    if (gate->slot_stride < rbg * I || up->slot_stride < rbg * I || down->slot_stride < rbd * H) return NAIWA_E_INVALID;
    // 16-byte loads of x and of Q4_K blocks, 4-byte loads of Q8_0 blocks
    if (((uintptr_t)gate->base | (uintptr_t)up->base | (uintptr_t)down->base | gate->slot_stride | up->slot_stride |
         down->slot_stride | (uintptr_t)x) & 15)
        return NAIWA_E_INVALID;
    if ((gate->dtype == NAIWA_Q4_K && (rbg % 16)) || (down->dtype == NAIWA_Q4_K && (rbd % 16))) return NAIWA_E_INVALID;
    if ((gate->dtype == NAIWA_Q8_0 && (rbg % 4)) || (down->dtype == NAIWA_Q8_0 && (rbd % 4))) return NAIWA_E_INVALID;

    // scratch: perm [n] | offsets [slots + 1] | bad | tiles 3 x max + n | xp bf16 [T, H] | h bf16 [n, I] |
    //          ypair f32 [n, H]
    const int64_t max_tiles = (n + kTM - 1) / kTM + slots;
    auto a256 = [](size_t b) { return (b + 255) & ~size_t(255); };
    const size_t o_perm = 0, o_off = a256(o_perm + (size_t)n * 4), o_bad = a256(o_off + (size_t)(slots + 1) * 4);
    const size_t o_tiles = a256(o_bad + 4), o_x = a256(o_tiles + (size_t)(3 * max_tiles + 1) * 4);
    const size_t o_h = a256(o_x + (size_t)T * H * 2), o_y = a256(o_h + (size_t)n * I * 2);
    const size_t total = a256(o_y + (size_t)n * H * 4);
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
    uint16_t* xp = (uint16_t*)(ws + o_x);
    uint16_t* hp = (uint16_t*)(ws + o_h);
    float* ypair = (float*)(ws + o_y);
    hipStream_t st = (hipStream_t)stream;

    if ((rc = naiwa_moe_gather(slot_ids, (int)n, slots, perm, offsets, (int*)(ws + o_bad), stream))) return rc;
    const unsigned prep_blocks = (unsigned)(((int64_t)T * (H / 8) + kThreads - 1) / kThreads);
    if (gate->dtype == NAIWA_Q4_K)
        prep_tiles_kernel<NAIWA_Q4_K><<<prep_blocks + 1, kThreads, 0, st>>>((const uint16_t*)x, T, H, xp, offsets,
                                                                            slots, tl);
    else
        prep_tiles_kernel<NAIWA_Q8_0><<<prep_blocks + 1, kThreads, 0, st>>>((const uint16_t*)x, T, H, xp, offsets,
                                                                            slots, tl);
    const Bank bg{(const uint8_t*)gate->base, gate->slot_stride, rbg}, bu{(const uint8_t*)up->base, up->slot_stride, rbg};
    const Bank bd{(const uint8_t*)down->base, down->slot_stride, rbd};
    const unsigned tiles8 = (unsigned)((max_tiles + 7) / 8 * 8);
    const dim3 g1((unsigned)(I / kTNG) * tiles8), g2((unsigned)(H / kTND) * tiles8);
    // XCD order when the experts average at most two tiles (few weight strips to share
    // between tiles, activation rows shared by every column block); with many tiles an
    // expert (a 4096-token Mixtral chunk: 16), the plain order keeps a column's weight
    // strip in one XCD's L2 across the tiles running at once.  DeepSeek-V2-Lite chunk:
    // FETCH -27 % (gate/up) and -26 % (down) at the same time; Mixtral 4096 tokens in
    // XCD order: 27.8K against 32.8K tok/s.
    const int xcd = n <= (int64_t)2 * kTM * slots ? 1 : 0;
    const bool g4 = gate->dtype == NAIWA_Q4_K, d4 = down->dtype == NAIWA_Q4_K;
    if (g4 && d4)
        launch_gateup<NAIWA_Q4_K, NAIWA_Q4_K>(g1, st, bg, bu, xp, H, I, k, perm, tl, act, hp, xcd);
    else if (g4)
        launch_gateup<NAIWA_Q4_K, NAIWA_Q8_0>(g1, st, bg, bu, xp, H, I, k, perm, tl, act, hp, xcd);
    else if (d4)
        launch_gateup<NAIWA_Q8_0, NAIWA_Q4_K>(g1, st, bg, bu, xp, H, I, k, perm, tl, act, hp, xcd);
    else
        launch_gateup<NAIWA_Q8_0, NAIWA_Q8_0>(g1, st, bg, bu, xp, H, I, k, perm, tl, act, hp, xcd);
    if (d4)
        down_kernel<NAIWA_Q4_K><<<g2, kGemm, 0, st>>>(bd, hp, H, I, perm, w, tl, ypair, xcd);
    else
        down_kernel<NAIWA_Q8_0><<<g2, kGemm, 0, st>>>(bd, hp, H, I, perm, w, tl, ypair, xcd);
    const int acc = (flags & NAIWA_PREFILL_ACCUMULATE) ? 1 : 0;
    const unsigned cs4 = (unsigned)((H / 4 + kThreads - 1) / kThreads), cs1 = (unsigned)((H + kThreads - 1) / kThreads);
    uint16_t* res = (flags & NAIWA_PREFILL_RESIDUAL) ? (uint16_t*)const_cast<void*>(x) : nullptr;
    if (((uintptr_t)out & 15) == 0)
        combine_kernel<4><<<dim3(T, cs4), kThreads, 0, st>>>(ypair, slot_ids, k, H, slots, acc, out, res);
    else
        combine_kernel<1><<<dim3(T, cs1), kThreads, 0, st>>>(ypair, slot_ids, k, H, slots, acc, out, res);
    return naiwa_hip_rc(hipGetLastError());
}
