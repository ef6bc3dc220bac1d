// NAIWA_STACK_FUSED: one persistent, cooperatively launched kernel runs a
// whole decode step through every MoE layer, x <- bf16(x + MoE_l(x)).
//
// Per layer, with every block resident (grid = CUs x blocks per CU):
//   A  route   every block reads the layer's router logits (int64 fixed-point
//              sums, see below), selects the top-k in one wave per token and
//              groups the (token, k) pairs by cache slot -- redundantly and
//              identically in every block, so no barrier is needed for it;
//   B  gate/up the (segment, intermediate row) pairs are dealt out evenly to
//              the blocks; each 16-lane group streams one gate and one up row
//              with 16-byte loads and writes h = act(g) * u (f32) per pair;
//   -- grid barrier --
//   C  down    each block owns 8 consecutive output features: it stages the
//              h vectors, dots every (feature, pair), adds the pairs of each
//              token in ascending slot order (no atomics), applies the
//              residual, stores bf16 x, and adds the next layer's router
//              partial sums for its 8 features;
//   -- grid barrier --
// Router logits: each chunk of 8 features is an f32 fma chain rounded to
// int64 with 32 fractional bits; chunks are added with integer atomics.
// Integer addition is associative, so the logits (and the top-k) are bit-
// identical to the CPU oracle's whatever order the blocks finish in.
#include <mutex>
#include <string.h>
#include <vector>

#include "router.h"
#include "rowdot.h"
#include "workspace.h"

namespace {

constexpr int kThreads = 256;           // 4 waves, 16 groups of 16 lanes
constexpr int kGroups = kThreads / NAIWA_GROUP;
constexpr int kMaxRows = 8;             // tokens per step served by this kernel
constexpr int kMaxK = 8;                // routed experts per token
constexpr int kMaxPairs = kMaxRows * kMaxK;
constexpr int kMaxE = 256;
constexpr int kChunk = NAIWA_ROUTER_CHUNK; // output features per phase-C block
constexpr int kCPairs = 16;             // h vectors staged per phase-C pass

struct LayerDev {
    const float* router;
    const uint8_t* gate;
    const uint8_t* up;
    const uint8_t* down;
    int64_t gate_stride, up_stride, down_stride;
    const int32_t* slot_of;
    int32_t slots;
    int32_t pad;
};

struct Params {
    const LayerDev* layers;
    int n_layers, rows, H, I, E, k, mode, act;
    uint16_t* x;                 // [rows, H] bf16, in/out
    float* h;                    // [kMaxPairs, I] f32
    unsigned long long* logit;   // [n_layers, rows, E] int64 fixed point
    unsigned int* bar;           // barrier counter
    int* status;                 // [0] barrier timeouts, [1] missing experts
    uint32_t* ids_out;           // [n_layers, rows, k] or null
    float* w_out;
    uint64_t spin_limit;         // wall-clock ticks before a barrier gives up
};

struct Smem {
    uint32_t pair_slot[kMaxPairs]; // slot of pair p = t*k + j
    float pair_w[kMaxPairs];
    uint32_t sorted[kMaxPairs];    // pairs in (slot, p) order
    uint32_t seg_begin[kMaxPairs + 1];
    int nseg;
    float partial[kChunk][kMaxPairs];
    float xnew[kMaxRows][kChunk];
};

__device__ __forceinline__ void grid_barrier(const Params& p, unsigned int& gen) {
    gen += gridDim.x;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(p.bar, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t t0 = wall_clock64();
        while (__hip_atomic_load(p.bar, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < gen) {
            if (wall_clock64() - t0 > p.spin_limit) {
                atomicAdd(&p.status[0], 1);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
    __threadfence();
}

// Router partial sums of the features [f0, f0 + kChunk) for every (token, expert).
__device__ inline void router_partials(const Params& p, const float* W, int layer, int f0,
                                       const float (*xv)[kChunk]) {
    unsigned long long* acc = p.logit + (size_t)layer * p.rows * p.E;
    for (int it = threadIdx.x; it < p.rows * p.E; it += kThreads) {
        const int t = it / p.E, e = it % p.E;
        const long long v = naiwa_router_chunk(W + (size_t)e * p.H + f0, xv[t]);
        if (v) atomicAdd(&acc[it], (unsigned long long)v);
        (void)t;
    }
}

template <int DG, int DD>
__global__ void __launch_bounds__(kThreads)
stack_kernel(Params p) {
    extern __shared__ __align__(16) uint8_t dyn[];
    __shared__ Smem sm;
    const int tid = threadIdx.x, grp = tid / NAIWA_GROUP, lr = tid % NAIWA_GROUP;
    const int lane = tid & 63, wave = tid >> 6;
    const int G = gridDim.x, bid = blockIdx.x;
    const int H = p.H, I = p.I, E = p.E, k = p.k, rows = p.rows;
    const int npairs = rows * k;
    const int xstage = naiwa_stage_bytes(DG, H);
    const int hstage = naiwa_stage_bytes(DD, I);
    unsigned int gen = 0;

    // ---- prologue: zero the logit accumulators, then layer 0's partials ----
    {
        const size_t n = (size_t)p.n_layers * rows * E;
        for (size_t i = (size_t)bid * kThreads + tid; i < n; i += (size_t)G * kThreads) p.logit[i] = 0ull;
    }
    grid_barrier(p, gen);
    for (int c = bid; c < H / kChunk; c += G) {
        __shared__ float x0[kMaxRows][kChunk];
        if (tid < rows * kChunk) {
            const int t = tid / kChunk, i = tid % kChunk;
            x0[t][i] = naiwa_bf16_to_f32(p.x[(size_t)t * H + c * kChunk + i]);
        }
        __syncthreads();
        router_partials(p, p.layers[0].router, 0, c * kChunk, x0);
        __syncthreads();
    }
    grid_barrier(p, gen);

    for (int l = 0; l < p.n_layers; ++l) {
        const LayerDev L = p.layers[l];
        // ---- A: route (every block, identically) ----
        unsigned long long* acc = p.logit + (size_t)l * rows * E;
        for (int t = wave; t < rows; t += kThreads / 64) {
            __shared__ float lg[kThreads / 64][kMaxE];
            for (int e = lane; e < E; e += 64)
                lg[wave][e] = naiwa_router_fix_to_f32((long long)__hip_atomic_load(
                    &acc[(size_t)t * E + e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            __builtin_amdgcn_wave_barrier();
            __shared__ uint32_t tid_ids[kMaxRows][kMaxK];
            __shared__ float tid_w[kMaxRows][kMaxK];
            naiwa_wave_topk(lg[wave], E, k, p.mode, tid_ids[t], tid_w[t]);
            __builtin_amdgcn_wave_barrier();
            if (lane < k) {
                const uint32_t e = tid_ids[t][lane];
                const int32_t s = L.slot_of ? L.slot_of[e] : (int32_t)e;
                const bool ok = s >= 0 && s < L.slots;
                sm.pair_slot[t * k + lane] = ok ? (uint32_t)s : 0u;
                sm.pair_w[t * k + lane] = ok ? tid_w[t][lane] : 0.0f;
                if (!ok && bid == 0) atomicAdd(&p.status[1], 1);
                if (bid == 0 && p.ids_out) {
                    p.ids_out[((size_t)l * rows + t) * k + lane] = e;
                    p.w_out[((size_t)l * rows + t) * k + lane] = tid_w[t][lane];
                }
            }
        }
        __syncthreads();
        // rank of pair q in (slot, q) order; zero-weight pairs are dropped
        if (wave == 0) {
            for (int q = lane; q < npairs; q += 64) {
                if (sm.pair_w[q] == 0.0f) continue;
                const uint32_t sq = sm.pair_slot[q];
                int rank = 0;
                for (int o = 0; o < npairs; ++o) {
                    if (sm.pair_w[o] == 0.0f) continue;
                    const uint32_t so = sm.pair_slot[o];
                    rank += so < sq || (so == sq && o < q);
                }
                sm.sorted[rank] = (uint32_t)q;
            }
        }
        __syncthreads();
        if (tid == 0) {
            int nvalid = 0;
            for (int q = 0; q < npairs; ++q) nvalid += sm.pair_w[q] != 0.0f;
            int ns = 0;
            for (int i = 0; i < nvalid; ++i) {
                if (i == 0 || sm.pair_slot[sm.sorted[i]] != sm.pair_slot[sm.sorted[i - 1]])
                    sm.seg_begin[ns++] = (uint32_t)i;
            }
            sm.seg_begin[ns] = (uint32_t)nvalid;
            sm.nseg = ns;
        }
        // stage x of every token (bf16 source)
        for (int t = 0; t < rows; ++t) {
            uint32_t* words = (uint32_t*)(dyn + t * xstage);
            naiwa_stage<DG>(p.x + (size_t)t * H, true, H, words, (float*)(words + H / 2), tid, kThreads);
        }
        __syncthreads();

        // ---- B: gate/up, rows dealt out evenly ----
        {
            const int nseg = sm.nseg;
            const int total = nseg * I;
            const int per = (total + G - 1) / G;
            const int q0 = bid * per, q1 = min(total, q0 + per);
            const int64_t rb = naiwa_row_bytes(DG == NAIWA_Q8_0_ODD ? NAIWA_Q8_0 : DG, H);
            const int nu = Fmt<DG>::units(H);
            constexpr int UM = Umax<DG>::v;
            for (int q = q0 + grp; q < q1; q += kGroups) {
                const int s = q / I, r = q % I;
                const uint32_t slot = sm.pair_slot[sm.sorted[sm.seg_begin[s]]];
                const uint8_t* grow = L.gate + (int64_t)slot * L.gate_stride + (int64_t)r * rb;
                const uint8_t* urow = L.up + (int64_t)slot * L.up_stride + (int64_t)r * rb;
                const int b = (int)sm.seg_begin[s], e = (int)sm.seg_begin[s + 1];
                float ag[kMaxRows], au[kMaxRows];
#pragma unroll
                for (int i = 0; i < kMaxRows; ++i) ag[i] = au[i] = 0.0f;
                for (int base = lr; base < nu; base += NAIWA_GROUP * UM) {
                    typename Fmt<DG>::Frag fg[UM], fu[UM];
#pragma unroll
                    for (int i = 0; i < UM; ++i) {
                        const int u = base + NAIWA_GROUP * i;
                        if (u < nu) {
                            fg[i] = Fmt<DG>::load(grow, u);
                            fu[i] = Fmt<DG>::load(urow, u);
                        }
                    }
#pragma unroll
                    for (int i = 0; i < UM; ++i) {
                        const int u = base + NAIWA_GROUP * i;
                        if (u >= nu) continue;
#pragma unroll
                        for (int tt = 0; tt < kMaxRows; ++tt) {
                            if (b + tt >= e) break;
                            const int t = (int)sm.sorted[b + tt] / k;
                            const uint32_t* words = (const uint32_t*)(dyn + t * xstage);
                            const float* sums = (const float*)(words + H / 2);
                            ag[tt] += Fmt<DG>::dot(fg[i], u, words, sums);
                            au[tt] += Fmt<DG>::dot(fu[i], u, words, sums);
                        }
                    }
                }
#pragma unroll
                for (int tt = 0; tt < kMaxRows; ++tt) {
                    if (b + tt >= e) break;
                    const float gv = naiwa_group_sum<NAIWA_GROUP>(ag[tt]);
                    const float uv = naiwa_group_sum<NAIWA_GROUP>(au[tt]);
                    if (lr == 0) p.h[(size_t)sm.sorted[b + tt] * I + r] = naiwa_act(p.act, gv) * uv;
                }
            }
        }
        grid_barrier(p, gen);

        // ---- C: down + ordered combine + residual + next router partials ----
        const int64_t drb = naiwa_row_bytes(DD == NAIWA_Q8_0_ODD ? NAIWA_Q8_0 : DD, I);
        const int nvalid = (int)sm.seg_begin[sm.nseg];
        for (int c = bid; c < H / kChunk; c += G) {
            const int f0 = c * kChunk;
            for (int b0 = 0; b0 < nvalid; b0 += kCPairs) {
                const int nb = min(kCPairs, nvalid - b0);
                __syncthreads();
                for (int i = 0; i < nb; ++i) {
                    uint32_t* words = (uint32_t*)(dyn + i * hstage);
                    naiwa_stage<DD>(p.h + (size_t)sm.sorted[b0 + i] * I, false, I, words,
                                    (float*)(words + I / 2), tid, kThreads);
                }
                __syncthreads();
                // (feature, staged pair) items over the 16 groups
                for (int it = grp; it < kChunk * nb; it += kGroups) {
                    const int fi = it % kChunk, pi = it / kChunk;
                    const uint32_t pr = sm.sorted[b0 + pi];
                    const uint8_t* drow = L.down + (int64_t)sm.pair_slot[pr] * L.down_stride +
                                          (int64_t)(f0 + fi) * drb;
                    const uint32_t* words = (const uint32_t*)(dyn + pi * hstage);
                    const float v = naiwa_row_dot<DD, Umax<DD>::v>(drow, I, words,
                                                                  (const float*)(words + I / 2), lr);
                    if (lr == 0) sm.partial[fi][b0 + pi] = v;
                }
            }
            __syncthreads();
            if (tid < rows * kChunk) {
                const int t = tid / kChunk, fi = tid % kChunk;
                float y = 0.0f;
                for (int i = 0; i < nvalid; ++i) {
                    const uint32_t pr = sm.sorted[i];
                    if ((int)pr / k == t) y += sm.pair_w[pr] * sm.partial[fi][i];
                }
                uint16_t* xp = p.x + (size_t)t * H + f0 + fi;
                const float xn = naiwa_bf16_to_f32(naiwa_f32_to_bf16(naiwa_bf16_to_f32(*xp) + y));
                *xp = (uint16_t)naiwa_f32_to_bf16(xn);
                sm.xnew[t][fi] = xn;
            }
            __syncthreads();
            if (l + 1 < p.n_layers) router_partials(p, p.layers[l + 1].router, l + 1, f0, sm.xnew);
        }
        grid_barrier(p, gen);
    }
}

struct FusedCache {
    std::mutex mu;
    LayerDev* dev_layers = nullptr;
    size_t cap = 0;
    std::vector<LayerDev> last;
};
FusedCache g_fused;

template <int DG, int DD>
int launch(const Params& prm, int blocks, size_t lds, hipStream_t st) {
    auto fn = stack_kernel<DG, DD>;
    Params copy = prm;
    void* args[] = {&copy};
    hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    e = hipLaunchCooperativeKernel((const void*)fn, dim3(blocks), dim3(kThreads), args, (unsigned)lds, st);
    return naiwa_hip_rc(e);
}

template <int DG, int DD>
int occupancy(size_t lds, int* per_cu) {
    return naiwa_hip_rc(hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, stack_kernel<DG, DD>,
                                                                     kThreads, lds));
}

__global__ void zero_u32(unsigned int* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

} // namespace

static int g_fused_blocks_per_cu = 2;

extern "C" int naiwa_stack_set_blocks_per_cu(int n) {
    if (n < 1 || n > 8) return NAIWA_E_INVALID;
    g_fused_blocks_per_cu = n;
    return NAIWA_OK;
}

// Status of the last fused launches: barrier timeouts and routed experts that
// had no resident slot.  Synchronizes the device.
extern "C" int naiwa_stack_status(int* barrier_timeouts, int* missing_experts) {
    int rc = 0;
    int* status = (int*)naiwa_scratch(NAIWA_SCRATCH_STACK + 1, 4096, &rc);
    if (!status) return rc;
    int h[2] = {0, 0};
    hipError_t e = hipMemcpy(h, status, sizeof(h), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return (int)e;
    if (barrier_timeouts) *barrier_timeouts = h[0];
    if (missing_experts) *missing_experts = h[1];
    return NAIWA_OK;
}

int naiwa_stack_fused(const naiwa_layer* layers, int n_layers, void* x, int rows, int H, int E, int k,
                      int mode, int act, uint32_t* ids_out, float* w_out, int64_t stream) {
    if (rows > kMaxRows || k > kMaxK || E > kMaxE) return NAIWA_E_UNSUPPORTED;
    if (H % kChunk || (ids_out == nullptr) != (w_out == nullptr)) return NAIWA_E_INVALID;
    if (mode < 0 || mode > 2 || (act != NAIWA_ACT_SILU && act != NAIWA_ACT_GELU_PYTORCH_TANH))
        return NAIWA_E_UNSUPPORTED;
    const naiwa_layer& L0 = layers[0];
    const int I = L0.gate.n;
    for (int l = 0; l < n_layers; ++l) {
        const naiwa_layer& L = layers[l];
        if (!L.router || !L.gate.base || !L.up.base || !L.down.base) return NAIWA_E_INVALID;
        if (L.gate.k != H || L.up.k != H || L.down.n != H || L.gate.n != I || L.up.n != I || L.down.k != I)
            return NAIWA_E_INVALID;
        if (L.gate.dtype != L0.gate.dtype || L.up.dtype != L0.gate.dtype || L.down.dtype != L0.down.dtype)
            return NAIWA_E_UNSUPPORTED;
        if (L.gate.slots != L.up.slots || L.gate.slots != L.down.slots) return NAIWA_E_INVALID;
        if (!L.slot_of_expert && L.gate.slots < E) return NAIWA_E_INVALID;
        const int64_t rg = naiwa_row_bytes(L.gate.dtype, H), rd = naiwa_row_bytes(L.down.dtype, I);
        if (rg < 0 || rd < 0 || L.gate.slot_stride < rg * I || L.up.slot_stride < rg * I ||
            L.down.slot_stride < rd * H)
            return NAIWA_E_INVALID;
        if (((uintptr_t)L.gate.base | (uintptr_t)L.up.base | (uintptr_t)L.down.base | L.gate.slot_stride |
             L.up.slot_stride | L.down.slot_stride) & 15)
            return NAIWA_E_INVALID;
        if (((uintptr_t)L.router & 15) || H % 32 || I % 32) return NAIWA_E_INVALID;
    }
    const int fg = naiwa_kernel_fmt(L0.gate.dtype, H), fd = naiwa_kernel_fmt(L0.down.dtype, I);
    if (fg == NAIWA_Q8_0_ODD) return NAIWA_E_UNSUPPORTED;
    const size_t lds_x = (size_t)rows * naiwa_stage_bytes(fg, H);
    const size_t lds_h = (size_t)kCPairs * naiwa_stage_bytes(fd, I);
    const size_t lds = lds_x > lds_h ? lds_x : lds_h;
    if (lds > 96 * 1024) return NAIWA_E_UNSUPPORTED;

    hipStream_t st = (hipStream_t)stream;
    int rc = 0;
    // scratch: h [kMaxPairs * I] f32 | logits [n_layers * rows * E] int64
    const size_t h_bytes = ((size_t)kMaxPairs * I * 4 + 255) & ~size_t(255);
    const size_t lg_bytes = (size_t)n_layers * rows * E * 8;
    uint8_t* ws = (uint8_t*)naiwa_scratch(NAIWA_SCRATCH_STACK, h_bytes + lg_bytes, &rc);
    if (!ws) return rc;
    int* misc = (int*)naiwa_scratch(NAIWA_SCRATCH_STACK + 1, 4096, &rc);
    if (!misc) return rc;

    // layer descriptors on the device (re-uploaded only when they change)
    std::vector<LayerDev> desc(n_layers);
    for (int l = 0; l < n_layers; ++l) {
        const naiwa_layer& L = layers[l];
        desc[l] = LayerDev{L.router, (const uint8_t*)L.gate.base, (const uint8_t*)L.up.base,
                           (const uint8_t*)L.down.base, L.gate.slot_stride, L.up.slot_stride,
                           L.down.slot_stride, L.slot_of_expert, L.gate.slots, 0};
    }
    LayerDev* dev_layers = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_fused.mu);
        const size_t bytes = desc.size() * sizeof(LayerDev);
        if (g_fused.cap < bytes) {
            if (g_fused.dev_layers) {
                hipError_t e = hipDeviceSynchronize();
                if (e != hipSuccess) return (int)e;
                (void)hipFree(g_fused.dev_layers);
            }
            g_fused.dev_layers = nullptr;
            g_fused.cap = 0;
            g_fused.last.clear();
            if (hipMalloc(&g_fused.dev_layers, bytes) != hipSuccess) return NAIWA_E_NOMEM;
            g_fused.cap = bytes;
        }
        if (g_fused.last.size() != desc.size() ||
            memcmp(g_fused.last.data(), desc.data(), bytes) != 0) {
            hipError_t e = hipMemcpy(g_fused.dev_layers, desc.data(), bytes, hipMemcpyHostToDevice);
            if (e != hipSuccess) return (int)e;
            g_fused.last = desc;
        }
        dev_layers = g_fused.dev_layers;
    }

    int dev = 0, cus = 0, khz = 0;
    if ((rc = naiwa_hip_rc(hipGetDevice(&dev)))) return rc;
    if ((rc = naiwa_hip_rc(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)))) return rc;
    if ((rc = naiwa_hip_rc(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev)))) return rc;
    int per_cu = 0;
    if (fg == NAIWA_Q4_K && fd == NAIWA_Q4_K) rc = occupancy<NAIWA_Q4_K, NAIWA_Q4_K>(lds, &per_cu);
    else if (fg == NAIWA_Q4_K && fd == NAIWA_Q8_0) rc = occupancy<NAIWA_Q4_K, NAIWA_Q8_0>(lds, &per_cu);
    else if (fg == NAIWA_Q4_K && fd == NAIWA_Q8_0_ODD) rc = occupancy<NAIWA_Q4_K, NAIWA_Q8_0_ODD>(lds, &per_cu);
    else if (fg == NAIWA_Q8_0 && fd == NAIWA_Q8_0) rc = occupancy<NAIWA_Q8_0, NAIWA_Q8_0>(lds, &per_cu);
    else if (fg == NAIWA_Q8_0 && fd == NAIWA_Q8_0_ODD) rc = occupancy<NAIWA_Q8_0, NAIWA_Q8_0_ODD>(lds, &per_cu);
    else return NAIWA_E_UNSUPPORTED;
    if (rc) return rc;
    const int bpc = per_cu < g_fused_blocks_per_cu ? per_cu : g_fused_blocks_per_cu;
    if (bpc < 1) return NAIWA_E_UNSUPPORTED;
    const int blocks = cus * bpc;

    Params prm;
    prm.layers = dev_layers;
    prm.n_layers = n_layers;
    prm.rows = rows;
    prm.H = H;
    prm.I = I;
    prm.E = E;
    prm.k = k;
    prm.mode = mode;
    prm.act = act;
    prm.x = (uint16_t*)x;
    prm.h = (float*)ws;
    prm.logit = (unsigned long long*)(ws + h_bytes);
    prm.bar = (unsigned int*)(misc + 16);
    prm.status = misc;
    prm.ids_out = ids_out;
    prm.w_out = w_out;
    prm.spin_limit = (uint64_t)khz * 2000ull; // 2 s
    zero_u32<<<1, 64, 0, st>>>((unsigned int*)misc, 32);
    if (fg == NAIWA_Q4_K && fd == NAIWA_Q4_K) return launch<NAIWA_Q4_K, NAIWA_Q4_K>(prm, blocks, lds, st);
    if (fg == NAIWA_Q4_K && fd == NAIWA_Q8_0) return launch<NAIWA_Q4_K, NAIWA_Q8_0>(prm, blocks, lds, st);
    if (fg == NAIWA_Q4_K && fd == NAIWA_Q8_0_ODD) return launch<NAIWA_Q4_K, NAIWA_Q8_0_ODD>(prm, blocks, lds, st);
    if (fg == NAIWA_Q8_0 && fd == NAIWA_Q8_0) return launch<NAIWA_Q8_0, NAIWA_Q8_0>(prm, blocks, lds, st);
    return launch<NAIWA_Q8_0, NAIWA_Q8_0_ODD>(prm, blocks, lds, st);
}
