// naiwa_moe_gather: the token->expert gather as a stable counting sort by
// expert id.  The reference groups hits per bank in row-major order
// (src/moe/stages/gpu.rs:100-133); here every (token, k) pair of a step is
// grouped by expert id, ties kept in flat index order, so the permutation and
// the per-expert offsets are bit-exact against the CPU counting sort.
#include "segments.h"

namespace {

__global__ void __launch_bounds__(NAIWA_SEG_THREADS)
gather_kernel(const uint32_t* ids, int n, int E, uint32_t* perm, uint32_t* offsets, int* bad) {
    __shared__ NaiwaSegSmem sm;
    naiwa_segment(sm, ids, nullptr, n, E, perm, offsets, nullptr, nullptr, nullptr, bad);
}

} // namespace

extern "C" int naiwa_moe_gather(const uint32_t* ids, int n, int E, uint32_t* perm_out,
                                uint32_t* offsets_out, int* bad_out, int64_t stream) {
    if (n < 0 || n > 65536 || E <= 0 || E > NAIWA_SEG_MAX_KEYS) return NAIWA_E_INVALID;
    if (!offsets_out || (n > 0 && (!ids || !perm_out))) return NAIWA_E_INVALID;
    gather_kernel<<<1, NAIWA_SEG_THREADS, 0, (hipStream_t)stream>>>(ids, n, E, perm_out, offsets_out,
                                                                     bad_out);
    return naiwa_hip_rc(hipGetLastError());
}
