// The CPU expert path for cache misses the staging ring does not take: the
// contract of the reference's fused_moe_decode (src/moe/stages/cpu_miss.rs:13-20,
// called at :45): rows of f32 activations, each with `width` (expert, weight)
// pairs; pass 1 computes h = act(gate . x) * (up . x) for every distinct
// (expert, row) with a nonzero weight, pass 2 adds w * (down . h) per row in
// the pairs' order.  Weights are the GGUF blocks of the host expert stacks
// (Q4_K or Q8_0), dequantised on the fly against f32 activations.
//
// Work is split over a persistent pool of host threads: pass 1 by (pair, chunk
// of intermediate rows), pass 2 by (row, chunk of output features), so every
// output element is written by exactly one task and sums in a fixed order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

#include "../../include/naiwa_cached.h"
#include "common.h"

namespace {

float f16_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else { // subnormal: normalise
            e = 127 - 15 + 1;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                --e;
            }
            bits = s | (e << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = s | 0x7F800000u | (m << 13);
    } else {
        bits = s | ((e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

inline uint16_t ld16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// Scale and min of sub-block j (0..7) of a Q4_K block header (GGML get_scale_min_k4).
inline void q4k_scale_min(const uint8_t* sc, int j, int* s, int* m) {
    if (j < 4) {
        *s = sc[j] & 63;
        *m = sc[j + 4] & 63;
    } else {
        *s = (sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4);
        *m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

// ---- dots of one quantized row with f32 activations -------------------------------

// sums[j]: the sum of the activations of 32-value group j (Q4_K's min term).
float dot_q4k_scalar(const uint8_t* row, const float* x, const float* sums, int k) {
    float acc = 0.0f;
    for (int b = 0; b < k / 256; ++b) {
        const uint8_t* blk = row + 144 * b;
        const float d = f16_to_f32(ld16(blk)), dmin = f16_to_f32(ld16(blk + 2));
        const uint8_t* sc = blk + 4;
        const uint8_t* qs = blk + 16;
        const float* xb = x + 256 * b;
        for (int c = 0; c < 4; ++c) {
            float lo = 0.0f, hi = 0.0f;
            for (int i = 0; i < 32; ++i) {
                lo += (float)(qs[32 * c + i] & 0x0F) * xb[64 * c + i];
                hi += (float)(qs[32 * c + i] >> 4) * xb[64 * c + 32 + i];
            }
            int s0, m0, s1, m1;
            q4k_scale_min(sc, 2 * c, &s0, &m0);
            q4k_scale_min(sc, 2 * c + 1, &s1, &m1);
            acc += d * ((float)s0 * lo + (float)s1 * hi) -
                   dmin * ((float)m0 * sums[8 * b + 2 * c] + (float)m1 * sums[8 * b + 2 * c + 1]);
        }
    }
    return acc;
}

float dot_q8_0_scalar(const uint8_t* row, const float* x, int k) {
    float acc = 0.0f;
    for (int b = 0; b < k / 32; ++b) {
        const uint8_t* blk = row + 34 * b;
        const float d = f16_to_f32(ld16(blk));
        const int8_t* q = (const int8_t*)(blk + 2);
        float s = 0.0f;
        for (int i = 0; i < 32; ++i) s += (float)q[i] * x[32 * b + i];
        acc += d * s;
    }
    return acc;
}

#if defined(__x86_64__)
__attribute__((target("avx2,fma"))) inline float hsum8(__m256 v) {
    const __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    const __m128 t = _mm_add_ps(s, _mm_movehl_ps(s, s));
    return _mm_cvtss_f32(_mm_add_ss(t, _mm_movehdup_ps(t)));
}

// 32 unsigned bytes (0..15) times 32 floats.
__attribute__((target("avx2,fma"))) inline __m256 dot32_u8(__m256i q, const float* x) {
    const __m128i lo = _mm256_castsi256_si128(q), hi = _mm256_extracti128_si256(q, 1);
    __m256 a = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(lo)), _mm256_loadu_ps(x));
    a = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(lo, 8))), _mm256_loadu_ps(x + 8), a);
    a = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(hi)), _mm256_loadu_ps(x + 16), a);
    a = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(hi, 8))), _mm256_loadu_ps(x + 24), a);
    return a;
}

// Q4_K: the 8-lane partial dots of each 32-value sub-block are scaled by d * scale
// and kept in one vector accumulator (one horizontal sum per row); the min terms
// (dmin * min * group sum) are summed apart and subtracted at the end.
__attribute__((target("avx2,fma,f16c"))) float dot_q4k_avx2(const uint8_t* row, const float* x, const float* sums,
                                                          int k) {
    const __m256i mask = _mm256_set1_epi8(0x0F);
    __m256 acc = _mm256_setzero_ps();
    float macc = 0.0f;
    for (int b = 0; b < k / 256; ++b) {
        const uint8_t* blk = row + 144 * b;
        const float d = _cvtsh_ss(ld16(blk)), dmin = _cvtsh_ss(ld16(blk + 2));
        const uint8_t* sc = blk + 4;
        const float* xb = x + 256 * b;
        int s[8], m[8];
        float ms = 0.0f;
        for (int j = 0; j < 8; ++j) {
            q4k_scale_min(sc, j, &s[j], &m[j]);
            ms += (float)m[j] * sums[8 * b + j];
        }
        macc += dmin * ms;
        for (int c = 0; c < 4; ++c) {
            const __m256i q = _mm256_loadu_si256((const __m256i*)(blk + 16 + 32 * c));
            const __m256 lo = dot32_u8(_mm256_and_si256(q, mask), xb + 64 * c);
            const __m256 hi = dot32_u8(_mm256_and_si256(_mm256_srli_epi16(q, 4), mask), xb + 64 * c + 32);
            acc = _mm256_fmadd_ps(lo, _mm256_set1_ps(d * (float)s[2 * c]), acc);
            acc = _mm256_fmadd_ps(hi, _mm256_set1_ps(d * (float)s[2 * c + 1]), acc);
        }
    }
    return hsum8(acc) - macc;
}

__attribute__((target("avx2,fma,f16c"))) float dot_q8_0_avx2(const uint8_t* row, const float* x, int k) {
    __m256 acc = _mm256_setzero_ps();
    for (int b = 0; b < k / 32; ++b) {
        const uint8_t* blk = row + 34 * b;
        const __m256 d = _mm256_set1_ps(_cvtsh_ss(ld16(blk)));
        const __m128i q0 = _mm_loadu_si128((const __m128i*)(blk + 2)), q1 = _mm_loadu_si128((const __m128i*)(blk + 18));
        __m256 s = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(q0)), _mm256_loadu_ps(x + 32 * b));
        s = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(q0, 8))), _mm256_loadu_ps(x + 32 * b + 8), s);
        s = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(q1)), _mm256_loadu_ps(x + 32 * b + 16), s);
        s = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(q1, 8))), _mm256_loadu_ps(x + 32 * b + 24), s);
        acc = _mm256_fmadd_ps(d, s, acc);
    }
    return hsum8(acc);
}

bool have_avx2() {
    static const bool v =
        __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c");
    return v;
}
#endif

// The dot of row `row` (K values, format dt) with x; sums: 32-value group sums of x.
float row_dot(int dt, const uint8_t* row, const float* x, const float* sums, int k) {
#if defined(__x86_64__)
    if (have_avx2()) return dt == NAIWA_Q4_K ? dot_q4k_avx2(row, x, sums, k) : dot_q8_0_avx2(row, x, k);
#endif
    return dt == NAIWA_Q4_K ? dot_q4k_scalar(row, x, sums, k) : dot_q8_0_scalar(row, x, k);
}

void group_sums(const float* x, int k, float* sums) {
    for (int j = 0; j < k / 32; ++j) {
        float s = 0.0f;
        for (int i = 0; i < 32; ++i) s += x[32 * j + i];
        sums[j] = s;
    }
}

float act_fn(int act, float g) {
    if (act == NAIWA_ACT_GELU_PYTORCH_TANH) {
        const float k0 = 0.7978845608028654f, k1 = 0.044715f;
        return 0.5f * g * (1.0f + std::tanh(k0 * (g + k1 * g * g * g)));
    }
    return g / (1.0f + std::exp(-g));
}

// ---- a persistent pool of host threads -------------------------------------------------

class Pool {
  public:
    static Pool& get() {
        static Pool p;
        return p;
    }
    // fn(i) for i in [0, n) over the workers and the caller; returns when all are done.
    // One parallel_for at a time (callers are serialised).
    void parallel_for(int n, const std::function<void(int)>& fn) {
        std::lock_guard<std::mutex> call(call_mu_);
        if (workers_.empty() || n <= 1) {
            for (int i = 0; i < n; ++i) fn(i);
            return;
        }
        {
            std::lock_guard<std::mutex> lock(mu_);
            fn_ = &fn;
            n_ = n;
            next_.store(0);
            done_ = 0;
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> lock(mu_);
        done_cv_.wait(lock, [&] { return done_ == (int)workers_.size(); });
        fn_ = nullptr;
    }

  private:
    Pool() {
        const unsigned hw = std::thread::hardware_concurrency();
        const int n = (int)std::min(31u, hw > 1 ? hw - 1 : 0u);
        for (int i = 0; i < n; ++i) workers_.emplace_back([this] { loop(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> lock(mu_);
            stop_ = true;
            ++gen_;
        }
        cv_.notify_all();
        for (auto& t : workers_) t.join();
    }
    void work() {
        for (int i = next_.fetch_add(1); i < n_; i = next_.fetch_add(1)) (*fn_)(i);
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lock(mu_);
                cv_.wait(lock, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
            }
            work();
            {
                std::lock_guard<std::mutex> lock(mu_);
                ++done_;
            }
            done_cv_.notify_one();
        }
    }
    std::mutex call_mu_, mu_;
    std::condition_variable cv_, done_cv_;
    std::vector<std::thread> workers_;
    const std::function<void(int)>* fn_ = nullptr;
    std::atomic<int> next_{0};
    int n_ = 0, done_ = 0;
    uint64_t gen_ = 0;
    bool stop_ = false;
};

bool fmt_ok(int dt, int k) {
    return (dt == NAIWA_Q4_K && k % 256 == 0) || (dt == NAIWA_Q8_0 && k % 32 == 0);
}

} // namespace

extern "C" int naiwa_cpu_moe_decode(const naiwa_host_experts* ex, const float* xs, const uint32_t* ids,
                                    const float* w, int rows, int width, int act, float* out) {
    if (!ex || !xs || !out || rows < 0 || width < 0 || (rows * width > 0 && (!ids || !w))) return NAIWA_E_INVALID;
    if (!ex->gate || !ex->up || !ex->down || ex->num_experts <= 0 || ex->hidden <= 0 || ex->inter <= 0)
        return NAIWA_E_INVALID;
    if (act != NAIWA_ACT_SILU && act != NAIWA_ACT_GELU_PYTORCH_TANH) return NAIWA_E_UNSUPPORTED;
    const int H = ex->hidden, I = ex->inter;
    if (!fmt_ok(ex->gate_dtype, H) || !fmt_ok(ex->up_dtype, H) || !fmt_ok(ex->down_dtype, I))
        return NAIWA_E_UNSUPPORTED;
    for (int i = 0; i < rows * width; ++i)
        if (ids[i] >= (uint32_t)ex->num_experts) return NAIWA_E_BAD_ID;
    const int64_t rg = naiwa_row_bytes(ex->gate_dtype, H), ru = naiwa_row_bytes(ex->up_dtype, H),
                  rd = naiwa_row_bytes(ex->down_dtype, I);
    const int64_t sg = ex->gate_stride ? ex->gate_stride : rg * I, su = ex->up_stride ? ex->up_stride : ru * I,
                  sd = ex->down_stride ? ex->down_stride : rd * H;

    // the distinct (expert, row) pairs with a nonzero weight, in row-major order
    std::vector<int> pair_of((size_t)rows * width, -1);
    std::vector<std::pair<uint32_t, int>> pairs; // (expert, row)
    for (int t = 0; t < rows; ++t)
        for (int j = 0; j < width; ++j) {
            const int q = t * width + j;
            if (w[q] == 0.0f) continue;
            int found = -1;
            for (int jj = 0; jj < j; ++jj) {
                const int qq = t * width + jj;
                if (w[qq] != 0.0f && ids[qq] == ids[q]) found = pair_of[(size_t)qq];
            }
            if (found < 0) {
                found = (int)pairs.size();
                pairs.emplace_back(ids[q], t);
            }
            pair_of[(size_t)q] = found;
        }
    std::vector<float> xsum((size_t)rows * (H / 32));
    for (int t = 0; t < rows; ++t) group_sums(xs + (size_t)t * H, H, xsum.data() + (size_t)t * (H / 32));

    // pass 1: h[pair] = act(gate . x_row) * (up . x_row), by chunks of intermediate rows
    const int np = (int)pairs.size();
    std::vector<float> h((size_t)np * I), hsum((size_t)np * (I / 32));
    constexpr int kRowsPerTask = 32;
    const int ich = (I + kRowsPerTask - 1) / kRowsPerTask;
    Pool::get().parallel_for(np * ich, [&](int task) {
        const int p = task / ich, c = task % ich;
        const uint32_t e = pairs[(size_t)p].first;
        const int t = pairs[(size_t)p].second;
        const float* x = xs + (size_t)t * H;
        const float* s = xsum.data() + (size_t)t * (H / 32);
        const uint8_t* G = (const uint8_t*)ex->gate + (int64_t)e * sg;
        const uint8_t* U = (const uint8_t*)ex->up + (int64_t)e * su;
        for (int i = c * kRowsPerTask; i < std::min(I, (c + 1) * kRowsPerTask); ++i) {
            const float g = row_dot(ex->gate_dtype, G + i * rg, x, s, H);
            const float u = row_dot(ex->up_dtype, U + i * ru, x, s, H);
            h[(size_t)p * I + i] = act_fn(act, g) * u;
        }
    });
    for (int p = 0; p < np; ++p) group_sums(h.data() + (size_t)p * I, I, hsum.data() + (size_t)p * (I / 32));

    // pass 2: out[row] = sum over the row's pairs (in order) of w * (down . h), by chunks of features
    const int hch = (H + kRowsPerTask - 1) / kRowsPerTask;
    Pool::get().parallel_for(rows * hch, [&](int task) {
        const int t = task / hch, c = task % hch;
        float* y = out + (size_t)t * H;
        for (int f = c * kRowsPerTask; f < std::min(H, (c + 1) * kRowsPerTask); ++f) {
            float acc = 0.0f;
            for (int j = 0; j < width; ++j) {
                const int q = t * width + j;
                const int p = pair_of[(size_t)q];
                if (p < 0) continue;
                const uint8_t* D = (const uint8_t*)ex->down + (int64_t)ids[q] * sd;
                acc += w[q] * row_dot(ex->down_dtype, D + f * rd, h.data() + (size_t)p * I,
                                      hsum.data() + (size_t)p * (I / 32), I);
            }
            y[f] = acc;
        }
    });
    return NAIWA_OK;
}
