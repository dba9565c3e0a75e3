// gefenx_host.cpp -- host-side parts of the C ABI: error state, quantisation
// table construction, exact-DP codebook solver, workspace sizing.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <limits>
#include <thread>
#include <vector>

#include "gefenx_common.h"
#include "gefenx_dp.h"
#include "gefenx_internal.h"
#include "gefenx.h"

namespace gx {

thread_local char g_last_error[512] = "";

int set_error(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

// ------------------------------------------------------------ quantisation

static inline uint32_t f2u(float x) { uint32_t u; std::memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; std::memcpy(&x, &u, 4); return x; }

float round_bf16(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return u2f(u | 0x00400000u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u2f(u & 0xffff0000u);
}

float round_f16(float x) {
    if (std::isnan(x)) return x;
    float a = std::fabs(x);
    if (a >= 65520.0f) return std::copysign(std::numeric_limits<float>::infinity(), x);
    if (a < 2.98023223876953125e-08f) return std::copysign(0.0f, x);
    int e;
    std::frexp(a, &e);
    int ue = std::max(e - 1, -14);
    float ulp = std::ldexp(1.0f, ue - 10);
    return std::copysign(std::nearbyint(a / ulp) * ulp, x);
}

// The reference's nearest-codeword rule for one value (searchsorted 'left',
// then the `|x-c[l]| <= |x-c[r]|` tie to the lower index): gefen.py:288-334.
static int reference_nearest(const float* cb, int k, float x) {
    if (k <= 1) return 0;
    int lo = 0, hi = k;
    while (lo < hi) {
        int mid = lo + ((hi - lo) >> 1);
        if (!(cb[mid] >= x)) lo = mid + 1; else hi = mid;
    }
    int left = std::min(std::max(lo - 1, 0), k - 1);
    int right = std::min(lo, k - 1);
    volatile float dl = std::fabs(x - cb[left]);
    volatile float dr = std::fabs(x - cb[right]);
    return (dl <= dr) ? left : right;
}

// Monotone integer key of a non-NaN float (order-preserving bijection).
static inline int64_t fkey(float x) {
    uint32_t u = f2u(x);
    return (u & 0x80000000u) ? -(int64_t)(u & 0x7fffffffu) - 1 : (int64_t)u;
}
static inline float keyf(int64_t k) {
    return k < 0 ? u2f((uint32_t)(-(k + 1)) | 0x80000000u) : u2f((uint32_t)k);
}

// Kernel bucket of x: clamp(floor((x + 1) * 2048), 0, 4095), evaluated in fp32
// exactly as the device does.
static inline int bucket_of(float x) {
    volatile float t = x + 1.0f;
    volatile float s = t * (float)(kBuckets / 2);
    float f = std::floor(s);
    if (!(f >= 0.0f)) return 0;
    if (f > (float)(kBuckets - 1)) return kBuckets - 1;
    return (int)f;
}

}  // namespace gx

using namespace gx;

extern "C" {

int gefenx_abi_version(void) { return GEFENX_ABI_VERSION; }

const char* gefenx_last_error(void) { return g_last_error; }

size_t gefenx_qtable_bytes(void) { return sizeof(QTable); }

int gefenx_search_lut(const float* codebook, int k, int buckets, int16_t* lut_out) {
    if (!codebook || !lut_out || k < 1 || k > kCodebookMax || buckets < 2)
        return set_error(GEFENX_EINVAL, "gefenx_search_lut: bad arguments (k=%d buckets=%d)", k, buckets);
    // _codebook_search_lut: kernels/automatic_gefen_fused.py:81-121
    std::vector<float> eb((size_t)k);
    for (int i = 0; i < k; ++i) {
        volatile float t = codebook[i] + 1.0f;
        volatile float s = t * (float)(buckets / 2);
        float f = std::floor(s);
        if (!(f >= 0.0f)) f = 0.0f;
        if (f > (float)(buckets - 1)) f = (float)(buckets - 1);
        eb[(size_t)i] = f;
    }
    for (int b = 0; b <= buckets; ++b) {
        int cnt = 0;
        while (cnt < k && eb[(size_t)cnt] < (float)b) ++cnt;  // entries are monotone
        lut_out[b] = (int16_t)cnt;
    }
    return GEFENX_OK;
}

int gefenx_qtable_build(const float* codebook, int k, int dtype, void* table_out) {
    if (!codebook || !table_out)
        return set_error(GEFENX_EINVAL, "gefenx_qtable_build: null pointer");
    if (k < 1 || k > kCodebookMax)
        return set_error(GEFENX_EINVAL, "gefenx_qtable_build: codebook size %d outside [1, 256]", k);
    if (dtype != F32 && dtype != F16 && dtype != BF16)
        return set_error(GEFENX_EDTYPE, "gefenx_qtable_build: unsupported dtype %d", dtype);
    for (int i = 0; i < k; ++i) {
        if (std::isnan(codebook[i]))
            return set_error(GEFENX_EINVAL, "gefenx_qtable_build: codebook[%d] is NaN", i);
        if (i && codebook[i] < codebook[i - 1])
            return set_error(GEFENX_EINVAL, "gefenx_qtable_build: codebook not sorted at %d", i);
    }
    QTable* t = static_cast<QTable*>(table_out);
    std::memset(t, 0, sizeof(QTable));
    t->k = k;
    t->dtype = dtype;
    t->n_thr = k - 1;
    for (int i = 0; i < kCodebookMax; ++i) {
        float c = codebook[std::min(i, k - 1)];
        t->cb[i] = c;
        t->cbr[i] = dtype == BF16 ? round_bf16(c) : dtype == F16 ? round_f16(c) : c;
    }
    // Thresholds: normalised momentum always lies in [-1, 1] (|u| <= max|u|),
    // where the reference rule is monotone non-decreasing in x; thr[i] is the
    // largest x in [-1, 1] whose nearest index is <= i (bisection on the
    // ordered fp32 keys).  -inf when even x = -1 maps above i.
    const int64_t k_lo = fkey(-1.0f), k_hi = fkey(1.0f);
    for (int i = 0; i < k - 1; ++i) {
        float thr;
        if (reference_nearest(codebook, k, 1.0f) <= i) {
            thr = 1.0f;
        } else if (reference_nearest(codebook, k, -1.0f) > i) {
            thr = -std::numeric_limits<float>::infinity();
        } else {
            int64_t lo = k_lo, hi = k_hi;  // invariant: f(lo) <= i, f(hi) > i
            while (hi - lo > 1) {
                int64_t mid = lo + (hi - lo) / 2;
                if (reference_nearest(codebook, k, keyf(mid)) <= i) lo = mid; else hi = mid;
            }
            thr = keyf(lo);
        }
        t->thr[i] = thr;
    }
    for (int i = k - 1; i < kCodebookMax; ++i) t->thr[i] = std::numeric_limits<float>::infinity();
    // Bucket index: base = #{thr with bucket < b}, count = #{thr with bucket == b}.
    std::vector<int> bt((size_t)std::max(k - 1, 1));
    for (int i = 0; i < k - 1; ++i) bt[(size_t)i] = bucket_of(t->thr[i]);
    int j = 0;
    t->max_cnt = 0;
    for (int b = 0; b < kBuckets; ++b) {
        while (j < k - 1 && bt[(size_t)j] < b) ++j;
        int base = j, cnt = 0;
        while (j + cnt < k - 1 && bt[(size_t)(j + cnt)] == b) ++cnt;
        t->bucket[b] = (uint32_t)base | ((uint32_t)cnt << 16);
        t->max_cnt = std::max(t->max_cnt, cnt);
    }
    for (int b = 0; b < kFqEntries; ++b) {
        const uint32_t e = t->bucket[std::min(b, kBuckets - 1)];
        const uint32_t base = e & 0xffffu;
        const float t0 = (int)base < k - 1 ? t->thr[base] : std::numeric_limits<float>::infinity();
        t->fq[2 * b] = f2u(t0);
        t->fq[2 * b + 1] = base;
    }
    int rc = gefenx_search_lut(codebook, k, kBuckets, t->lut);
    if (rc != GEFENX_OK) return rc;
    for (int i = kLutEntries; i < kLutEntries + 7; ++i) t->lut[i] = (int16_t)k;
    return GEFENX_OK;
}

size_t gefenx_workspace_bytes(int kind, int64_t rows, int64_t cols, int64_t num_blocks) {
    if (rows < 0 || cols < 0 || num_blocks < 0) return 0;
    switch (kind) {
        case GEFENX_WS_FACTORED: return FactoredWs::make(rows, cols, num_blocks).total;
        case GEFENX_WS_BLOCK: return BlockWs::make(num_blocks, rows * cols).total;
        case GEFENX_WS_MOMENTUM: return MomentumWs::make(num_blocks).total;
        default: return 0;
    }
}

// Exact DP (quantization.py:75-139): dp[c][end] = min over start of
// dp[c-1][start-1] + cost(start..end).  Each cluster level depends only on the
// previous one, so the `end` loop of a level is split across host threads; the
// per-(level, end) arithmetic and its first-minimum rule are unchanged.
int gefenx_exact_dp(const float* active_centers, const float* active_counts,
                    int n_points, int k, int force_endpoints, float* codebook_out) {
    if (!active_centers || !active_counts || !codebook_out || n_points < 1 || k < 1)
        return set_error(GEFENX_EINVAL, "gefenx_exact_dp: bad arguments (n=%d k=%d)", n_points, k);
    for (int i = 0; i < n_points; ++i)
        if (!(active_counts[i] > 0.0f))
            return set_error(GEFENX_EINVAL, "exact DP expects strictly positive counts for all active histogram bins.");
    if (k > n_points) {
        dp_padded(active_centers, n_points, k, force_endpoints, codebook_out);
        return GEFENX_OK;
    }
    const int n = n_points;
    const DpPrefix pre = dp_prefix(active_centers, active_counts, n);
    const size_t W = (size_t)n + 1;
    std::vector<double> prev(W, std::numeric_limits<double>::infinity()), cur(W);
    std::vector<int32_t> bt((size_t)(k + 1) * W, -1);
    prev[0] = 0.0;
    unsigned hw = std::thread::hardware_concurrency();
    const int nthreads = (int)std::max(1u, std::min(hw ? hw : 1u, 16u));
    for (int c = 1; c <= k; ++c) {
        std::fill(cur.begin(), cur.end(), std::numeric_limits<double>::infinity());
        const bool endpoint = force_endpoints && (c == 1 || c == k);
        const double fc = (c == 1) ? -1.0 : 1.0;
        auto work = [&](int tid) {
            for (int end = c + tid; end <= n; end += nthreads) {
                double best = std::numeric_limits<double>::infinity();
                int32_t best_start = -1;
                for (int s = c; s <= end; ++s) {
                    const double cand = prev[(size_t)s - 1] +
                                        dp_cost(pre.pw.data(), pre.pwx.data(), pre.pwx2.data(), s, end, endpoint, fc);
                    if (cand < best) { best = cand; best_start = s; }
                }
                cur[(size_t)end] = best;
                bt[(size_t)c * W + (size_t)end] = best_start;
            }
        };
        if (nthreads > 1 && (int64_t)(n - c + 1) * (int64_t)(n - c + 1) > 200000) {
            std::vector<std::thread> pool;
            for (int t = 0; t < nthreads; ++t) pool.emplace_back(work, t);
            for (auto& th : pool) th.join();
        } else {
            for (int t = 0; t < nthreads; ++t) work(t);
        }
        std::swap(prev, cur);
    }
    if (!dp_backtrack(pre, bt.data(), W, n, k, force_endpoints, codebook_out))
        return set_error(GEFENX_EINVAL, "gefenx_exact_dp: infeasible segmentation");
    return GEFENX_OK;
}

}  // extern "C"
