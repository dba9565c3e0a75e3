// gefenx_dp.h -- host parts of the exact-DP codebook solver shared by the
// host (gefenx_exact_dp) and device (gefenx_exact_dp_device) entry points:
// the float64 prefix sums, the padded codebook for k > n, the cost of one
// segment and the backtracking.  quantization.py:59-72, 75-139, 197-253.
#pragma once

#include <algorithm>
#include <cstdint>
#include <vector>

namespace gx {

// Sequential float64 prefix sums of w, w*c, w*c^2 over the active bins
// (torch.cumsum order); index 0 holds 0.
struct DpPrefix {
    std::vector<double> pw, pwx, pwx2;
};

inline DpPrefix dp_prefix(const float* centers, const float* counts, int n) {
    DpPrefix p;
    p.pw.assign((size_t)n + 1, 0.0);
    p.pwx.assign((size_t)n + 1, 0.0);
    p.pwx2.assign((size_t)n + 1, 0.0);
    double aw = 0.0, awx = 0.0, awx2 = 0.0;
    for (int i = 0; i < n; ++i) {
        const double w = (double)counts[i];
        const double c = (double)centers[i];
        const double wx = w * c;
        const double cc = c * c;
        const double wx2 = w * cc;
        aw += w; awx += wx; awx2 += wx2;
        p.pw[(size_t)i + 1] = aw; p.pwx[(size_t)i + 1] = awx; p.pwx2[(size_t)i + 1] = awx2;
    }
    return p;
}

// Fewer active bins than centres: the bins repeated, endpoints forced, sorted.
inline void dp_padded(const float* centers, int n, int k, int force_endpoints, float* out) {
    std::vector<float> cb((size_t)k);
    for (int i = 0; i < k; ++i) cb[(size_t)i] = centers[std::min(i, n - 1)];
    if (force_endpoints) { cb[0] = -1.0f; cb[(size_t)k - 1] = 1.0f; }
    std::sort(cb.begin(), cb.end());
    std::copy(cb.begin(), cb.end(), out);
}

// Cost of bins [s, end] (1-based, inclusive) as centre c of k.  Forced
// endpoint centres use sum w (x - f)^2 expanded; the others the weighted
// variance sum w x^2 - (sum w x)^2 / sum w.  Written for host and device with
// the same operation order.
#if defined(__HIP__)
__host__ __device__
#endif
inline double dp_cost(const double* pw, const double* pwx, const double* pwx2, int s, int end, bool endpoint,
                      double fc) {
    const double sw = pw[end] - pw[s - 1];
    const double swx = pwx[end] - pwx[s - 1];
    const double swx2 = pwx2[end] - pwx2[s - 1];
    if (endpoint) {
        const double t1 = 2.0 * fc;
        const double t2 = t1 * swx;
        const double t3 = fc * fc;
        const double t4 = t3 * sw;
        return (swx2 - t2) + t4;
    }
    const double sq = swx * swx;
    return swx2 - sq / sw;
}

// Walk the first-minimum starts back from bin n: the centres are the segment
// means (forced endpoints -1 / +1), sorted.  bt row c, column end: start of
// centre c's segment when it ends at `end`.  Returns false when a segment is
// missing (infeasible).
inline bool dp_backtrack(const DpPrefix& p, const int32_t* bt, size_t W, int n, int k, int force_endpoints,
                         float* out) {
    std::vector<float> cb((size_t)k);
    int64_t end = n;
    for (int c = k; c >= 1; --c) {
        const int64_t s = bt[(size_t)c * W + (size_t)end];
        if (force_endpoints && c == 1) cb[(size_t)c - 1] = -1.0f;
        else if (force_endpoints && c == k) cb[(size_t)c - 1] = 1.0f;
        else {
            if (s < 1) return false;
            const double sw = p.pw[(size_t)end] - p.pw[(size_t)s - 1];
            const double swx = p.pwx[(size_t)end] - p.pwx[(size_t)s - 1];
            cb[(size_t)c - 1] = (float)(swx / sw);
        }
        end = s - 1;
    }
    std::sort(cb.begin(), cb.end());
    std::copy(cb.begin(), cb.end(), out);
    return true;
}

}  // namespace gx
