/*
 * gefen_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU-resident (fused=False) Gefen
 * optimizer step, used exclusively as the checker for the HIP product path.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library; the product (gefen-x_amd/) never links, imports or calls it.
 *
 * Every function cites the reference file:line it follows (paths relative to
 * the reference repo root, src/gefen/ omitted).  Numerics follow the torch CPU
 * kernels the reference calls:
 *   - Tensor.lerp with a scalar weight w < 0.5 is fma(w, end - self, self)
 *     (ATen vectorised lerp), else fma(w - 1, end - self, end);
 *   - searchsorted(side='left') is a lower_bound on `!(c[mid] >= x)`;
 *   - `scalar / tensor` and `reciprocal` are correctly rounded fp32 divides;
 *   - `a.add_(b, alpha=s)` is fma(b, s, a);
 *   - dequantised coefficients are rounded through the grad dtype
 *     (gefen.py:337-373 returns like_tensor.dtype).
 * Summation order: torch's CPU cascade sums depend on the host's vector width,
 * so the oracle accumulates in double and rounds once; comparisons against the
 * oracle for sums (v_row, v_col, vmean, mean(v_row)) carry a tolerance.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2 };

/* ---------------------------------------------------------------- rounding */

static uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* fp32 -> bf16 -> fp32, round-to-nearest-even (c10::BFloat16 semantics). */
float orc_bf16_round(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return u2f(u | 0x00400000u); /* NaN */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return u2f(u & 0xffff0000u);
}

/* fp32 -> binary16 -> fp32, round-to-nearest-even (IEEE semantics). */
float orc_f16_round(float x) {
    if (isnan(x)) return x;
    float a = fabsf(x);
    if (a >= 65520.0f) return copysignf(INFINITY, x); /* rounds to inf */
    if (a < 5.9604644775390625e-08f * 0.5f) return copysignf(0.0f, x);
    int e;
    frexpf(a, &e); /* a = m * 2^e, m in [0.5,1) */
    int exp_unbiased = e - 1;
    if (exp_unbiased < -14) exp_unbiased = -14; /* subnormal spacing */
    float ulp = ldexpf(1.0f, exp_unbiased - 10);
    /* a / ulp is exact (power-of-two scale); rint is round-half-even */
    float r = rintf(a / ulp) * ulp;
    return copysignf(r, x);
}

float orc_round(float x, int dtype) {
    if (dtype == ORC_BF16) return orc_bf16_round(x);
    if (dtype == ORC_F16) return orc_f16_round(x);
    return x;
}

void orc_round_array(float* x, int64_t n, int dtype) {
    for (int64_t i = 0; i < n; ++i) x[i] = orc_round(x[i], dtype);
}

/* ----------------------------------------------------------- codebook search */

/* torch.searchsorted(codebook, x) (side='left'): gefen.py:318 */
int orc_lower_bound(const float* cb, int k, float x) {
    int lo = 0, hi = k;
    while (lo < hi) {
        int mid = lo + ((hi - lo) >> 1);
        if (!(cb[mid] >= x)) lo = mid + 1; else hi = mid;
    }
    return lo;
}

/* gefen_nearest_codebook_indices, one element: gefen.py:288-334 */
uint8_t orc_nearest(const float* cb, int k, float x) {
    if (k <= 1) return 0;
    int idx = orc_lower_bound(cb, k, x);
    int left = idx - 1;
    if (left < 0) left = 0;
    if (left > k - 1) left = k - 1;
    int right = idx;
    if (right > k - 1) right = k - 1;
    float dl = fabsf(x - cb[left]);
    float dr = fabsf(x - cb[right]);
    return (uint8_t)((dl <= dr) ? left : right);
}

void orc_nearest_array(const float* cb, int k, const float* x, int64_t n, uint8_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_nearest(cb, k, x[i]);
}

/* _codebook_search_lut: kernels/automatic_gefen_fused.py:81-121.
 * lut[b] = #{entries whose bucket < b}, bucket(c) = clamp(floor((c+1)*B/2)). */
void orc_search_lut(const float* cb, int k, int buckets, int16_t* lut) {
    for (int b = 0; b <= buckets; ++b) {
        int cnt = 0;
        for (int i = 0; i < k; ++i) {
            float eb = floorf((cb[i] + 1.0f) * (float)(buckets / 2));
            if (eb < 0.0f) eb = 0.0f;
            if (eb > (float)(buckets - 1)) eb = (float)(buckets - 1);
            if (eb < (float)b) ++cnt;
        }
        lut[b] = (int16_t)cnt;
    }
}

/* ------------------------------------------------------- momentum recurrence */

/* Tensor.lerp(end, w) with a scalar weight (ATen LerpKernel, vectorised form). */
static float lerp_f(float self, float end, float w) {
    if (fabsf(w) < 0.5f) return fmaf(w, end - self, self);
    return fmaf(w - 1.0f, end - self, end);
}

/*
 * _automatic_momentum_update_merged / _automatic_momentum_update:
 * gefen.py:3438-3486 and 3329-3436 (identical arithmetic).
 *   cm  = dtype_round(c[idx]) * mag                 (3394-3400, 3465-3469)
 *   u   = cm.lerp(g, 1 - beta1)                     (3403-3405, 3470)
 *   mag'= amax |u| over the block (NaN propagates)  (3409-3414, 3472-3476)
 *   x   = mag' > 0 ? u / mag' : 0                   (3416-3418, 3478-3480)
 *   idx'= nearest(x)                                (3421-3422, 3482-3483)
 *   q   = dtype_round(c[idx']) * mag'               (3428-3429, 3485-3486)
 * g holds the grad values already widened to fp32; dtype is the grad dtype.
 * idx and mag are updated in place; q (may be NULL) receives the reconstructed
 * momentum.  u_out (may be NULL) receives the pre-quantisation momentum.
 */
/* Rounding of the requantisation: nearest (the default) or the fused
 * kernels' stochastic rounding with a seed (kernels/automatic_gefen_fused_kernel.cu:
 * 160-211, 273-328), keyed by the element's flat index in its tensor.  Set by
 * orc_set_rounding before a step call; single-threaded use. */
static int g_sr_on = 0;
static uint64_t g_sr_seed = 0;
uint8_t orc_sr_quantize(const float* cb, int k, float x, uint64_t seed, int64_t element_idx);

void orc_set_rounding(int stochastic, uint64_t seed) {
    g_sr_on = stochastic ? 1 : 0;
    g_sr_seed = seed;
}

static uint8_t requantize(const float* cb, int k, float x, int64_t element_idx) {
    return g_sr_on ? orc_sr_quantize(cb, k, x, g_sr_seed, element_idx) : orc_nearest(cb, k, x);
}

/* Threads for the loops below (OpenMP).  Every parallel loop keeps each
 * element's operation order -- per-row and per-column sums stay sequential in
 * their own index order, the block max is an exact max -- so any thread count
 * gives bit-identical results. */
void orc_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }

/* Blocks at least this long are split across threads; shorter blocks are
 * handed out whole. */
#define ORC_PAR_BLOCK 16384

static void momentum_block(const float* g, uint8_t* idx, float* mag, int64_t b, int64_t period,
                           const float* cb, int k, int dtype, float w, float* q, float* u_out,
                           float* u, int inner_parallel) {
    const int64_t base = b * period;
    const float m_old = mag[b];
    float amax = 0.0f;
    int saw_nan = 0;
#pragma omp parallel for if (inner_parallel) reduction(max : amax) reduction(| : saw_nan) schedule(static)
    for (int64_t j = 0; j < period; ++j) {
        float c = orc_round(cb[idx[base + j]], dtype);
        float cm = c * m_old;
        float uu = lerp_f(cm, g[base + j], w);
        u[j] = uu;
        if (u_out) u_out[base + j] = uu;
        float a = fabsf(uu);
        if (isnan(a)) saw_nan = 1;
        else if (a > amax) amax = a;
    }
    float m_new = saw_nan ? NAN : amax;
    mag[b] = m_new;
    const int nonzero = (m_new > 0.0f);
#pragma omp parallel for if (inner_parallel) schedule(static)
    for (int64_t j = 0; j < period; ++j) {
        float x = nonzero ? u[j] / m_new : 0.0f;
        uint8_t ni = requantize(cb, k, x, base + j);
        idx[base + j] = ni;
        if (q) q[base + j] = orc_round(cb[ni], dtype) * m_new;
    }
}

void orc_momentum_update(const float* g, uint8_t* idx, float* mag, int64_t nb,
                         int64_t period, const float* cb, int k, int dtype,
                         float w, float* q, float* u_out) {
    if (period >= ORC_PAR_BLOCK) {
        float* u = (float*)malloc(sizeof(float) * (size_t)period);
        for (int64_t b = 0; b < nb; ++b) momentum_block(g, idx, mag, b, period, cb, k, dtype, w, q, u_out, u, 1);
        free(u);
        return;
    }
#pragma omp parallel if (nb > 1)
    {
        float* u = (float*)malloc(sizeof(float) * (size_t)(period > 0 ? period : 1));
#pragma omp for schedule(static)
        for (int64_t b = 0; b < nb; ++b) momentum_block(g, idx, mag, b, period, cb, k, dtype, w, q, u_out, u, 0);
        free(u);
    }
}

/* ------------------------------------------------- Muon quantised momentum */

/*
 * GefenMuon._prepare_muon_momentum, decomposed path: gefen_muon.py:1136-1141
 * with _quantize_momentum_ (gefen_muon.py:948-974).  Every intermediate is a
 * tensor of the grad dtype D, so each op rounds to D:
 *   cm  = D(D(c[idx]) * mag)                          (dequant, mul_)
 *   u   = D(lerp(cm, g, 1 - beta))                    (lerp_)
 *   mag'= amax |u| over the block (NaN propagates)    (copy_ into fp32 state)
 *   x   = mag' > 0 ? D(u / max(mag', tiny)) : 0       (div_, masked_fill_)
 *   idx'= nearest(x)
 *   out = D(D(c[idx']) * mag')                        (copy_, mul_)
 *   nesterov: out = D(fma(a, g, D(out * beta))), a = D((float)(1 - beta))
 *             (gefen_muon.py:1143-1144: mul_(beta).add_(g, alpha=1-beta); torch
 *             converts `alpha` to the tensor dtype, a `mul_` scalar stays fp32)
 * g holds the grad values widened to fp32.  idx / mag are updated in place.
 */
void orc_muon_momentum(const float* g, uint8_t* idx, float* mag, int64_t nb,
                       int64_t period, const float* cb, int k, int dtype,
                       double beta, int nesterov, float* out) {
    const float w = (float)(1.0 - beta);
    const float beta_f = (float)beta;
    const float alpha_d = orc_round(w, dtype);
    const float tiny = 1.17549435e-38f;
    float* u = (float*)malloc(sizeof(float) * (size_t)(period > 0 ? period : 1));
    for (int64_t b = 0; b < nb; ++b) {
        const int64_t base = b * period;
        const float m_old = mag[b];
        float amax = 0.0f;
        int saw_nan = 0;
        for (int64_t j = 0; j < period; ++j) {
            const float c = orc_round(cb[idx[base + j]], dtype);
            const float cm = orc_round(c * m_old, dtype);
            const float uu = orc_round(lerp_f(cm, g[base + j], w), dtype);
            u[j] = uu;
            const float a = fabsf(uu);
            if (isnan(a)) saw_nan = 1;
            else if (j == 0 || a > amax) amax = a;
        }
        const float m_new = saw_nan ? NAN : amax;
        mag[b] = m_new;
        const float den = m_new < tiny ? tiny : m_new;  /* clamp(min=tiny); NaN stays NaN */
        for (int64_t j = 0; j < period; ++j) {
            float x = orc_round(u[j] / den, dtype);
            if (m_new <= 0.0f) x = 0.0f;
            const uint8_t ni = requantize(cb, k, x, base + j);
            idx[base + j] = ni;
            float o = orc_round(orc_round(cb[ni], dtype) * m_new, dtype);
            if (nesterov) o = orc_round(fmaf(alpha_d, g[base + j], orc_round(o * beta_f, dtype)), dtype);
            out[base + j] = o;
        }
    }
    free(u);
}

/* ------------------------------------------------------- factored step (2D) */

/*
 * Decomposed factored update: gefen.py:2959-3018.
 *   row_ms = sum_j g^2 / cols, col_ms = sum_i g^2 / rows  (2973-2994)
 *   v <- fma(ms, 1-beta2, v*beta2)                          (2995-2996)
 *   v_hat = (v_row ⊗ v_col) / max(mean(v_row), FLT_MIN)     (2998-3000)
 *   step  = (1/bc1) * 1/(sqrt(v_hat/bc2) + eps)             (3001-3002)
 *   p     = dtype(p * (1 - lr*wd)) if wd > 0                (3015-3016)
 *   p     = dtype(p - (q*step)*lr)                          (3017-3018)
 * Host scalars arrive exactly as the reference computes them in Python
 * doubles: beta1, beta2, lr, eps, bc1 = 1-beta1^step, bc2 = 1-beta2^fstep, wd.
 * p and g are fp32 arrays holding the dtype's values; p is re-rounded to dtype.
 */
void orc_factored_step(float* p, const float* g, uint8_t* idx, float* mag,
                       float* v_row, float* v_col, int64_t rows, int64_t cols,
                       int64_t period, const float* cb, int k, int dtype,
                       double beta1, double beta2, double lr, double eps,
                       double bc1, double bc2, double wd) {
    const int64_t n = rows * cols;
    const int64_t nb = n / period;
    const float beta2_f = (float)beta2;
    const float alpha_f = (float)(1.0 - beta2);
    /* row sums, each over its columns in order */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows; ++i) {
        double racc = 0.0;
        for (int64_t j = 0; j < cols; ++j) {
            float gv = g[i * cols + j];
            float sq = gv * gv;
            racc += (double)sq;
        }
        float row_ms = (float)racc / (float)cols;
        v_row[i] = fmaf(row_ms, alpha_f, v_row[i] * beta2_f);
    }
    /* column sums, each over its rows in order; a thread owns a stripe of
     * 64 columns and walks it row by row */
    const int64_t stripes = (cols + 63) / 64;
#pragma omp parallel for schedule(static)
    for (int64_t st = 0; st < stripes; ++st) {
        double cacc[64];
        const int64_t j0 = st * 64;
        const int64_t nj = cols - j0 < 64 ? cols - j0 : 64;
        for (int64_t t = 0; t < nj; ++t) cacc[t] = 0.0;
        for (int64_t i = 0; i < rows; ++i) {
            const float* gr = g + i * cols + j0;
            for (int64_t t = 0; t < nj; ++t) {
                float sq = gr[t] * gr[t];
                cacc[t] += (double)sq;
            }
        }
        for (int64_t t = 0; t < nj; ++t) {
            float col_ms = (float)cacc[t] / (float)rows;
            v_col[j0 + t] = fmaf(col_ms, alpha_f, v_col[j0 + t] * beta2_f);
        }
    }
    double vsum = 0.0;
    for (int64_t i = 0; i < rows; ++i) vsum += (double)v_row[i];
    float mean_r = (float)vsum / (float)rows;
    if (!(mean_r >= 1.17549435e-38f)) mean_r = (mean_r != mean_r) ? mean_r : 1.17549435e-38f;

    float* q = (float*)malloc(sizeof(float) * (size_t)n);
    orc_momentum_update(g, idx, mag, nb, period, cb, k, dtype, (float)(1.0 - beta1), q, NULL);

    const float bc2_f = (float)bc2;
    const float eps_f = (float)eps;
    const float inv_bc1_f = (float)(1.0 / bc1);
    const float lr_f = (float)lr;
    const float wdf_f = (float)(1.0 - lr * wd);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows; ++i) {
        for (int64_t j = 0; j < cols; ++j) {
            const int64_t e = i * cols + j;
            float vh = (v_row[i] * v_col[j]) / mean_r;
            float h = sqrtf(vh / bc2_f) + eps_f;
            float step = (1.0f / h) * inv_bc1_f;
            float pv = p[e];
            if (wd > 0.0) pv = orc_round(pv * wdf_f, dtype);
            float upd = (q[e] * step) * lr_f;
            p[e] = orc_round(pv - upd, dtype);
        }
    }
    free(q);
}

/* ---------------------------------------------------- block-vmean step (1D) */

/*
 * automatic_vmean_update(use_fused=False): gefen.py:129-191.
 * bf16 grads square in bf16 and take a bf16 mean (fp32 sum, /P, cast back);
 * fp16 grads are promoted to fp32 first; fp32 squares in fp32.
 */
void orc_vmean_update(float* vmean, const float* g, int64_t nb, int64_t period,
                      int dtype, double beta2) {
    const float beta2_f = (float)beta2;
    const float alpha_f = (float)(1.0 - beta2);
#pragma omp parallel for if (nb > 1) schedule(static)
    for (int64_t b = 0; b < nb; ++b) {
        double acc = 0.0;
        for (int64_t j = 0; j < period; ++j) {
            float gv = g[b * period + j];
            float sq = gv * gv;
            if (dtype == ORC_BF16) sq = orc_bf16_round(sq);
            acc += (double)sq;
        }
        float mean = (float)acc / (float)period;
        if (dtype == ORC_BF16) mean = orc_bf16_round(mean);
        vmean[b] = fmaf(mean, alpha_f, vmean[b] * beta2_f);
    }
}

/*
 * Non-fused block step: gefen.py:3776-3818 (+ vmean update 3626-3628 and the
 * streamed momentum/apply 3329-3436).
 *   p = dtype(p*(1-lr*wd)) if wd > 0
 *   h = sqrt(vmean)/sqrt(bc2) + eps ; step = (1/h) * (1/bc1)
 *   p = dtype(p - (q*step_b)*lr)
 */
void orc_block_step(float* p, const float* g, uint8_t* idx, float* mag,
                    float* vmean, int64_t n, int64_t period, const float* cb,
                    int k, int dtype, double beta1, double beta2, double lr,
                    double eps, double bc1, double bc2, double wd) {
    const int64_t nb = n / period;
    orc_vmean_update(vmean, g, nb, period, dtype, beta2);
    const float wdf_f = (float)(1.0 - lr * wd);
    if (wd > 0.0) {
#pragma omp parallel for schedule(static)
        for (int64_t e = 0; e < n; ++e) p[e] = orc_round(p[e] * wdf_f, dtype);
    }
    const float sbc2_f = (float)sqrt(bc2);
    const float eps_f = (float)eps;
    const float inv_bc1_f = (float)(1.0 / bc1);
    const float lr_f = (float)lr;
    float* q = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    orc_momentum_update(g, idx, mag, nb, period, cb, k, dtype, (float)(1.0 - beta1), q, NULL);
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < nb; ++b) {
        float h = sqrtf(vmean[b]) / sbc2_f + eps_f;
        float step = (1.0f / h) * inv_bc1_f;
        for (int64_t j = 0; j < period; ++j) {
            const int64_t e = b * period + j;
            float upd = (q[e] * step) * lr_f;
            p[e] = orc_round(p[e] - upd, dtype);
        }
    }
    free(q);
}

/* ----------------------------------------------- step-1 codebook histogram */

/*
 * learn_gefen_exact_codebook_from_grad_periods, torch histogram branch:
 * gefen.py:455-469.  counts has `bins` int64 entries and is accumulated.
 * multiply = 0: floor((x + 1) / f32(2 / bins)) (the torch path); 1:
 * floor((x + 1) * (0.5f * bins)) (the reference's histogram kernel,
 * kernels/exact_histogram_fused_kernel.cu:66-76).  The two agree whenever
 * bins is a power of two.
 */
void orc_exact_histogram_form(const float* g, int64_t n, int64_t period, int bins,
                              int64_t* counts, int multiply) {
    const float bin_width = (float)(2.0 / (double)bins);
    const float scale = 0.5f * (float)bins;
    const int64_t nb = n / period;
    for (int64_t b = 0; b < nb; ++b) {
        const float* blk = g + b * period;
        float amax = 0.0f;
        int saw_nan = 0;
        for (int64_t j = 0; j < period; ++j) {
            float a = fabsf(blk[j]);
            if (isnan(a)) saw_nan = 1;
            else if (a > amax) amax = a;
        }
        const int nonzero = !saw_nan && amax > 0.0f;
        for (int64_t j = 0; j < period; ++j) {
            float x = nonzero ? blk[j] / amax : 0.0f;
            float t = multiply ? floorf((x + 1.0f) * scale) : floorf((x + 1.0f) / bin_width);
            int64_t bi;
            if (isnan(t)) bi = 0; /* long() of NaN then clamp(0, bins-1) */
            else if (t < 0.0f) bi = 0;
            else if (t > (float)(bins - 1)) bi = bins - 1;
            else bi = (int64_t)t;
            counts[bi] += 1;
        }
    }
}

void orc_exact_histogram(const float* g, int64_t n, int64_t period, int bins, int64_t* counts) {
    orc_exact_histogram_form(g, n, period, bins, counts, 0);
}

/* ------------------------------------------------------------ exact DP */

/*
 * quantization.exact_dp numba/python kernel: quantization.py:75-139, 142-194.
 * Optimal 1-D weighted k-means by DP in float64 with forced +-1 endpoints,
 * strict `<` keeps the first minimum.  prefix arrays have n_points+1 entries.
 * Writes the unsorted codebook (the caller sorts, quantization.py:252).
 */
int orc_exact_dp_kernel(const double* pw, const double* pwx, const double* pwx2,
                        int n_points, int k, int force_endpoints, float* codebook) {
    const int64_t W = (int64_t)k + 1;
    double* dp = (double*)malloc(sizeof(double) * (size_t)(n_points + 1) * (size_t)W);
    int64_t* bt = (int64_t*)malloc(sizeof(int64_t) * (size_t)(n_points + 1) * (size_t)W);
    if (!dp || !bt) { free(dp); free(bt); return -1; }
    for (int64_t i = 0; i < (int64_t)(n_points + 1) * W; ++i) { dp[i] = INFINITY; bt[i] = -1; }
    dp[0] = 0.0;
    for (int c = 1; c <= k; ++c) {
        for (int end = c; end <= n_points; ++end) {
            double best = INFINITY;
            int64_t best_start = -1;
            for (int s = c; s <= end; ++s) {
                double sw = pw[end] - pw[s - 1];
                double swx = pwx[end] - pwx[s - 1];
                double swx2 = pwx2[end] - pwx2[s - 1];
                double cost;
                if (force_endpoints && c == 1) {
                    double fc = -1.0;
                    cost = swx2 - 2.0 * fc * swx + fc * fc * sw;
                } else if (force_endpoints && c == k) {
                    double fc = 1.0;
                    cost = swx2 - 2.0 * fc * swx + fc * fc * sw;
                } else {
                    cost = swx2 - (swx * swx) / sw;
                }
                double cand = dp[(int64_t)(s - 1) * W + (c - 1)] + cost;
                if (cand < best) { best = cand; best_start = s; }
            }
            dp[(int64_t)end * W + c] = best;
            bt[(int64_t)end * W + c] = best_start;
        }
    }
    int64_t end = n_points;
    for (int c = k; c >= 1; --c) {
        int64_t s = bt[end * W + c];
        if (force_endpoints && c == 1) codebook[c - 1] = -1.0f;
        else if (force_endpoints && c == k) codebook[c - 1] = 1.0f;
        else {
            double sw = pw[end] - pw[s - 1];
            double swx = pwx[end] - pwx[s - 1];
            codebook[c - 1] = (float)(swx / sw);
        }
        end = s - 1;
    }
    free(dp); free(bt);
    return 0;
}

/* ------------------------------------------------------ stochastic rounding */

/* gefen_sr_uniform: kernels/automatic_gefen_fused_kernel.cu:141-151
 * (SplitMix64 finalizer over seed + golden_gamma * (idx + 1)). */
float orc_sr_uniform(uint64_t seed, int64_t element_idx) {
    uint64_t z = seed + 0x9E3779B97F4A7C15ULL * ((uint64_t)element_idx + 1ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    z = z ^ (z >> 31);
    return (float)(z >> 40) * (1.0f / 16777216.0f);
}

/* quantize_codebook_index, stochastic branch:
 * kernels/automatic_gefen_fused_kernel.cu:160-211. */
uint8_t orc_sr_quantize(const float* cb, int k, float x, uint64_t seed, int64_t element_idx) {
    /* the kernel's own lower_bound moves right on `c[mid] < x` (:173-181) */
    int r = 0, hi_ = k;
    while (r < hi_) {
        int mid = r + ((hi_ - r) >> 1);
        if (cb[mid] < x) r = mid + 1; else hi_ = mid;
    }
    if (r > k - 1) r = k - 1;
    int l = r - 1;
    if (l < 0) l = 0;
    if (l == r) return (uint8_t)r;
    float lo = cb[l], hi = cb[r];
    float span = hi - lo;
    float v = x;
    if (v < lo) v = lo; else if (v > hi) v = hi;
    float p_up = (span > 0.0f) ? (v - lo) / span : 0.0f;
    float u = orc_sr_uniform(seed, element_idx);
    return (uint8_t)((u < p_up) ? r : l);
}

/* ------------------------------------------------ standalone factored EMA */

/*
 * gefen_factored_v_ema_cuda: kernels/automatic_gefen_fused_kernel.cu:1990-2042,
 * 2792-2850 -- the GPU aten chain v.mul_(beta2).add_(sq.div_(n), alpha=1-beta2):
 * t = sq * RN(1/n) (a scalar divide is a reciprocal multiply there),
 * vb = RN(v * beta2), v' = fma(1 - beta2, t, vb).
 */
void orc_factored_v_ema(float* v, const float* sq, int64_t count, int64_t n, double beta2) {
    const float inv = 1.0f / (float)(double)n;
    const float b2 = (float)beta2;
    const float a2 = (float)(1.0 - beta2);
    for (int64_t i = 0; i < count; ++i) {
        const float t = sq[i] * inv;
        const float vb = v[i] * b2;
        v[i] = fmaf(a2, t, vb);
    }
}

/* ------------------------------------------- partial update (legacy pair) */

/*
 * automatic_gefen_fused_update_cuda / _v2_cuda: kernels/automatic_gefen_fused_kernel.cu:
 * 331-415 -- the quantised-momentum recurrence of the CPU step (gefen.py:3438-3486)
 * followed by p <- D(p - (q * stepsize[b]) * lr), no weight decay; lr == 0 leaves
 * p untouched.  stepsize: fp32 [nb].
 */
void orc_partial_update(float* p, const float* g, uint8_t* idx, float* mag, const float* stepsize,
                        int64_t n, int64_t period, const float* cb, int k, int dtype, double beta1,
                        double lr) {
    const int64_t nb = n / period;
    float* q = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    orc_momentum_update(g, idx, mag, nb, period, cb, k, dtype, (float)(1.0 - beta1), q, NULL);
    const float lr_f = (float)lr;
    if (lr_f != 0.0f) {
        for (int64_t b = 0; b < nb; ++b) {
            for (int64_t j = 0; j < period; ++j) {
                const int64_t e = b * period + j;
                p[e] = orc_round(p[e] - (q[e] * stepsize[b]) * lr_f, dtype);
            }
        }
    }
    free(q);
}
