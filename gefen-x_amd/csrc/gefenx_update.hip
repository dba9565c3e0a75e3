// gefenx_update.hip -- fused Gefen update kernels for MI355X (gfx950, wave64).
//
// Per parameter the step is three launches on the caller's stream:
//   stats    one pass over grad + stored indices: per-block max |u| (u = the
//            updated momentum) and the second-moment sums (row/column sums of
//            g^2 for the factored path, per-block sums for the block path);
//   finalize tiny: EMA of the second moment, mean(v_row), new magnitudes,
//            per-block stepsizes; re-zeroes the workspace accumulators;
//   apply    one pass: recompute u, normalise by the new magnitude,
//            requantise through the exact threshold table, write the indices
//            and the parameter (decoupled weight decay folded in).
// The math follows the reference's decomposed step (gefen.py:2959-3018,
// 3329-3486, 3776-3818); see gefenx_device.h for the bit-exact momentum and
// quantisation primitives.
#include "gefenx_device.h"
#include "gefenx_internal.h"
#include "gefenx_profile.h"
#include "../../include/gefenx.h"

#include <algorithm>
#include <cmath>

namespace gx {

constexpr int kThreads = 256;
constexpr int kChunk = 8;
constexpr int kTileCols = kThreads * kChunk;  // 2048 columns per stats tile
constexpr int kMaxTileRows = 32;

struct StepScalars {
    float lr, inv_bc2, inv_bc1, wdf;
};

__device__ __forceinline__ StepScalars read_scalars(StepScalars host, const float* dev) {
    if (dev != nullptr) {
        host.lr = dev[0];
        host.inv_bc2 = dev[1];
        host.inv_bc1 = dev[2];
        host.wdf = dev[3];
    }
    return host;
}

// Per-thread running block max of |u| (as ordered uint bits: NaN > inf > finite,
// so the integer max propagates NaN like torch's amax).
struct BlockMax {
    int64_t blk;
    uint32_t bits;
    float mag_old;
};

__device__ __forceinline__ void blockmax_flush(uint32_t* __restrict__ magbits, const BlockMax& bm) {
    if (bm.blk >= 0 && bm.bits != 0u) atomicMax(magbits + bm.blk, bm.bits);
}

// Wave-level final flush: one atomic per wave when every lane holds the same block.
__device__ __forceinline__ void blockmax_final(uint32_t* __restrict__ magbits, const BlockMax& bm) {
    const int lane = threadIdx.x & 63;
    const int64_t blk0 = __shfl(bm.blk, 0, 64);
    const bool same = __all(bm.blk == blk0);
    if (same) {
        const uint32_t m = wave_max_u(bm.bits);
        if (lane == 0 && blk0 >= 0 && m != 0u) atomicMax(magbits + blk0, m);
    } else {
        blockmax_flush(magbits, bm);
    }
}

// ====================================================================
// Factored stats: grid (ceil(C / 2048), ceil(R / tile_rows)), 256 threads.
// Thread t owns columns [c0, c0+8) of every row of its tile.
// ====================================================================
struct FactStatsArgs {
    const void* grad;
    const uint8_t* idx;
    const float* mag_old;
    const QTable* qt;
    int64_t R, C, gs0, gs1, P;
    double invP;
    int tile_rows;
    int fast;  // contiguous, C % 8 == 0, 16-byte aligned grad
    double* row_sq;
    double* col_sq;
    uint32_t* magbits;
    MomentumCoef mc;
};

template <int DT>
__global__ void __launch_bounds__(kThreads) k_factored_stats(FactStatsArgs a) {
    using T = typename Elem<DT>::T;
    __shared__ float s_cbr[kCodebookMax];
    __shared__ float s_row[kMaxTileRows][kThreads / 64];
    for (int i = threadIdx.x; i < kCodebookMax; i += kThreads) s_cbr[i] = a.qt->cbr[i];
    __syncthreads();

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int64_t c0 = (int64_t)blockIdx.x * kTileCols + (int64_t)tid * kChunk;
    const int64_t r_begin = (int64_t)blockIdx.y * a.tile_rows;
    const int64_t r_end = std::min<int64_t>(r_begin + a.tile_rows, a.R);
    const T* g = static_cast<const T*>(a.grad);

    float colacc[kChunk];
#pragma unroll
    for (int k = 0; k < kChunk; ++k) colacc[k] = 0.0f;
    BlockMax bm{-1, 0u, 0.0f};
    const int nvalid = (int)std::max<int64_t>(0, std::min<int64_t>(kChunk, a.C - c0));

    for (int64_t r = r_begin; r < r_end; ++r) {
        float rowacc = 0.0f;
        if (nvalid > 0) {
            const int64_t e0 = r * a.C + c0;
            float gv[kChunk];
            uint32_t ix[kChunk];
            if (a.fast && nvalid == kChunk) {
                load8<DT>(g + e0, gv);
                load_idx8(a.idx + e0, ix);
            } else {
#pragma unroll
                for (int k = 0; k < kChunk; ++k) {
                    if (k < nvalid) {
                        gv[k] = to_f32<DT>(g[r * a.gs0 + (c0 + k) * a.gs1]);
                        ix[k] = a.idx[e0 + k];
                    } else {
                        gv[k] = 0.0f;
                        ix[k] = 0u;
                    }
                }
            }
            int64_t blk = div_floor(e0, a.P, a.invP);
            int64_t pin = e0 - blk * a.P;
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                if (k < nvalid) {
                    if (blk != bm.blk) {
                        blockmax_flush(a.magbits, bm);
                        bm.blk = blk;
                        bm.bits = 0u;
                        bm.mag_old = a.mag_old[blk];
                    }
                    const float u = momentum_value(s_cbr[ix[k]], bm.mag_old, gv[k], a.mc);
                    const uint32_t ub = __float_as_uint(u) & 0x7fffffffu;
                    bm.bits = ub > bm.bits ? ub : bm.bits;
                    const float sq = gv[k] * gv[k];
                    rowacc += sq;
                    colacc[k] += sq;
                    if (++pin == a.P) { pin = 0; ++blk; }
                }
            }
        }
        const float rs = wave_sum(rowacc);
        if (lane == 0) s_row[r - r_begin][wave] = rs;
    }
    blockmax_final(a.magbits, bm);
    for (int k = 0; k < nvalid; ++k) atomicAdd(a.col_sq + c0 + k, (double)colacc[k]);
    __syncthreads();
    const int nrows = (int)(r_end - r_begin);
    if (tid < nrows) {
        double s = 0.0;
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w) s += (double)s_row[tid][w];
        atomicAdd(a.row_sq + r_begin + tid, s);
    }
}

// ====================================================================
// Factored finalize: block 0 = rows/cols/mean, blocks 1.. = magnitudes.
// v <- fma(sum/n, 1-beta2, v*beta2)  (gefen.py:2994-2996)
// ====================================================================
struct FactFinArgs {
    double* row_sq;
    double* col_sq;
    float* v_row;
    float* v_col;
    int64_t R, C, nb;
    float beta2, alpha2;
    uint32_t* magbits;
    float* mag;      // m_magnitude: receives the new magnitudes
    float* mag_old;  // workspace: receives the old magnitudes
    float* scal;     // workspace scalars: [0] = max(mean(v_row), FLT_MIN)
};

__global__ void __launch_bounds__(kThreads) k_factored_finalize(FactFinArgs a) {
    const int tid = threadIdx.x;
    if (blockIdx.x == 0) {
        __shared__ double s_part[kThreads / 64];
        double acc = 0.0;
        const float fC = (float)a.C, fR = (float)a.R;
        for (int64_t i = tid; i < a.R; i += kThreads) {
            const float ms = (float)a.row_sq[i] / fC;
            a.row_sq[i] = 0.0;
            const float v = __builtin_fmaf(ms, a.alpha2, a.v_row[i] * a.beta2);
            a.v_row[i] = v;
            acc += (double)v;
        }
        for (int64_t j = tid; j < a.C; j += kThreads) {
            const float ms = (float)a.col_sq[j] / fR;
            a.col_sq[j] = 0.0;
            a.v_col[j] = __builtin_fmaf(ms, a.alpha2, a.v_col[j] * a.beta2);
        }
        acc = wave_sum_d(acc);
        if ((tid & 63) == 0) s_part[tid >> 6] = acc;
        __syncthreads();
        if (tid == 0) {
            double s = 0.0;
            for (int w = 0; w < kThreads / 64; ++w) s += s_part[w];
            float mean = (float)s / fR;
            if (!(mean >= 1.17549435e-38f) && mean == mean) mean = 1.17549435e-38f;
            a.scal[0] = mean;
        }
        return;
    }
    for (int64_t b = (int64_t)(blockIdx.x - 1) * kThreads + tid; b < a.nb;
         b += (int64_t)(gridDim.x - 1) * kThreads) {
        const float old = a.mag[b];
        a.mag_old[b] = old;
        a.mag[b] = __uint_as_float(a.magbits[b]);
        a.magbits[b] = 0u;
    }
}

// ====================================================================
// Block stats: flat over logical chunks; per-block sum of squares (squares
// rounded through bf16 for bf16 grads, gefen.py:180-190) and max |u|.
// ====================================================================
struct BlockStatsArgs {
    const void* grad;
    const uint8_t* idx;
    const float* mag_old;
    const QTable* qt;
    int64_t N, P;
    double invP;
    int fast;
    double* blk_sq;
    uint32_t* magbits;
    MomentumCoef mc;
};

template <int DT>
__global__ void __launch_bounds__(kThreads) k_block_stats(BlockStatsArgs a) {
    using T = typename Elem<DT>::T;
    __shared__ float s_cbr[kCodebookMax];
    for (int i = threadIdx.x; i < kCodebookMax; i += kThreads) s_cbr[i] = a.qt->cbr[i];
    __syncthreads();
    const T* g = static_cast<const T*>(a.grad);
    const int64_t nchunks = (a.N + kChunk - 1) / kChunk;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    BlockMax bm{-1, 0u, 0.0f};
    double bsum = 0.0;
    for (int64_t ch = (int64_t)blockIdx.x * kThreads + threadIdx.x; ch < nchunks; ch += stride) {
        const int64_t e0 = ch * kChunk;
        const int nvalid = (int)std::min<int64_t>(kChunk, a.N - e0);
        float gv[kChunk];
        uint32_t ix[kChunk];
        if (a.fast && nvalid == kChunk) {
            load8<DT>(g + e0, gv);
            load_idx8(a.idx + e0, ix);
        } else {
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                gv[k] = k < nvalid ? to_f32<DT>(g[e0 + k]) : 0.0f;
                ix[k] = k < nvalid ? (uint32_t)a.idx[e0 + k] : 0u;
            }
        }
        int64_t blk = div_floor(e0, a.P, a.invP);
        int64_t pin = e0 - blk * a.P;
        float csum = 0.0f;
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if (k < nvalid) {
                if (blk != bm.blk) {
                    if (bm.blk >= 0) {
                        bsum += (double)csum;
                        csum = 0.0f;
                        if (bsum != 0.0) atomicAdd(a.blk_sq + bm.blk, bsum);
                        bsum = 0.0;
                    }
                    blockmax_flush(a.magbits, bm);
                    bm.blk = blk;
                    bm.bits = 0u;
                    bm.mag_old = a.mag_old[blk];
                }
                const float u = momentum_value(s_cbr[ix[k]], bm.mag_old, gv[k], a.mc);
                const uint32_t ub = __float_as_uint(u) & 0x7fffffffu;
                bm.bits = ub > bm.bits ? ub : bm.bits;
                float sq = gv[k] * gv[k];
                if constexpr (DT == BF16) sq = round_dt<BF16>(sq);
                csum += sq;
                if (++pin == a.P) { pin = 0; ++blk; }
            }
        }
        bsum += (double)csum;
    }
    // Final flush: combine the wave when all lanes hold the same block.
    const int lane = threadIdx.x & 63;
    const int64_t blk0 = __shfl(bm.blk, 0, 64);
    if (__all(bm.blk == blk0)) {
        const double s = wave_sum_d(bsum);
        if (lane == 0 && blk0 >= 0 && s != 0.0) atomicAdd(a.blk_sq + blk0, s);
    } else if (bm.blk >= 0 && bsum != 0.0) {
        atomicAdd(a.blk_sq + bm.blk, bsum);
    }
    blockmax_final(a.magbits, bm);
}

// vmean EMA + per-block stepsize (gefen.py:180-190, 3794-3805).
struct BlockFinArgs {
    double* blk_sq;
    float* vmean;
    int64_t nb, P;
    float beta2, alpha2, eps;
    int bf16_mean;
    StepScalars sc;
    const float* step_scalars;
    uint32_t* magbits;
    float* mag;
    float* mag_old;
    float* step;
};

__global__ void __launch_bounds__(kThreads) k_block_finalize(BlockFinArgs a) {
    const StepScalars sc = read_scalars(a.sc, a.step_scalars);
    const float fP = (float)a.P;
    for (int64_t b = (int64_t)blockIdx.x * kThreads + threadIdx.x; b < a.nb;
         b += (int64_t)gridDim.x * kThreads) {
        float mean = (float)a.blk_sq[b] / fP;
        a.blk_sq[b] = 0.0;
        if (a.bf16_mean) mean = round_dt<BF16>(mean);
        const float v = __builtin_fmaf(mean, a.alpha2, a.vmean[b] * a.beta2);
        a.vmean[b] = v;
        const float h = sqrtf(v) * sc.inv_bc2 + a.eps;
        a.step[b] = (1.0f / h) * sc.inv_bc1;
        const float old = a.mag[b];
        a.mag_old[b] = old;
        a.mag[b] = __uint_as_float(a.magbits[b]);
        a.magbits[b] = 0u;
    }
}

// ====================================================================
// Apply: flat over logical chunks of 8.  MODE 0 = factored, 1 = block.
// ====================================================================
struct ApplyArgs {
    void* p;
    const void* grad;
    uint8_t* idx;
    const float* mag_old;
    const float* mag_new;
    const float* v_row;   // factored
    const float* v_col;   // factored
    const float* scal;    // factored: [0] = clamped mean(v_row)
    const float* step;    // block: per-block stepsize
    const QTable* qt;
    int64_t N, C, P;
    double invC, invP;
    int64_t ps0, ps1, gs0, gs1;
    int fast;        // contiguous p and grad, 16-byte aligned, C % 8 == 0 (or 1D)
    int write_p;     // 0 when lr == 0 and wd_factor == 1
    float eps;
    StepScalars sc;
    const float* step_scalars;
    MomentumCoef mc;
    uint64_t seed;
    const int64_t* seed_dev;
};

template <int DT, int MODE, bool SR>
__global__ void __launch_bounds__(kThreads) k_apply(ApplyArgs a) {
    using T = typename Elem<DT>::T;
    __shared__ SharedTables st;
    __shared__ SharedSR ssr;
    stage_tables(st, a.qt);
    if constexpr (SR) stage_sr(ssr, a.qt);
    __syncthreads();
    const uint32_t kmax = (uint32_t)(a.qt->k - 1);
    const int kk = a.qt->k;
    const StepScalars sc = read_scalars(a.sc, a.step_scalars);
    uint64_t seed = a.seed;
    if constexpr (SR) {
        if (a.seed_dev != nullptr) seed = (uint64_t)a.seed_dev[0];
    }
    float inv_mean = 0.0f;
    if constexpr (MODE == 0) inv_mean = 1.0f / a.scal[0];

    T* p = static_cast<T*>(a.p);
    const T* g = static_cast<const T*>(a.grad);
    const int64_t nchunks = (a.N + kChunk - 1) / kChunk;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t ch = (int64_t)blockIdx.x * kThreads + threadIdx.x; ch < nchunks; ch += stride) {
        const int64_t e0 = ch * kChunk;
        const int nvalid = (int)std::min<int64_t>(kChunk, a.N - e0);
        int64_t row = 0, col = e0;
        if (MODE == 0 || !a.fast) {
            row = div_floor(e0, a.C, a.invC);
            col = e0 - row * a.C;
        }
        int64_t blk = div_floor(e0, a.P, a.invP);
        int64_t pin = e0 - blk * a.P;
        float gv[kChunk], pv[kChunk];
        uint32_t ix[kChunk];
        const bool vec = a.fast && nvalid == kChunk;
        if (vec) {
            load8<DT>(g + e0, gv);
            if (a.write_p) load8<DT>(p + e0, pv);
            load_idx8(a.idx + e0, ix);
        } else {
            int64_t r = row, c = col;
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                if (k < nvalid) {
                    gv[k] = to_f32<DT>(g[r * a.gs0 + c * a.gs1]);
                    pv[k] = a.write_p ? to_f32<DT>(p[r * a.ps0 + c * a.ps1]) : 0.0f;
                    ix[k] = a.idx[e0 + k];
                    if (++c == a.C) { c = 0; ++r; }
                } else {
                    gv[k] = 0.0f;
                    pv[k] = 0.0f;
                    ix[k] = 0u;
                }
            }
        }
        float m_old = a.mag_old[blk];
        float m_new = a.mag_new[blk];
        float bstep = 0.0f;
        if constexpr (MODE == 1) bstep = a.step[blk];
        float vr = 0.0f;
        if constexpr (MODE == 0) vr = a.v_row[row];
        int64_t r = row, c = col;
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if (k < nvalid) {
                const float u = momentum_value(st.cbr[ix[k]], m_old, gv[k], a.mc);
                const float x = (m_new > 0.0f) ? u / m_new : 0.0f;
                uint32_t ni;
                if constexpr (SR) ni = quant_stochastic(x, ssr.cb, ssr.lut, kk, seed, e0 + k);
                else ni = quant_nearest(x, st.bkt, st.thr, kmax);
                ix[k] = ni;
                if (a.write_p) {
                    const float q = st.cbr[ni] * m_new;
                    float stepv;
                    if constexpr (MODE == 0) {
                        const float vhat = (vr * a.v_col[c]) * inv_mean;
                        const float h = sqrtf(vhat * sc.inv_bc2) + a.eps;
                        stepv = (1.0f / h) * sc.inv_bc1;
                    } else {
                        stepv = bstep;
                    }
                    const float upd = (q * stepv) * sc.lr;
                    float pw = pv[k];
                    if (sc.wdf != 1.0f) pw = round_dt<DT>(pw * sc.wdf);
                    pv[k] = pw - upd;
                }
                if (++c == a.C) {
                    c = 0;
                    ++r;
                    if constexpr (MODE == 0) {
                        if (k + 1 < nvalid) vr = a.v_row[r];
                    }
                }
                if (++pin == a.P) {
                    pin = 0;
                    ++blk;
                    if (k + 1 < nvalid) {
                        m_old = a.mag_old[blk];
                        m_new = a.mag_new[blk];
                        if constexpr (MODE == 1) bstep = a.step[blk];
                    }
                }
            }
        }
        if (vec) {
            store_idx8(a.idx + e0, ix);
            if (a.write_p) store8<DT>(p + e0, pv);
        } else {
            int64_t rr = row, cc = col;
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                if (k < nvalid) {
                    a.idx[e0 + k] = (uint8_t)ix[k];
                    if (a.write_p) p[rr * a.ps0 + cc * a.ps1] = from_f32<DT>(pv[k]);
                    if (++cc == a.C) { cc = 0; ++rr; }
                }
            }
        }
    }
}

// ====================================================================
// Host launchers
// ====================================================================

static MomentumCoef make_coef(double beta1) {
    MomentumCoef mc;
    mc.w = (float)(1.0 - beta1);
    mc.wm1 = mc.w - 1.0f;
    mc.small = std::fabs(mc.w) < 0.5f ? 1 : 0;
    return mc;
}

static inline bool aligned(const void* ptr, size_t a) {
    return (reinterpret_cast<uintptr_t>(ptr) % a) == 0;
}

static int launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GEFENX_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
    return GEFENX_OK;
}

static int grid_for(int64_t work_items, int per_block, int cap) {
    int64_t g = (work_items + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int)g;
}

constexpr int kApplyGridCap = 8192;

template <int MODE, bool SR>
static void launch_apply_dt(int dtype, const ApplyArgs& a, int grid, hipStream_t s) {
    switch (dtype) {
        case F32: hipLaunchKernelGGL((k_apply<F32, MODE, SR>), dim3(grid), dim3(kThreads), 0, s, a); break;
        case F16: hipLaunchKernelGGL((k_apply<F16, MODE, SR>), dim3(grid), dim3(kThreads), 0, s, a); break;
        default: hipLaunchKernelGGL((k_apply<BF16, MODE, SR>), dim3(grid), dim3(kThreads), 0, s, a); break;
    }
}

template <int MODE>
static void launch_apply(int dtype, bool sr, const ApplyArgs& a, hipStream_t s) {
    const int64_t nchunks = (a.N + kChunk - 1) / kChunk;
    const int grid = grid_for(nchunks, kThreads, kApplyGridCap);
    if (sr) launch_apply_dt<MODE, true>(dtype, a, grid, s);
    else launch_apply_dt<MODE, false>(dtype, a, grid, s);
}

static size_t elem_size(int dtype) { return dtype == F32 ? 4 : 2; }

int factored_update(void* p, const void* grad, int dtype, int64_t R, int64_t C,
                    int64_t ps0, int64_t ps1, int64_t gs0, int64_t gs1,
                    uint8_t* m_codebook, float* m_magnitude, float* v_row, float* v_col,
                    int64_t period, const void* qtable, double beta1, double beta2,
                    double lr, double eps, double inv_bc2, double inv_bc1, double wdf,
                    int stochastic_round, int64_t rng_seed, const float* step_scalars,
                    const int64_t* seed_dev, void* workspace, size_t ws_bytes, hipStream_t s) {
    const int64_t N = R * C;
    const int64_t nb = N / period;
    const FactoredWs L = FactoredWs::make(R, C, nb);
    if (ws_bytes < L.total)
        return set_error(GEFENX_EINVAL, "factored update: workspace %zu bytes < required %zu", ws_bytes, L.total);
    char* ws = static_cast<char*>(workspace);
    double* row_sq = reinterpret_cast<double*>(ws + L.off_row);
    double* col_sq = reinterpret_cast<double*>(ws + L.off_col);
    uint32_t* magbits = reinterpret_cast<uint32_t*>(ws + L.off_magbits);
    float* mag_old = reinterpret_cast<float*>(ws + L.off_magold);
    float* scal = reinterpret_cast<float*>(ws + L.off_scal);
    const QTable* qt = static_cast<const QTable*>(qtable);
    const MomentumCoef mc = make_coef(beta1);
    const bool contig_g = (gs1 == 1 && gs0 == C);
    const bool contig_p = (ps1 == 1 && ps0 == C);

    // stats
    FactStatsArgs sa;
    sa.grad = grad; sa.idx = m_codebook; sa.mag_old = m_magnitude; sa.qt = qt;
    sa.R = R; sa.C = C; sa.gs0 = gs0; sa.gs1 = gs1; sa.P = period; sa.invP = 1.0 / (double)period;
    sa.fast = contig_g && (C % kChunk == 0) && aligned(grad, 16) && aligned(m_codebook, 8);
    sa.row_sq = row_sq; sa.col_sq = col_sq; sa.magbits = magbits; sa.mc = mc;
    const int64_t col_tiles = (C + kTileCols - 1) / kTileCols;
    int64_t tile_rows = (R * col_tiles) / 2048;  // aim for >= ~2048 workgroups
    tile_rows = std::max<int64_t>(1, std::min<int64_t>(kMaxTileRows, tile_rows));
    sa.tile_rows = (int)tile_rows;
    const int64_t row_tiles = (R + tile_rows - 1) / tile_rows;
    if (row_tiles > 2147483647LL || col_tiles > 65535)
        return set_error(GEFENX_EINVAL, "factored update: shape [%lld, %lld] exceeds the launch grid",
                         (long long)R, (long long)C);
    dim3 sgrid((unsigned)col_tiles, (unsigned)row_tiles);
    const double es = (double)elem_size(dtype);
    int ph = prof_begin(GEFENX_K_STATS, (double)N * (es + 1.0), 0.0, s);
    switch (dtype) {
        case F32: hipLaunchKernelGGL(k_factored_stats<F32>, sgrid, dim3(kThreads), 0, s, sa); break;
        case F16: hipLaunchKernelGGL(k_factored_stats<F16>, sgrid, dim3(kThreads), 0, s, sa); break;
        default: hipLaunchKernelGGL(k_factored_stats<BF16>, sgrid, dim3(kThreads), 0, s, sa); break;
    }
    prof_end(ph, s);
    int rc = launch_check("k_factored_stats");
    if (rc) return rc;

    // finalize
    FactFinArgs fa;
    fa.row_sq = row_sq; fa.col_sq = col_sq; fa.v_row = v_row; fa.v_col = v_col;
    fa.R = R; fa.C = C; fa.nb = nb; fa.beta2 = (float)beta2; fa.alpha2 = (float)(1.0 - beta2);
    fa.magbits = magbits; fa.mag = m_magnitude; fa.mag_old = mag_old; fa.scal = scal;
    const int fgrid = 1 + grid_for(nb, kThreads * 8, 1024);
    ph = prof_begin(GEFENX_K_FINALIZE, 8.0 * (double)(R + C + nb), 0.0, s);
    hipLaunchKernelGGL(k_factored_finalize, dim3(fgrid), dim3(kThreads), 0, s, fa);
    prof_end(ph, s);
    rc = launch_check("k_factored_finalize");
    if (rc) return rc;

    // apply
    ApplyArgs aa{};
    aa.p = p; aa.grad = grad; aa.idx = m_codebook; aa.mag_old = mag_old; aa.mag_new = m_magnitude;
    aa.v_row = v_row; aa.v_col = v_col; aa.scal = scal; aa.step = nullptr; aa.qt = qt;
    aa.N = N; aa.C = C; aa.P = period; aa.invC = 1.0 / (double)C; aa.invP = 1.0 / (double)period;
    aa.ps0 = ps0; aa.ps1 = ps1; aa.gs0 = gs0; aa.gs1 = gs1;
    aa.fast = contig_g && contig_p && (C % kChunk == 0) && aligned(grad, 16) && aligned(p, 16) &&
              aligned(m_codebook, 8);
    aa.write_p = (step_scalars != nullptr) || !(lr == 0.0 && (float)wdf == 1.0f);
    aa.eps = (float)eps;
    aa.sc = StepScalars{(float)lr, (float)inv_bc2, (float)inv_bc1, (float)wdf};
    aa.step_scalars = step_scalars;
    aa.mc = mc;
    aa.seed = (uint64_t)rng_seed;
    aa.seed_dev = seed_dev;
    // algorithmic bytes of the whole step: p r/w, g r, idx r/w per element
    // plus the fp32 state vectors read and written
    ph = prof_begin(GEFENX_K_APPLY, (double)N * (3.0 * es + 2.0) + 8.0 * (double)(R + C + nb), 0.0, s);
    launch_apply<0>(dtype, stochastic_round != 0, aa, s);
    prof_end(ph, s);
    return launch_check("k_apply(factored)");
}

int block_update(void* p, const void* grad, int dtype, int64_t N, int64_t period,
                 uint8_t* m_codebook, float* m_magnitude, float* vmean, const void* qtable,
                 double beta1, double beta2, double lr, double eps, double inv_sqrt_bc2,
                 double inv_bc1, double wdf, int stochastic_round, int64_t rng_seed,
                 const float* step_scalars, const int64_t* seed_dev, void* workspace,
                 size_t ws_bytes, hipStream_t s) {
    const int64_t nb = N / period;
    const BlockWs L = BlockWs::make(nb);
    if (ws_bytes < L.total)
        return set_error(GEFENX_EINVAL, "block update: workspace %zu bytes < required %zu", ws_bytes, L.total);
    char* ws = static_cast<char*>(workspace);
    double* blk_sq = reinterpret_cast<double*>(ws + L.off_sq);
    uint32_t* magbits = reinterpret_cast<uint32_t*>(ws + L.off_magbits);
    float* mag_old = reinterpret_cast<float*>(ws + L.off_magold);
    float* step = reinterpret_cast<float*>(ws + L.off_step);
    const QTable* qt = static_cast<const QTable*>(qtable);
    const MomentumCoef mc = make_coef(beta1);

    BlockStatsArgs sa;
    sa.grad = grad; sa.idx = m_codebook; sa.mag_old = m_magnitude; sa.qt = qt;
    sa.N = N; sa.P = period; sa.invP = 1.0 / (double)period;
    sa.fast = aligned(grad, 16) && aligned(m_codebook, 8);
    sa.blk_sq = blk_sq; sa.magbits = magbits; sa.mc = mc;
    const int64_t nchunks = (N + kChunk - 1) / kChunk;
    const int sgrid = grid_for(nchunks, kThreads * 4, kApplyGridCap);
    const double es = (double)elem_size(dtype);
    int ph = prof_begin(GEFENX_K_STATS, (double)N * (es + 1.0), 0.0, s);
    switch (dtype) {
        case F32: hipLaunchKernelGGL(k_block_stats<F32>, dim3(sgrid), dim3(kThreads), 0, s, sa); break;
        case F16: hipLaunchKernelGGL(k_block_stats<F16>, dim3(sgrid), dim3(kThreads), 0, s, sa); break;
        default: hipLaunchKernelGGL(k_block_stats<BF16>, dim3(sgrid), dim3(kThreads), 0, s, sa); break;
    }
    prof_end(ph, s);
    int rc = launch_check("k_block_stats");
    if (rc) return rc;

    BlockFinArgs fa;
    fa.blk_sq = blk_sq; fa.vmean = vmean; fa.nb = nb; fa.P = period;
    fa.beta2 = (float)beta2; fa.alpha2 = (float)(1.0 - beta2); fa.eps = (float)eps;
    fa.bf16_mean = (dtype == BF16) ? 1 : 0;
    fa.sc = StepScalars{(float)lr, (float)inv_sqrt_bc2, (float)inv_bc1, (float)wdf};
    fa.step_scalars = step_scalars;
    fa.magbits = magbits; fa.mag = m_magnitude; fa.mag_old = mag_old; fa.step = step;
    ph = prof_begin(GEFENX_K_FINALIZE, 16.0 * (double)nb, 0.0, s);
    hipLaunchKernelGGL(k_block_finalize, dim3(grid_for(nb, kThreads, 4096)), dim3(kThreads), 0, s, fa);
    prof_end(ph, s);
    rc = launch_check("k_block_finalize");
    if (rc) return rc;

    ApplyArgs aa{};
    aa.p = p; aa.grad = grad; aa.idx = m_codebook; aa.mag_old = mag_old; aa.mag_new = m_magnitude;
    aa.step = step; aa.qt = qt;
    aa.N = N; aa.C = N; aa.P = period; aa.invC = 1.0 / (double)N; aa.invP = 1.0 / (double)period;
    aa.ps0 = N; aa.ps1 = 1; aa.gs0 = N; aa.gs1 = 1;
    aa.fast = aligned(grad, 16) && aligned(p, 16) && aligned(m_codebook, 8);
    aa.write_p = (step_scalars != nullptr) || !(lr == 0.0 && (float)wdf == 1.0f);
    aa.eps = (float)eps;
    aa.sc = fa.sc;
    aa.step_scalars = step_scalars;
    aa.mc = mc;
    aa.seed = (uint64_t)rng_seed;
    aa.seed_dev = seed_dev;
    ph = prof_begin(GEFENX_K_APPLY, (double)N * (3.0 * es + 2.0) + 16.0 * (double)nb, 0.0, s);
    launch_apply<1>(dtype, stochastic_round != 0, aa, s);
    prof_end(ph, s);
    return launch_check("k_apply(block)");
}

}  // namespace gx

using namespace gx;

static int check_dtype(int dtype, const char* fn) {
    if (dtype == F64)
        return set_error(GEFENX_EDTYPE, "%s: not implemented for 'Double' (fp32/fp16/bf16 only)", fn);
    if (dtype != F32 && dtype != F16 && dtype != BF16)
        return set_error(GEFENX_EINVAL, "%s: unknown dtype code %d", fn, dtype);
    return GEFENX_OK;
}

extern "C" {

int gefenx_factored_update(
    void* p, const void* grad, int dtype, int64_t rows, int64_t cols,
    int64_t ps0, int64_t ps1, int64_t gs0, int64_t gs1,
    uint8_t* m_codebook, float* m_magnitude, float* v_row, float* v_col,
    int64_t period, const void* qtable_dev,
    double beta1, double beta2, double lr, double eps,
    double inv_bias_correction_2, double inv_bias_correction_1,
    double weight_decay_factor, int stochastic_round, int64_t rng_seed,
    const float* step_scalars, const int64_t* seed_dev,
    void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_dtype(dtype, "gefenx_factored_update");
    if (rc) return rc;
    if (rows < 0 || cols < 0) return set_error(GEFENX_EINVAL, "gefenx_factored_update: negative shape");
    const int64_t N = rows * cols;
    if (N == 0) return GEFENX_OK;  // empty tensors are a no-op
    if (period <= 0 || N % period != 0)
        return set_error(GEFENX_EINVAL, "gefenx_factored_update: period %lld does not divide numel %lld",
                         (long long)period, (long long)N);
    if (!p || !grad || !m_codebook || !m_magnitude || !v_row || !v_col || !qtable_dev || !workspace)
        return set_error(GEFENX_EINVAL, "gefenx_factored_update: null pointer argument");
    return factored_update(p, grad, dtype, rows, cols, ps0, ps1, gs0, gs1, m_codebook, m_magnitude,
                           v_row, v_col, period, qtable_dev, beta1, beta2, lr, eps,
                           inv_bias_correction_2, inv_bias_correction_1, weight_decay_factor,
                           stochastic_round, rng_seed, step_scalars, seed_dev, workspace,
                           workspace_bytes, static_cast<hipStream_t>(stream));
}

int gefenx_block_update(
    void* p, const void* grad, int dtype, int64_t numel, int64_t period,
    uint8_t* m_codebook, float* m_magnitude, float* vmean, const void* qtable_dev,
    double beta1, double beta2, double lr, double eps,
    double inv_sqrt_bias_correction_2, double inv_bias_correction_1,
    double weight_decay_factor, int stochastic_round, int64_t rng_seed,
    const float* step_scalars, const int64_t* seed_dev,
    void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_dtype(dtype, "gefenx_block_update");
    if (rc) return rc;
    if (numel < 0) return set_error(GEFENX_EINVAL, "gefenx_block_update: negative numel");
    if (numel == 0) return GEFENX_OK;
    if (period <= 0 || numel % period != 0)
        return set_error(GEFENX_EINVAL, "gefenx_block_update: period %lld does not divide numel %lld",
                         (long long)period, (long long)numel);
    if (!p || !grad || !m_codebook || !m_magnitude || !vmean || !qtable_dev || !workspace)
        return set_error(GEFENX_EINVAL, "gefenx_block_update: null pointer argument");
    return block_update(p, grad, dtype, numel, period, m_codebook, m_magnitude, vmean, qtable_dev,
                        beta1, beta2, lr, eps, inv_sqrt_bias_correction_2, inv_bias_correction_1,
                        weight_decay_factor, stochastic_round, rng_seed, step_scalars, seed_dev,
                        workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
