// gefenx_update.hip -- fused Gefen update kernels for MI355X (gfx950, wave64).
//
// Per parameter the step is three launches on the caller's stream:
//   stats    one pass over grad + stored indices: per-block max |u| (u = the
//            updated momentum) and the second-moment sums (per-tile row/column
//            partial sums of g^2 for the factored path, per-block sums for the
//            block path);
//   finalize tiny: EMA of the second moment, mean(v_row), new magnitudes and
//            their reciprocals, per-block stepsizes; re-zeroes the workspace
//            accumulators;
//   apply    one pass: recompute u, normalise by the new magnitude,
//            requantise through the exact threshold table, write the indices
//            and the parameter (decoupled weight decay folded in).
// The math follows the reference's decomposed step (gefen.py:2959-3018,
// 3329-3486, 3776-3818); gefenx_device.h holds the bit-exact momentum,
// division and quantisation primitives.
#include "gefenx_device.h"
#include "gefenx_internal.h"
#include "gefenx_profile.h"
#include "../../include/gefenx.h"

#include <algorithm>
#include <cmath>

namespace gx {

constexpr int kThreads = 256;
constexpr int kChunk = 8;

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

// Wave-uniform running block max of |u| as ordered uint bits (NaN > inf >
// finite, so the integer max propagates NaN like torch's amax).  `blk` is
// identical in every lane; `bits` is each lane's partial.
struct WaveMax {
    int64_t blk;
    uint32_t bits;
};

__device__ __forceinline__ void wavemax_flush(uint32_t* __restrict__ magbits, WaveMax& wm) {
    if (wm.blk >= 0) {
        const uint32_t m = wave_max_u(wm.bits);
        if ((threadIdx.x & 63) == 0 && m != 0u) atomicMax(magbits + wm.blk, m);
    }
    wm.bits = 0u;
}

// ====================================================================
// Factored stats.  Workgroup = 4 waves over a tile of `tile_rows` rows x 512
// columns: lane l owns columns [c0 + 8l, c0 + 8l + 8), wave w takes rows
// r0 + w, r0 + w + 4, ...  Row sums reduce per wave (one value per row per
// column tile), column sums reduce across the 4 waves in LDS; both are
// written as float64 partials (no atomics, deterministic), summed by the
// finalize kernel.
// ====================================================================
struct FactStatsArgs {
    const void* grad;
    const uint8_t* idx;
    const float* mag_old;
    const QTable* qt;
    int64_t R, C, gs0, gs1, P;
    double invP;
    int64_t tile_rows, ct;
    int fast;  // contiguous grad, C % 8 == 0, P % 8 == 0, aligned
    double* row_part;  // [ct][R]
    double* col_part;  // [rt][C]
    uint32_t* magbits; // [shards][nb]
    int64_t nb, shards;
    MomentumCoef mc;
};

template <int DT, bool FAST>
__global__ void __launch_bounds__(kThreads) k_factored_stats(FactStatsArgs a) {
    using T = typename Elem<DT>::T;
    __shared__ float s_cbr[kCodebookMax];
    __shared__ double s_col[kThreads / 64 - 1][kFactTileCols];
    for (int i = threadIdx.x; i < kCodebookMax; i += kThreads) s_cbr[i] = a.qt->cbr[i];
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t ctile = (int64_t)blockIdx.x % a.ct;
    const int64_t rtile = (int64_t)blockIdx.x / a.ct;
    const int64_t c0 = ctile * kFactTileCols + (int64_t)lane * kChunk;
    const int64_t r_begin = rtile * a.tile_rows;
    const int64_t r_end = std::min<int64_t>(r_begin + a.tile_rows, a.R);
    const int nvalid = (int)std::max<int64_t>(0, std::min<int64_t>(kChunk, a.C - c0));
    const T* g = static_cast<const T*>(a.grad);
    uint32_t* mb = a.magbits + ((int64_t)blockIdx.x % a.shards) * a.nb;

    double colacc[kChunk];
#pragma unroll
    for (int k = 0; k < kChunk; ++k) colacc[k] = 0.0;
    WaveMax wm{-1, 0u};
    float mag_cur = 0.0f;

    // kU rows of a wave are loaded before any is reduced, so each lane keeps
    // kU grad + index loads in flight.
    constexpr int kU = 4;
    constexpr int64_t kWaves = kThreads / 64;
    for (int64_t rg = r_begin + wave; rg < r_end; rg += kU * kWaves) {
    Raw8<DT> graw[kU];
    RawIdx8 iraw[kU];
    float gvu[kU][kChunk];
    uint32_t ixu[kU][kChunk];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const int64_t r = rg + (int64_t)u * kWaves;
        const int64_t e0 = r * a.C + c0;
        if constexpr (FAST) {
            if (r < r_end && nvalid == kChunk) {
                load_raw8<DT>(g + e0, graw[u]);
                iraw[u] = load_raw_idx8(a.idx + e0);
            } else {
                graw[u] = Raw8<DT>{};
                iraw[u] = RawIdx8{0u, 0u};
            }
        } else {
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                if (r < r_end && k < nvalid) {
                    gvu[u][k] = to_f32<DT>(g[r * a.gs0 + (c0 + k) * a.gs1]);
                    ixu[u][k] = a.idx[e0 + k];
                } else {
                    gvu[u][k] = 0.0f;
                    ixu[u][k] = 0u;
                }
            }
        }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const int64_t r = rg + (int64_t)u * kWaves;
        if (r >= r_end) break;
        const int64_t e0 = r * a.C + c0;
        float gv[kChunk];
        uint32_t ix[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if constexpr (FAST) {
                gv[k] = raw_elem<DT>(graw[u], k);
                ix[k] = raw_idx(iraw[u], k);
            } else {
                gv[k] = gvu[u][k];
                ix[k] = ixu[u][k];
            }
        }
        // block of this row strip: uniform across the wave when the wave's
        // 512 columns never cross a block boundary
        const int64_t e_first = r * a.C + ctile * kFactTileCols;
        const int64_t blk0 = div_floor(e_first, a.P, a.invP);
        const int64_t span = std::min<int64_t>(kFactTileCols, a.C - ctile * kFactTileCols);
        const bool uniform = (e_first + span - 1) < (blk0 + 1) * a.P;
        float rowacc = 0.0f;
        if (uniform) {
            if (blk0 != wm.blk) {
                wavemax_flush(mb, wm);
                wm.blk = blk0;
                mag_cur = a.mag_old[blk0];
            }
            uint32_t m = wm.bits;
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                if (k < nvalid) {
                    const float u = momentum_value(s_cbr[ix[k]], mag_cur, gv[k], a.mc);
                    const uint32_t ub = __float_as_uint(u) & 0x7fffffffu;
                    m = ub > m ? ub : m;
                    const float sq = gv[k] * gv[k];
                    rowacc += sq;
                    colacc[k] += (double)sq;
                }
            }
            wm.bits = m;
        } else {
            // blocks smaller than the strip: per-lane runs, one atomic per run
            wavemax_flush(mb, wm);
            wm.blk = -1;
            if (nvalid > 0) {
                int64_t blk = div_floor(e0, a.P, a.invP);
                int64_t pin = e0 - blk * a.P;
                float mo = a.mag_old[blk];
                uint32_t m = 0u;
#pragma unroll
                for (int k = 0; k < kChunk; ++k) {
                    if (k < nvalid) {
                        const float u = momentum_value(s_cbr[ix[k]], mo, gv[k], a.mc);
                        const uint32_t ub = __float_as_uint(u) & 0x7fffffffu;
                        m = ub > m ? ub : m;
                        const float sq = gv[k] * gv[k];
                        rowacc += sq;
                        colacc[k] += (double)sq;
                        if (++pin == a.P) {
                            if (m) atomicMax(mb + blk, m);
                            m = 0u;
                            pin = 0;
                            ++blk;
                            if (k + 1 < nvalid) mo = a.mag_old[blk];
                        }
                    }
                }
                if (m) atomicMax(mb + blk, m);
            }
        }
        const double rs = wave_sum_d((double)rowacc);
        if (lane == 0) a.row_part[ctile * a.R + r] = rs;
    }
    }
    // final block-max flush: one atomic per workgroup when the waves agree
    __shared__ int64_t s_wblk[kThreads / 64];
    __shared__ uint32_t s_wbits[kThreads / 64];
    const uint32_t wbits = wave_max_u(wm.bits);
    if (lane == 0) {
        s_wblk[wave] = wm.blk;
        s_wbits[wave] = wbits;
    }
    // column partials: waves 1..3 park theirs in LDS, wave 0 adds and stores
    if (wave > 0) {
#pragma unroll
        for (int k = 0; k < kChunk; ++k) s_col[wave - 1][lane * kChunk + k] = colacc[k];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        bool same = true;
        uint32_t m = 0u;
        for (int w = 0; w < kThreads / 64; ++w) {
            same = same && (s_wblk[w] == s_wblk[0]);
            m = s_wbits[w] > m ? s_wbits[w] : m;
        }
        if (same) {
            if (s_wblk[0] >= 0 && m) atomicMax(mb + s_wblk[0], m);
        } else {
            for (int w = 0; w < kThreads / 64; ++w)
                if (s_wblk[w] >= 0 && s_wbits[w]) atomicMax(mb + s_wblk[w], s_wbits[w]);
        }
    }
    if (wave == 0) {
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            double s = colacc[k];
#pragma unroll
            for (int w = 0; w < kThreads / 64 - 1; ++w) s += s_col[w][lane * kChunk + k];
            if (k < nvalid) a.col_part[rtile * a.C + c0 + k] = s;
        }
    }
}

// ====================================================================
// Factored finalize.  Workgroups [0, nr): v_row EMA from the ct row partials,
// one float64 partial of sum(v_row) per workgroup; [nr, nr+nc): v_col EMA
// from the rt column partials; the rest: new magnitudes (max over shards),
// their reciprocals, the old magnitudes.
// v <- fma(sum/n, 1-beta2, v*beta2)  (gefen.py:2994-2996)
// ====================================================================
struct FactFinArgs {
    const double* row_part;
    const double* col_part;
    float* v_row;
    float* v_col;
    int64_t R, C, nb, ct, rt, shards;
    int64_t nr, nc;   // row / column workgroup counts
    float beta2, alpha2;
    uint32_t* magbits;
    float* mag;      // m_magnitude: receives the new magnitudes
    float* mag_old;  // workspace: receives the old magnitudes
    float* minv;     // workspace: reciprocal of the new magnitudes
    double* vsum;    // workspace: [nr] partials of sum(v_row)
};

__global__ void __launch_bounds__(kThreads) k_factored_finalize(FactFinArgs a) {
    const int tid = threadIdx.x;
    const int64_t wg = blockIdx.x;
    if (wg < a.nr) {
        __shared__ double s_part[kThreads / 64];
        const int64_t i = wg * kFinRowsPerWg + tid;
        double v64 = 0.0;
        if (i < a.R) {
            double s = 0.0;
            for (int64_t t = 0; t < a.ct; ++t) s += a.row_part[t * a.R + i];
            const float ms = (float)s / (float)a.C;
            const float v = __builtin_fmaf(ms, a.alpha2, a.v_row[i] * a.beta2);
            a.v_row[i] = v;
            v64 = (double)v;
        }
        v64 = wave_sum_d(v64);
        if ((tid & 63) == 0) s_part[tid >> 6] = v64;
        __syncthreads();
        if (tid == 0) {
            double s = 0.0;
            for (int w = 0; w < kThreads / 64; ++w) s += s_part[w];
            a.vsum[wg] = s;
        }
        return;
    }
    if (wg < a.nr + a.nc) {
        // 64 columns per workgroup; wave w adds row tiles t = w, w+4, ...
        __shared__ double s_cp[kThreads / 64][64];
        const int lane = tid & 63;
        const int wave = tid >> 6;
        const int64_t j = (wg - a.nr) * 64 + lane;
        double s = 0.0;
        if (j < a.C)
            for (int64_t t = wave; t < a.rt; t += kThreads / 64) s += a.col_part[t * a.C + j];
        s_cp[wave][lane] = s;
        __syncthreads();
        if (wave == 0 && j < a.C) {
            double tot = 0.0;
            for (int w = 0; w < kThreads / 64; ++w) tot += s_cp[w][lane];
            const float ms = (float)tot / (float)a.R;
            a.v_col[j] = __builtin_fmaf(ms, a.alpha2, a.v_col[j] * a.beta2);
        }
        return;
    }
    const int64_t gtid = (wg - a.nr - a.nc) * kThreads + tid;
    const int64_t gstride = ((int64_t)gridDim.x - a.nr - a.nc) * kThreads;
    for (int64_t b = gtid; b < a.nb; b += gstride) {
        const float old = a.mag[b];
        a.mag_old[b] = old;
        uint32_t bits = 0u;
        for (int64_t sh = 0; sh < a.shards; ++sh) {
            const uint32_t v = a.magbits[sh * a.nb + b];
            bits = v > bits ? v : bits;
            a.magbits[sh * a.nb + b] = 0u;
        }
        const float m = __uint_as_float(bits);
        a.mag[b] = m;
        a.minv[b] = block_recip(m);
    }
}

// Deterministic mean(v_row) from the finalize partials, clamped at FLT_MIN
// (gefen.py:2998-3000); every workgroup of the apply kernel recomputes it.
__device__ __forceinline__ float mean_from_partials(const double* __restrict__ vsum, int64_t nr, int64_t R) {
    __shared__ double s_red[kThreads];
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < nr; i += kThreads) acc += vsum[i];
    s_red[threadIdx.x] = acc;
    __syncthreads();
    for (int off = kThreads / 2; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off) s_red[threadIdx.x] += s_red[threadIdx.x + off];
        __syncthreads();
    }
    float mean = (float)s_red[0] / (float)R;
    if (!(mean >= 1.17549435e-38f) && mean == mean) mean = 1.17549435e-38f;
    return mean;
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
    uint32_t* magbits;  // [shards][nb]
    int64_t nb, shards;
    MomentumCoef mc;
};

template <int DT>
__global__ void __launch_bounds__(kThreads) k_block_stats(BlockStatsArgs a) {
    using T = typename Elem<DT>::T;
    __shared__ float s_cbr[kCodebookMax];
    for (int i = threadIdx.x; i < kCodebookMax; i += kThreads) s_cbr[i] = a.qt->cbr[i];
    __syncthreads();
    const T* g = static_cast<const T*>(a.grad);
    uint32_t* mb = a.magbits + ((int64_t)blockIdx.x % a.shards) * a.nb;
    const int64_t nchunks = (a.N + kChunk - 1) / kChunk;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    int64_t cur = -1;
    uint32_t cbits = 0u;
    double bsum = 0.0;
    float mo = 0.0f;
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
                if (blk != cur) {
                    if (cur >= 0) {
                        bsum += (double)csum;
                        csum = 0.0f;
                        if (bsum != 0.0) atomicAdd(a.blk_sq + cur, bsum);
                        if (cbits) atomicMax(mb + cur, cbits);
                    }
                    bsum = 0.0;
                    cbits = 0u;
                    cur = blk;
                    mo = a.mag_old[blk];
                }
                const float u = momentum_value(s_cbr[ix[k]], mo, gv[k], a.mc);
                const uint32_t ub = __float_as_uint(u) & 0x7fffffffu;
                cbits = ub > cbits ? ub : cbits;
                float sq = gv[k] * gv[k];
                if constexpr (DT == BF16) sq = round_dt<BF16>(sq);
                csum += sq;
                if (++pin == a.P) { pin = 0; ++blk; }
            }
        }
        bsum += (double)csum;
    }
    const int lane = threadIdx.x & 63;
    const int64_t c0 = __shfl(cur, 0, 64);
    if (__all(cur == c0)) {
        const double s = wave_sum_d(bsum);
        const uint32_t m = wave_max_u(cbits);
        if (lane == 0 && c0 >= 0) {
            if (s != 0.0) atomicAdd(a.blk_sq + c0, s);
            if (m) atomicMax(mb + c0, m);
        }
    } else if (cur >= 0) {
        if (bsum != 0.0) atomicAdd(a.blk_sq + cur, bsum);
        if (cbits) atomicMax(mb + cur, cbits);
    }
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
    float* minv;
    int64_t shards;
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
        uint32_t bits = 0u;
        for (int64_t sh = 0; sh < a.shards; ++sh) {
            const uint32_t v = a.magbits[sh * a.nb + b];
            bits = v > bits ? v : bits;
            a.magbits[sh * a.nb + b] = 0u;
        }
        const float m = __uint_as_float(bits);
        a.mag[b] = m;
        a.minv[b] = block_recip(m);
    }
}

// ====================================================================
// Apply: grid-stride over logical chunks of 8 elements.  MODE 0 factored,
// MODE 1 block.  FAST: contiguous p/grad, C % 8 == 0, P % 8 == 0, aligned --
// a chunk then never crosses a row or a block, and (row, col, blk) advance
// by constant strides between iterations (no per-chunk division).
// ====================================================================
struct ApplyArgs {
    void* p;
    const void* grad;
    uint8_t* idx;
    const float* mag_old;
    const float* mag_new;
    const float* minv;
    const float* v_row;   // factored
    const float* v_col;   // factored
    const double* vsum;   // factored: [nr] partials of sum(v_row)
    int64_t nr, R;
    const float* step;    // block: per-block stepsize
    const QTable* qt;
    int64_t N, C, P;
    double invC, invP;
    int64_t ps0, ps1, gs0, gs1;
    // FAST iteration strides: S = gridDim.x * 256 * 8 elements = dR*C + dC = dB*P + dP
    int64_t dR, dC, dB, dP;
    int write_p;     // 0 when lr == 0 and wd_factor == 1
    float eps;
    StepScalars sc;
    const float* step_scalars;
    MomentumCoef mc;
    uint64_t seed;
    const int64_t* seed_dev;
};

// Logical position of a chunk: row/column (factored) and block/offset.
struct Pos {
    int64_t row, col, blk, pin;
};

template <int MODE>
__device__ __forceinline__ Pos advance(const ApplyArgs& a, Pos q) {
    if constexpr (MODE == 0) {
        q.col += a.dC;
        q.row += a.dR;
        if (q.col >= a.C) { q.col -= a.C; ++q.row; }
    }
    q.pin += a.dP;
    q.blk += a.dB;
    if (q.pin >= a.P) { q.pin -= a.P; ++q.blk; }
    return q;
}

__device__ __forceinline__ void load_vcol(const float* __restrict__ vc, float v[8]) {
    const f32x4* q = reinterpret_cast<const f32x4*>(vc);
    const f32x4 v0 = q[0], v1 = q[1];
    v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
    v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
}

// One chunk of 8 elements that shares a row and a block (fast path).  The
// division u / m_new goes through the block reciprocal (div_by_block's
// Markstein step) for every lane; a wave where any lane is outside that
// step's safe range (tiny |u|, unusable reciprocal: zero, subnormal, huge,
// inf or NaN magnitude) redoes the chunk with the fully guarded helpers.
template <int DT, int MODE, bool SR>
__device__ __forceinline__ void apply_chunk(const ApplyArgs& a, const SharedTables& st,
                                            const SharedSR& ssr, int64_t e0, const Pos& ps,
                                            const Raw8<DT>& gr, const Raw8<DT>& pr,
                                            const RawIdx8& ir, const float vcv[kChunk],
                                            uint32_t ix[kChunk], float pv[kChunk],
                                            float row_scale, float c1, bool wd,
                                            const StepScalars& sc, bool dense, uint32_t kmax,
                                            int kk, uint64_t seed) {
    const float m_old = a.mag_old[ps.blk];
    const float m_new = a.mag_new[ps.blk];
    const float y = a.minv[ps.blk];
    const float tb = 0x1.00001p-100f * fmaxf(m_new, 1.0f);
    float xs[kChunk];
    bool bad = (y == 0.0f);
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
        const float u = momentum_value(st.cbr[raw_idx(ir, k)], m_old, raw_elem<DT>(gr, k), a.mc);
        const float q0 = u * y;
        const float r = __builtin_fmaf(-q0, m_new, u);
        xs[k] = __builtin_fmaf(r, y, q0);
        bad = bad || !(fabsf(u) >= tb);
    }
    if (__any(bad)) {
        const bool nz = m_new > 0.0f;
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            const float u = momentum_value(st.cbr[raw_idx(ir, k)], m_old, raw_elem<DT>(gr, k), a.mc);
            const float x = nz ? div_by_block(u, m_new, y) : 0.0f;
            if constexpr (SR) ix[k] = quant_stochastic(x, ssr.cb, ssr.lut, kk, seed, e0 + k);
            else ix[k] = quant_nearest(x, st.bkt, st.thr, kmax);
        }
    } else {
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if constexpr (SR) ix[k] = quant_stochastic(xs[k], ssr.cb, ssr.lut, kk, seed, e0 + k);
            else ix[k] = quant_fast(xs[k], st, dense);
        }
    }
    if (a.write_p) {
        float rs = 0.0f, bstep = 0.0f;
        if constexpr (MODE == 0) rs = a.v_row[ps.row] * row_scale;
        else bstep = a.step[ps.blk] * sc.lr;
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            const float q = st.cbr[ix[k]] * m_new;
            float s;
            if constexpr (MODE == 0) {
                const float h = __builtin_amdgcn_sqrtf(rs * vcv[k]) + a.eps;
                s = __builtin_amdgcn_rcpf(h) * c1;
            } else {
                s = bstep;
            }
            float pw = raw_elem<DT>(pr, k);
            if (wd) pw = round_dt<DT>(pw * sc.wdf);
            pv[k] = pw - q * s;
        }
    }
}

template <int DT, int MODE, bool SR, bool FAST>
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
    float row_scale = 0.0f;  // mean(v_row)^-1 * (1/bc2)
    if constexpr (MODE == 0) row_scale = (1.0f / mean_from_partials(a.vsum, a.nr, a.R)) * sc.inv_bc2;
    const float c1 = sc.inv_bc1 * sc.lr;
    const bool wd = sc.wdf != 1.0f;

    T* p = static_cast<T*>(a.p);
    const T* g = static_cast<const T*>(a.grad);
    const int64_t nchunks = (a.N + kChunk - 1) / kChunk;
    int64_t ch = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    if (ch >= nchunks) return;

    if constexpr (FAST) {
        // Two chunks per iteration (ch and ch + stride): both chunks' loads are
        // issued before either is computed, so every lane keeps ~80 bytes of
        // HBM reads in flight.  (row, col, blk, pin) of a chunk advance to the
        // chunk one stride later by constant increments (no division).
        Pos pa;
        {
            const int64_t e0 = ch * kChunk;
            pa.row = 0;
            pa.col = e0;
            if constexpr (MODE == 0) {
                pa.row = div_floor(e0, a.C, a.invC);
                pa.col = e0 - pa.row * a.C;
            }
            pa.blk = div_floor(e0, a.P, a.invP);
            pa.pin = e0 - pa.blk * a.P;
        }
        const bool dense = a.qt->max_cnt > 2;
        for (; ch < nchunks; ch += 2 * stride) {
            const bool has_b = ch + stride < nchunks;
            const Pos pb = advance<MODE>(a, pa);
            const int64_t ea = ch * kChunk, eb = (ch + stride) * kChunk;
            Raw8<DT> rga, rpa, rgb, rpb;
            RawIdx8 ria, rib;
            float va[kChunk], vb[kChunk];
            load_raw8<DT>(g + ea, rga);
            ria = load_raw_idx8(a.idx + ea);
            if (a.write_p) {
                load_raw8<DT>(p + ea, rpa);
                if constexpr (MODE == 0) load_vcol(a.v_col + pa.col, va);
            }
            if (has_b) {
                load_raw8<DT>(g + eb, rgb);
                rib = load_raw_idx8(a.idx + eb);
                if (a.write_p) {
                    load_raw8<DT>(p + eb, rpb);
                    if constexpr (MODE == 0) load_vcol(a.v_col + pb.col, vb);
                }
            }
            uint32_t ix[kChunk];
            float pv[kChunk];
            apply_chunk<DT, MODE, SR>(a, st, ssr, ea, pa, rga, rpa, ria, va, ix, pv, row_scale, c1, wd, sc,
                                      dense, kmax, kk, seed);
            store_idx8(a.idx + ea, ix);
            if (a.write_p) store8<DT>(p + ea, pv);
            if (has_b) {
                apply_chunk<DT, MODE, SR>(a, st, ssr, eb, pb, rgb, rpb, rib, vb, ix, pv, row_scale, c1, wd,
                                          sc, dense, kmax, kk, seed);
                store_idx8(a.idx + eb, ix);
                if (a.write_p) store8<DT>(p + eb, pv);
            }
            pa = advance<MODE>(a, pb);
        }
    } else {
        for (; ch < nchunks; ch += stride) {
            const int64_t e0 = ch * kChunk;
            const int nvalid = (int)std::min<int64_t>(kChunk, a.N - e0);
            int64_t row = div_floor(e0, a.C, a.invC);
            int64_t col = e0 - row * a.C;
            int64_t blk = div_floor(e0, a.P, a.invP);
            int64_t pin = e0 - blk * a.P;
            float gv[kChunk], pv[kChunk];
            uint32_t ix[kChunk];
            {
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
            float y = a.minv[blk];
            float bstep = 0.0f;
            if constexpr (MODE == 1) bstep = a.step[blk] * sc.lr;
            float rs = 0.0f;
            if constexpr (MODE == 0) rs = a.v_row[row] * row_scale;
            int64_t r = row, c = col;
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                if (k < nvalid) {
                    const float u = momentum_value(st.cbr[ix[k]], m_old, gv[k], a.mc);
                    const float x = (m_new > 0.0f) ? div_by_block(u, m_new, y) : 0.0f;
                    uint32_t ni;
                    if constexpr (SR) ni = quant_stochastic(x, ssr.cb, ssr.lut, kk, seed, e0 + k);
                    else ni = quant_nearest(x, st.bkt, st.thr, kmax);
                    ix[k] = ni;
                    if (a.write_p) {
                        const float q = st.cbr[ni] * m_new;
                        float s;
                        if constexpr (MODE == 0) {
                            const float h = __builtin_amdgcn_sqrtf(rs * a.v_col[c]) + a.eps;
                            s = __builtin_amdgcn_rcpf(h) * c1;
                        } else {
                            s = bstep;
                        }
                        float pw = pv[k];
                        if (wd) pw = round_dt<DT>(pw * sc.wdf);
                        pv[k] = pw - q * s;
                    }
                    if (++c == a.C) {
                        c = 0;
                        ++r;
                        if constexpr (MODE == 0) {
                            if (k + 1 < nvalid) rs = a.v_row[r] * row_scale;
                        }
                    }
                    if (++pin == a.P) {
                        pin = 0;
                        ++blk;
                        if (k + 1 < nvalid) {
                            m_old = a.mag_old[blk];
                            m_new = a.mag_new[blk];
                            y = a.minv[blk];
                            if constexpr (MODE == 1) bstep = a.step[blk] * sc.lr;
                        }
                    }
                }
            }
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

constexpr int kApplyGridCap = 4096;

template <int MODE, bool SR, bool FAST>
static void launch_apply_dt(int dtype, const ApplyArgs& a, int grid, hipStream_t s) {
    switch (dtype) {
        case F32: hipLaunchKernelGGL((k_apply<F32, MODE, SR, FAST>), dim3(grid), dim3(kThreads), 0, s, a); break;
        case F16: hipLaunchKernelGGL((k_apply<F16, MODE, SR, FAST>), dim3(grid), dim3(kThreads), 0, s, a); break;
        default: hipLaunchKernelGGL((k_apply<BF16, MODE, SR, FAST>), dim3(grid), dim3(kThreads), 0, s, a); break;
    }
}

template <int MODE>
static void launch_apply(int dtype, bool sr, bool fast, ApplyArgs a, hipStream_t s) {
    const int64_t nchunks = (a.N + kChunk - 1) / kChunk;
    const int grid = grid_for(nchunks, kThreads, kApplyGridCap);
    const int64_t S = (int64_t)grid * kThreads * kChunk;
    a.dR = S / a.C;
    a.dC = S - a.dR * a.C;
    a.dB = S / a.P;
    a.dP = S - a.dB * a.P;
    if (fast) {
        if (sr) launch_apply_dt<MODE, true, true>(dtype, a, grid, s);
        else launch_apply_dt<MODE, false, true>(dtype, a, grid, s);
    } else {
        if (sr) launch_apply_dt<MODE, true, false>(dtype, a, grid, s);
        else launch_apply_dt<MODE, false, false>(dtype, a, grid, s);
    }
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
    const FactTiles tiles = FactTiles::make(R, C);
    if (ws_bytes < L.total)
        return set_error(GEFENX_EINVAL, "factored update: workspace %zu bytes < required %zu", ws_bytes, L.total);
    char* ws = static_cast<char*>(workspace);
    double* row_part = reinterpret_cast<double*>(ws + L.off_rowp);
    double* col_part = reinterpret_cast<double*>(ws + L.off_colp);
    uint32_t* magbits = reinterpret_cast<uint32_t*>(ws + L.off_magbits);
    float* mag_old = reinterpret_cast<float*>(ws + L.off_magold);
    float* minv = reinterpret_cast<float*>(ws + L.off_minv);
    double* vsum = reinterpret_cast<double*>(ws + L.off_vsum);
    const int64_t shards = mag_shards(nb);
    const QTable* qt = static_cast<const QTable*>(qtable);
    const MomentumCoef mc = make_coef(beta1);
    const bool contig_g = (gs1 == 1 && gs0 == C);
    const bool contig_p = (ps1 == 1 && ps0 == C);
    const double es = (double)elem_size(dtype);

    FactStatsArgs sa;
    sa.grad = grad; sa.idx = m_codebook; sa.mag_old = m_magnitude; sa.qt = qt;
    sa.R = R; sa.C = C; sa.gs0 = gs0; sa.gs1 = gs1; sa.P = period; sa.invP = 1.0 / (double)period;
    sa.tile_rows = tiles.tile_rows; sa.ct = tiles.ct;
    sa.fast = contig_g && (C % kChunk == 0) && aligned(grad, 16) && aligned(m_codebook, 8);
    sa.row_part = row_part; sa.col_part = col_part; sa.magbits = magbits; sa.mc = mc;
    sa.nb = nb; sa.shards = shards;
    const int64_t nwg = tiles.ct * tiles.rt;
    if (nwg > 2147483647LL)
        return set_error(GEFENX_EINVAL, "factored update: shape [%lld, %lld] exceeds the launch grid",
                         (long long)R, (long long)C);
    int ph = prof_begin(GEFENX_K_STATS, (double)N * (es + 1.0), 0.0, s);
#define GX_STATS(DTV)                                                                                   \
    if (sa.fast) hipLaunchKernelGGL((k_factored_stats<DTV, true>), dim3((unsigned)nwg), dim3(kThreads), 0, s, sa); \
    else hipLaunchKernelGGL((k_factored_stats<DTV, false>), dim3((unsigned)nwg), dim3(kThreads), 0, s, sa)
    switch (dtype) {
        case F32: GX_STATS(F32); break;
        case F16: GX_STATS(F16); break;
        default: GX_STATS(BF16); break;
    }
#undef GX_STATS
    prof_end(ph, s);
    int rc = launch_check("k_factored_stats");
    if (rc) return rc;

    FactFinArgs fa;
    fa.row_part = row_part; fa.col_part = col_part; fa.v_row = v_row; fa.v_col = v_col;
    fa.R = R; fa.C = C; fa.nb = nb; fa.ct = tiles.ct; fa.rt = tiles.rt;
    fa.beta2 = (float)beta2; fa.alpha2 = (float)(1.0 - beta2);
    fa.magbits = magbits; fa.mag = m_magnitude; fa.mag_old = mag_old; fa.minv = minv; fa.vsum = vsum;
    fa.shards = shards;
    fa.nr = (R + kFinRowsPerWg - 1) / kFinRowsPerWg;
    fa.nc = (C + 63) / 64;
    const int64_t fgrid = fa.nr + fa.nc + grid_for(nb, kThreads * 4, 1024);
    ph = prof_begin(GEFENX_K_FINALIZE, 8.0 * (double)(R + C + nb), 0.0, s);
    hipLaunchKernelGGL(k_factored_finalize, dim3((unsigned)fgrid), dim3(kThreads), 0, s, fa);
    prof_end(ph, s);
    rc = launch_check("k_factored_finalize");
    if (rc) return rc;

    ApplyArgs aa{};
    aa.p = p; aa.grad = grad; aa.idx = m_codebook; aa.mag_old = mag_old; aa.mag_new = m_magnitude;
    aa.minv = minv; aa.v_row = v_row; aa.v_col = v_col; aa.vsum = vsum; aa.nr = fa.nr; aa.R = R;
    aa.step = nullptr; aa.qt = qt;
    aa.N = N; aa.C = C; aa.P = period; aa.invC = 1.0 / (double)C; aa.invP = 1.0 / (double)period;
    aa.ps0 = ps0; aa.ps1 = ps1; aa.gs0 = gs0; aa.gs1 = gs1;
    const bool fast = contig_g && contig_p && (C % kChunk == 0) && (period % kChunk == 0) &&
                      aligned(grad, 16) && aligned(p, 16) && aligned(m_codebook, 8) && aligned(v_col, 16);
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
    launch_apply<0>(dtype, stochastic_round != 0, fast, aa, s);
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
    float* minv = reinterpret_cast<float*>(ws + L.off_minv);
    const QTable* qt = static_cast<const QTable*>(qtable);
    const MomentumCoef mc = make_coef(beta1);
    const double es = (double)elem_size(dtype);

    BlockStatsArgs sa;
    sa.grad = grad; sa.idx = m_codebook; sa.mag_old = m_magnitude; sa.qt = qt;
    sa.N = N; sa.P = period; sa.invP = 1.0 / (double)period;
    sa.fast = aligned(grad, 16) && aligned(m_codebook, 8);
    sa.blk_sq = blk_sq; sa.magbits = magbits; sa.mc = mc;
    sa.nb = nb; sa.shards = mag_shards(nb);
    const int64_t nchunks = (N + kChunk - 1) / kChunk;
    const int sgrid = grid_for(nchunks, kThreads * 4, kApplyGridCap);
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
    fa.magbits = magbits; fa.mag = m_magnitude; fa.mag_old = mag_old; fa.step = step; fa.minv = minv;
    fa.shards = mag_shards(nb);
    ph = prof_begin(GEFENX_K_FINALIZE, 16.0 * (double)nb, 0.0, s);
    hipLaunchKernelGGL(k_block_finalize, dim3(grid_for(nb, kThreads, 4096)), dim3(kThreads), 0, s, fa);
    prof_end(ph, s);
    rc = launch_check("k_block_finalize");
    if (rc) return rc;

    ApplyArgs aa{};
    aa.p = p; aa.grad = grad; aa.idx = m_codebook; aa.mag_old = mag_old; aa.mag_new = m_magnitude;
    aa.minv = minv; aa.step = step; aa.qt = qt;
    aa.N = N; aa.C = N; aa.P = period; aa.invC = 1.0 / (double)N; aa.invP = 1.0 / (double)period;
    aa.ps0 = N; aa.ps1 = 1; aa.gs0 = N; aa.gs1 = 1;
    const bool fast = (period % kChunk == 0) && aligned(grad, 16) && aligned(p, 16) && aligned(m_codebook, 8);
    aa.write_p = (step_scalars != nullptr) || !(lr == 0.0 && (float)wdf == 1.0f);
    aa.eps = (float)eps;
    aa.sc = fa.sc;
    aa.step_scalars = step_scalars;
    aa.mc = mc;
    aa.seed = (uint64_t)rng_seed;
    aa.seed_dev = seed_dev;
    ph = prof_begin(GEFENX_K_APPLY, (double)N * (3.0 * es + 2.0) + 16.0 * (double)nb, 0.0, s);
    launch_apply<1>(dtype, stochastic_round != 0, fast, aa, s);
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
