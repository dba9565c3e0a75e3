// gefenx_update.hip -- fused Gefen update kernels for MI355X (gfx950, wave64).
//
// Per parameter the step has three phases:
//   stats    one pass over grad + stored indices: per-block max |u| (u = the
//            updated momentum) and the second-moment sums (per-tile row/column
//            partial sums of g^2 for the factored path, per-block sums for the
//            block path);
//   finalize tiny: EMA of the second moment, new magnitudes and their
//            reciprocals, per-block stepsizes (block path), partial sums of
//            v_row; re-zeroes the workspace accumulators;
//   apply    one pass: recompute u, normalise by the new magnitude,
//            requantise through the exact threshold table, write the indices
//            and the parameter (decoupled weight decay folded in).
// Every phase is a device function of (TensorWork, workgroup index): the
// single-parameter entry points launch it for one descriptor passed by value,
// the multi-tensor launcher (gefenx_multi_tensor_step) launches it for a
// cohort of parameters whose workgroups are laid end to end.
// The math follows the reference's decomposed step (gefen.py:2959-3018,
// 3329-3486, 3776-3818); gefenx_device.h holds the bit-exact momentum,
// division and quantisation primitives.
#include "gefenx_device.h"
#include "gefenx_internal.h"
#include "gefenx_profile.h"
#include "gefenx.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <tuple>
#include <vector>

namespace gx {

constexpr int kThreads = 256;
constexpr int kChunk = 8;
constexpr int64_t kWaves = kThreads / 64;
constexpr int64_t kApplyChunksPerThread = 8;   // apply: 4 iterations of 2 chunks
constexpr int64_t kFinBlocksPerWg = 1024;
constexpr int64_t kDefaultCohortElems = 0;  // one cohort per step (see cohort_limit)

struct StepScalars {
    float lr, inv_bc2, inv_bc1, wdf;
};

// Everything one phase needs about one parameter.  Built on the host
// (build_work) from the C-ABI arguments; lives in kernel arguments (single
// parameter) or in device memory (multi-tensor).
struct TensorWork {
    void* p;
    const void* grad;
    uint8_t* idx;
    float* mag;          // m_magnitude
    float* v0;           // factored: v_row; block: vmean
    float* v1;           // factored: v_col
    double* row_part;    // factored workspace
    double* col_part;
    double* vsum;
    double* blk_sq;      // block workspace
    float* step;
    uint32_t* magbits;
    float* mag_old;
    float* minv;
    float* vcs;          // factored: sqrt(v_col), written by finalize
    uint32_t* fin;       // factored: {finalize counter, bits of mean(v_row)}
    struct DetRec* det_rec;  // block: per-workgroup first / last block partials
    const QTable* qt;
    const float* step_scalars;
    const int64_t* seed_dev;
    int64_t R, C, N, P, nb;
    double invC, invP;
    int64_t ps0, ps1, gs0, gs1;
    int64_t ct, rt, tile_rows, shards;
    int64_t stats_wgs, nr, nc, nbw, fin_wgs, apply_wgs;
    int64_t det_elems;   // block stats: elements per workgroup
    int64_t dR, dC, dB, dP;  // apply: chunk advance for a stride of apply_wgs*256*8 elements
    int64_t fR, fC, fB, fP;  // fast apply: advance for a stride of 256*8 elements
    uint64_t seed;
    int32_t dtype, mode;
    int32_t fast_stats, fast_apply;  // kernel variant: 0 general, 1 contiguous, 2 transposed view
    int32_t write_p, sr, bf16_mean, det_epl;  // det_epl: block stats elements per item (8 or 1)
    int32_t det_vec;     // block stats items: vector loads (grad 16-byte, indices 8-byte aligned)
    int32_t row_apply;   // factored contiguous apply over row segments (apply_rows)
    int32_t partial;     // block path with the caller's per-block stepsize (no vmean)
    int32_t fin_wide;    // block finalize: one workgroup per block (blocks span many stats records)
    int32_t csplit;      // factored finalize: threads per column (1, 2, 4 or 8), each over a run of row tiles
    float eps, beta2, alpha2;
    float bc2_div;       // reference-order divisor (factored bc2, block sqrt(bc2)) or 0
    StepScalars sc;
    MomentumCoef mc;
};

__device__ __forceinline__ StepScalars read_scalars(const TensorWork& w) {
    StepScalars s = w.sc;
    if (w.step_scalars != nullptr) {
        s.lr = w.step_scalars[0];
        s.inv_bc2 = w.step_scalars[1];
        s.inv_bc1 = w.step_scalars[2];
        s.wdf = w.step_scalars[3];
    }
    return s;
}

// The factored stepsize of one element in the rounding order of the
// reference's decomposed step (gefen.py:2996-3006): vh = (v_row*v_col)/mean,
// h = sqrt(vh/bc2) + eps, (1/h) * (1/bc1), one fp32 rounding per operation.
// The divisions by the tensor-wide mean and bc2 take div_by_const; sqrt and
// 1/h are the correctly rounded operations.  Used for fp32 parameters when
// the host gave bc2 (w.bc2_div); otherwise the kernels take the cheaper
// sqrt(v_row*s) * sqrt(v_col) form, within 1e-6 of this.
struct RefStep {
    float mean, rmean, bc2, rbc2, eps, inv_bc1;
    bool on;
};

__device__ __forceinline__ RefStep make_ref_step(const TensorWork& w, const StepScalars& sc, float mean) {
    RefStep r;
    r.on = w.bc2_div > 0.0f;
    r.mean = mean;
    r.rmean = block_recip(mean);
    r.bc2 = w.bc2_div;
    r.rbc2 = block_recip(w.bc2_div);
    r.eps = w.eps;
    r.inv_bc1 = sc.inv_bc1;
    return r;
}

__device__ __forceinline__ float ref_step(const RefStep& r, float v_row, float v_col) {
    const float vh = div_by_const(v_row * v_col, r.mean, r.rmean);
    const float h = sqrtf(div_by_const(vh, r.bc2, r.rbc2)) + r.eps;
    return (1.0f / h) * r.inv_bc1;
}

// Wave-uniform running block max of |u| as ordered uint bits (NaN > inf >
// finite, so the integer max propagates NaN like torch's amax).
struct WaveMax {
    int64_t blk;
    uint32_t bits;
};

__device__ __forceinline__ void wavemax_flush(uint32_t* __restrict__ mb, WaveMax& wm) {
    if (wm.blk >= 0) {
        const uint32_t m = wave_max_u(wm.bits);
        if ((threadIdx.x & 63) == 0 && m != 0u) gatomic_max(mb + wm.blk, m);
    }
    wm.bits = 0u;
}

// Flush a wave-uniform running block max: one atomic per wave.
__device__ __forceinline__ void wavemax_flush63(uint32_t* __restrict__ mb, WaveMax& wm) {
    if (wm.blk >= 0) {
        const uint32_t m = wave_max_u63(wm.bits);
        if ((threadIdx.x & 63) == 63 && m != 0u) gatomic_max(mb + wm.blk, m);
    }
    wm.bits = 0u;
}

// ====================================================================
// Factored stats: workgroup = 4 waves over a tile of tile_rows rows x 1024
// columns; lane l owns the chunks at columns c0 + 8l and c0 + 512 + 8l, wave
// w takes rows r0 + w, r0 + w + 4, ... two at a time.  Per row: squares and
// the momentum max over the lane's 16 elements, then a float64 DPP reduction
// of the row sum (one value per row per column tile).  Column sums: fp32 in
// registers over 8 rows, then float64; the 4 waves combine in LDS at the end.
// Both go out as float64 partials (no float atomics, deterministic).
// FAST: contiguous, 16-byte aligned grad, C % 8 == 0, P % 8 == 0.
// ====================================================================
struct FactStatsLds {
    float cbr[kCodebookMax];
    double col[kWaves][kChunk][2][64];  // float64 column sums: [wave][k][h][lane]
    int64_t wblk[kWaves];
    uint32_t wbits[kWaves];
};

template <int DT, bool FAST, int LF>
__device__ __forceinline__ void stats_factored(const TensorWork& wr, int64_t wg, FactStatsLds& lds) {
    using T = typename Elem<DT>::T;
    // fp32 grads: every square into a float64 accumulator, as the reference
    // sums them; 16-bit grads: exact squares in 8-row / 16-column fp32 partials
    using Acc = std::conditional_t<DT == F32, double, float>;
    constexpr int H = 2;  // chunks per lane per row
    float* s_cbr = lds.cbr;
    auto& s_col = lds.col;
    int64_t* s_wblk = lds.wblk;
    uint32_t* s_wbits = lds.wbits;
    const QTable* qt = wr.qt;
    if (threadIdx.x < kCodebookMax) s_cbr[threadIdx.x] = *gbl(qt->cbr + threadIdx.x);

    const T* g = static_cast<const T*>(wr.grad);
    const uint8_t* idxp = wr.idx;
    const float* mag_old = wr.mag;
    double* row_part = wr.row_part;
    double* col_part = wr.col_part;
    const int64_t R = wr.R, C = wr.C, P = wr.P, gs0 = wr.gs0, gs1 = wr.gs1;
    const int64_t ct = wr.ct, tile_rows = wr.tile_rows, nb = wr.nb;
    const double invP = wr.invP;
    const MomentumCoef mc = wr.mc;
    uint32_t* mb = wr.magbits + (wg % wr.shards) * nb;
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: row state in SGPRs
    const int64_t ctile = wg % ct;
    const int64_t rtile = wg / ct;
    const int64_t tc0 = ctile * kFactTileCols;
    const int64_t span = std::min<int64_t>(kFactTileCols, C - tc0);
    int64_t cc[H], ccl[H];
    int nv[H];
#pragma unroll
    for (int h = 0; h < H; ++h) {
        cc[h] = tc0 + h * (kFactTileCols / 2) + (int64_t)lane * kChunk;
        nv[h] = (int)std::max<int64_t>(0, std::min<int64_t>(kChunk, C - cc[h]));
        // FAST loads every chunk unconditionally: a chunk past C (nv == 0,
        // skipped by the math) reads the row's last chunk instead
        ccl[h] = nv[h] > 0 ? cc[h] : C - kChunk;
    }
    const int64_t r_begin = rtile * tile_rows;
    const int64_t r_end = std::min<int64_t>(r_begin + tile_rows, R);

    // block position of the first element of the wave's row segment, and its
    // advance for 4 rows: (blk, pin) += divmod(4C, P)
    int64_t blk = 0, pin = 0;
    {
        const int64_t e = (r_begin + wave) * C + tc0;
        blk = div_floor(e, P, invP);
        pin = e - blk * P;
    }
    const int64_t d4 = 4 * C;
    const int64_t dB4 = div_floor(d4, P, invP);
    const int64_t dP4 = d4 - dB4 * P;

    // column sums: in registers over 8 rows, then added into the wave's
    // float64 slots in LDS (each lane owns its 16 columns' slots)
    Acc colf[H][kChunk];
#pragma unroll
    for (int h = 0; h < H; ++h)
#pragma unroll
        for (int k = 0; k < kChunk; ++k) { colf[h][k] = 0; s_col[wave][k][h][lane] = 0.0; }
    auto flush_cols = [&]() {
#pragma unroll
        for (int h = 0; h < H; ++h)
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                s_col[wave][k][h][lane] += (double)colf[h][k];
                colf[h][k] = 0;
            }
    };
    int nrows_f = 0;
    WaveMax wm{-1, 0u};
    float mag_cur = 0.0f;
    bool mag_ok = false;
    // chunk h of every lane inside C (hall) / of some lane (hany): wave-uniform
    bool hall[H], hany[H];
#pragma unroll
    for (int h = 0; h < H; ++h) {
        hall[h] = tc0 + (h + 1) * (kFactTileCols / 2) <= C;
        hany[h] = tc0 + h * (kFactTileCols / 2) < C;
    }

    // One batch = the wave's next two rows (r0, r0 + 4): raw grads and
    // indices, plus (FAST) the old magnitude of each row segment's first
    // block.  FAST keeps the next batch in flight while the current one is
    // reduced, so a wave never waits for a load it issued in the same step.
    struct Batch {
        Raw8<DT> graw[2][H];
        RawIdx8 iraw[2][H];
        float gsc[2][H][kChunk];
        uint32_t isc[2][H][kChunk];
        float mo[2];
    };
    int64_t pblk = blk, ppin = pin;  // block position of the next batch to load
    auto load_batch = [&](int64_t rr0, Batch& b) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t r = rr0 + (int64_t)u * kWaves;
            if constexpr (FAST) {
                // rows past the tile re-read the tile's last row; the math
                // stops before them (C % 8 == 0, so nv is 0 or 8)
                const int64_t rl = r < r_end ? r : r_end - 1;
#pragma unroll
                for (int h = 0; h < H; ++h) {
                    const int64_t el = rl * C + ccl[h];
                    load_raw8<DT>(g + el, b.graw[u][h]);
                    b.iraw[u][h] = load_raw_idx8(idxp + el);
                }
                b.mo[u] = sload(mag_old + (pblk < nb ? pblk : nb - 1));  // uniform: scalar load
                ppin += dP4;
                pblk += dB4;
                if (ppin >= P) { ppin -= P; ++pblk; }
            } else {
#pragma unroll
                for (int h = 0; h < H; ++h) {
                    const int64_t e0 = r * C + cc[h];
#pragma unroll
                    for (int k = 0; k < kChunk; ++k) {
                        const bool ok = r < r_end && k < nv[h];
                        b.gsc[u][h][k] = ok ? to_f32<DT>(*gbl(g + r * gs0 + (cc[h] + k) * gs1)) : 0.0f;
                        b.isc[u][h][k] = ok ? (uint32_t)*gbl(idxp + e0 + k) : 0u;
                    }
                }
            }
        }
    };
    auto reduce_batch = [&](int64_t rr0, const Batch& b) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t r = rr0 + (int64_t)u * kWaves;
            if (r >= r_end) break;
            Acc rs[H];
            const bool uniform = (pin + span - 1) < P;
            if (uniform) {
                if (blk != wm.blk) {
                    wavemax_flush63(mb, wm);
                    wm.blk = blk;
                    if constexpr (FAST) {
                        mag_cur = b.mo[u];
                        mag_ok = (__float_as_uint(mag_cur) & 0x7fffffffu) < 0x7e967699u;  // |m| < 1e38, not NaN
                    } else {
                        mag_cur = *gbl(mag_old + blk);
                    }
                }
                if constexpr (FAST) {
                    // |u| max as floats (v_max3 with |.| modifiers).  Exact when
                    // every u is finite, which holds when the old magnitude is
                    // below 1e38 and every g^2 is finite (then |g - cm| cannot
                    // overflow); otherwise the row is redone with the ordered
                    // integer max, which ranks NaN above inf like torch's amax.
                    float mf = 0.0f;
                    auto chunk = [&](int h, auto masked) {
                        rs[h] = 0;
#pragma unroll
                        for (int k = 0; k < kChunk; ++k) {
                            float gv = raw_elem<DT>(b.graw[u][h], k);
                            if constexpr (decltype(masked)::value) gv = nv[h] > 0 ? gv : 0.0f;
                            const float uu = momentum_value<LF>(s_cbr[raw_idx(b.iraw[u][h], k)], mag_cur, gv, mc);
                            if constexpr (decltype(masked)::value) mf = nv[h] > 0 ? __builtin_fmaxf(mf, fabsf(uu)) : mf;
                            else mf = __builtin_fmaxf(mf, fabsf(uu));
                            sq_add(rs[h], gv);
                            sq_add(colf[h][k], gv);
                        }
                    };
#pragma unroll
                    for (int h = 0; h < H; ++h) {
                        if (hall[h]) chunk(h, std::false_type{});
                        else if (hany[h]) chunk(h, std::true_type{});
                        else rs[h] = 0;
                    }
                    // integer test: NaN and inf both fail it, whatever the
                    // compiler assumes about float compares (a square that
                    // overflows fp32 is inf in either accumulator)
                    const bool fin = (__float_as_uint((float)(rs[0] + rs[1])) & 0x7fffffffu) < 0x7f800000u;
                    if (__builtin_expect(mag_ok && __all(fin), 1)) {
                        const uint32_t mb_ = __float_as_uint(mf);
                        wm.bits = mb_ > wm.bits ? mb_ : wm.bits;
                    } else {
                        uint32_t m = wm.bits;
#pragma unroll
                        for (int h = 0; h < H; ++h) {
                            if (nv[h] == 0) continue;
#pragma unroll
                            for (int k = 0; k < kChunk; ++k) {
                                const float uu = momentum_value<LF>(s_cbr[raw_idx(b.iraw[u][h], k)], mag_cur,
                                                                    raw_elem<DT>(b.graw[u][h], k), mc);
                                const uint32_t ub = __float_as_uint(uu) & 0x7fffffffu;
                                m = ub > m ? ub : m;
                            }
                        }
                        wm.bits = m;
                    }
                } else {
                    uint32_t m = wm.bits;
#pragma unroll
                    for (int h = 0; h < H; ++h) {
                        rs[h] = 0;
                        if (nv[h] == 0) continue;  // columns past C (last tile)
#pragma unroll
                        for (int k = 0; k < kChunk; ++k) {
                            if (k >= nv[h]) continue;
                            const float gv = b.gsc[u][h][k];
                            const float uu = momentum_value<LF>(s_cbr[b.isc[u][h][k]], mag_cur, gv, mc);
                            const uint32_t ub = __float_as_uint(uu) & 0x7fffffffu;
                            m = ub > m ? ub : m;
                            sq_add(rs[h], gv);
                            sq_add(colf[h][k], gv);
                        }
                    }
                    wm.bits = m;
                }
            } else {
                // blocks end inside this row segment: per-lane runs, one atomic per run
                wavemax_flush63(mb, wm);
                wm.blk = -1;
#pragma unroll
                for (int h = 0; h < H; ++h) {
                    rs[h] = 0;
                    if (nv[h] == 0) continue;
                    const int64_t off = pin + (cc[h] - tc0);
                    const int64_t db = div_floor(off, P, invP);
                    int64_t bb = blk + db;
                    int64_t pp = off - db * P;
                    float mo = *gbl(mag_old + bb);
                    uint32_t m = 0u;
#pragma unroll
                    for (int k = 0; k < kChunk; ++k) {
                        if (k < nv[h]) {
                            float gv;
                            uint32_t ix;
                            if constexpr (FAST) { gv = raw_elem<DT>(b.graw[u][h], k); ix = raw_idx(b.iraw[u][h], k); }
                            else { gv = b.gsc[u][h][k]; ix = b.isc[u][h][k]; }
                            const float uu = momentum_value<LF>(s_cbr[ix], mo, gv, mc);
                            const uint32_t ub = __float_as_uint(uu) & 0x7fffffffu;
                            m = ub > m ? ub : m;
                            sq_add(rs[h], gv);
                            sq_add(colf[h][k], gv);
                            if (++pp == P) {
                                if (m) gatomic_max(mb + bb, m);
                                m = 0u;
                                pp = 0;
                                ++bb;
                                if (k + 1 < nv[h]) mo = *gbl(mag_old + bb);
                            }
                        }
                    }
                    if (m) gatomic_max(mb + bb, m);
                }
            }
            double rsum = 0.0;
#pragma unroll
            for (int h = 0; h < H; ++h) rsum += (double)rs[h];
            rsum = wave_sum_d63(rsum);
            if (lane == 63) *gbl(row_part + ctile * R + r) = rsum;
            if (++nrows_f == 8) {
                flush_cols();
                nrows_f = 0;
            }
            pin += dP4;
            blk += dB4;
            if (pin >= P) { pin -= P; ++blk; }
        }
    };

    constexpr int64_t kStep = 2 * kWaves;
    int64_t r0 = r_begin + wave;
    if (r0 < r_end) {
        Batch ba, bb;
        load_batch(r0, ba);
        if constexpr (FAST) {
            // The prefetch is unconditional (past the tile it re-reads the
            // tile's last row, which is still in cache), so every step has
            // the same loads in flight and the compiler can wait for the
            // current batch alone instead of draining the queue.
            for (;;) {
                load_batch(r0 + kStep, bb);
                reduce_batch(r0, ba);
                r0 += kStep;
                if (r0 >= r_end) break;
                load_batch(r0 + kStep, ba);
                reduce_batch(r0, bb);
                r0 += kStep;
                if (r0 >= r_end) break;
            }
        } else {
            for (;;) {
                reduce_batch(r0, ba);
                r0 += kStep;
                if (r0 >= r_end) break;
                load_batch(r0, ba);
            }
        }
    }
    flush_cols();

    // final block-max flush: one atomic per workgroup when the waves agree
    const uint32_t wbits = wm.blk >= 0 ? wave_max_u63(wm.bits) : 0u;
    if (lane == 63) {
        s_wblk[wave] = wm.blk;
        s_wbits[wave] = wbits;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        bool same = true;
        uint32_t m = 0u;
        for (int ww = 0; ww < kWaves; ++ww) {
            same = same && (s_wblk[ww] == s_wblk[0]);
            m = s_wbits[ww] > m ? s_wbits[ww] : m;
        }
        if (same) {
            if (s_wblk[0] >= 0 && m) gatomic_max(mb + s_wblk[0], m);
        } else {
            for (int ww = 0; ww < kWaves; ++ww)
                if (s_wblk[ww] >= 0 && s_wbits[ww]) gatomic_max(mb + s_wblk[ww], s_wbits[ww]);
        }
    }
    // column partials of the tile: waves summed in order 0..3; thread t
    // stores columns t, t + 256, ... (coalesced)
#pragma unroll
    for (int j = 0; j < kFactTileCols / kThreads; ++j) {
        const int c = threadIdx.x + j * kThreads;
        const int h = c / (kFactTileCols / 2), cl = c % (kFactTileCols / 2);
        const int ln = cl / kChunk, k = cl % kChunk;
        double sum = s_col[0][k][h][ln];
#pragma unroll
        for (int ww = 1; ww < kWaves; ++ww) sum += s_col[ww][k][h][ln];
        if (c < span) *gbl(col_part + rtile * C + tc0 + c) = sum;
    }
}

// ====================================================================
// Transposed views: g (and p) with strides (1, ld), ld >= R -- the layout of
// x.t() for a contiguous [C, R] tensor x.  Logical row-major order still
// fixes the blocks, the indices and v_row / v_col, but g and p run along
// logical columns.  The view kernels walk 64 x 64 logical tiles, one per
// wave at a time; lane l = 8b + a owns the 8 x 8 sub-block at tile rows
// 8a .. 8a+7 and tile columns 8b .. 8b+7.  It loads g (and p) as 8 vectors
// along storage rows (tile column 8b+k, rows 8a .. 8a+7: the 8 lanes of one
// b read one 128-byte run for 16-bit types) and the indices as 8 logical
// chunks (row 8a+j, columns 8b .. 8b+7: the 8 lanes of one a read one
// 64-byte run).  Element (j, k) of the sub-block is element j of g vector k
// and element k of index chunk j, so no data passes through LDS.  Chunk j
// (8 elements of one logical row) lies in one block since P % 8 == 0.
// Requires R, C, P multiples of 8 and 16-byte aligned storage rows.
// ====================================================================
constexpr int kTv = 64;
constexpr int kTvTilesPerWave = 2;  // apply: consecutive tiles per wave
constexpr int kTvLdsBlocks = 512;   // stats: LDS block accumulators per workgroup
constexpr int kTvFew = 4;           // blocks a tile may touch on the scalar-load path

// A value every lane of the wave holds, moved to scalar registers.
__device__ __forceinline__ int64_t uniform64(int64_t v) {
    const uint64_t u = (uint64_t)v;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(u >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Blocks of a lane's 8 chunks (rows r .. r+7 at column c) relative to b_lo;
// (dB, dP) = divmod(C, P) advances one row.
__device__ __forceinline__ void tv_chunk_blocks(int64_t r, int64_t c, int64_t C, int64_t P, double invP,
                                                int64_t dB, int64_t dP, int64_t b_lo, int q[kChunk]) {
    const int64_t e = r * C + c;
    int64_t b = div_floor(e, P, invP);
    int64_t pin = e - b * P;
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
        q[j] = (int)(b - b_lo);
        pin += dP;
        b += dB;
        if (pin >= P) { pin -= P; ++b; }
    }
}

__device__ __forceinline__ float tv_pick(int q, const float v[kTvFew]) {
    return q == 0 ? v[0] : (q == 1 ? v[1] : (q == 2 ? v[2] : v[3]));
}

// The first kTvFew values of a per-block array from block b_lo on (indices
// clamped to the array), as scalar loads.
__device__ __forceinline__ void tv_sload_few(const float* arr, int64_t b_lo, int64_t nb, float v[kTvFew]) {
#pragma unroll
    for (int i = 0; i < kTvFew; ++i) v[i] = sload(arr + (b_lo + i < nb ? b_lo + i : nb - 1));
}

// Reduce-scatter of 8 float64 values over the 8 lanes of a group (lane bits
// 0-2): lane i ends with the group's sum of v[i].  Partners at the three
// steps: i ^ 7 (row_half_mirror), i ^ 2, i ^ 1 (quad_perm); a fixed order of
// float64 adds.
__device__ __forceinline__ double tv_scatter_lo(const double v[kChunk], int i) {
    const bool hi = (i & 4) != 0, mid = (i & 2) != 0, lo = (i & 1) != 0;
    double w[4], x[2];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const double send = hi ? v[t] : v[t + 4];
        w[t] = (hi ? v[t + 4] : v[t]) + dpp64<0x141, 0xf>(send);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const double send = mid ? w[t] : w[t + 2];
        x[t] = (mid ? w[t + 2] : w[t]) + dpp64<0x4E, 0xf>(send);
    }
    const double send = lo ? x[0] : x[1];
    return (lo ? x[1] : x[0]) + dpp64<0xB1, 0xf>(send);
}

// The same over lane bits 3-5 (partners lane ^ 32, lane ^ 16, lane ^ 8):
// lane 8i + a ends with the sum of v[i] over its 8 lanes a + 8i'.
__device__ __forceinline__ double tv_scatter_hi(const double v[kChunk], int i) {
    const bool hi = (i & 4) != 0, mid = (i & 2) != 0, lo = (i & 1) != 0;
    double w[4], x[2];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const double send = hi ? v[t] : v[t + 4];
        w[t] = (hi ? v[t + 4] : v[t]) + __shfl_xor(send, 32, 64);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const double send = mid ? w[t] : w[t + 2];
        x[t] = (mid ? w[t + 2] : w[t]) + __shfl_xor(send, 16, 64);
    }
    const double send = lo ? x[0] : x[1];
    return (lo ? x[1] : x[0]) + dpp64<0x128, 0xf>(send);  // row_ror:8 = lane ^ 8 within 16
}

template <int MODE>
struct TvStatsLds {
    float cbr[kCodebookMax];
    double colp[MODE == 0 ? kWaves : 1][MODE == 0 ? kFactTileCols : 1];
    uint32_t bmax[kTvLdsBlocks];
    double bsum[MODE == 1 ? kTvLdsBlocks : 1];
};

// Stats of a transposed view.  Workgroup (ctile, rtile) covers the same
// kFactTileCols columns as the contiguous factored kernel (so row_part keeps
// its layout) and tile_rows (<= 256) rows; wave w takes the 64-row band w and
// walks the workgroup's columns in 64 x 64 tiles, so the 4 waves read 512-byte
// runs of the same storage rows at about the same time (measured 6% faster
// than 4 waves on 4 column ranges) and a wave reads the two halves of each
// 128-byte index line in consecutive tiles.  MODE 0 (factored): squares in
// fp32 over a chunk's 8 columns and over a vector's 8 rows (float64 for fp32
// grads), then float64: a row's sum over the columns collects in its lanes
// and leaves as the row partial (reduce-scatter over the 8 column groups),
// a column's over the band in one lane (reduce-scatter over the 8 row
// groups of each tile), and the 4 bands' column sums meet in LDS in band
// order.  Block max |u| (and, MODE 1, the block's sum of squares, each square
// rounded to bf16 for bf16 grads, in float64): when a tile touches at most
// kTvFew blocks (the common case) its old magnitudes are scalar loads, the
// lanes keep one value per block and the wave reduces each; otherwise per
// chunk.  Either way the values go to the workgroup's LDS accumulators (<= 512
// blocks) or the shards.
template <int DT, int MODE, int LF>
__device__ __forceinline__ void stats_tv(const TensorWork& wr, int64_t wg, TvStatsLds<MODE>& lds) {
    using T = typename Elem<DT>::T;
    using Acc = std::conditional_t<DT == F32, double, float>;
    const QTable* qt = wr.qt;
    if (threadIdx.x < kCodebookMax) lds.cbr[threadIdx.x] = *gbl(qt->cbr + threadIdx.x);
    if constexpr (MODE == 0) {
        for (int k = threadIdx.x; k < kWaves * kFactTileCols; k += kThreads) (&lds.colp[0][0])[k] = 0.0;
    }
    const float* s_cbr = lds.cbr;

    const T* g = static_cast<const T*>(wr.grad);
    const uint8_t* idxp = wr.idx;
    const float* mag_old = wr.mag;
    double* row_part = wr.row_part;
    double* col_part = wr.col_part;
    const int64_t R = wr.R, C = wr.C, P = wr.P, ld = wr.gs1, nb = wr.nb;
    const double invP = wr.invP;
    const MomentumCoef mc = wr.mc;
    uint32_t* mb = wr.magbits + (wg % wr.shards) * nb;
    double* bsq = MODE == 1 ? wr.blk_sq + (wg % wr.shards) * nb : nullptr;
    const int64_t ctile = wg % wr.ct, rtile = wg / wr.ct;
    const int64_t c_begin = ctile * kFactTileCols;
    const int64_t c_end = std::min<int64_t>(c_begin + kFactTileCols, C);
    const int64_t r_begin = rtile * wr.tile_rows;
    const int64_t r_end = std::min<int64_t>(r_begin + wr.tile_rows, R);
    // blocks of the workgroup's region: few of them (large periods) reduce
    // in LDS and leave with one atomic per block and workgroup
    const int64_t b_wlo = div_floor(r_begin * C + c_begin, P, invP);
    const int64_t b_span = div_floor((r_end - 1) * C + (c_end - 1), P, invP) - b_wlo + 1;
    const bool lds_blk = b_span <= kTvLdsBlocks;
    if (lds_blk) {
        for (int k = threadIdx.x; k < b_span; k += kThreads) {
            lds.bmax[k] = 0u;
            if constexpr (MODE == 1) lds.bsum[k] = 0.0;
        }
    }
    const int lane = threadIdx.x & 63, la = lane & 7, lb = lane >> 3;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t cw0 = c_begin, cw1 = c_end;
    const int ncs = (int)((c_end - c_begin + kTv - 1) / kTv);
    const int64_t rw0 = r_begin + (int64_t)wave * kTv;
    const int ntile = rw0 < r_end ? ncs : 0;
    const int64_t dB = div_floor(C, P, invP);
    const int64_t dP = C - dB * P;
    __syncthreads();

    auto put_max = [&](int64_t b, uint32_t m) {
        if (m == 0u) return;
        if (lds_blk) atomicMax(&lds.bmax[b - b_wlo], m);
        else gatomic_max(mb + b, m);
    };
    auto put_sum = [&](int64_t b, double v) {
        if (v == 0.0) return;
        if (lds_blk) atomicAdd(&lds.bsum[b - b_wlo], v);
        else gatomic_add(bsq + b, v);
    };

    struct Tile {
        Raw8<DT> gv[kChunk];  // storage-row vectors: tile column 8b+k, rows 8a .. 8a+7
        RawIdx8 iv[kChunk];   // index chunks: row 8a+j, columns 8b .. 8b+7
    };
    // lanes outside the region read its last sub-block instead (the math
    // skips them)
    auto load_tile = [&](int s, Tile& t) {
        const int64_t r = rw0 + 8 * la;
        const int64_t c = cw0 + (int64_t)s * kTv + 8 * lb;
        const int64_t rl = r < r_end ? r : r_end - kChunk, cl = c < cw1 ? c : cw1 - kChunk;
#pragma unroll
        for (int k = 0; k < kChunk; ++k) load_raw8<DT>(g + (cl + k) * ld + rl, t.gv[k]);
#pragma unroll
        for (int j = 0; j < kChunk; ++j) t.iv[j] = load_raw_idx8_cached(idxp + (rl + j) * C + cl);
    };

    double racc[kChunk];  // MODE 0: row sums of the lane's 8 rows over the columns so far
#pragma unroll
    for (int j = 0; j < kChunk; ++j) racc[j] = 0.0;

    auto reduce_tile = [&](int s, const Tile& t) {
        const int cs = s;
        const int64_t r0 = rw0, c0 = cw0 + (int64_t)cs * kTv;
        const int64_t r = r0 + 8 * la, c = c0 + 8 * lb;
        const bool ok = r < r_end && c < cw1;
        const int64_t r_last = std::min<int64_t>(r0 + kTv, r_end) - 1;
        const int64_t c_last = std::min<int64_t>(c0 + kTv, cw1) - 1;
        const int64_t b_lo = uniform64(div_floor(r0 * C + c0, P, invP));
        const int64_t b_hi = uniform64(div_floor(r_last * C + c_last, P, invP));
        Acc colf[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; ++k) colf[k] = 0;
        // one chunk: max |u| bits, fp32 (MODE 0) or float64 (MODE 1) square sums
        auto chunk = [&](int j, float mo, uint32_t& m, Acc& rs, double& bs) {
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                const float gv = raw_elem<DT>(t.gv[k], j);
                const float uu = momentum_value<LF>(s_cbr[raw_idx(t.iv[j], k)], mo, gv, mc);
                const uint32_t ub = __float_as_uint(uu) & 0x7fffffffu;
                m = ub > m ? ub : m;
                if constexpr (MODE == 0) {
                    sq_add(rs, gv);
                    sq_add(colf[k], gv);
                } else {
                    float sq = gv * gv;
                    if constexpr (DT == BF16) sq = round_dt<BF16>(sq);
                    bs += (double)sq;
                }
            }
        };
        if (b_hi - b_lo < kTvFew) {
            float mo[kTvFew];
            tv_sload_few(mag_old, b_lo, nb, mo);
            uint32_t mx[kTvFew] = {0u, 0u, 0u, 0u};
            double bx[kTvFew] = {0.0, 0.0, 0.0, 0.0};
            if (ok) {
                int q[kChunk];
                tv_chunk_blocks(r, c, C, P, invP, dB, dP, b_lo, q);
#pragma unroll
                for (int j = 0; j < kChunk; ++j) {
                    uint32_t m = 0u;
                    Acc rs = 0;
                    double bs = 0.0;
                    chunk(j, tv_pick(q[j], mo), m, rs, bs);
                    if constexpr (MODE == 0) racc[j] += (double)rs;
#pragma unroll
                    for (int i = 0; i < kTvFew; ++i) {
                        if (q[j] == i) {
                            mx[i] = m > mx[i] ? m : mx[i];
                            if constexpr (MODE == 1) bx[i] += bs;
                        }
                    }
                }
            }
            const int nq = (int)(b_hi - b_lo) + 1;
#pragma unroll
            for (int i = 0; i < kTvFew; ++i) {
                if (i < nq) {
                    const uint32_t m = wave_max_u63(mx[i]);
                    double v = 0.0;
                    if constexpr (MODE == 1) v = wave_sum_d63(bx[i]);
                    if (lane == 63) {
                        put_max(b_lo + i, m);
                        if constexpr (MODE == 1) put_sum(b_lo + i, v);
                    }
                }
            }
        } else if (ok) {
            // many blocks in the tile (P small against C): per chunk
            const int64_t e = r * C + c;
            int64_t b = div_floor(e, P, invP);
            int64_t pin = e - b * P;
#pragma unroll
            for (int j = 0; j < kChunk; ++j) {
                uint32_t m = 0u;
                Acc rs = 0;
                double bs = 0.0;
                chunk(j, *gbl(mag_old + b), m, rs, bs);
                if constexpr (MODE == 0) racc[j] += (double)rs;
                put_max(b, m);
                if constexpr (MODE == 1) put_sum(b, bs);
                pin += dP;
                b += dB;
                if (pin >= P) { pin -= P; ++b; }
            }
        }
        if constexpr (MODE == 0) {
            // column 8b + a of this tile, over its rows
            double cv[kChunk];
#pragma unroll
            for (int k = 0; k < kChunk; ++k) cv[k] = (double)colf[k];
            const double col = tv_scatter_lo(cv, la);
            lds.colp[wave][cs * kTv + 8 * lb + la] = col;
            if (cs == ncs - 1) {
                const double row = tv_scatter_hi(racc, lb);
                const int64_t rr = r0 + 8 * la + lb;
                if (rr < r_end) *gbl(row_part + ctile * R + rr) = row;
            }
        }
    };

    if (ntile > 0) {
        // one tile in flight per wave: a second register set (the next
        // tile's loads issued before this one's math) measured no faster at
        // two waves per SIMD than one set at three
        Tile t;
        for (int s = 0; s < ntile; ++s) {
            load_tile(s, t);
            reduce_tile(s, t);
        }
    }
    __syncthreads();
    if constexpr (MODE == 0) {
        for (int64_t k = threadIdx.x; k < c_end - c_begin; k += kThreads) {
            double v = lds.colp[0][k];
#pragma unroll
            for (int ww = 1; ww < kWaves; ++ww) v += lds.colp[ww][k];
            *gbl(col_part + rtile * C + c_begin + k) = v;
        }
    }
    if (lds_blk) {
        for (int k = threadIdx.x; k < b_span; k += kThreads) {
            const uint32_t m = lds.bmax[k];
            if (m != 0u) gatomic_max(mb + b_wlo + k, m);
            if constexpr (MODE == 1) {
                const double v = lds.bsum[k];
                if (v != 0.0) gatomic_add(bsq + b_wlo + k, v);
            }
        }
    }
}

template <int DT, int MODE>
__device__ __forceinline__ void stats_tv_wg(const TensorWork& w, int64_t wg) {
    __shared__ TvStatsLds<MODE> lds;
    if (w.mc.small) stats_tv<DT, MODE, kLerpSmall>(w, wg, lds);
    else stats_tv<DT, MODE, kLerpLarge>(w, wg, lds);
}

// ====================================================================
// Block stats (block path): per-block sum of squared grads (rounded through
// bf16 for bf16 grads, gefen.py:180-190) and max |u|, summed in an order that
// does not depend on scheduling, so a run is bit-reproducible.
// Workgroup wg owns elements [wg*E, (wg+1)*E), E = kDetIters * 256 * EPL.  In
// iteration i, lane l of wave v takes the EPL elements of item
// j = i*256 + v*64 + l, all in one block (EPL = 8 needs P % 8 == 0 and
// N % 8 == 0; otherwise EPL = 1).  A wave's 64 items are combined per block
// by a segmented suffix sum (Hillis-Steele steps masked at block starts: a
// fixed schedule of float64 adds).  A block that starts and ends inside those
// 64 items is complete and is stored; the first and last block partials of
// each wave and iteration go to LDS, where wave 0 combines the workgroup's 64
// of them the same way.  The workgroup's own first and last block partials
// go to its record; finalize adds a block's stored sum and the records of
// the workgroups it spans, in workgroup order.  Max |u| takes one atomic max
// per block and wave (a max is exact in any order).
// ====================================================================
constexpr int kDetIters = 8;
static_assert(kThreads == kCodebookMax, "one codebook entry per thread");
// Stats records per block from which the block finalize takes a workgroup per block.
constexpr int64_t kFinWideRecords = 32;
static_assert(2 * kDetIters * kWaves == 64, "the workgroup's run partials fill one wave");

// Lane-order run starts (bit l: lane l begins a new key) and the segmented
// suffix sum / max: each lane ends with the sum (max) of its run from itself
// to the run's last lane, so a run's first lane holds the run's total.
__device__ __forceinline__ uint64_t run_heads(int64_t key) {
    const int lane = threadIdx.x & 63;
    const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)key, 1, 64);
    const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)((uint64_t)key >> 32), 1, 64);
    const int64_t prev = (int64_t)(((uint64_t)hi << 32) | lo);
    return (uint64_t)__ballot(lane == 0 || prev != key);
}

__device__ __forceinline__ double seg_suffix_sum(double v, uint64_t heads) {
    const int lane = threadIdx.x & 63;
    const uint64_t after = lane < 63 ? heads >> (lane + 1) : 0ull;  // run starts past this lane
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const double o = __shfl_down(v, d, 64);
        const bool ok = lane + d < 64 && (after & ((1ull << d) - 1ull)) == 0ull;
        v = ok ? v + o : v;
    }
    return v;
}

__device__ __forceinline__ uint32_t seg_suffix_max(uint32_t m, uint64_t heads) {
    const int lane = threadIdx.x & 63;
    const uint64_t after = lane < 63 ? heads >> (lane + 1) : 0ull;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = (uint32_t)__shfl_down((int)m, d, 64);
        const bool ok = lane + d < 64 && (after & ((1ull << d) - 1ull)) == 0ull;
        m = (ok && o > m) ? o : m;
    }
    return m;
}

// Flush a wave's running block max (wave-uniform key and value): one atomic
// into the workgroup's shard.
__device__ __forceinline__ void flush_det_max(uint32_t* mb, int64_t key, int64_t nb, uint32_t m) {
    if ((threadIdx.x & 63) == 0 && key >= 0 && key < nb && m != 0u) gatomic_max(mb + key, m);
}

// A workgroup whose elements all lie in one block (every block of at least
// E elements, most of them): no per-element block index and no segmented
// scans.  The old magnitude is one scalar load; each lane sums its items in
// iteration order, the waves combine by a fixed DPP pattern, then in wave
// order -- the same order on every run.  FULL: the workgroup's E elements
// all lie inside the tensor, so no load sits behind a branch.
template <int DT, int EPL, bool FULL>
__device__ __forceinline__ void stats_block_one(const TensorWork& w, int64_t wg, int64_t kb, float* s_cbr,
                                                double* s_sum) {
    using T = typename Elem<DT>::T;
    const T* g = static_cast<const T*>(w.grad);
    const int64_t N = w.N;
    const MomentumCoef mc = w.mc;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t base = wg * (int64_t)(kDetIters * kThreads * EPL);
    const float mo = sload(w.mag + kb);
    // the codebook goes into a register first and into LDS after the element
    // loads are issued (loaded in this block, so the LDS write waits for it alone)
    const float cbr_v = *gbl(w.qt->cbr + threadIdx.x % kCodebookMax);
    Raw8<DT> gr[kDetIters];
    RawIdx8 ir[kDetIters];
    float graw[kDetIters];
    uint32_t iraw[kDetIters];
#pragma unroll
    for (int i = 0; i < kDetIters; ++i) {
        const int64_t e0 = base + ((int64_t)i * kThreads + threadIdx.x) * EPL;
        if (FULL || e0 < N) {
            if constexpr (EPL == kChunk) {
                if (w.det_vec) {
                    load_raw8<DT>(g + e0, gr[i]);
                    ir[i] = load_raw_idx8(w.idx + e0);
                } else {  // grad or indices not 16 / 8-byte aligned: the same items, element loads
                    load_raw8_elems<DT>(g + e0, gr[i]);
                    ir[i] = load_raw_idx8_elems(w.idx + e0);
                }
            } else {
                graw[i] = to_f32<DT>(*gbl(g + e0));
                iraw[i] = *gbl(w.idx + e0);
            }
        }
        if constexpr (FULL) __builtin_amdgcn_sched_barrier(0);  // iteration order kept: iteration i lands i-th
    }
    s_cbr[threadIdx.x % kCodebookMax] = cbr_v;  // every thread: no branch, so the waits stay exact
    __syncthreads();
    double lsum = 0.0;
    uint32_t lmax = 0u;
#pragma unroll
    for (int i = 0; i < kDetIters; ++i) {
        const int64_t e0 = base + ((int64_t)i * kThreads + threadIdx.x) * EPL;
        if (FULL || e0 < N) {
            double cs = 0.0;  // every square into float64, as the reference sums them
            if constexpr (EPL == kChunk) {
#pragma unroll
                for (int k = 0; k < kChunk; ++k) {
                    const float gv = raw_elem<DT>(gr[i], k);
                    const float u = momentum_value(s_cbr[raw_idx(ir[i], k)], mo, gv, mc);
                    const uint32_t ub = __float_as_uint(u) & 0x7fffffffu;
                    lmax = ub > lmax ? ub : lmax;
                    float sq = gv * gv;
                    if constexpr (DT == BF16) sq = round_dt<BF16>(sq);
                    cs += (double)sq;
                }
            } else {
                const float gv = graw[i];
                const float u = momentum_value(s_cbr[iraw[i]], mo, gv, mc);
                const uint32_t ub = __float_as_uint(u) & 0x7fffffffu;
                lmax = ub > lmax ? ub : lmax;
                float sq = gv * gv;
                if constexpr (DT == BF16) sq = round_dt<BF16>(sq);
                cs = (double)sq;
            }
            lsum += cs;
        }
    }
    lsum = wave_sum_d(lsum);
    const uint32_t wmax = wave_max_u63(lmax);  // in lane 63
    uint32_t* mb = w.magbits + (wg % w.shards) * w.nb;
    if (lane == 63 && wmax != 0u) gatomic_max(mb + kb, wmax);
    if (lane == 0) s_sum[wave] = lsum;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int v = 0; v < kWaves; ++v) t += s_sum[v];
        DetRec* rec = w.det_rec + wg;
        rec->kf = kb;
        rec->sf = t;
        rec->kl = -1;
        rec->sl = 0.0;
    }
}

template <int DT, int EPL>
__device__ __forceinline__ void stats_block_det(const TensorWork& w, int64_t wg) {
    using T = typename Elem<DT>::T;
    __shared__ float s_cbr[kCodebookMax];
    __shared__ int64_t s_key[2 * kDetIters * kWaves];
    __shared__ double s_sum[2 * kDetIters * kWaves];
    const int64_t N = w.N, P = w.P, nb = w.nb;
    constexpr int64_t E = (int64_t)kDetIters * kThreads * EPL;
    const int64_t base = wg * E;
    const int64_t wg_end = base + E < N ? base + E : N;
    const int64_t kfirst = div_floor(base, P, w.invP);
    if (kfirst == div_floor(wg_end - 1, P, w.invP)) {
        if (base + E <= N) stats_block_one<DT, EPL, true>(w, wg, kfirst, s_cbr, s_sum);
        else stats_block_one<DT, EPL, false>(w, wg, kfirst, s_cbr, s_sum);
        return;
    }
    const float cbr_v = *gbl(w.qt->cbr + threadIdx.x % kCodebookMax);  // to LDS after the element loads
    const T* g = static_cast<const T*>(w.grad);
    const MomentumCoef mc = w.mc;
    // max |u|: a wave carries the max of its current block across iterations
    // and flushes it into its workgroup's shard when the block changes, so a
    // block spanning many workgroups takes one atomic per wave, spread over
    // the shards (finalize takes the max over them)
    uint32_t* mb = w.magbits + (wg % w.shards) * nb;
    double* bsq = w.blk_sq;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    // every iteration's loads first
    Raw8<DT> gr[kDetIters];
    RawIdx8 ir[kDetIters];
    float graw[kDetIters];
    uint32_t iraw[kDetIters];
    float mo[kDetIters];
    int64_t keys[kDetIters];
#pragma unroll
    for (int i = 0; i < kDetIters; ++i) {
        const int64_t e0 = base + ((int64_t)i * kThreads + threadIdx.x) * EPL;
        keys[i] = nb;  // past the end: a sentinel key, never stored
        if (e0 < N) {
            keys[i] = div_floor(e0, P, w.invP);
            mo[i] = *gbl(w.mag + keys[i]);
            if constexpr (EPL == kChunk) {
                if (w.det_vec) {
                    load_raw8<DT>(g + e0, gr[i]);
                    ir[i] = load_raw_idx8(w.idx + e0);
                } else {  // grad or indices not 16 / 8-byte aligned: the same items, element loads
                    load_raw8_elems<DT>(g + e0, gr[i]);
                    ir[i] = load_raw_idx8_elems(w.idx + e0);
                }
            } else {
                graw[i] = to_f32<DT>(*gbl(g + e0));
                iraw[i] = *gbl(w.idx + e0);
            }
        }
    }
    s_cbr[threadIdx.x % kCodebookMax] = cbr_v;  // every thread: no branch, so the waits stay exact
    __syncthreads();  // s_cbr
    int64_t ck = -1;   // carried block and its running max (wave-uniform)
    uint32_t cm = 0u;
#pragma unroll
    for (int i = 0; i < kDetIters; ++i) {
        const int64_t e0 = base + ((int64_t)i * kThreads + threadIdx.x) * EPL;
        const int64_t key = keys[i];
        double val = 0.0;
        uint32_t mx = 0u;
        if (e0 < N) {
            double cs = 0.0;  // every square into float64, as the reference sums them
            if constexpr (EPL == kChunk) {
#pragma unroll
                for (int k = 0; k < kChunk; ++k) {
                    const float gv = raw_elem<DT>(gr[i], k);
                    const float u = momentum_value(s_cbr[raw_idx(ir[i], k)], mo[i], gv, mc);
                    const uint32_t ub = __float_as_uint(u) & 0x7fffffffu;
                    mx = ub > mx ? ub : mx;
                    float sq = gv * gv;
                    if constexpr (DT == BF16) sq = round_dt<BF16>(sq);
                    cs += (double)sq;
                }
            } else {
                const float gv = graw[i];
                const float u = momentum_value(s_cbr[iraw[i]], mo[i], gv, mc);
                mx = __float_as_uint(u) & 0x7fffffffu;
                float sq = gv * gv;
                if constexpr (DT == BF16) sq = round_dt<BF16>(sq);
                cs = (double)sq;
            }
            val = cs;
        }
        const uint64_t heads = run_heads(key);
        const double sv = seg_suffix_sum(val, heads);
        const uint32_t sm = seg_suffix_max(mx, heads);
        const bool start = (heads >> lane) & 1ull;
        const int last = 63 - __clzll((long long)heads);
        // max: the first run continues the carried block or flushes it; runs
        // strictly inside these 64 items are complete; the last run is carried
        const int64_t k0 = __shfl(key, 0, 64);
        const uint32_t m0 = (uint32_t)__shfl((int)sm, 0, 64);
        if (k0 == ck) {
            cm = m0 > cm ? m0 : cm;
        } else {
            flush_det_max(mb, ck, nb, cm);
            ck = k0;
            cm = m0;
        }
        if (last != 0) {
            flush_det_max(mb, ck, nb, cm);
            if (start && lane != last && lane != 0 && key < nb && sm != 0u) gatomic_max(mb + key, sm);
            ck = __shfl(key, last, 64);
            cm = (uint32_t)__shfl((int)sm, last, 64);
        }
        if (start && lane != 0 && lane != last && key < nb) bsq[key] = sv;  // complete inside these items
        const int q = 2 * (i * kWaves + wave);
        if (lane == 0) {
            s_key[q] = key;
            s_sum[q] = sv;
        }
        if (lane == last) {  // a single run: the second slot repeats the key with nothing to add
            s_key[q + 1] = key;
            s_sum[q + 1] = lane == 0 ? 0.0 : sv;
        }
    }
    flush_det_max(mb, ck, nb, cm);
    __syncthreads();
    if (wave == 0) {
        const int64_t key = s_key[lane];
        const uint64_t heads = run_heads(key);
        const double sv = seg_suffix_sum(s_sum[lane], heads);
        const bool start = (heads >> lane) & 1ull;
        const int last = 63 - __clzll((long long)heads);
        if (start && lane != 0 && lane != last && key < nb) bsq[key] = sv;
        DetRec* rec = w.det_rec + wg;
        if (lane == 0) {
            rec->kf = key < nb ? key : -1;
            rec->sf = sv;
            if (last == 0) {
                rec->kl = -1;
                rec->sl = 0.0;
            }
        }
        if (lane == last && last != 0) {
            rec->kl = key < nb ? key : -1;
            rec->sl = sv;
        }
    }
}

__device__ __forceinline__ bool block_stats_fast_ok(const TensorWork& w) {
    return w.det_epl == kChunk;
}

template <int DT>
__device__ __forceinline__ void stats_block_wg(const TensorWork& w, int64_t wg) {
    if (block_stats_fast_ok(w)) stats_block_det<DT, kChunk>(w, wg);
    else stats_block_det<DT, 1>(w, wg);
}

// New magnitude (max over the shards), its reciprocal and the old magnitude.
__device__ __forceinline__ void finalize_magnitude(const TensorWork& w, int64_t b) {
    const float old = w.mag[b];
    w.mag_old[b] = old;
    uint32_t bits = 0u;
    drain_shards(w.magbits, w.shards, w.nb, b, [&](uint32_t v) { bits = v > bits ? v : bits; });
    const float m = __uint_as_float(bits);
    w.mag[b] = m;
    w.minv[b] = block_recip(m);
}

// Sum of p[0], p[stride], ..., p[(n-1)*stride] in index order (the sequential
// sum, bit for bit), the loads issued four at a time.
__device__ __forceinline__ double ordered_sum(const double* __restrict__ p, int64_t n, int64_t stride) {
    double s = 0.0;
    int64_t t = 0;
    for (; t + 4 <= n; t += 4) {
        double a[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) a[k] = *gbl(p + (t + k) * stride);
#pragma unroll
        for (int k = 0; k < 4; ++k) s += a[k];
    }
    for (; t < n; ++t) s += *gbl(p + t * stride);
    return s;
}

// ====================================================================
// Factored finalize.  Workgroups [0, nr): v_row EMA from the ct row partials
// plus one float64 partial of sum(v_row); [nr, nr+nc): v_col EMA from the rt
// column partials in row-tile order, csplit threads per column: thread p sums
// the p-th run of ceil(rt / csplit) partials in order, then the runs are
// added in order (one run, the plain sequential sum, when rt <= 32); the
// rest: magnitudes.
// v <- fma(sum/n, 1-beta2, v*beta2)  (gefen.py:2994-2996)
// ====================================================================
__device__ __forceinline__ void finalize_factored(const TensorWork& w, int64_t wg) {
    const int tid = threadIdx.x;
    if (wg < w.nr) {
        __shared__ double s_part[kWaves];
        const int64_t i = wg * kFinRowsPerWg + tid;
        double v64 = 0.0;
        if (i < w.R) {
            const double s = ordered_sum(w.row_part + i, w.ct, w.R);
            const float ms = (float)s / (float)w.C;
            const float v = __builtin_fmaf(ms, w.alpha2, w.v0[i] * w.beta2);
            w.v0[i] = v;
            v64 = (double)v;
        }
        v64 = wave_sum_d(v64);
        if ((tid & 63) == 0) s_part[tid >> 6] = v64;
        __syncthreads();
        if (tid == 0) {
            double s = 0.0;
            for (int ww = 0; ww < kWaves; ++ww) s += s_part[ww];
            w.vsum[wg] = s;
        }
        return;
    }
    if (wg < w.nr + w.nc) {
        __shared__ double s_run[kThreads];
        const int sp = w.csplit;
        const int cpw = kThreads / sp;  // columns per workgroup
        const int part = tid / cpw;
        const int64_t j = (wg - w.nr) * cpw + tid % cpw;
        const int64_t per = (w.rt + sp - 1) / sp;
        const int64_t t0 = std::min<int64_t>((int64_t)part * per, w.rt);
        const int64_t t1 = std::min<int64_t>(t0 + per, w.rt);
        double tot = j < w.C ? ordered_sum(w.col_part + t0 * w.C + j, t1 - t0, w.C) : 0.0;
        if (sp > 1) {
            s_run[tid] = tot;
            __syncthreads();
            if (part == 0)
                for (int q = 1; q < sp; ++q) tot += s_run[q * cpw + tid];
        }
        if (part == 0 && j < w.C) {
            const float ms = (float)tot / (float)w.R;
            const float v = __builtin_fmaf(ms, w.alpha2, w.v1[j] * w.beta2);
            w.v1[j] = v;
            w.vcs[j] = sqrtf(v);
        }
        return;
    }
    const int64_t gtid = (wg - w.nr - w.nc) * kThreads + tid;
    const int64_t gstride = w.nbw * kThreads;
    for (int64_t b = gtid; b < w.nb; b += gstride) finalize_magnitude(w, b);
}

// vmean EMA + per-block stepsize of block b from its sum of squares
// (gefen.py:180-190, 3794-3805), then its magnitude.
__device__ __forceinline__ void finalize_block_one(const TensorWork& w, const StepScalars& sc, int64_t b, double sq) {
    float mean = (float)sq / (float)w.P;
    if (w.bf16_mean) mean = round_dt<BF16>(mean);
    const float v = __builtin_fmaf(mean, w.alpha2, w.v0[b] * w.beta2);
    w.v0[b] = v;
    // the reference divides by sqrt(bc2) (gefen.py:3794-3805); without that
    // divisor from the host, multiply by the scalar row's 1/sqrt(bc2)
    const float h = (w.bc2_div > 0.0f ? sqrtf(v) / w.bc2_div : sqrtf(v) * sc.inv_bc2) + w.eps;
    w.step[b] = (1.0f / h) * sc.inv_bc1;
    finalize_magnitude(w, b);
}

// Wide form: workgroup b sums block b's stored sum and the records of the
// workgroups it spans (thread t takes records t, t+256, ... in order, then a
// fixed-order reduction), so a block of tens of millions of elements is not
// one thread's serial walk.
__device__ __forceinline__ void finalize_block_wide(const TensorWork& w, int64_t b) {
    __shared__ double s_part[kWaves];
    const int tid = threadIdx.x;
    double part = 0.0;
    if (!w.partial) {
        const int64_t wlo = (b * w.P) / w.det_elems;
        const int64_t whi = ((b + 1) * w.P - 1) / w.det_elems;
        for (int64_t r = wlo + tid; r <= whi; r += kThreads) {
            const DetRec d = w.det_rec[r];
            if (d.kf == b) part += d.sf;
            if (d.kl == b) part += d.sl;
        }
    }
    part = wave_sum_d(part);
    if ((tid & 63) == 0) s_part[tid >> 6] = part;
    __syncthreads();
    if (tid != 0) return;
    double sq = 0.0;
    drain_shards(w.blk_sq, w.shards, w.nb, b, [&](double v) { sq += v; });
    if (w.partial) {  // the stepsize comes from the caller: magnitudes only
        finalize_magnitude(w, b);
        return;
    }
    for (int ww = 0; ww < kWaves; ++ww) sq += s_part[ww];
    finalize_block_one(w, read_scalars(w), b, sq);
}

// vmean EMA + per-block stepsize (gefen.py:180-190, 3794-3805) + magnitudes.
__device__ __forceinline__ void finalize_block(const TensorWork& w, int64_t wg) {
    if (w.fin_wide) {
        if (wg < w.nb) finalize_block_wide(w, wg);
        return;
    }
    const StepScalars sc = read_scalars(w);
    for (int64_t b = wg * kThreads + threadIdx.x; b < w.nb; b += w.nbw * kThreads) {
        // the fixed-order stats store a block's sum (in shard 0) when the
        // block is complete inside one workgroup, or leave it in the records
        // of the workgroups it spans; the transposed-view stats accumulate
        // into the shards
        double sq = 0.0;
        drain_shards(w.blk_sq, w.shards, w.nb, b, [&](double v) { sq += v; });
        if (w.partial) {  // the stepsize comes from the caller: magnitudes only
            finalize_magnitude(w, b);
            continue;
        }
        if (w.det_rec != nullptr) {
            const int64_t wlo = (b * w.P) / w.det_elems;
            const int64_t whi = ((b + 1) * w.P - 1) / w.det_elems;
            for (int64_t r = wlo; r <= whi; ++r) {
                const DetRec d = w.det_rec[r];
                if (d.kf == b) sq += d.sf;
                if (d.kl == b) sq += d.sl;
            }
        }
        finalize_block_one(w, sc, b, sq);
    }
}

// mean(v_row) of one factored parameter from the finalize partials, in a
// fixed order, clamped at FLT_MIN (gefen.py:2998-3000); one workgroup.
__device__ __forceinline__ void mean_phase(const TensorWork& w) {
    __shared__ double s_part[kWaves];
    const int tid = threadIdx.x;
    double acc = 0.0;
    for (int64_t k = tid; k < w.nr; k += kThreads) acc += *gbl(w.vsum + k);
    acc = wave_sum_d(acc);
    if ((tid & 63) == 0) s_part[tid >> 6] = acc;
    __syncthreads();
    if (tid == 0) {
        double t = 0.0;
        for (int ww = 0; ww < kWaves; ++ww) t += s_part[ww];
        float mean = (float)t / (float)w.R;
        if (!(mean >= 1.17549435e-38f) && mean == mean) mean = 1.17549435e-38f;
        w.fin[1] = __float_as_uint(mean);
    }
}

// mean(v_row) as finalize stored it (already clamped at FLT_MIN).
__device__ __forceinline__ float stored_mean(const TensorWork& w) {
    return __uint_as_float(*gbl(w.fin + 1));
}

// ====================================================================
// Apply: grid-stride over logical chunks of 8 elements with nwg workgroups.
// MODE 0 factored, MODE 1 block.  FAST: contiguous p/grad, C % 8 == 0,
// P % 8 == 0, aligned -- a chunk then never crosses a row or a block, and
// (row, col, blk, pin) advance by constant strides (no per-chunk division).
// ====================================================================
struct Pos {
    int64_t row, col, blk, pin;
};

template <int MODE>
__device__ __forceinline__ Pos advance(const TensorWork& w, Pos q) {
    if constexpr (MODE == 0) {
        q.col += w.dC;
        q.row += w.dR;
        if (q.col >= w.C) { q.col -= w.C; ++q.row; }
    }
    q.pin += w.dP;
    q.blk += w.dB;
    if (q.pin >= w.P) { q.pin -= w.P; ++q.blk; }
    return q;
}

__device__ __forceinline__ void load_vcol(const float* __restrict__ vc, float v[8]) {
    const GX_GLOBAL f32x4* q = gbl(reinterpret_cast<const f32x4*>(vc));
    const f32x4 v0 = q[0], v1 = q[1];
    v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
    v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
}

struct ApplyCtx {
    float row_scale;  // (1 / mean(v_row)) * (1/bc2)
    float c1;         // (1/bc1) * lr
    RefStep ref;      // fp32 factored: the reference-order stepsize
    bool wd;
    StepScalars sc;
    bool dense;
    uint32_t kmax;
    int kk;
    uint64_t seed;
};

// One chunk of 8 elements sharing a row and a block (fast path).  u / m_new
// goes through the block reciprocal (div_by_block's Markstein step) in every
// lane; a wave where any lane is outside that step's safe range (tiny |u|;
// zero, subnormal, huge, inf or NaN magnitude) redoes the chunk with the
// fully guarded helpers.
template <int DT, int MODE, bool SR>
__device__ __forceinline__ void apply_chunk(const TensorWork& w, const SharedTables& st,
                                            const SharedSR& ssr, const ApplyCtx& cx, int64_t e0,
                                            const Pos& ps, const Raw8<DT>& gr, const Raw8<DT>& pr,
                                            const RawIdx8& ir, const float vcv[kChunk],
                                            uint32_t ix[kChunk], float pv[kChunk]) {
    const float m_old = w.mag_old[ps.blk];
    const float m_new = w.mag[ps.blk];
    const float y = w.minv[ps.blk];
    const float tb = 0x1.00001p-100f * fmaxf(m_new, 1.0f);
    float xs[kChunk];
    bool bad = (y == 0.0f);
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
        const float u = momentum_value(st.cbr[raw_idx(ir, k)], m_old, raw_elem<DT>(gr, k), w.mc);
        const float q0 = u * y;
        const float r = __builtin_fmaf(-q0, m_new, u);
        xs[k] = __builtin_fmaf(r, y, q0);
        bad = bad || !(fabsf(u) >= tb);
    }
    if (__any(bad)) {
        const bool nz = m_new > 0.0f;
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            const float u = momentum_value(st.cbr[raw_idx(ir, k)], m_old, raw_elem<DT>(gr, k), w.mc);
            const float x = nz ? div_by_block(u, m_new, y) : 0.0f;
            if constexpr (SR) ix[k] = quant_stochastic(x, ssr.cb, ssr.lut, cx.kk, cx.seed, e0 + k);
            else ix[k] = quant_nearest(x, st.bkt, st.thr, cx.kmax);
        }
    } else {
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if constexpr (SR) ix[k] = quant_stochastic(xs[k], ssr.cb, ssr.lut, cx.kk, cx.seed, e0 + k);
            else ix[k] = quant_fast(xs[k], st, cx.dense);
        }
    }
    if (w.write_p) {
        float rs = 0.0f, bstep = 0.0f, vr = 0.0f;
        if constexpr (MODE == 0) {
            vr = w.v0[ps.row];
            rs = vr * cx.row_scale;
        } else {
            bstep = w.step[ps.blk];
        }
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            const float q = st.cbr[ix[k]] * m_new;
            float pw = raw_elem<DT>(pr, k);
            if (cx.wd) pw = round_dt<DT>(pw * cx.sc.wdf);
            if constexpr (MODE == 0) {
                if (DT == F32 && cx.ref.on) {
                    pv[k] = pw - (q * ref_step(cx.ref, vr, vcv[k])) * cx.sc.lr;
                } else {
                    const float h = __builtin_amdgcn_sqrtf(rs * vcv[k]) + w.eps;
                    pv[k] = pw - q * (__builtin_amdgcn_rcpf(h) * cx.c1);
                }
            } else {
                pv[k] = pw - (q * bstep) * cx.sc.lr;  // the reference's order (gefen.py:3806-3818)
            }
        }
    }
}

template <int DT, int MODE, bool SR, bool FAST>
__device__ __forceinline__ void apply_phase(const TensorWork& w, int64_t wg, int64_t nwg,
                                            const SharedTables& st, const SharedSR& ssr) {
    using T = typename Elem<DT>::T;
    ApplyCtx cx;
    cx.sc = read_scalars(w);
    cx.kmax = (uint32_t)(w.qt->k - 1);
    cx.kk = w.qt->k;
    cx.dense = w.qt->max_cnt > 2;
    cx.seed = w.seed;
    if constexpr (SR) {
        if (w.seed_dev != nullptr) cx.seed = (uint64_t)w.seed_dev[0];
    }
    cx.row_scale = 0.0f;
    cx.ref.on = false;
    if constexpr (MODE == 0) {
        const float mean = stored_mean(w);
        cx.row_scale = (1.0f / mean) * cx.sc.inv_bc2;
        if constexpr (DT == F32) cx.ref = make_ref_step(w, cx.sc, mean);
    }
    cx.c1 = cx.sc.inv_bc1 * cx.sc.lr;
    cx.wd = cx.sc.wdf != 1.0f;

    T* p = static_cast<T*>(w.p);
    const T* g = static_cast<const T*>(w.grad);
    const int64_t nchunks = (w.N + kChunk - 1) / kChunk;
    int64_t ch = wg * kThreads + threadIdx.x;
    const int64_t stride = nwg * kThreads;
    if (ch >= nchunks) return;

    if constexpr (FAST) {
        // Two chunks per iteration (ch and ch + stride): both chunks' loads are
        // issued before either is computed.
        Pos pa;
        {
            const int64_t e0 = ch * kChunk;
            pa.row = 0;
            pa.col = e0;
            if constexpr (MODE == 0) {
                pa.row = div_floor(e0, w.C, w.invC);
                pa.col = e0 - pa.row * w.C;
            }
            pa.blk = div_floor(e0, w.P, w.invP);
            pa.pin = e0 - pa.blk * w.P;
        }
        for (; ch < nchunks; ch += 2 * stride) {
            const bool has_b = ch + stride < nchunks;
            const Pos pb = advance<MODE>(w, pa);
            const int64_t ea = ch * kChunk, eb = (ch + stride) * kChunk;
            Raw8<DT> rga, rpa, rgb, rpb;
            RawIdx8 ria, rib;
            float va[kChunk], vb[kChunk];
            load_raw8<DT>(g + ea, rga);
            ria = load_raw_idx8(w.idx + ea);
            if (w.write_p) {
                load_raw8<DT>(p + ea, rpa);
                if constexpr (MODE == 0) load_vcol(w.v1 + pa.col, va);
            }
            if (has_b) {
                load_raw8<DT>(g + eb, rgb);
                rib = load_raw_idx8(w.idx + eb);
                if (w.write_p) {
                    load_raw8<DT>(p + eb, rpb);
                    if constexpr (MODE == 0) load_vcol(w.v1 + pb.col, vb);
                }
            }
            uint32_t ix[kChunk];
            float pv[kChunk];
            apply_chunk<DT, MODE, SR>(w, st, ssr, cx, ea, pa, rga, rpa, ria, va, ix, pv);
            store_idx8(w.idx + ea, ix);
            if (w.write_p) store8<DT>(p + ea, pv);
            if (has_b) {
                apply_chunk<DT, MODE, SR>(w, st, ssr, cx, eb, pb, rgb, rpb, rib, vb, ix, pv);
                store_idx8(w.idx + eb, ix);
                if (w.write_p) store8<DT>(p + eb, pv);
            }
            pa = advance<MODE>(w, pb);
        }
    } else {
        for (; ch < nchunks; ch += stride) {
            const int64_t e0 = ch * kChunk;
            const int nvalid = (int)std::min<int64_t>(kChunk, w.N - e0);
            int64_t row = div_floor(e0, w.C, w.invC);
            int64_t col = e0 - row * w.C;
            int64_t blk = div_floor(e0, w.P, w.invP);
            int64_t pin = e0 - blk * w.P;
            float gv[kChunk], pv[kChunk];
            uint32_t ix[kChunk];
            {
                int64_t r = row, c = col;
#pragma unroll
                for (int k = 0; k < kChunk; ++k) {
                    if (k < nvalid) {
                        gv[k] = to_f32<DT>(g[r * w.gs0 + c * w.gs1]);
                        pv[k] = w.write_p ? to_f32<DT>(p[r * w.ps0 + c * w.ps1]) : 0.0f;
                        ix[k] = w.idx[e0 + k];
                        if (++c == w.C) { c = 0; ++r; }
                    } else {
                        gv[k] = 0.0f;
                        pv[k] = 0.0f;
                        ix[k] = 0u;
                    }
                }
            }
            float m_old = w.mag_old[blk];
            float m_new = w.mag[blk];
            float y = w.minv[blk];
            float bstep = 0.0f;
            if constexpr (MODE == 1) bstep = w.step[blk];
            float rs = 0.0f, vr = 0.0f;
            if constexpr (MODE == 0) {
                vr = w.v0[row];
                rs = vr * cx.row_scale;
            }
            int64_t r = row, c = col;
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                if (k < nvalid) {
                    const float u = momentum_value(st.cbr[ix[k]], m_old, gv[k], w.mc);
                    const float x = (m_new > 0.0f) ? div_by_block(u, m_new, y) : 0.0f;
                    uint32_t ni;
                    if constexpr (SR) ni = quant_stochastic(x, ssr.cb, ssr.lut, cx.kk, cx.seed, e0 + k);
                    else ni = quant_nearest(x, st.bkt, st.thr, cx.kmax);
                    ix[k] = ni;
                    if (w.write_p) {
                        const float q = st.cbr[ni] * m_new;
                        float pw = pv[k];
                        if (cx.wd) pw = round_dt<DT>(pw * cx.sc.wdf);
                        if constexpr (MODE == 0) {
                            if (DT == F32 && cx.ref.on) {
                                pv[k] = pw - (q * ref_step(cx.ref, vr, w.v1[c])) * cx.sc.lr;
                            } else {
                                const float h = __builtin_amdgcn_sqrtf(rs * w.v1[c]) + w.eps;
                                pv[k] = pw - q * (__builtin_amdgcn_rcpf(h) * cx.c1);
                            }
                        } else {
                            pv[k] = pw - (q * bstep) * cx.sc.lr;
                        }
                    }
                    if (++c == w.C) {
                        c = 0;
                        ++r;
                        if constexpr (MODE == 0) {
                            if (k + 1 < nvalid) {
                                vr = w.v0[r];
                                rs = vr * cx.row_scale;
                            }
                        }
                    }
                    if (++pin == w.P) {
                        pin = 0;
                        ++blk;
                        if (k + 1 < nvalid) {
                            m_old = w.mag_old[blk];
                            m_new = w.mag[blk];
                            y = w.minv[blk];
                            if constexpr (MODE == 1) bstep = w.step[blk];
                        }
                    }
                }
            }
            int64_t rr = row, cc = col;
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                if (k < nvalid) {
                    w.idx[e0 + k] = (uint8_t)ix[k];
                    if (w.write_p) p[rr * w.ps0 + cc * w.ps1] = from_f32<DT>(pv[k]);
                    if (++cc == w.C) { cc = 0; ++rr; }
                }
            }
        }
    }
}

// ====================================================================
// Fast apply (the hot path): contiguous p/grad, C % 8 == 0, P % 8 == 0,
// nearest rounding, a table with at most one threshold per bucket.
// Workgroup `wg` owns chunks [wg*256*kApplyChunksPerThread, ...): thread t
// takes chunks t, t+256, ... of that range, two at a time with all loads
// issued before any math.  Per element the only LDS traffic is the old
// codeword, one 8-byte quantiser entry {thr[base], base} and the new
// codeword; the step uses sqrt(v_col) precomputed by finalize and one
// sqrt(v_row * scale) per chunk.
// ====================================================================
struct FastTables {
    uint2 fq[kFqEntries];
    float cbr[kCodebookMax];
};

// All loads of a thread's share are issued before the first LDS write.
__device__ __forceinline__ void stage_fast(FastTables& s, const QTable* __restrict__ t) {
    constexpr int kVec = kFqEntries / 2;                   // uint4 per table
    constexpr int kPer = (kVec + kThreads - 1) / kThreads;
    const GX_GLOBAL u32x4* src = gbl(reinterpret_cast<const u32x4*>(t->fq));
    u32x4* dst = reinterpret_cast<u32x4*>(s.fq);
    u32x4 v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = threadIdx.x + j * kThreads;
        if (i < kVec) v[j] = src[i];
    }
    const float c = threadIdx.x < kCodebookMax ? *gbl(t->cbr + threadIdx.x) : 0.0f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = threadIdx.x + j * kThreads;
        if (i < kVec) dst[i] = v[j];
    }
    if (threadIdx.x < kCodebookMax) s.cbr[threadIdx.x] = c;
}

// Everything the fast loop touches, copied out of the descriptor once: the
// stores to p / indices could alias the descriptor memory, so fields read
// through it would be re-fetched after every store.
template <int DT>
struct FastArgs {
    using T = typename Elem<DT>::T;
    T* p;
    const T* g;
    uint8_t* idx;
    const float* mag_old;
    const float* mag;
    const float* minv;
    const float* vrow;   // factored: v_row
    const float* vcs;    // factored: sqrt(v_col)
    const float* bstep;  // block: per-block stepsize
    const QTable* qt;
    int64_t C, P, fR, fC, fB, fP;
    float row_scale, c1, eps, wdf, lr;
    bool wd;
    MomentumCoef mc;
    RefStep ref;         // fp32 factored: the reference-order stepsize (vcs then holds v_col itself)
};

// Inputs of one chunk, loaded one pipeline stage ahead of its math.
template <int DT>
struct ChunkIn {
    Raw8<DT> g, p;
    RawIdx8 i;
    float vc[kChunk];
    float m_old, m_new, y, rv;  // rv: v_row (factored) or the block stepsize (block)
};

template <int DT, int MODE>
__device__ __forceinline__ Pos advance_fast(const FastArgs<DT>& a, Pos q) {
    if constexpr (MODE == 0) {
        q.col += a.fC;
        q.row += a.fR;
        if (q.col >= a.C) { q.col -= a.C; ++q.row; }
    }
    q.pin += a.fP;
    q.blk += a.fB;
    if (q.pin >= a.P) { q.pin -= a.P; ++q.blk; }
    return q;
}

// Nearest index through the global threshold table (rare fallback).
__device__ __forceinline__ uint32_t quant_global(float x, const QTable* __restrict__ qt) {
    return quant_nearest(x, qt->bucket, qt->thr, (uint32_t)(qt->k - 1));
}

// Issue the loads of one chunk: the small per-row/per-block values first, so
// that waiting for them never waits for the streams issued after them.
template <int DT, int MODE>
__device__ __forceinline__ void fast_load(const FastArgs<DT>& a, const Pos& ps, int64_t e0, ChunkIn<DT>& in) {
    in.m_old = *gbl(a.mag_old + ps.blk);
    in.m_new = *gbl(a.mag + ps.blk);
    in.y = *gbl(a.minv + ps.blk);
    if constexpr (MODE == 0) {
        in.rv = *gbl(a.vrow + ps.row);
        load_vcol(a.vcs + ps.col, in.vc);
    } else {
        in.rv = *gbl(a.bstep + ps.blk);
    }
    load_raw8<DT>(a.g + e0, in.g);
    in.i = load_raw_idx8(a.idx + e0);
    load_raw8<DT>(a.p + e0, in.p);
}

// Requantise and apply one chunk: new indices in ix, new parameter values
// in pv.  g and p are the chunk's grads and parameters as floats, iv its old
// indices, vc its columns' sqrt(v_col) (v_col on the fp32 reference path),
// rv its v_row (factored) or block stepsize (block).  GENERAL_Q: the table
// may hold several thresholds per bucket (the fq entries do not describe
// it), so every element takes the exact search.
template <int DT, int MODE, int LF>
__device__ __forceinline__ void chunk_math(const FastArgs<DT>& a, const FastTables& ft, const float g[kChunk],
                                           const float p[kChunk], const RawIdx8& iv, const float vc[kChunk],
                                           float m_old, float m_new, float y, float rv, bool general_q,
                                           uint32_t ix[kChunk], float pv[kChunk]) {
    const float tb = 0x1.00001p-100f * fmaxf(m_new, 1.0f);
    float xs[kChunk];
    bool bad = (y == 0.0f) || general_q;
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
        const float u = momentum_value<LF>(ft.cbr[raw_idx(iv, k)], m_old, g[k], a.mc);
        const float q0 = u * y;
        const float r = __builtin_fmaf(-q0, m_new, u);
        xs[k] = __builtin_fmaf(r, y, q0);
        bad = bad || !(fabsf(u) >= tb);
    }
    if (__builtin_expect(__any(bad), 0)) {
        const bool nz = m_new > 0.0f;
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            const float u = momentum_value<LF>(ft.cbr[raw_idx(iv, k)], m_old, g[k], a.mc);
            const float x = nz ? div_by_block(u, m_new, y) : 0.0f;
            ix[k] = quant_global(x, a.qt);
        }
    } else {
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            int b = (int)__builtin_fmaf(xs[k], (float)(kBuckets / 2), (float)(kBuckets / 2));
            b = b < 0 ? 0 : (b > kFqEntries - 1 ? kFqEntries - 1 : b);  // |x| <= 1 already (v_med3)
            const uint2 e = ft.fq[b];
            ix[k] = e.y + (__uint_as_float(e.x) < xs[k] ? 1u : 0u);
        }
    }
    if constexpr (MODE == 0 && DT == F32) {
        if (a.ref.on) {  // reference order; vc holds v_col
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                const float q = ft.cbr[ix[k]] * m_new;
                float pw = p[k];
                if (a.wd) pw = round_dt<DT>(pw * a.wdf);
                pv[k] = pw - (q * ref_step(a.ref, rv, vc[k])) * a.lr;
            }
            return;
        }
    }
    float sr = 0.0f;
    if constexpr (MODE == 0) sr = __builtin_amdgcn_sqrtf(rv * a.row_scale);
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
        const float q = ft.cbr[ix[k]] * m_new;
        float pw = p[k];
        if (a.wd) pw = round_dt<DT>(pw * a.wdf);
        if constexpr (MODE == 0) {
            pv[k] = pw - q * (__builtin_amdgcn_rcpf(__builtin_fmaf(sr, vc[k], a.eps)) * a.c1);
        } else {
            pv[k] = pw - (q * rv) * a.lr;  // the reference's order (gefen.py:3806-3818)
        }
    }
}

template <int DT, int MODE, int LF>
__device__ __forceinline__ void fast_math(const FastArgs<DT>& a, const FastTables& ft, const ChunkIn<DT>& in,
                                          bool general_q, uint32_t ix[kChunk], float pv[kChunk]) {
    float g[kChunk], p[kChunk];
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
        g[k] = raw_elem<DT>(in.g, k);
        p[k] = raw_elem<DT>(in.p, k);
    }
    chunk_math<DT, MODE, LF>(a, ft, g, p, in.i, in.vc, in.m_old, in.m_new, in.y, in.rv, general_q, ix, pv);
}

// Requantise and apply one chunk, then store its indices and parameters.
template <int DT, int MODE, int LF>
__device__ __forceinline__ void fast_compute(const FastArgs<DT>& a, const FastTables& ft, int64_t e0,
                                             const ChunkIn<DT>& in) {
    uint32_t ix[kChunk];
    float pv[kChunk];
    fast_math<DT, MODE, LF>(a, ft, in, false, ix, pv);
    store_idx8(a.idx + e0, ix);
    store8<DT>(a.p + e0, pv);
}

// Workgroup `wg` of one parameter's fast apply.  Two chunks are computed per
// iteration while the next two are already loading.
template <int DT>
__device__ __forceinline__ FastArgs<DT> make_fast_args(const TensorWork& w, float row_scale) {
    FastArgs<DT> a;
    const StepScalars sc = read_scalars(w);
    a.p = static_cast<typename Elem<DT>::T*>(w.p);
    a.g = static_cast<const typename Elem<DT>::T*>(w.grad);
    a.idx = w.idx;
    a.mag_old = w.mag_old;
    a.mag = w.mag;
    a.minv = w.minv;
    a.vrow = w.v0;
    a.vcs = w.vcs;
    a.bstep = w.step;
    a.qt = w.qt;
    a.C = w.C; a.P = w.P; a.fR = w.fR; a.fC = w.fC; a.fB = w.fB; a.fP = w.fP;
    a.row_scale = row_scale;
    a.c1 = sc.inv_bc1 * sc.lr;
    a.eps = w.eps;
    a.wdf = sc.wdf;
    a.lr = sc.lr;
    a.wd = sc.wdf != 1.0f;
    a.mc = w.mc;
    a.ref.on = false;
    if constexpr (DT == F32) {
        if (w.mode == 0 && w.bc2_div > 0.0f) {
            a.ref = make_ref_step(w, sc, stored_mean(w));
            a.vcs = w.v1;
        }
    }
    return a;
}

template <int DT, int MODE, int LF>
__device__ __forceinline__ void apply_fast(const TensorWork& w, int64_t wg, const FastTables& ft,
                                           float row_scale) {
    const FastArgs<DT> a = make_fast_args<DT>(w, row_scale);
    const int64_t nchunks = w.N / kChunk;
    const int64_t first = wg * (kThreads * kApplyChunksPerThread) + threadIdx.x;
    if (first >= nchunks) return;
    // chunks of this thread: first + i*256 for i < n (n >= 1)
    const int n = (int)std::min<int64_t>(kApplyChunksPerThread, (nchunks - first + kThreads - 1) / kThreads);
    Pos p0;
    {
        const int64_t e0 = first * kChunk;
        p0.row = 0;
        p0.col = e0;
        if constexpr (MODE == 0) {
            p0.row = div_floor(e0, w.C, w.invC);
            p0.col = e0 - p0.row * w.C;
        }
        p0.blk = div_floor(e0, w.P, w.invP);
        p0.pin = e0 - p0.blk * w.P;
    }
    Pos p1 = advance_fast<DT, MODE>(a, p0);
    ChunkIn<DT> A, B;
    if ((wg + 1) * (kThreads * kApplyChunksPerThread) <= nchunks) {
        // A full workgroup (all but a tensor's last): straight-line code with
        // every load and store unconditional, so each wait names exactly the
        // chunk about to be computed and the next two chunks stay in flight.
        // (A load or store behind a branch makes the compiler assume, at the
        // join, the path with fewer operations in flight, and the waits then
        // drain the prefetched chunks as well.)
        fast_load<DT, MODE>(a, p0, first * kChunk, A);
        fast_load<DT, MODE>(a, p1, (first + kThreads) * kChunk, B);
#pragma unroll
        for (int i = 0; i < (int)kApplyChunksPerThread; i += 2) {
            const int64_t ea = (first + (int64_t)i * kThreads) * kChunk;
            const int64_t eb = ea + kThreads * kChunk;
            const Pos p2 = advance_fast<DT, MODE>(a, p1);
            const Pos p3 = advance_fast<DT, MODE>(a, p2);
            fast_compute<DT, MODE, LF>(a, ft, ea, A);
            if (i + 2 < (int)kApplyChunksPerThread) fast_load<DT, MODE>(a, p2, ea + 2 * kThreads * kChunk, A);
            fast_compute<DT, MODE, LF>(a, ft, eb, B);
            if (i + 3 < (int)kApplyChunksPerThread) fast_load<DT, MODE>(a, p3, eb + 2 * kThreads * kChunk, B);
            p1 = p3;
        }
        return;
    }
    fast_load<DT, MODE>(a, p0, first * kChunk, A);
    if (n > 1) fast_load<DT, MODE>(a, p1, (first + kThreads) * kChunk, B);
#pragma unroll 1
    for (int i = 0; i < n; i += 2) {
        const int64_t ea = (first + (int64_t)i * kThreads) * kChunk;
        const int64_t eb = ea + kThreads * kChunk;
        const Pos p2 = advance_fast<DT, MODE>(a, p1);
        const Pos p3 = advance_fast<DT, MODE>(a, p2);
        fast_compute<DT, MODE, LF>(a, ft, ea, A);
        if (i + 2 < n) fast_load<DT, MODE>(a, p2, ea + 2 * kThreads * kChunk, A);
        if (i + 1 < n) fast_compute<DT, MODE, LF>(a, ft, eb, B);
        if (i + 3 < n) fast_load<DT, MODE>(a, p3, eb + 2 * kThreads * kChunk, B);
        p0 = p2;
        p1 = p3;
    }
}

// Factored apply over row segments (contiguous p and grad, C >= 512).  The
// tasks are 512-column segments of 8 rows, segment-fastest; wave v of
// workgroup wg takes task 4*wg + v.  A lane keeps its 8 columns' sqrt(v_col)
// in registers for the task's rows, v_row is a scalar load per row, and when
// the segment lies inside one block in every row of the task, so are the
// block's magnitudes and reciprocal: per 8 elements the lane loads only g, p
// and the indices (the per-chunk v_col and block loads of apply_fast cost
// ~6% of the apply time).  Two rows are in flight while one is computed.
constexpr int64_t kRowSegCols = 64 * kChunk;
constexpr int kRowsPerTask = 8;

template <int DT, int LF>
__device__ __forceinline__ void apply_rows(const TensorWork& w, int64_t wg, const FastTables& ft, float row_scale) {
    const FastArgs<DT> a = make_fast_args<DT>(w, row_scale);
    const int64_t C = w.C, R = w.R, P = w.P;
    const int64_t nseg = (C + kRowSegCols - 1) / kRowSegCols;
    const int64_t t = wg * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t rt = t / nseg;
    const int64_t cs = (t - rt * nseg) * kRowSegCols;
    const int64_t r0 = rt * kRowsPerTask;
    if (r0 >= R) return;
    const int64_t seglen = std::min<int64_t>(kRowSegCols, C - cs);
    const int64_t c = cs + (int64_t)(threadIdx.x & 63) * kChunk;
    const bool active = c < C;
    const int64_t cl = active ? c : cs;  // idle lanes of a short segment re-read its first chunk
    const int nrows = (int)std::min<int64_t>(kRowsPerTask, R - r0);
    // block and offset of the segment's first element, row by row
    // (wave-uniform): one block per row when pin + seglen <= P
    const int64_t e_first = r0 * C + cs;
    int64_t bk[kRowsPerTask];
    bool uniform = true;
    {
        int64_t b = div_floor(e_first, P, w.invP);
        int64_t pin = e_first - b * P;
        const int64_t dB = div_floor(C, P, w.invP);
        const int64_t dP = C - dB * P;
#pragma unroll
        for (int i = 0; i < kRowsPerTask; ++i) {
            bk[i] = b;
            uniform = uniform && (i >= nrows || pin + seglen <= P);
            pin += dP;
            b += dB;
            if (pin >= P) { pin -= P; ++b; }
        }
    }
    if (nrows == kRowsPerTask && seglen == kRowSegCols && uniform) {
        float vc[kChunk];
        load_vcol(a.vcs + c, vc);
        auto load_row = [&](int i, ChunkIn<DT>& in) {
            const int64_t r = r0 + i;
            const int64_t e0 = r * C + c;
            in.m_old = sload(a.mag_old + bk[i]);
            in.m_new = sload(a.mag + bk[i]);
            in.y = sload(a.minv + bk[i]);
            in.rv = sload(a.vrow + r);
            load_raw8<DT>(a.g + e0, in.g);
            in.i = load_raw_idx8(a.idx + e0);
            load_raw8<DT>(a.p + e0, in.p);
        };
        ChunkIn<DT> A, B;
        load_row(0, A);
        load_row(1, B);
#pragma unroll
        for (int i = 0; i < kRowsPerTask; i += 2) {
#pragma unroll
            for (int k = 0; k < kChunk; ++k) { A.vc[k] = vc[k]; B.vc[k] = vc[k]; }
            fast_compute<DT, 0, LF>(a, ft, (r0 + i) * C + c, A);
            if (i + 2 < kRowsPerTask) load_row(i + 2, A);
            fast_compute<DT, 0, LF>(a, ft, (r0 + i + 1) * C + c, B);
            if (i + 3 < kRowsPerTask) load_row(i + 3, B);
        }
        return;
    }
    // a short segment, fewer rows, or a block boundary inside the segment:
    // one row at a time, per-lane block values
#pragma unroll 1
    for (int i = 0; i < nrows; ++i) {
        const int64_t r = r0 + i;
        const int64_t e0 = r * C + cl;
        Pos ps;
        ps.row = r;
        ps.col = cl;
        ps.blk = div_floor(e0, P, w.invP);
        ps.pin = e0 - ps.blk * P;
        ChunkIn<DT> in;
        fast_load<DT, 0>(a, ps, e0, in);
        uint32_t ix[kChunk];
        float pv[kChunk];
        fast_math<DT, 0, LF>(a, ft, in, false, ix, pv);
        if (active) {
            store_idx8(a.idx + e0, ix);
            store8<DT>(a.p + e0, pv);
        }
    }
}

// Apply of a transposed view, MODE 0 factored / 1 block (nearest rounding; a
// table with several thresholds per bucket takes the exact search for every
// element).  Wave v of workgroup wg takes kTvTilesPerWave consecutive 64 x 64
// tiles in tile-row-fastest order, so a workgroup reads 1 KB runs of its 64
// storage rows.  (The other half of each 128-byte index line belongs to the
// next tile column and is fetched again; orders that read both halves in
// the same step shorten those runs and measured ~20% slower.)  Per tile a
// lane loads its sub-block's g and p
// vectors and index chunks, sqrt(v_col) of its 8 columns and v_row of its 8
// rows (factored) and the block values: scalar loads of the tile's first
// kTvFew blocks when it touches no more, else per chunk.  Then chunk by
// chunk it requantises and applies (indices stored per chunk) and collects
// the new parameters into storage-row vectors, stored at the end.
template <int DT, int MODE, int LF>
__device__ __forceinline__ void apply_tv(const TensorWork& w, int64_t wg, const FastTables& ft, float row_scale) {
    const FastArgs<DT> a = make_fast_args<DT>(w, row_scale);
    const int64_t R = w.R, C = w.C, P = w.P, ldg = w.gs1, ldp = w.ps1, nb = w.nb;
    const double invP = w.invP;
    const int64_t nrt = (R + kTv - 1) / kTv;
    const int64_t ntiles = nrt * ((C + kTv - 1) / kTv);
    const int lane = threadIdx.x & 63, la = lane & 7, lb = lane >> 3;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool general_q = w.qt->max_cnt > 1;
    const int64_t dB = div_floor(C, P, invP);
    const int64_t dP = C - dB * P;
    const int64_t t0 = (wg * kWaves + wave) * (int64_t)kTvTilesPerWave;
#pragma unroll 1
    for (int it = 0; it < kTvTilesPerWave; ++it) {
        const int64_t T = t0 + it;
        if (T >= ntiles) break;
        const int64_t r0 = (T % nrt) * kTv, c0 = (T / nrt) * kTv;
        const int64_t r = r0 + 8 * la, c = c0 + 8 * lb;
        const bool ok = r < R && c < C;
        // lanes outside the tensor load the last sub-block and store nothing
        const int64_t rl = r < R ? r : R - kChunk, cl = c < C ? c : C - kChunk;
        Raw8<DT> gv[kChunk], pv[kChunk];
        RawIdx8 iv[kChunk];
        float vc[kChunk], vr[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            load_raw8<DT>(a.g + (cl + k) * ldg + rl, gv[k]);
            load_raw8<DT>(a.p + (cl + k) * ldp + rl, pv[k]);
        }
#pragma unroll
        for (int j = 0; j < kChunk; ++j) iv[j] = load_raw_idx8_cached(a.idx + (rl + j) * C + cl);
        if constexpr (MODE == 0) {
            load_vcol(a.vcs + cl, vc);
            load_vcol(a.vrow + rl, vr);
        } else {
#pragma unroll
            for (int k = 0; k < kChunk; ++k) vc[k] = vr[k] = 0.0f;
        }
        // block values of the lane's chunks
        float mo[kChunk], mn[kChunk], y[kChunk], bs[kChunk];
        const int64_t r_last = std::min<int64_t>(r0 + kTv, R) - 1, c_last = std::min<int64_t>(c0 + kTv, C) - 1;
        const int64_t b_lo = uniform64(div_floor(r0 * C + c0, P, invP));
        const int64_t b_hi = uniform64(div_floor(r_last * C + c_last, P, invP));
        if (b_hi - b_lo < kTvFew) {
            float fo[kTvFew], fn[kTvFew], fy[kTvFew], fs[kTvFew];
            tv_sload_few(a.mag_old, b_lo, nb, fo);
            tv_sload_few(a.mag, b_lo, nb, fn);
            tv_sload_few(a.minv, b_lo, nb, fy);
            if constexpr (MODE == 1) tv_sload_few(a.bstep, b_lo, nb, fs);
            int q[kChunk];
            tv_chunk_blocks(rl, cl, C, P, invP, dB, dP, b_lo, q);
#pragma unroll
            for (int j = 0; j < kChunk; ++j) {
                mo[j] = tv_pick(q[j], fo);
                mn[j] = tv_pick(q[j], fn);
                y[j] = tv_pick(q[j], fy);
                bs[j] = MODE == 1 ? tv_pick(q[j], fs) : 0.0f;
            }
        } else {
            const int64_t e = rl * C + cl;
            int64_t b = div_floor(e, P, invP);
            int64_t pin = e - b * P;
#pragma unroll
            for (int j = 0; j < kChunk; ++j) {
                mo[j] = *gbl(a.mag_old + b);
                mn[j] = *gbl(a.mag + b);
                y[j] = *gbl(a.minv + b);
                bs[j] = MODE == 1 ? *gbl(a.bstep + b) : 0.0f;
                pin += dP;
                b += dB;
                if (pin >= P) { pin -= P; ++b; }
            }
        }
        float po[kChunk][kChunk];  // new parameters: po[k][j] = element (j, k)
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            float gj[kChunk], pj[kChunk];
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                gj[k] = raw_elem<DT>(gv[k], j);
                pj[k] = raw_elem<DT>(pv[k], j);
            }
            uint32_t ix[kChunk];
            float pn[kChunk];
            chunk_math<DT, MODE, LF>(a, ft, gj, pj, iv[j], vc, mo[j], mn[j], y[j], MODE == 0 ? vr[j] : bs[j],
                                     general_q, ix, pn);
            if (ok) store_idx8(a.idx + (r + j) * C + c, ix);
#pragma unroll
            for (int k = 0; k < kChunk; ++k) po[k][j] = pn[k];
        }
        if (ok) {
#pragma unroll
            for (int k = 0; k < kChunk; ++k) store8<DT>(a.p + (c + k) * ldp + r, po[k]);
        }
    }
}

template <int DT, int MODE>
__device__ __forceinline__ void apply_tv_wg(const TensorWork& w, int64_t wg, FastTables& ft) {
    stage_fast(ft, w.qt);
    float row_scale = 0.0f;
    if constexpr (MODE == 0) {
        const StepScalars sc = read_scalars(w);
        row_scale = (1.0f / stored_mean(w)) * sc.inv_bc2;
    }
    __syncthreads();
    if (w.mc.small) apply_tv<DT, MODE, kLerpSmall>(w, wg, ft, row_scale);
    else apply_tv<DT, MODE, kLerpLarge>(w, wg, ft, row_scale);
}

// LDS of the apply kernels: the fast tables or the general ones, never both.
union ApplyLds {
    FastTables f;
    struct {
        SharedTables st;
        SharedSR ssr;
    } g;
};

// One apply workgroup: the fast path when the parameter and the table allow
// it, the general path (grid-stride over all chunks, any strides, stochastic
// rounding, dense tables) otherwise.
template <int DT, int MODE, bool SR, bool FAST>
__device__ __forceinline__ void apply_wg(const TensorWork& w, int64_t wg, int64_t nwg, ApplyLds& lds) {
    const QTable* qt = w.qt;
    if constexpr (FAST && !SR) {
        if (w.write_p && qt->max_cnt <= 1) {
            stage_fast(lds.f, qt);
            float row_scale = 0.0f;
            if constexpr (MODE == 0) {
                const StepScalars sc = read_scalars(w);
                row_scale = (1.0f / stored_mean(w)) * sc.inv_bc2;
            }
            __syncthreads();
            if constexpr (MODE == 0) {
                if (w.row_apply) {
                    if (w.mc.small) apply_rows<DT, kLerpSmall>(w, wg, lds.f, row_scale);
                    else apply_rows<DT, kLerpLarge>(w, wg, lds.f, row_scale);
                    return;
                }
            }
            if (w.mc.small) apply_fast<DT, MODE, kLerpSmall>(w, wg, lds.f, row_scale);
            else apply_fast<DT, MODE, kLerpLarge>(w, wg, lds.f, row_scale);
            return;
        }
    }
    stage_tables(lds.g.st, qt);
    if constexpr (SR) stage_sr(lds.g.ssr, qt);
    __syncthreads();
    apply_phase<DT, MODE, SR, FAST>(w, wg, nwg, lds.g.st, lds.g.ssr);
}

// ====================================================================
// Kernels.  Single parameter: descriptor by value.  Multi-tensor: a
// segment table maps launch workgroups to (descriptor, local workgroup).
// ====================================================================
struct Seg {
    int32_t t;         // descriptor index
    int32_t pad_;
    int64_t wg_begin;  // first launch workgroup of this descriptor
};

// Launch workgroup -> segment.  coarse[j] is the segment holding workgroup
// j << gshift (the host picks gshift so the table stays small), so a lookup
// is one load plus a binary search inside one granule (usually empty).
struct SegTable {
    const Seg* segs;
    const int32_t* coarse;
    int nseg;
    int gshift;
};

__device__ __forceinline__ Seg find_seg(const SegTable& tb, int64_t wg) {
    const int64_t j = wg >> tb.gshift;
    int lo = gbl(tb.coarse)[j];
    int hi = gbl(tb.coarse)[j + 1] + 1;  // last seg with wg_begin <= wg lies in [lo, hi)
    hi = hi > tb.nseg ? tb.nseg : hi;
    const Seg* sg = tb.segs;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (*gbl(&sg[mid].wg_begin) <= wg) lo = mid; else hi = mid;
    }
    Seg r;
    r.t = *gbl(&sg[lo].t);
    r.pad_ = 0;
    r.wg_begin = *gbl(&sg[lo].wg_begin);
    return r;
}

// Workgroup b of a launch of G, renumbered so that each XCD (the hardware
// deals consecutive workgroups to the 8 XCDs in turn) runs one contiguous
// range of the launch's logical workgroups.
__device__ __forceinline__ int64_t xcd_contiguous(int64_t b, int64_t G) {
    const int64_t q = G / 8, r = G % 8, x = b % 8;
    return x * q + (x < r ? x : r) + b / 8;
}

// One LDS image for both lerp forms (each instantiation would otherwise
// declare its own).
template <int DT, bool FAST>
__device__ __forceinline__ void stats_factored_wg(const TensorWork& w, int64_t wg) {
    __shared__ FactStatsLds lds;
    if (w.mc.small) stats_factored<DT, FAST, kLerpSmall>(w, wg, lds);
    else stats_factored<DT, FAST, kLerpLarge>(w, wg, lds);
}

template <int DT, bool FAST>
__global__ void __launch_bounds__(kThreads) k_factored_stats(TensorWork w) {
    stats_factored_wg<DT, FAST>(w, blockIdx.x);
}

template <int DT>
__global__ void __launch_bounds__(kThreads) k_factored_stats_tv(TensorWork w) {
    stats_tv_wg<DT, 0>(w, blockIdx.x);
}

template <int DT>
__global__ void __launch_bounds__(kThreads) k_apply_tv(TensorWork w) {
    __shared__ FastTables ft;
    apply_tv_wg<DT, 0>(w, blockIdx.x, ft);
}

template <int DT>
__global__ void __launch_bounds__(kThreads) k_block_stats(TensorWork w) {
    stats_block_wg<DT>(w, blockIdx.x);
}

__global__ void __launch_bounds__(kThreads) k_finalize(TensorWork w) {
    if (w.mode == 0) finalize_factored(w, blockIdx.x);
    else finalize_block(w, blockIdx.x);
}

__global__ void __launch_bounds__(kThreads) k_mean(TensorWork w) { mean_phase(w); }

template <int DT, int MODE, bool SR, bool FAST>
__global__ void __launch_bounds__(kThreads) k_apply(TensorWork w) {
    __shared__ ApplyLds lds;
    apply_wg<DT, MODE, SR, FAST>(w, blockIdx.x, gridDim.x, lds);
}

// Factored stats of a launch group; the group's block-path tensors of the
// same dtype (not transposed views) ride in the same launch.
template <int DT, bool FAST>
__global__ void __launch_bounds__(kThreads) k_mt_factored_stats(const TensorWork* __restrict__ ws,
                                                                SegTable tb) {
    const Seg sg = find_seg(tb, blockIdx.x);
    const TensorWork& w = ws[sg.t];
    const int64_t local = (int64_t)blockIdx.x - sg.wg_begin;
    if (w.mode != 0) {
        stats_block_wg<DT>(w, local);
        return;
    }
    stats_factored_wg<DT, FAST>(w, local);
}

template <int DT, int MODE>
__global__ void __launch_bounds__(kThreads) k_mt_stats_tv(const TensorWork* __restrict__ ws, SegTable tb) {
    const Seg sg = find_seg(tb, blockIdx.x);
    stats_tv_wg<DT, MODE>(ws[sg.t], (int64_t)blockIdx.x - sg.wg_begin);
}

template <int DT, int MODE>
// Workgroups in XCD-contiguous order: a tile's index chunks are the first or
// second half of 128-byte lines whose other half a workgroup a few places
// later reads, which then hits the same L2 (measured on the Qwen3-4B views:
// 2.07 -> 1.76 GB read per launch, the algorithmic bytes, at the same speed).
__global__ void __launch_bounds__(kThreads) k_mt_apply_tv(const TensorWork* __restrict__ ws, SegTable tb) {
    __shared__ FastTables ft;
    const int64_t L = xcd_contiguous(blockIdx.x, gridDim.x);
    const Seg sg = find_seg(tb, L);
    apply_tv_wg<DT, MODE>(ws[sg.t], L - sg.wg_begin, ft);
}

__global__ void __launch_bounds__(kThreads) k_mt_finalize(const TensorWork* __restrict__ ws,
                                                          SegTable tb) {
    const Seg sg = find_seg(tb, blockIdx.x);
    const TensorWork& w = ws[sg.t];
    const int64_t local = (int64_t)blockIdx.x - sg.wg_begin;
    if (w.mode == 0) finalize_factored(w, local);
    else finalize_block(w, local);
}

__global__ void __launch_bounds__(kThreads) k_mt_mean(const TensorWork* __restrict__ ws, SegTable tb) {
    const Seg sg = find_seg(tb, blockIdx.x);
    mean_phase(ws[sg.t]);
}

// Apply of a launch group; with MODE 0 the group's block-path tensors of the
// same dtype and variant (not transposed views) ride in the same launch.
template <int DT, int MODE, bool SR, bool FAST>
// Each XCD runs a contiguous range of the launch's workgroups, i.e. streams
// its own part of each tensor (measured on the Llama-3-8B set: apply
// 11.51-11.61 -> 11.42-11.44 ms, with a smaller spread between processes).
__global__ void __launch_bounds__(kThreads) k_mt_apply(const TensorWork* __restrict__ ws,
                                                       SegTable tb) {
    __shared__ ApplyLds lds;
    const int64_t L = xcd_contiguous(blockIdx.x, gridDim.x);
    const Seg sg = find_seg(tb, L);
    const TensorWork& w = ws[sg.t];
    const int64_t local = L - sg.wg_begin;
    if (MODE == 0 && w.mode != 0) {
        apply_wg<DT, 1, SR, FAST>(w, local, w.apply_wgs, lds);
        return;
    }
    apply_wg<DT, MODE, SR, FAST>(w, local, w.apply_wgs, lds);
}

// ====================================================================
// Host side
// ====================================================================

static MomentumCoef make_coef_w(float w1) {
    MomentumCoef mc;
    mc.w = w1;
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

static inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

static size_t elem_size(int dtype) { return dtype == F32 ? 4 : 2; }

// Fill the derived fields of a descriptor.  Everything that depends only on
// shapes, strides, pointers and the workspace layout is computed here.
struct WorkInput {
    void* p;
    const void* grad;
    int dtype;
    int mode;  // 0 factored, 1 block
    int64_t R, C, ps0, ps1, gs0, gs1, period;
    uint8_t* idx;
    float* mag;
    float* v0;
    float* v1;
    const void* qt;
    float lerp_w, beta2, alpha2, eps;
    float bc2_div;  // reference-order divisor or 0 (gefenx_tensor_desc.bc2_div)
    StepScalars sc;
    int sr;
    uint64_t seed;
    const float* step_scalars;
    const int64_t* seed_dev;
    void* workspace;
    size_t ws_bytes;
};

// The divisor of the reference's decomposed step (bc2, or sqrt(bc2) on the
// block path) from the reciprocal the C ABI passes, in double then rounded
// once: (float)(1/(1/x)) equals (float)x unless x lies within ~2^-52 of an
// fp32 rounding midpoint (none for beta2 in {0.5, 0.9, 0.95, ..., 0.9999}
// over 200,000 steps).  Python descriptors carry the same value.
static float reference_divisor(double inv) {
    if (!(inv > 0.0) || !std::isfinite(inv)) return 0.0f;
    return (float)(1.0 / inv);
}

static int build_work(const WorkInput& in, TensorWork& w) {
    std::memset(&w, 0, sizeof(w));
    const int64_t N = in.R * in.C;
    const int64_t nb = N / in.period;
    w.p = in.p; w.grad = in.grad; w.idx = in.idx; w.mag = in.mag; w.v0 = in.v0; w.v1 = in.v1;
    w.qt = static_cast<const QTable*>(in.qt);
    w.step_scalars = in.step_scalars; w.seed_dev = in.seed_dev;
    w.R = in.R; w.C = in.C; w.N = N; w.P = in.period; w.nb = nb;
    w.invC = 1.0 / (double)in.C; w.invP = 1.0 / (double)in.period;
    w.ps0 = in.ps0; w.ps1 = in.ps1; w.gs0 = in.gs0; w.gs1 = in.gs1;
    w.shards = mag_shards(nb);
    w.seed = in.seed;
    w.dtype = in.dtype; w.mode = in.mode; w.sr = in.sr;
    w.bf16_mean = in.dtype == BF16 ? 1 : 0;
    w.eps = in.eps; w.beta2 = in.beta2; w.alpha2 = in.alpha2;
    // the divisor describes the host scalars; a device scalar row carries 1/bc2 only
    w.bc2_div = in.step_scalars == nullptr && in.bc2_div > 0.0f ? in.bc2_div : 0.0f;
    w.sc = in.sc;
    w.mc = make_coef_w(in.lerp_w);
    w.write_p = (in.step_scalars != nullptr) || !(in.sc.lr == 0.0f && in.sc.wdf == 1.0f);
    char* ws = static_cast<char*>(in.workspace);
    const int64_t nchunks = ceil_div(N, kChunk);
    // transposed views: strides (1, ld), storage rows 16-byte aligned
    const int64_t es = (int64_t)elem_size(in.dtype);
    const bool tv_shape = in.R > 1 && in.R % kChunk == 0 && in.C % kChunk == 0 && in.period % kChunk == 0 &&
                          aligned(in.idx, 8);
    const bool tv_g = in.gs0 == 1 && in.gs1 >= in.R && (in.gs1 * es) % 16 == 0 && aligned(in.grad, 16);
    const bool tv_p = in.ps0 == 1 && in.ps1 >= in.R && (in.ps1 * es) % 16 == 0 && aligned(in.p, 16);
    if (in.mode == 0) {
        const FactoredWs L = FactoredWs::make(in.R, in.C, nb);
        if (in.ws_bytes < L.total)
            return set_error(GEFENX_EINVAL, "factored update: workspace %zu bytes < required %zu", in.ws_bytes, L.total);
        const FactTiles t = FactTiles::make(in.R, in.C);
        w.row_part = reinterpret_cast<double*>(ws + L.off_rowp);
        w.col_part = reinterpret_cast<double*>(ws + L.off_colp);
        w.magbits = reinterpret_cast<uint32_t*>(ws + L.off_magbits);
        w.mag_old = reinterpret_cast<float*>(ws + L.off_magold);
        w.minv = reinterpret_cast<float*>(ws + L.off_minv);
        w.vsum = reinterpret_cast<double*>(ws + L.off_vsum);
        w.vcs = reinterpret_cast<float*>(ws + L.off_vcs);
        w.fin = reinterpret_cast<uint32_t*>(ws + L.off_fin);
        w.ct = t.ct; w.rt = t.rt; w.tile_rows = t.tile_rows;
        w.stats_wgs = t.ct * t.rt;
        w.nr = ceil_div(in.R, kFinRowsPerWg);
        w.nbw = std::max<int64_t>(1, std::min<int64_t>(1024, ceil_div(nb, kFinBlocksPerWg)));
        const bool contig_g = (in.gs1 == 1 && in.gs0 == in.C);
        const bool contig_p = (in.ps1 == 1 && in.ps0 == in.C);
        w.fast_stats = contig_g && (in.C % kChunk == 0) && aligned(in.grad, 16) && aligned(in.idx, 8);
        w.fast_apply = contig_g && contig_p && (in.C % kChunk == 0) && (in.period % kChunk == 0) &&
                       aligned(in.grad, 16) && aligned(in.p, 16) && aligned(in.idx, 8) && aligned(in.v1, 16);
        if (!w.fast_stats && tv_shape && tv_g) {
            w.fast_stats = 2;
            w.rt = t.rt_tv;
            w.tile_rows = t.tv_rows;
            w.stats_wgs = t.ct * t.rt_tv;
        }
        // column sums over many row tiles (embeddings: ~250-300) split into
        // up to 8 runs (of <= 32 partials up to 256 row tiles), so no thread
        // waits on a long load chain
        w.csplit = 1;
        while (w.csplit < 8 && ceil_div(w.rt, (int64_t)w.csplit) > 32) w.csplit *= 2;
        w.nc = ceil_div(in.C, kThreads / w.csplit);
        w.fin_wgs = w.nr + w.nc + w.nbw;
        // the view apply reads v_row and sqrt(v_col) (v_col on the fp32
        // reference path) 8 floats at a time
        if (!w.fast_apply && tv_shape && tv_g && tv_p && !in.sr && w.write_p && aligned(in.v0, 16) &&
            aligned(in.v1, 16))
            w.fast_apply = 2;
    } else {
        const BlockWs L = BlockWs::make(nb, N);
        if (in.ws_bytes < L.total)
            return set_error(GEFENX_EINVAL, "block update: workspace %zu bytes < required %zu", in.ws_bytes, L.total);
        w.blk_sq = reinterpret_cast<double*>(ws + L.off_sq);
        w.magbits = reinterpret_cast<uint32_t*>(ws + L.off_magbits);
        w.mag_old = reinterpret_cast<float*>(ws + L.off_magold);
        w.step = reinterpret_cast<float*>(ws + L.off_step);
        w.minv = reinterpret_cast<float*>(ws + L.off_minv);
        w.det_rec = reinterpret_cast<DetRec*>(ws + L.off_rec);
        // fixed-order stats: 8 elements per item when chunks never cross a
        // block (P and N multiples of 8), else 1.  The summation order then
        // depends on the shape alone, not on where the grad starts in memory
        // (a view into a flat bucket sums like a fresh tensor); a misaligned
        // grad or index array loads its items element by element.
        w.det_epl = (in.period % kChunk == 0 && N % kChunk == 0) ? (int32_t)kChunk : 1;
        w.det_vec = aligned(in.grad, 16) && aligned(in.idx, 8) ? 1 : 0;
        w.det_elems = (int64_t)kDetIters * kThreads * w.det_epl;
        w.stats_wgs = std::max<int64_t>(1, ceil_div(N, w.det_elems));
        w.nbw = std::max<int64_t>(1, std::min<int64_t>(4096, ceil_div(nb, kThreads)));
        w.fin_wgs = w.nbw;
        w.fast_stats = aligned(in.grad, 16) && aligned(in.idx, 8);
        w.fast_apply = (in.period % kChunk == 0) && aligned(in.grad, 16) && aligned(in.p, 16) &&
                       aligned(in.idx, 8);
        if (in.R > 1) {
            // a 2D descriptor that is not contiguous (the callers flatten the
            // contiguous ones): the grad must be contiguous (flat stats) or a
            // transposed view; p any strides (general apply) or a view too
            const bool g_contig = in.gs1 == 1 && in.gs0 == in.C;
            const bool p_contig = in.ps1 == 1 && in.ps0 == in.C;
            if (tv_shape && tv_g) {
                const FactTiles t = FactTiles::make(in.R, in.C);
                w.ct = t.ct; w.rt = t.rt_tv; w.tile_rows = t.tv_rows;
                w.stats_wgs = t.ct * t.rt_tv;
                w.fast_stats = 2;
                w.det_rec = nullptr;  // the view tiles accumulate into the shards
            } else if (!g_contig) {
                return set_error(GEFENX_EINVAL,
                                 "block update: grad strides (%lld, %lld) of [%lld, %lld] are neither contiguous nor "
                                 "a transposed view with rows, cols and period multiples of 8",
                                 (long long)in.gs0, (long long)in.gs1, (long long)in.R, (long long)in.C);
            }
            w.fast_apply = (tv_shape && tv_g && tv_p && !in.sr && w.write_p) ? 2
                         : (g_contig && p_contig) ? w.fast_apply : 0;
        }
        // blocks that span many stats workgroups sum their records with a
        // whole workgroup each (a thread would walk thousands of them)
        if (w.det_rec != nullptr && w.P / w.det_elems + 2 >= kFinWideRecords) {
            w.fin_wide = 1;
            w.nbw = nb;
            w.fin_wgs = nb;
        }
    }
    w.apply_wgs = std::max<int64_t>(1, ceil_div(nchunks, kThreads * kApplyChunksPerThread));
    // contiguous factored tensors of at least one 512-column segment per row:
    // row segments (apply_rows); any grid size works for the general apply
    w.row_apply = (in.mode == 0 && w.fast_apply == 1 && in.R > 1 && in.C >= kRowSegCols) ? 1 : 0;
    if (w.row_apply)
        w.apply_wgs = ceil_div(ceil_div(in.C, kRowSegCols) * ceil_div(in.R, (int64_t)kRowsPerTask), (int64_t)kWaves);
    if (w.fast_apply == 2)
        w.apply_wgs = ceil_div(ceil_div(in.R, kTv) * ceil_div(in.C, kTv), (int64_t)kWaves * kTvTilesPerWave);
    const int64_t S = w.apply_wgs * kThreads * kChunk;
    w.dR = S / w.C;
    w.dC = S - w.dR * w.C;
    w.dB = S / w.P;
    w.dP = S - w.dB * w.P;
    const int64_t F = kThreads * kChunk;
    w.fR = F / w.C;
    w.fC = F - w.fR * w.C;
    w.fB = F / w.P;
    w.fP = F - w.fB * w.P;
    return GEFENX_OK;
}

// Algorithmic bytes of one parameter's step: p r/w, g r, idx r/w per element
// plus the fp32 state vectors read and written.
static double algo_bytes(const TensorWork& w) {
    const double es = (double)elem_size(w.dtype);
    const double vec = w.mode == 0 ? 8.0 * (double)(w.R + w.C + w.nb) : 16.0 * (double)w.nb;
    return (double)w.N * (3.0 * es + 2.0) + vec;
}

template <int MODE, bool SR, bool FAST>
static void launch_apply_one(int dtype, const TensorWork& w, hipStream_t s) {
    const dim3 grid((unsigned)w.apply_wgs), block(kThreads);
    switch (dtype) {
        case F32: hipLaunchKernelGGL((k_apply<F32, MODE, SR, FAST>), grid, block, 0, s, w); break;
        case F16: hipLaunchKernelGGL((k_apply<F16, MODE, SR, FAST>), grid, block, 0, s, w); break;
        default: hipLaunchKernelGGL((k_apply<BF16, MODE, SR, FAST>), grid, block, 0, s, w); break;
    }
}

template <int MODE>
static void launch_apply_single(const TensorWork& w, hipStream_t s) {
    if (MODE == 0 && w.fast_apply == 2) {
        const dim3 grid((unsigned)w.apply_wgs), block(kThreads);
        switch (w.dtype) {
            case F32: hipLaunchKernelGGL(k_apply_tv<F32>, grid, block, 0, s, w); break;
            case F16: hipLaunchKernelGGL(k_apply_tv<F16>, grid, block, 0, s, w); break;
            default: hipLaunchKernelGGL(k_apply_tv<BF16>, grid, block, 0, s, w); break;
        }
        return;
    }
    if (w.fast_apply) {
        if (w.sr) launch_apply_one<MODE, true, true>(w.dtype, w, s);
        else launch_apply_one<MODE, false, true>(w.dtype, w, s);
    } else {
        if (w.sr) launch_apply_one<MODE, true, false>(w.dtype, w, s);
        else launch_apply_one<MODE, false, false>(w.dtype, w, s);
    }
}

// Run the three phases of one parameter (single-parameter entry points).
static int run_single(const TensorWork& w, hipStream_t s) {
    const double es = (double)elem_size(w.dtype);
    int ph = prof_begin(w.mode == 0 ? GEFENX_K_STATS : GEFENX_K_BLOCK_STATS, (double)w.N * (es + 1.0), 0.0, s);
    const dim3 block(kThreads);
    if (w.mode == 0) {
        const dim3 grid((unsigned)w.stats_wgs);
#define GX_FSTATS(DTV)                                                                          \
    if (w.fast_stats == 2) hipLaunchKernelGGL(k_factored_stats_tv<DTV>, grid, block, 0, s, w);  \
    else if (w.fast_stats) hipLaunchKernelGGL((k_factored_stats<DTV, true>), grid, block, 0, s, w);  \
    else hipLaunchKernelGGL((k_factored_stats<DTV, false>), grid, block, 0, s, w)
        switch (w.dtype) {
            case F32: GX_FSTATS(F32); break;
            case F16: GX_FSTATS(F16); break;
            default: GX_FSTATS(BF16); break;
        }
#undef GX_FSTATS
    } else {
        const dim3 grid((unsigned)w.stats_wgs);
        switch (w.dtype) {
            case F32: hipLaunchKernelGGL(k_block_stats<F32>, grid, block, 0, s, w); break;
            case F16: hipLaunchKernelGGL(k_block_stats<F16>, grid, block, 0, s, w); break;
            default: hipLaunchKernelGGL(k_block_stats<BF16>, grid, block, 0, s, w); break;
        }
    }
    prof_end(ph, s);
    int rc = launch_check("stats");
    if (rc) return rc;
    ph = prof_begin(GEFENX_K_FINALIZE, 16.0 * (double)(w.R + w.C + w.nb), 0.0, s);
    hipLaunchKernelGGL(k_finalize, dim3((unsigned)w.fin_wgs), block, 0, s, w);
    if (w.mode == 0) hipLaunchKernelGGL(k_mean, dim3(1), block, 0, s, w);
    prof_end(ph, s);
    rc = launch_check("finalize");
    if (rc) return rc;
    ph = prof_begin(w.mode == 0 ? GEFENX_K_APPLY : GEFENX_K_BLOCK_APPLY, algo_bytes(w), 0.0, s);
    if (w.mode == 0) launch_apply_single<0>(w, s);
    else launch_apply_single<1>(w, s);
    prof_end(ph, s);
    return launch_check("apply");
}

// ------------------------------------------------------------ multi-tensor

// Launch-group key: tensors of one cohort that share a kernel variant.
struct GroupKey {
    int mode, dtype, fast, sr;
    bool operator<(const GroupKey& o) const {
        return std::tie(mode, dtype, fast, sr) < std::tie(o.mode, o.dtype, o.fast, o.sr);
    }
};

struct Launch {
    int phase;       // 0 stats, 1 finalize, 2 apply, 3 mean(v_row)
    int cohort;      // index of the cohort the launch belongs to
    GroupKey key;
    size_t seg_off;  // index of the first Seg in the segment array
    int nseg;
    size_t coarse_off;  // index of the first coarse entry
    int gshift;
    int64_t wgs;
    double bytes;
};

// Pinned, double-buffered staging for the per-step descriptor upload.
struct Staging {
    void* host[2] = {nullptr, nullptr};
    size_t cap[2] = {0, 0};
    hipEvent_t done[2] = {nullptr, nullptr};
    int next = 0;
};
static std::mutex g_stage_mu;
static std::map<int, Staging> g_stage;  // per device; never freed (process lifetime)

// Cohorts: consecutive parameters whose summed element count stays within
// the limit.  Each cohort runs stats -> finalize -> mean -> apply; with more
// than one cohort, the stats of cohort k+1 run on a side stream while cohort
// k applies.  Default: one cohort per step (on the Llama-3-8B set, 256M-element
// cohorts overlapped this way measured no faster: both passes already share
// the same HBM ceiling).  GEFENX_COHORT_ELEMS sets the limit (<= 0: one
// cohort); GEFENX_PIPELINE=0 keeps every launch on the caller's stream.
// Both are read at every plan build (a getenv per step), so a process can
// change them between steps.
static int64_t cohort_limit() {
    const char* e = std::getenv("GEFENX_COHORT_ELEMS");
    int64_t v = e ? std::atoll(e) : kDefaultCohortElems;
    return v > 0 ? v : (int64_t)1 << 62;
}

static bool pipeline_enabled() {
    const char* e = std::getenv("GEFENX_PIPELINE");
    return !(e && std::atoi(e) == 0);
}

struct MtLayout {
    std::vector<TensorWork> works;
    std::vector<Seg> segs;
    std::vector<int32_t> coarse;
    std::vector<Launch> launches;
};

static void plan_multi(const std::vector<TensorWork>& works, MtLayout& L) {
    L.works = works;
    L.segs.clear();
    L.coarse.clear();
    L.launches.clear();
    const int n = (int)works.size();
    const int64_t limit = cohort_limit();
    int c0 = 0, cohort = 0;
    while (c0 < n) {
        int c1 = c0;
        int64_t acc = 0;
        while (c1 < n && (c1 == c0 || acc + works[(size_t)c1].N <= limit)) acc += works[(size_t)c1++].N;
        // phases in launch order: 0 stats, 1 finalize, 3 mean(v_row), 2 apply
        for (int phase : {0, 1, 3, 2}) {
            std::map<GroupKey, std::vector<int>> groups;
            for (int t = c0; t < c1; ++t) {
                const TensorWork& w = works[(size_t)t];
                GroupKey k{w.mode, w.dtype, 0, 0};
                if (phase == 0) k.fast = w.fast_stats;
                if (phase == 2) { k.fast = w.fast_apply; k.sr = w.sr; }
                if (phase == 1 || phase == 3) k = GroupKey{0, 0, 0, 0};
                // block-path tensors other than transposed views join the
                // factored launches of their dtype (the kernels branch per
                // tensor): two launches fewer per step when both paths occur
                if (w.mode == 1 && phase == 0 && k.fast != 2) k = GroupKey{0, w.dtype, 1, 0};
                if (w.mode == 1 && phase == 2 && k.fast != 2) k.mode = 0;
                if (phase == 3 && w.mode != 0) continue;
                groups[k].push_back(t);
            }
            // transposed-view stats before the contiguous ones: their index
            // loads go through L2, so the contiguous stats' partials, which
            // the finalize reads next, stay cached (measured on the Qwen3-4B
            // set: stats 2.04 -> 1.98 ms, finalize 65 -> 58 us)
            std::vector<std::pair<GroupKey, std::vector<int>>> ordered(groups.begin(), groups.end());
            if (phase == 0) {
                std::stable_sort(ordered.begin(), ordered.end(), [](const auto& a, const auto& b) {
                    return (a.first.fast == 2) > (b.first.fast == 2);
                });
                // inside a launch, tensors with the largest stats tiles first
                // and the smallest last, so the launch's last round of
                // workgroups, which leaves CUs idle, is one of short tiles
                for (auto& kv : ordered)
                    std::stable_sort(kv.second.begin(), kv.second.end(), [&](int a, int b) {
                        const TensorWork& wa = works[(size_t)a];
                        const TensorWork& wb = works[(size_t)b];
                        return (double)wa.N * (double)wb.stats_wgs > (double)wb.N * (double)wa.stats_wgs;
                    });
            }
            for (auto& kv : ordered) {
                Launch l;
                l.phase = phase;
                l.cohort = cohort;
                l.key = kv.first;
                l.seg_off = L.segs.size();
                l.nseg = (int)kv.second.size();
                l.wgs = 0;
                l.bytes = 0.0;
                for (int t : kv.second) {
                    const TensorWork& w = works[(size_t)t];
                    L.segs.push_back(Seg{t, 0, l.wgs});
                    const int64_t wgs = phase == 0 ? w.stats_wgs : phase == 1 ? w.fin_wgs
                                      : phase == 3 ? 1 : w.apply_wgs;
                    l.wgs += wgs;
                    const double es = (double)elem_size(w.dtype);
                    l.bytes += phase == 0 ? (double)w.N * (es + 1.0)
                             : phase == 1 ? 16.0 * (double)(w.R + w.C + w.nb)
                             : phase == 3 ? 8.0 * (double)w.nr : algo_bytes(w);
                }
                // coarse table: at most 4 entries per segment (+2)
                int gs = 0;
                while ((l.wgs >> gs) > 4 * (int64_t)l.nseg) ++gs;
                l.gshift = gs;
                l.coarse_off = L.coarse.size();
                const int64_t ncoarse = (l.wgs >> gs) + 2;
                int cur = 0;
                for (int64_t j = 0; j < ncoarse; ++j) {
                    const int64_t wgj = j << gs;
                    while (cur + 1 < l.nseg && L.segs[l.seg_off + (size_t)cur + 1].wg_begin <= wgj) ++cur;
                    L.coarse.push_back(cur);
                }
                L.launches.push_back(l);
            }
        }
        c0 = c1;
        ++cohort;
    }
}

template <int MODE, bool SR, bool FAST>
static void launch_mt_apply(int dtype, dim3 grid, hipStream_t s, const TensorWork* ws, SegTable sg) {
    switch (dtype) {
        case F32: hipLaunchKernelGGL((k_mt_apply<F32, MODE, SR, FAST>), grid, dim3(kThreads), 0, s, ws, sg); break;
        case F16: hipLaunchKernelGGL((k_mt_apply<F16, MODE, SR, FAST>), grid, dim3(kThreads), 0, s, ws, sg); break;
        default: hipLaunchKernelGGL((k_mt_apply<BF16, MODE, SR, FAST>), grid, dim3(kThreads), 0, s, ws, sg); break;
    }
}

// Byte offsets of the descriptor image [works | segments | coarse index] that
// the multi-tensor launches read from device memory.
struct MtImage {
    size_t works, segs, coarse, end;
};

static MtImage image_layout(const MtLayout& L, size_t base) {
    MtImage im;
    im.works = base;
    im.segs = im.works + align256(sizeof(TensorWork) * L.works.size());
    im.coarse = im.segs + align256(sizeof(Seg) * L.segs.size());
    im.end = im.coarse + align256(sizeof(int32_t) * L.coarse.size());
    return im;
}

static void write_image(const MtLayout& L, const MtImage& im, char* h) {
    std::memcpy(h + im.works, L.works.data(), sizeof(TensorWork) * L.works.size());
    std::memcpy(h + im.segs, L.segs.data(), sizeof(Seg) * L.segs.size());
    std::memcpy(h + im.coarse, L.coarse.data(), sizeof(int32_t) * L.coarse.size());
}

static int launch_layout(const MtLayout& L, char* dev, const MtImage& im, hipStream_t s, bool prof);

static int run_multi(const MtLayout& L, void* scratch, size_t scratch_bytes, hipStream_t s) {
    const MtImage im = image_layout(L, 0);
    const size_t need = im.end;
    if (scratch_bytes < need)
        return set_error(GEFENX_EINVAL, "gefenx_multi_tensor_step: scratch %zu bytes < required %zu", scratch_bytes, need);
    int dev = 0;
    hipGetDevice(&dev);
    {
        std::lock_guard<std::mutex> lk(g_stage_mu);
        Staging& st = g_stage[dev];
        const int b = st.next;
        st.next ^= 1;
        if (st.done[b] == nullptr && hipEventCreateWithFlags(&st.done[b], hipEventDisableTiming) != hipSuccess)
            return set_error(GEFENX_ELAUNCH, "gefenx_multi_tensor_step: event creation failed");
        if (st.host[b] != nullptr) hipEventSynchronize(st.done[b]);  // previous upload from this buffer finished
        if (st.cap[b] < need) {
            if (st.host[b]) hipHostFree(st.host[b]);
            st.host[b] = nullptr;
            st.cap[b] = 0;
            if (hipHostMalloc(&st.host[b], need, hipHostMallocDefault) != hipSuccess)
                return set_error(GEFENX_ENOMEM, "gefenx_multi_tensor_step: pinned staging of %zu bytes failed", need);
            st.cap[b] = need;
        }
        char* h = static_cast<char*>(st.host[b]);
        write_image(L, im, h);
        if (hipMemcpyAsync(scratch, h, need, hipMemcpyHostToDevice, s) != hipSuccess)
            return set_error(GEFENX_ELAUNCH, "gefenx_multi_tensor_step: descriptor upload failed");
        hipEventRecord(st.done[b], s);
    }
    return launch_layout(L, static_cast<char*>(scratch), im, s, true);
}

// Enqueue one phase launch of a layout whose descriptor image is at dev.
static int enqueue_launch(const Launch& l, char* dev, const MtImage& im, hipStream_t s, bool prof) {
    const TensorWork* dws = reinterpret_cast<const TensorWork*>(dev + im.works);
    const Seg* dsegs = reinterpret_cast<const Seg*>(dev + im.segs);
    const int32_t* dcoarse = reinterpret_cast<const int32_t*>(dev + im.coarse);
    {
        if (l.wgs <= 0) return GEFENX_OK;
        if (l.wgs > 2147483647LL) return set_error(GEFENX_EINVAL, "gefenx_multi_tensor_step: launch too large");
        const dim3 grid((unsigned)l.wgs), block(kThreads);
        const SegTable sg{dsegs + l.seg_off, dcoarse + l.coarse_off, l.nseg, l.gshift};
        const int kinds[4] = {GEFENX_K_STATS, GEFENX_K_FINALIZE, GEFENX_K_APPLY, GEFENX_K_FINALIZE};
        int kind = kinds[l.phase];
        if (l.key.mode == 1 && l.phase == 0) kind = GEFENX_K_BLOCK_STATS;
        if (l.key.mode == 1 && l.phase == 2) kind = GEFENX_K_BLOCK_APPLY;
        int ph = prof ? prof_begin(kind, l.bytes, 0.0, s) : -1;
        if (l.phase == 0) {
            if (l.key.mode == 0) {
#define GX_MTS(DTV)                                                                                          \
    if (l.key.fast == 2) hipLaunchKernelGGL((k_mt_stats_tv<DTV, 0>), grid, block, 0, s, dws, sg); \
    else if (l.key.fast) hipLaunchKernelGGL((k_mt_factored_stats<DTV, true>), grid, block, 0, s, dws, sg); \
    else hipLaunchKernelGGL((k_mt_factored_stats<DTV, false>), grid, block, 0, s, dws, sg)
                switch (l.key.dtype) {
                    case F32: GX_MTS(F32); break;
                    case F16: GX_MTS(F16); break;
                    default: GX_MTS(BF16); break;
                }
#undef GX_MTS
            } else {
                // block path: only transposed views form groups of their own
                switch (l.key.dtype) {
                    case F32: hipLaunchKernelGGL((k_mt_stats_tv<F32, 1>), grid, block, 0, s, dws, sg); break;
                    case F16: hipLaunchKernelGGL((k_mt_stats_tv<F16, 1>), grid, block, 0, s, dws, sg); break;
                    default: hipLaunchKernelGGL((k_mt_stats_tv<BF16, 1>), grid, block, 0, s, dws, sg); break;
                }
            }
        } else if (l.phase == 3) {
            hipLaunchKernelGGL(k_mt_mean, grid, block, 0, s, dws, sg);
        } else if (l.phase == 1) {
            hipLaunchKernelGGL(k_mt_finalize, grid, block, 0, s, dws, sg);
        } else {
            const int dt = l.key.dtype;
            if (l.key.fast == 2) {
#define GX_MTA_TV(MODEV)                                                                                     \
    switch (dt) {                                                                                            \
        case F32: hipLaunchKernelGGL((k_mt_apply_tv<F32, MODEV>), grid, block, 0, s, dws, sg); break;      \
        case F16: hipLaunchKernelGGL((k_mt_apply_tv<F16, MODEV>), grid, block, 0, s, dws, sg); break;      \
        default: hipLaunchKernelGGL((k_mt_apply_tv<BF16, MODEV>), grid, block, 0, s, dws, sg); break;      \
    }
                if (l.key.mode == 0) { GX_MTA_TV(0) } else { GX_MTA_TV(1) }
#undef GX_MTA_TV
            } else {
                // factored and block-path tensors together (k_mt_apply<.., 0, ..>
                // branches per tensor)
                if (l.key.fast) {
                    if (l.key.sr) launch_mt_apply<0, true, true>(dt, grid, s, dws, sg);
                    else launch_mt_apply<0, false, true>(dt, grid, s, dws, sg);
                } else {
                    if (l.key.sr) launch_mt_apply<0, true, false>(dt, grid, s, dws, sg);
                    else launch_mt_apply<0, false, false>(dt, grid, s, dws, sg);
                }
            }
        }
        prof_end(ph, s);
        int rc = launch_check("multi-tensor launch");
        if (rc) return rc;
    }
    return GEFENX_OK;
}

// Side stream and event pool of one device for the cohort pipeline (default
// priority; created on first use, kept for the process lifetime).
struct Pipe {
    hipStream_t side = nullptr;
    std::vector<hipEvent_t> ev;
};
static std::mutex g_pipe_mu;
static std::map<int, Pipe> g_pipe;

static int pipe_get(size_t n_events, Pipe*& out) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lk(g_pipe_mu);
    Pipe& p = g_pipe[dev];
    if (p.side == nullptr && hipStreamCreateWithFlags(&p.side, hipStreamNonBlocking) != hipSuccess) {
        p.side = nullptr;
        return set_error(GEFENX_ELAUNCH, "gefenx_multi_tensor_step: side stream creation failed");
    }
    while (p.ev.size() < n_events) {
        hipEvent_t e = nullptr;
        if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess)
            return set_error(GEFENX_ELAUNCH, "gefenx_multi_tensor_step: event creation failed");
        p.ev.push_back(e);
    }
    out = &p;
    return GEFENX_OK;
}

// Enqueue the phase launches of L reading the descriptor image at dev.
// One cohort: everything on s in plan order.  Several: the stats, finalize
// and mean launches of every cohort go to the device's side stream, which
// first waits for all work enqueued on s so far; cohort k's applies wait on
// the event recorded after its mean launch, so the side stream runs the
// stats of later cohorts while s applies earlier ones.  s ends after the
// last apply, which follows every side-stream launch, so work enqueued on s
// afterwards sees the whole step.  Calls that overlap on one device must
// come from one host thread at a time (the side stream is shared).
static int launch_layout(const MtLayout& L, char* dev, const MtImage& im, hipStream_t s, bool prof) {
    const int n_cohorts = L.launches.empty() ? 0 : L.launches.back().cohort + 1;
    if (n_cohorts <= 1 || !pipeline_enabled()) {
        for (const Launch& l : L.launches) {
            int rc = enqueue_launch(l, dev, im, s, prof);
            if (rc) return rc;
        }
        return GEFENX_OK;
    }
    Pipe* pp = nullptr;
    int rc = pipe_get((size_t)n_cohorts + 1, pp);
    if (rc) return rc;
    hipStream_t side = pp->side;
    if (hipEventRecord(pp->ev[0], s) != hipSuccess || hipStreamWaitEvent(side, pp->ev[0], 0) != hipSuccess)
        return set_error(GEFENX_ELAUNCH, "gefenx_multi_tensor_step: stream fork failed");
    size_t i = 0;
    const size_t nl = L.launches.size();
    for (int c = 0; c < n_cohorts; ++c) {
        size_t j = i;
        for (; j < nl && L.launches[j].cohort == c; ++j)
            if (L.launches[j].phase != 2) {
                rc = enqueue_launch(L.launches[j], dev, im, side, prof);
                if (rc) return rc;
            }
        hipEvent_t ready = pp->ev[(size_t)c + 1];
        if (hipEventRecord(ready, side) != hipSuccess || hipStreamWaitEvent(s, ready, 0) != hipSuccess)
            return set_error(GEFENX_ELAUNCH, "gefenx_multi_tensor_step: cohort hand-off failed");
        for (size_t k = i; k < j; ++k)
            if (L.launches[k].phase == 2) {
                rc = enqueue_launch(L.launches[k], dev, im, s, prof);
                if (rc) return rc;
            }
        i = j;
    }
    return GEFENX_OK;
}

static size_t multi_scratch_bytes(int n_works, size_t n_segs) {
    // coarse tables: <= 4 entries per segment + 2 per launch, and every launch
    // holds at least one segment
    return align256(sizeof(TensorWork) * (size_t)n_works) + align256(sizeof(Seg) * n_segs) +
           align256(sizeof(int32_t) * 6 * n_segs);
}

// ------------------------------------------------------------ capturable plan

// Descriptor image upload as a kernel node: src is the plan's pinned host
// image (device-visible), dst the plan's device buffer; n16 16-byte words.
__global__ __launch_bounds__(kThreads) void k_image_copy(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                         int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n16; i += (int64_t)gridDim.x * kThreads)
        dst[i] = src[i];
}

__device__ __forceinline__ double capt_lr(const gefenx_capt_desc& c) {
    if (c.lr_dev == nullptr) return c.lr;
    switch (c.lr_dtype) {
        case F64: return *static_cast<const double*>(c.lr_dev);
        case F16: return (double)f16_to_f32(*static_cast<const uint16_t*>(c.lr_dev));
        case BF16: return (double)bf16_to_f32(*static_cast<const uint16_t*>(c.lr_dev));
        default: return (double)*static_cast<const float*>(c.lr_dev);
    }
}

// One thread per parameter: step counters += 1 (fp32, as torch's add_ on a
// 0-dim fp32 tensor), then the scalar row in float64 cast to fp32 --
// bc = 1 - beta^step, sqrt for the block path, reciprocal (the op chain of
// gefen.py:1984-1995).  lr: the device value when given (the weight-decay
// factor from its float64 value, gefen.py:1996-2001), else the host value
// (gefen.py:2003-2004).  Thread 0 also advances {global step, next seed,
// seed of this step}.
__global__ __launch_bounds__(kThreads) void k_capt_prologue(const gefenx_capt_desc* __restrict__ d, int n,
                                                            int64_t* __restrict__ counter) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i == 0 && counter != nullptr) {
        const int64_t seed = counter[1];
        counter[2] = seed;
        counter[1] = seed + 1;
        counter[0] = counter[0] + 1;
    }
    if (i >= n) return;
    const gefenx_capt_desc c = d[i];
    const float st = *c.step + 1.0f;
    *c.step = st;
    float st2 = st;
    if (c.bc2_step != nullptr) {
        st2 = *c.bc2_step + 1.0f;
        *c.bc2_step = st2;
    }
    double bc2 = 1.0 - pow(c.beta2, (double)st2);
    if (c.sqrt_bc2) bc2 = sqrt(bc2);
    const double bc1 = 1.0 - pow(c.beta1, (double)st);
    const double lr = capt_lr(c);
    c.scalars[0] = (float)lr;
    c.scalars[1] = (float)(1.0 / bc2);
    c.scalars[2] = (float)(1.0 / bc1);
    c.scalars[3] = c.weight_decay != 0.0 ? (float)(1.0 - lr * c.weight_decay) : 1.0f;
}

}  // namespace gx

// A fixed tensor set's descriptor image and launch list (include/gefenx.h).
struct gefenx_mt_plan {
    gx::MtLayout L;
    gx::MtImage im;
    size_t capt_off = 0;
    int n_capt = 0;
    int64_t* counter = nullptr;
    size_t bytes = 0;
    int device = 0;
    void* host = nullptr;      // pinned image
    void* host_dev = nullptr;  // its device-visible address
    bool uploaded = false;     // an eager launch copied the image into uploaded_to on uploaded_on
    void* uploaded_to = nullptr;
    hipStream_t uploaded_on = nullptr;
};

using namespace gx;

static int check_dtype(int dtype, const char* fn) {
    if (dtype == F64)
        return set_error(GEFENX_EDTYPE, "%s: not implemented for 'Double' (fp32/fp16/bf16 only)", fn);
    if (dtype != F32 && dtype != F16 && dtype != BF16)
        return set_error(GEFENX_EINVAL, "%s: unknown dtype code %d", fn, dtype);
    return GEFENX_OK;
}

// ------------------------------------------------------------ static scratch
// Device scratch of gefenx_factored_update_noalloc: a file-scope array, one
// copy per GPU the library runs on, held until the process ends.  In host
// code the array's name is not a device address: scratch_on_device() resolves
// it once per device (hipGetSymbolAddress with that device current) and every
// host use -- kernel arguments, the clearing launch -- goes through the
// resolved pointer.
static __device__ __align__(256) unsigned char scratch[GEFENX_NOALLOC_SCRATCH_BYTES];

constexpr int kScratchDevices = 64;
static void* g_scratch_addr[kScratchDevices];  // per device; nullptr until resolved
static std::mutex g_scratch_mu;

static int scratch_on_device(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices)
        return set_error(GEFENX_ELAUNCH, "gefenx_factored_update_noalloc: no usable current device");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_addr[dev] == nullptr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr)
            return set_error(GEFENX_ELAUNCH, "gefenx_factored_update_noalloc: hipGetSymbolAddress of the scratch "
                             "array failed on device %d: %s", dev, hipGetErrorString(e));
        g_scratch_addr[dev] = ptr;
    }
    *out = g_scratch_addr[dev];
    return GEFENX_OK;
}

// Zero n 32-bit words (a kernel, not a memset node, so a captured graph
// replays it like any other launch).
__global__ __launch_bounds__(kThreads) void k_zero_words(uint32_t* __restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        p[i] = 0u;
}

extern "C" {

// Validation and work description shared by the factored entry points.
static int factored_input(const char* fn, void* p, const void* grad, int dtype, int64_t rows, int64_t cols,
                          int64_t ps0, int64_t ps1, int64_t gs0, int64_t gs1, uint8_t* m_codebook,
                          float* m_magnitude, float* v_row, float* v_col, int64_t period, const void* qtable_dev,
                          double beta1, double beta2, double lr, double eps, double inv_bias_correction_2,
                          double inv_bias_correction_1, double weight_decay_factor, int stochastic_round,
                          int64_t rng_seed, const float* step_scalars, const int64_t* seed_dev, WorkInput& in,
                          bool& empty) {
    empty = false;
    int rc = check_dtype(dtype, fn);
    if (rc) return rc;
    if (rows < 0 || cols < 0) return set_error(GEFENX_EINVAL, "%s: negative shape", fn);
    const int64_t N = rows * cols;
    if (N == 0) {  // empty tensors are a no-op
        empty = true;
        return GEFENX_OK;
    }
    if (period <= 0 || N % period != 0)
        return set_error(GEFENX_EINVAL, "%s: period %lld does not divide numel %lld", fn, (long long)period,
                         (long long)N);
    if (!p || !grad || !m_codebook || !m_magnitude || !v_row || !v_col || !qtable_dev)
        return set_error(GEFENX_EINVAL, "%s: null pointer argument", fn);
    in = WorkInput{};
    in.p = p; in.grad = grad; in.dtype = dtype; in.mode = 0;
    in.R = rows; in.C = cols; in.ps0 = ps0; in.ps1 = ps1; in.gs0 = gs0; in.gs1 = gs1; in.period = period;
    in.idx = m_codebook; in.mag = m_magnitude; in.v0 = v_row; in.v1 = v_col; in.qt = qtable_dev;
    in.lerp_w = (float)(1.0 - beta1); in.beta2 = (float)beta2; in.alpha2 = (float)(1.0 - beta2);
    in.eps = (float)eps;
    in.sc = StepScalars{(float)lr, (float)inv_bias_correction_2, (float)inv_bias_correction_1,
                        (float)weight_decay_factor};
    in.bc2_div = reference_divisor(inv_bias_correction_2);
    in.sr = stochastic_round ? 1 : 0; in.seed = (uint64_t)rng_seed;
    in.step_scalars = step_scalars; in.seed_dev = seed_dev;
    return GEFENX_OK;
}

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
    WorkInput in;
    bool empty = false;
    int rc = factored_input("gefenx_factored_update", p, grad, dtype, rows, cols, ps0, ps1, gs0, gs1, m_codebook,
                            m_magnitude, v_row, v_col, period, qtable_dev, beta1, beta2, lr, eps,
                            inv_bias_correction_2, inv_bias_correction_1, weight_decay_factor, stochastic_round,
                            rng_seed, step_scalars, seed_dev, in, empty);
    if (rc || empty) return rc;
    if (!workspace) return set_error(GEFENX_EINVAL, "gefenx_factored_update: null workspace");
    in.workspace = workspace; in.ws_bytes = workspace_bytes;
    TensorWork w;
    rc = build_work(in, w);
    if (rc) return rc;
    return run_single(w, static_cast<hipStream_t>(stream));
}

int gefenx_factored_update_noalloc(
    void* p, const void* grad, int dtype, int64_t rows, int64_t cols,
    int64_t ps0, int64_t ps1, int64_t gs0, int64_t gs1,
    uint8_t* m_codebook, float* m_magnitude, float* v_row, float* v_col,
    int64_t period, const void* qtable_dev,
    double beta1, double beta2, double lr, double eps,
    double inv_bias_correction_2, double inv_bias_correction_1,
    double weight_decay_factor, int stochastic_round, int64_t rng_seed,
    const float* step_scalars, const int64_t* seed_dev, void* stream) {
    const char* fn = "gefenx_factored_update_noalloc";
    WorkInput in;
    bool empty = false;
    int rc = factored_input(fn, p, grad, dtype, rows, cols, ps0, ps1, gs0, gs1, m_codebook, m_magnitude, v_row,
                            v_col, period, qtable_dev, beta1, beta2, lr, eps, inv_bias_correction_2,
                            inv_bias_correction_1, weight_decay_factor, stochastic_round, rng_seed, step_scalars,
                            seed_dev, in, empty);
    if (rc || empty) return rc;
    const FactoredWs L = FactoredWs::make(rows, cols, rows * cols / period);
    if (L.total > (size_t)GEFENX_NOALLOC_SCRATCH_BYTES)
        return set_error(GEFENX_EINVAL, "%s: a [%lld, %lld] parameter with period %lld needs %zu bytes of scratch; "
                         "the static scratch holds %zu (use gefenx_factored_update with a workspace)", fn,
                         (long long)rows, (long long)cols, (long long)period, L.total,
                         (size_t)GEFENX_NOALLOC_SCRATCH_BYTES);
    void* ptr = nullptr;
    rc = scratch_on_device(&ptr);
    if (rc) return rc;
    in.workspace = ptr;
    in.ws_bytes = GEFENX_NOALLOC_SCRATCH_BYTES;
    TensorWork w;
    rc = build_work(in, w);
    if (rc) return rc;
    // the accumulators that must start at zero: block maxima and the
    // finalize counter (the previous call on this GPU left them zero unless
    // it failed part-way)
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* base = static_cast<char*>(ptr);
    const int64_t nmag = (int64_t)((L.off_magold - L.off_magbits) / sizeof(uint32_t));
    hipLaunchKernelGGL(k_zero_words, dim3((unsigned)std::min<int64_t>(1024, ceil_div(nmag, kThreads))),
                       dim3(kThreads), 0, s, reinterpret_cast<uint32_t*>(base + L.off_magbits), nmag);
    hipLaunchKernelGGL(k_zero_words, dim3(1), dim3(kThreads), 0, s, reinterpret_cast<uint32_t*>(base + L.off_fin),
                       (int64_t)(256 / sizeof(uint32_t)));
    rc = launch_check(fn);
    if (rc) return rc;
    return run_single(w, s);
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
    WorkInput in{};
    in.p = p; in.grad = grad; in.dtype = dtype; in.mode = 1;
    in.R = 1; in.C = numel; in.ps0 = numel; in.ps1 = 1; in.gs0 = numel; in.gs1 = 1; in.period = period;
    in.idx = m_codebook; in.mag = m_magnitude; in.v0 = vmean; in.v1 = nullptr; in.qt = qtable_dev;
    in.lerp_w = (float)(1.0 - beta1); in.beta2 = (float)beta2; in.alpha2 = (float)(1.0 - beta2);
    in.eps = (float)eps;
    in.sc = StepScalars{(float)lr, (float)inv_sqrt_bias_correction_2, (float)inv_bias_correction_1,
                        (float)weight_decay_factor};
    in.bc2_div = reference_divisor(inv_sqrt_bias_correction_2);
    in.sr = stochastic_round ? 1 : 0; in.seed = (uint64_t)rng_seed;
    in.step_scalars = step_scalars; in.seed_dev = seed_dev;
    in.workspace = workspace; in.ws_bytes = workspace_bytes;
    TensorWork w;
    rc = build_work(in, w);
    if (rc) return rc;
    return run_single(w, static_cast<hipStream_t>(stream));
}

int gefenx_momentum_apply(
    void* p, const void* grad, int dtype, int64_t numel, int64_t period,
    uint8_t* m_codebook, float* m_magnitude, const float* stepsize, const void* qtable_dev,
    double beta1, double lr, void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_dtype(dtype, "gefenx_momentum_apply");
    if (rc) return rc;
    if (numel < 0) return set_error(GEFENX_EINVAL, "gefenx_momentum_apply: negative numel");
    if (numel == 0) return GEFENX_OK;
    if (period <= 0 || numel % period != 0)
        return set_error(GEFENX_EINVAL, "gefenx_momentum_apply: period %lld does not divide numel %lld",
                         (long long)period, (long long)numel);
    if (!p || !grad || !m_codebook || !m_magnitude || !stepsize || !qtable_dev || !workspace)
        return set_error(GEFENX_EINVAL, "gefenx_momentum_apply: null pointer argument");
    WorkInput in{};
    in.p = p; in.grad = grad; in.dtype = dtype; in.mode = 1;
    in.R = 1; in.C = numel; in.ps0 = numel; in.ps1 = 1; in.gs0 = numel; in.gs1 = 1; in.period = period;
    in.idx = m_codebook; in.mag = m_magnitude; in.v0 = nullptr; in.v1 = nullptr; in.qt = qtable_dev;
    in.lerp_w = (float)(1.0 - beta1); in.beta2 = 0.0f; in.alpha2 = 0.0f; in.eps = 0.0f;
    in.sc = StepScalars{(float)lr, 1.0f, 1.0f, 1.0f};
    in.workspace = workspace; in.ws_bytes = workspace_bytes;
    TensorWork w;
    rc = build_work(in, w);
    if (rc) return rc;
    w.partial = 1;
    w.step = const_cast<float*>(stepsize);  // read by the apply, never written in this mode
    return run_single(w, static_cast<hipStream_t>(stream));
}

static int desc_to_work(const gefenx_tensor_desc& d, int i, const void* const* qtables, int sr,
                        int64_t seed, const float* step_scalars, const int64_t* seed_dev, TensorWork& w) {
    int rc = check_dtype(d.dtype, "gefenx_multi_tensor_step");
    if (rc) return rc;
    const int64_t N = d.rows * d.cols;
    if (d.rows < 0 || d.cols < 0 || d.period <= 0 || N % d.period != 0)
        return set_error(GEFENX_EINVAL, "gefenx_multi_tensor_step: descriptor %d has period %lld not dividing [%lld, %lld]",
                         i, (long long)d.period, (long long)d.rows, (long long)d.cols);
    if (!d.p || !d.grad || !d.m_codebook || !d.m_magnitude || !d.v0 || (d.factored && !d.v1) || !d.workspace)
        return set_error(GEFENX_EINVAL, "gefenx_multi_tensor_step: descriptor %d has a null pointer", i);
    const void* qt = qtables[d.dtype];
    if (!qt) return set_error(GEFENX_EINVAL, "gefenx_multi_tensor_step: no quantisation table for dtype %d", d.dtype);
    WorkInput in{};
    in.p = d.p; in.grad = d.grad; in.dtype = d.dtype; in.mode = d.factored ? 0 : 1;
    if (d.factored) {
        in.R = d.rows; in.C = d.cols; in.ps0 = d.ps0; in.ps1 = d.ps1; in.gs0 = d.gs0; in.gs1 = d.gs1;
    } else if (d.rows <= 1 || (d.ps1 == 1 && d.gs1 == 1 && d.ps0 == d.cols && d.gs0 == d.cols)) {
        in.R = 1; in.C = N; in.ps0 = N; in.ps1 = 1; in.gs0 = N; in.gs1 = 1;  // contiguous: flat
    } else {
        in.R = d.rows; in.C = d.cols; in.ps0 = d.ps0; in.ps1 = d.ps1; in.gs0 = d.gs0; in.gs1 = d.gs1;
    }
    in.period = d.period;
    in.idx = d.m_codebook; in.mag = d.m_magnitude; in.v0 = d.v0; in.v1 = d.v1; in.qt = qt;
    in.lerp_w = d.lerp_w; in.beta2 = d.beta2; in.alpha2 = d.alpha2; in.eps = d.eps;
    in.bc2_div = d.bc2_div;
    in.sc = StepScalars{d.lr, d.inv_bc2, d.inv_bc1, d.wd_factor};
    in.sr = sr ? 1 : 0; in.seed = (uint64_t)seed;
    in.step_scalars = step_scalars; in.seed_dev = seed_dev;
    in.workspace = d.workspace;
    in.ws_bytes = d.factored ? gefenx_workspace_bytes(GEFENX_WS_FACTORED, d.rows, d.cols, N / d.period)
                             : gefenx_workspace_bytes(GEFENX_WS_BLOCK, d.rows, d.cols, N / d.period);
    return build_work(in, w);
}

static int build_layout(const gefenx_tensor_desc* descs, int n, const void* const* qtables, int sr,
                        int64_t seed, const float* const* step_scalars, const int64_t* seed_dev, MtLayout& L) {
    if (n < 0 || (n > 0 && (!descs || !qtables)))
        return set_error(GEFENX_EINVAL, "gefenx_multi_tensor_step: bad descriptor array");
    std::vector<TensorWork> works;
    works.reserve((size_t)n);
    for (int i = 0; i < n; ++i) {
        if (descs[i].rows * descs[i].cols == 0) continue;  // empty tensors are a no-op
        TensorWork w;
        int rc = desc_to_work(descs[i], i, qtables, sr, seed, step_scalars ? step_scalars[i] : nullptr,
                              seed_dev, w);
        if (rc) return rc;
        works.push_back(w);
    }
    plan_multi(works, L);
    return GEFENX_OK;
}

size_t gefenx_multi_tensor_scratch_bytes(int n) {
    if (n <= 0) return 256;
    // each tensor is one segment of one launch per phase (4 phases)
    return multi_scratch_bytes(n, (size_t)n * 4);
}

int gefenx_multi_tensor_step(const gefenx_tensor_desc* descs, int n, const void* const* qtables_dev,
                             int stochastic_round, int64_t rng_seed, void* desc_scratch_dev,
                             size_t desc_scratch_bytes, void* stream) {
    MtLayout L;
    int rc = build_layout(descs, n, qtables_dev, stochastic_round, rng_seed, nullptr, nullptr, L);
    if (rc) return rc;
    if (L.works.empty()) return GEFENX_OK;
    if (!desc_scratch_dev) return set_error(GEFENX_EINVAL, "gefenx_multi_tensor_step: null scratch");
    return run_multi(L, desc_scratch_dev, desc_scratch_bytes, static_cast<hipStream_t>(stream));
}

int gefenx_mt_plan_create(const gefenx_tensor_desc* descs, int n, const float* const* step_scalars,
                          const void* const* qtables_dev, int stochastic_round, int64_t rng_seed,
                          const gefenx_capt_desc* capt, int n_capt, int64_t* counter_dev,
                          gefenx_mt_plan** plan_out) {
    if (!plan_out) return set_error(GEFENX_EINVAL, "gefenx_mt_plan_create: null plan_out");
    *plan_out = nullptr;
    if (n_capt < 0 || (n_capt > 0 && !capt))
        return set_error(GEFENX_EINVAL, "gefenx_mt_plan_create: bad capturable descriptor array");
    for (int i = 0; i < n_capt; ++i) {
        const gefenx_capt_desc& c = capt[i];
        if (!c.step || !c.scalars)
            return set_error(GEFENX_EINVAL, "gefenx_mt_plan_create: capturable descriptor %d has a null pointer", i);
        if (c.lr_dev && (c.lr_dtype < GEFENX_F32 || c.lr_dtype > GEFENX_F64))
            return set_error(GEFENX_EINVAL, "gefenx_mt_plan_create: capturable descriptor %d: lr dtype code %d", i,
                             c.lr_dtype);
    }
    const int64_t* seed_dev = counter_dev ? counter_dev + 2 : nullptr;
    auto plan = std::make_unique<gefenx_mt_plan>();
    int rc = build_layout(descs, n, qtables_dev, stochastic_round, rng_seed, step_scalars, seed_dev, plan->L);
    if (rc) return rc;
    plan->im = image_layout(plan->L, 0);
    plan->capt_off = plan->im.end;
    plan->n_capt = n_capt;
    plan->counter = counter_dev;
    (void)hipGetDevice(&plan->device);
    plan->bytes = std::max<size_t>(plan->capt_off + align256(sizeof(gefenx_capt_desc) * (size_t)n_capt), 256);
    // Pinned allocation is host work; let it through while this thread's
    // stream is being captured.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    (void)hipThreadExchangeStreamCaptureMode(&mode);
    const hipError_t e = hipHostMalloc(&plan->host, plan->bytes, hipHostMallocDefault);
    (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess) {
        plan->host = nullptr;
        return set_error(GEFENX_ENOMEM, "gefenx_mt_plan_create: pinned image of %zu bytes failed", plan->bytes);
    }
    if (hipHostGetDevicePointer(&plan->host_dev, plan->host, 0) != hipSuccess) {
        (void)hipHostFree(plan->host);
        plan->host = nullptr;
        return set_error(GEFENX_ELAUNCH, "gefenx_mt_plan_create: pinned image has no device address");
    }
    char* h = static_cast<char*>(plan->host);
    std::memset(h, 0, plan->bytes);
    write_image(plan->L, plan->im, h);
    if (n_capt > 0) std::memcpy(h + plan->capt_off, capt, sizeof(gefenx_capt_desc) * (size_t)n_capt);
    *plan_out = plan.release();
    return GEFENX_OK;
}

size_t gefenx_mt_plan_device_bytes(const gefenx_mt_plan* plan) { return plan ? plan->bytes : 0; }

int gefenx_mt_plan_launch(gefenx_mt_plan* plan, void* dev_buf, size_t dev_bytes, void* stream) {
    if (!plan || !dev_buf) return set_error(GEFENX_EINVAL, "gefenx_mt_plan_launch: null plan or buffer");
    if (dev_bytes < plan->bytes)
        return set_error(GEFENX_EINVAL, "gefenx_mt_plan_launch: buffer %zu bytes < required %zu", dev_bytes,
                         plan->bytes);
    if (reinterpret_cast<uintptr_t>(dev_buf) % 256 != 0)
        return set_error(GEFENX_EINVAL, "gefenx_mt_plan_launch: buffer not 256-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess)
        return set_error(GEFENX_ELAUNCH, "gefenx_mt_plan_launch: stream capture query failed");
    const bool capturing = cs != hipStreamCaptureStatusNone;
    const dim3 block(kThreads);
    if (capturing || !plan->uploaded || plan->uploaded_to != dev_buf || plan->uploaded_on != s) {
        const int64_t n16 = (int64_t)(plan->bytes / 16);
        const unsigned grid = (unsigned)std::min<int64_t>((n16 + kThreads - 1) / kThreads, 1024);
        hipLaunchKernelGGL(k_image_copy, dim3(grid), block, 0, s, static_cast<const uint4*>(plan->host_dev),
                           static_cast<uint4*>(dev_buf), n16);
        int rc = launch_check("plan image copy");
        if (rc) return rc;
        if (!capturing) {
            plan->uploaded = true;
            plan->uploaded_to = dev_buf;
            plan->uploaded_on = s;
        }
    }
    char* dev = static_cast<char*>(dev_buf);
    if (plan->n_capt > 0 || plan->counter != nullptr) {
        const unsigned grid = (unsigned)std::max(1, (plan->n_capt + kThreads - 1) / kThreads);
        hipLaunchKernelGGL(k_capt_prologue, dim3(grid), block, 0, s,
                           reinterpret_cast<const gefenx_capt_desc*>(dev + plan->capt_off), plan->n_capt,
                           plan->counter);
        int rc = launch_check("capturable prologue");
        if (rc) return rc;
    }
    if (plan->L.works.empty()) return GEFENX_OK;
    return launch_layout(plan->L, dev, plan->im, s, !capturing);
}

void gefenx_mt_plan_destroy(gefenx_mt_plan* plan) {
    if (!plan) return;
    if (plan->host) {
        // the last launch's image copy may still be reading the pinned image
        int cur = 0;
        (void)hipGetDevice(&cur);
        (void)hipSetDevice(plan->device);
        (void)hipDeviceSynchronize();
        (void)hipHostFree(plan->host);
        (void)hipSetDevice(cur);
    }
    delete plan;
}

}  // extern "C"
