// gefenx_muon.hip -- the Muon half of the step on MI355X (gfx950):
//
//   momentum     advance the 8-bit quantised momentum of a 2D parameter by one
//                EMA step and emit the dense momentum (optionally Nesterov)
//                that Newton-Schulz orthogonalises.  Two passes: the block
//                max of |u|, then requantise + emit (gefen_muon.py:1064-1146,
//                948-974; every intermediate rounds to the grad dtype D, as
//                the reference's tensors of dtype D do).
//   newton-schulz  X = bf16(M) (transposed when tall), X /= max(||X||, eps),
//                then per iteration G = XX^T, B = bG + cGG, X = aX + BX, each
//                product rounded to bf16 (gefen_muon.py:236-291).  Every
//                product is an "NT" GEMM C = A B^T with K contiguous in both
//                operands: G = X X^T; GG = G G^T (G is symmetric); BX =
//                B (X^T)^T -- so the kernel keeps X and X^T side by side and
//                the X update writes both.  G and B = bG + cGG are symmetric:
//                only their lower-triangle tiles are computed, each mirrored
//                as it is stored (about 30% fewer MFMAs per iteration).  bf16
//                MFMA 32x32x16, fp32 accumulation, LDS double buffering.
//   normuon      per-row EMA of the mean square of the update, rescaled to
//                keep the Frobenius norm (gefen_muon.py:1192-1230).
//   apply        p = D(p * (1 - lr*wd)); p = D(fma(update, alpha, p)),
//                alpha = D(-adjusted_lr) (gefen_muon.py:1286-1300).
#include "gefenx_device.h"
#include "gefenx_internal.h"
#include "gefenx_profile.h"
#include "gefenx.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

namespace gx {
namespace muon {

constexpr int kT = 256;
constexpr float kTiny = 1.17549435e-38f;

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

static int launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GEFENX_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
    return GEFENX_OK;
}

// ==================================================================
// Quantised momentum
// ==================================================================
// A launch covers a batch of matrices of one shape [R, C] (blockIdx.y picks
// the matrix): the grad, state and workspace pointers, the period and the
// grad strides are per matrix, the scalars shared.  The dense momentum of
// matrix i goes to out + i * N (row-major, the Newton-Schulz input stack).
constexpr int kMaxBatch = 16;

struct MomItem {
    const void* g;
    int64_t gs0, gs1;   // grad strides in elements (logical row-major order)
    uint8_t* idx;
    float* mag;         // m_magnitude (old on entry, new after finalize)
    uint32_t* magbits;  // workspace: sharded block max |u| (ordered bits)
    float* mag_old;
    float* minv;        // RN(1 / max(mag_new, tiny)) or 0 when unusable
    int64_t P, nb, shards;
    double invP;
};
struct MomBatch {
    MomItem it[kMaxBatch];
};

struct MomArgs {
    void* out;        // dense momentum [n, N], grad dtype
    const QTable* qt;
    const int64_t* seed_dev;
    int64_t N, C;
    double invC;
    uint64_t seed;
    float w;          // (float)(1 - beta)
    float beta;       // (float)beta
    float alpha_d;    // D((float)(1 - beta)): torch's add_ alpha in the grad dtype
    int nesterov;
};

// u = D(lerp(D(D(c) * m_old), g, w)); cr already rounded through D.
template <int DT>
__device__ __forceinline__ float mom_u(float cr, float m_old, float g, float w) {
    const float cm = round_dt<DT>(cr * m_old);
    const float d = g - cm;
    const float l = fabsf(w) < 0.5f ? __builtin_fmaf(w, d, cm) : __builtin_fmaf(w - 1.0f, d, g);
    return round_dt<DT>(l);
}

// Offset of logical element e of a [R, C] view with strides (gs0, gs1).
__device__ __forceinline__ int64_t view_offset(int64_t e, int64_t C, double invC, int64_t s0, int64_t s1) {
    const int64_t r = div_floor(e, C, invC);
    return r * s0 + (e - r * C) * s1;
}

// Any layout: grid-stride over the matrix's elements.
template <int DT>
__global__ void __launch_bounds__(kT) k_mom_max(MomArgs a, MomBatch bt) {
    using T = typename Elem<DT>::T;
    const MomItem& it = bt.it[blockIdx.y];
    __shared__ float s_cbr[kCodebookMax];
    if (threadIdx.x < kCodebookMax) s_cbr[threadIdx.x] = *gbl(a.qt->cbr + threadIdx.x);
    __syncthreads();
    const T* g = static_cast<const T*>(it.g);
    const bool dense = it.gs1 == 1 && it.gs0 == a.C;
    uint32_t* mb = it.magbits + ((int64_t)blockIdx.x % it.shards) * it.nb;
    const int64_t stride = (int64_t)gridDim.x * kT;
    int64_t cur = -1;
    uint32_t cbits = 0u;
    float mo = 0.0f;
    for (int64_t e = (int64_t)blockIdx.x * kT + threadIdx.x; e < a.N; e += stride) {
        const int64_t b = div_floor(e, it.P, it.invP);
        if (b != cur) {
            if (cur >= 0 && cbits) gatomic_max(mb + cur, cbits);
            cur = b;
            cbits = 0u;
            mo = *gbl(it.mag + b);
        }
        const int64_t ge = dense ? e : view_offset(e, a.C, a.invC, it.gs0, it.gs1);
        const float gv = to_f32<DT>(*gbl(g + ge));
        const float u = mom_u<DT>(s_cbr[*gbl(it.idx + e)], mo, gv, a.w);
        const uint32_t ub = __float_as_uint(u) & 0x7fffffffu;  // ordered: NaN > inf > finite
        cbits = ub > cbits ? ub : cbits;
    }
    if (cur >= 0 && cbits) gatomic_max(mb + cur, cbits);
}

__global__ void __launch_bounds__(kT) k_mom_finalize(MomBatch bt) {
    const MomItem& it = bt.it[blockIdx.y];
    for (int64_t b = (int64_t)blockIdx.x * kT + threadIdx.x; b < it.nb; b += (int64_t)gridDim.x * kT) {
        it.mag_old[b] = it.mag[b];
        uint32_t bits = 0u;
        drain_shards(it.magbits, it.shards, it.nb, b, [&](uint32_t v) { bits = v > bits ? v : bits; });
        const float m = __uint_as_float(bits);
        it.mag[b] = m;
        it.minv[b] = block_recip(m < kTiny ? kTiny : m);
    }
}

// Requantise one element: x = D(u / m_new) (0 when the block is all zero,
// NaN when its magnitude is), then the nearest or stochastic codeword.
template <int DT>
__device__ __forceinline__ float mom_x(float u, float m_new, float y) {
    float x = 0.0f;
    if (m_new > 0.0f) x = round_dt<DT>(div_by_block(u, m_new < kTiny ? kTiny : m_new, y));
    else if (m_new != m_new) x = u / m_new;  // NaN magnitude: NaN (masked_fill only zeroes mag <= 0)
    return x;
}

// Dense momentum of codeword ni: D(D(c) * m_new), Nesterov D(fma(alpha, g, D(o * beta))).
template <int DT>
__device__ __forceinline__ float mom_out(float cr, float m_new, float gv, const MomArgs& a) {
    float o = round_dt<DT>(cr * m_new);
    if (a.nesterov) o = round_dt<DT>(__builtin_fmaf(a.alpha_d, gv, round_dt<DT>(o * a.beta)));
    return o;
}

template <int DT, bool SR>
__global__ void __launch_bounds__(kT) k_mom_emit(MomArgs a, MomBatch bt) {
    using T = typename Elem<DT>::T;
    const MomItem& it = bt.it[blockIdx.y];
    __shared__ float s_cbr[kCodebookMax];
    __shared__ float s_cb[kCodebookMax];
    __shared__ int16_t s_lut[SR ? kLutEntries + 7 : 1];
    const QTable* qt = a.qt;
    for (int i = threadIdx.x; i < kCodebookMax; i += kT) {
        s_cbr[i] = *gbl(qt->cbr + i);
        s_cb[i] = *gbl(qt->cb + i);
    }
    if constexpr (SR)
        for (int i = threadIdx.x; i < kLutEntries + 7; i += kT) s_lut[i] = *gbl(qt->lut + i);
    __syncthreads();
    uint64_t seed = a.seed;
    if (SR && a.seed_dev != nullptr) seed = (uint64_t)*gbl(a.seed_dev);
    const int k = qt->k;
    const uint32_t kmax = (uint32_t)(k - 1);
    const T* g = static_cast<const T*>(it.g);
    const bool dense = it.gs1 == 1 && it.gs0 == a.C;
    T* out = static_cast<T*>(a.out) + (int64_t)blockIdx.y * a.N;
    const int64_t stride = (int64_t)gridDim.x * kT;
    for (int64_t e = (int64_t)blockIdx.x * kT + threadIdx.x; e < a.N; e += stride) {
        const int64_t b = div_floor(e, it.P, it.invP);
        const float m_old = *gbl(it.mag_old + b);
        const float m_new = *gbl(it.mag + b);
        const float y = *gbl(it.minv + b);
        const int64_t ge = dense ? e : view_offset(e, a.C, a.invC, it.gs0, it.gs1);
        const float gv = to_f32<DT>(*gbl(g + ge));
        const float u = mom_u<DT>(s_cbr[*gbl(it.idx + e)], m_old, gv, a.w);
        const float x = mom_x<DT>(u, m_new, y);
        uint32_t ni;
        if constexpr (SR) ni = quant_stochastic(x, s_cb, s_lut, k, seed, e);
        else ni = quant_nearest(x, qt->bucket, qt->thr, kmax);
        *gbl(it.idx + e) = (uint8_t)ni;
        *gbl(out + e) = from_f32<DT>(mom_out<DT>(s_cbr[ni], m_new, gv, a));
    }
}

// ---------------------------------------------------- fast momentum path
// Contiguous grad, P % 8 == 0, N % 8 == 0, 16-byte aligned grad / momentum,
// 8-byte aligned indices: 8-element chunks never cross a block.  Workgroup w
// of a matrix owns chunks [w * 256 * kMomCpt, ...); thread t takes chunks t,
// t + 256, ... so a wave covers 512 consecutive elements per step.  Every
// chunk's loads are issued before the first chunk's math.
constexpr int kChunk = 8;
constexpr int kMomCpt = 8;
static_assert(kT == kCodebookMax, "one codebook entry per thread");

struct BlkPos {
    int64_t blk, pin;
};

__device__ __forceinline__ BlkPos blk_advance(BlkPos q, int64_t dB, int64_t dP, int64_t P) {
    q.pin += dP;
    q.blk += dB;
    if (q.pin >= P) { q.pin -= P; ++q.blk; }
    return q;
}

// FULL: every chunk of the workgroup lies inside the matrix (all but its last
// workgroup), so no load or store sits behind a branch and each wait names
// exactly the chunk about to be used (a load behind a branch makes the
// compiler assume, at the join, the path with fewer loads in flight, and
// the first wait then drains every chunk's loads).
template <int DT, bool FULL>
__device__ __forceinline__ void mom_max_body(const MomArgs& a, const MomItem& it, float* s_cbr, float cbr_v) {
    using T = typename Elem<DT>::T;
    const T* g = static_cast<const T*>(it.g);
    const uint8_t* idxp = it.idx;
    const float w = a.w;
    const int64_t P = it.P;
    uint32_t* mb = it.magbits + ((int64_t)blockIdx.x % it.shards) * it.nb;
    const int64_t nch = a.N / kChunk;
    const int64_t first = (int64_t)blockIdx.x * (kT * kMomCpt) + threadIdx.x;
    const int64_t F = (int64_t)kT * kChunk;
    const int64_t dB = F / P, dP = F - (F / P) * P;
    BlkPos pos;
    {
        const int64_t e0 = first * kChunk;
        pos.blk = div_floor(e0, P, it.invP);
        pos.pin = e0 - pos.blk * P;
    }
    Raw8<DT> gr[kMomCpt];
    RawIdx8 ir[kMomCpt];
    float mo[kMomCpt];
    int64_t blk[kMomCpt];
#pragma unroll
    for (int i = 0; i < kMomCpt; ++i) {
        const int64_t ch = first + (int64_t)i * kT;
        blk[i] = pos.blk;
        if (FULL || ch < nch) {
            load_raw8<DT>(g + ch * kChunk, gr[i]);
            ir[i] = load_raw_idx8(idxp + ch * kChunk);
            mo[i] = *gbl(it.mag + pos.blk);
        }
        pos = blk_advance(pos, dB, dP, P);
        if constexpr (FULL) __builtin_amdgcn_sched_barrier(0);  // chunk order kept: chunk i's data lands i-th
    }
    s_cbr[threadIdx.x % kCodebookMax] = cbr_v;  // every thread: no branch, so the waits stay exact
    __syncthreads();  // s_cbr
    int64_t wblk = -1;   // wave-uniform running block
    uint32_t wbits = 0u;
#pragma unroll
    for (int i = 0; i < kMomCpt; ++i) {
        const bool valid = FULL || first + (int64_t)i * kT < nch;
        uint32_t m = 0u;
        if (valid) {
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                const float u = mom_u<DT>(s_cbr[raw_idx(ir[i], k)], mo[i], raw_elem<DT>(gr[i], k), w);
                const uint32_t ub = __float_as_uint(u) & 0x7fffffffu;
                m = ub > m ? ub : m;
            }
        }
        // lane 0 holds the wave's lowest chunk, valid whenever any lane is
        const int64_t b0 = __shfl(blk[i], 0, 64);
        if (__all(!valid || blk[i] == b0)) {
            if (b0 != wblk) {
                if (wblk >= 0) {
                    const uint32_t r = wave_max_u63(wbits);
                    if ((threadIdx.x & 63) == 63 && r) gatomic_max(mb + wblk, r);
                }
                wblk = b0;
                wbits = 0u;
            }
            wbits = m > wbits ? m : wbits;
        } else {
            if (wblk >= 0) {
                const uint32_t r = wave_max_u63(wbits);
                if ((threadIdx.x & 63) == 63 && r) gatomic_max(mb + wblk, r);
            }
            wblk = -1;
            wbits = 0u;
            if (valid && m) gatomic_max(mb + blk[i], m);
        }
    }
    if (wblk >= 0) {
        const uint32_t r = wave_max_u63(wbits);
        if ((threadIdx.x & 63) == 63 && r) gatomic_max(mb + wblk, r);
    }
}

template <int DT>
__global__ void __launch_bounds__(kT) k_mom_max_fast(MomArgs a, MomBatch bt) {
    const MomItem& it = bt.it[blockIdx.y];
    __shared__ float s_cbr[kCodebookMax];
    const float cbr_v = *gbl(a.qt->cbr + threadIdx.x % kCodebookMax);  // written to LDS after the chunk loads
    if (((int64_t)blockIdx.x + 1) * (kT * kMomCpt) <= a.N / kChunk) mom_max_body<DT, true>(a, it, s_cbr, cbr_v);
    else mom_max_body<DT, false>(a, it, s_cbr, cbr_v);
}

template <int DT, bool SR>
struct EmitLds {
    uint2 fq[SR ? 1 : kFqEntries];
    float cbr[kCodebookMax];
    float cb[SR ? kCodebookMax : 1];
    int16_t lut[SR ? kLutEntries + 7 : 1];
};

// FULL: as in mom_max_body.  The nearest-rounding table is read into
// registers before the chunks' loads are issued and written to LDS after, so
// the LDS writes wait for the table alone, not for every chunk.
template <int DT, bool SR, bool NEST, bool FULL>
__device__ __forceinline__ void mom_emit_body(const MomArgs& a, const MomItem& it, EmitLds<DT, SR>& lds) {
    using T = typename Elem<DT>::T;
    uint2* s_fq = lds.fq;
    float* s_cbr = lds.cbr;
    float* s_cb = lds.cb;
    int16_t* s_lut = lds.lut;
    const QTable* qt = a.qt;
    constexpr int kFqVec = kFqEntries / 2;                // u32x4 per table
    constexpr int kFqPer = (kFqVec + kT - 1) / kT;
    u32x4 fqv[SR ? 1 : kFqPer];
    if constexpr (!SR) {
        const GX_GLOBAL u32x4* src = gbl(reinterpret_cast<const u32x4*>(qt->fq));
#pragma unroll
        for (int j = 0; j < kFqPer; ++j) {
            const int i = threadIdx.x + j * kT;
            fqv[j] = src[i < kFqVec ? i : kFqVec - 1];  // unconditional: no branch before the chunk loads
        }
    }
    const float cbr_v = *gbl(qt->cbr + threadIdx.x % kCodebookMax);  // unconditional: no branch before the loads
    const T* g = static_cast<const T*>(it.g);
    T* out = static_cast<T*>(a.out) + (int64_t)blockIdx.y * a.N;
    uint8_t* idxp = it.idx;
    const int64_t P = it.P;
    const int64_t nch = a.N / kChunk;
    const int64_t first = (int64_t)blockIdx.x * (kT * kMomCpt) + threadIdx.x;
    const int64_t F = (int64_t)kT * kChunk;
    const int64_t dB = F / P, dP = F - (F / P) * P;
    BlkPos pos;
    {
        const int64_t e0 = first * kChunk;
        pos.blk = div_floor(e0, P, it.invP);
        pos.pin = e0 - pos.blk * P;
    }
    // this thread's chunks: loads first, then the tables into LDS
    Raw8<DT> gr[kMomCpt];
    RawIdx8 ir[kMomCpt];
    float mold[kMomCpt], mnew[kMomCpt], yv[kMomCpt];
#pragma unroll
    for (int i = 0; i < kMomCpt; ++i) {
        const int64_t ch = first + (int64_t)i * kT;
        if (FULL || ch < nch) {
            mold[i] = *gbl(it.mag_old + pos.blk);
            mnew[i] = *gbl(it.mag + pos.blk);
            yv[i] = *gbl(it.minv + pos.blk);
            load_raw8<DT>(g + ch * kChunk, gr[i]);
            ir[i] = load_raw_idx8(idxp + ch * kChunk);
        }
        pos = blk_advance(pos, dB, dP, P);
        if constexpr (FULL) __builtin_amdgcn_sched_barrier(0);  // chunk order kept: chunk i's data lands i-th
    }
    if constexpr (SR) {
        for (int i = threadIdx.x; i < kLutEntries + 7; i += kT) s_lut[i] = *gbl(qt->lut + i);
        if (threadIdx.x < kCodebookMax) s_cb[threadIdx.x] = *gbl(qt->cb + threadIdx.x);
    } else {
        u32x4* dst = reinterpret_cast<u32x4*>(s_fq);
#pragma unroll
        for (int j = 0; j < kFqPer; ++j) {
            const int i = threadIdx.x + j * kT;
            if (j + 1 < kFqPer || i < kFqVec) dst[i] = fqv[j];
        }
    }
    s_cbr[threadIdx.x % kCodebookMax] = cbr_v;  // every thread: no branch, so the waits stay exact
    __syncthreads();
    uint64_t seed = a.seed;
    if (SR && a.seed_dev != nullptr) seed = (uint64_t)*gbl(a.seed_dev);
    const bool fastq = qt->max_cnt <= 1;
    const uint32_t kmax = (uint32_t)(qt->k - 1);
    const float w = a.w;
#pragma unroll
    for (int i = 0; i < kMomCpt; ++i) {
        const int64_t ch = first + (int64_t)i * kT;
        if (!FULL && ch >= nch) break;
        const int64_t e0 = ch * kChunk;
        const float m_new = mnew[i], y = yv[i];
        // x = D(u / m_new) through the block reciprocal (Markstein step) in
        // every lane; a wave where any lane is outside that step's safe range
        // (tiny |u|; zero, subnormal, huge or NaN magnitude: y == 0) redoes the
        // chunk element by element with the guarded helpers
        const float tb = 0x1.00001p-100f * fmaxf(m_new, 1.0f);
        float us[kChunk], xs[kChunk];
        bool bad = y == 0.0f;
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            const float u = mom_u<DT>(s_cbr[raw_idx(ir[i], k)], mold[i], raw_elem<DT>(gr[i], k), w);
            const float q0 = u * y;
            const float r = __builtin_fmaf(-q0, m_new, u);
            us[k] = u;
            xs[k] = round_dt<DT>(__builtin_fmaf(r, y, q0));
            bad = bad || !(fabsf(u) >= tb);
        }
        uint32_t ix[kChunk];
        if (__builtin_expect(__any(bad), 0)) {
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                const float x = mom_x<DT>(us[k], m_new, y);
                if constexpr (SR) ix[k] = quant_stochastic(x, s_cb, s_lut, qt->k, seed, e0 + k);
                else ix[k] = quant_nearest(x, qt->bucket, qt->thr, kmax);
            }
        } else if constexpr (SR) {
#pragma unroll
            for (int k = 0; k < kChunk; ++k) ix[k] = quant_stochastic(xs[k], s_cb, s_lut, qt->k, seed, e0 + k);
        } else if (fastq) {
            // |x| <= 1 here: one bucket entry {threshold, base index} per element
#pragma unroll
            for (int k = 0; k < kChunk; ++k) {
                int b = (int)__builtin_fmaf(xs[k], (float)(kBuckets / 2), (float)(kBuckets / 2));
                b = b < 0 ? 0 : (b > kFqEntries - 1 ? kFqEntries - 1 : b);
                const uint2 e = s_fq[b];
                ix[k] = e.y + (__uint_as_float(e.x) < xs[k] ? 1u : 0u);
            }
        } else {
#pragma unroll
            for (int k = 0; k < kChunk; ++k) ix[k] = quant_nearest(xs[k], qt->bucket, qt->thr, kmax);
        }
        float cr[kChunk], o[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; ++k) cr[k] = s_cbr[ix[k]];
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            o[k] = round_dt<DT>(cr[k] * m_new);
            if constexpr (NEST)
                o[k] = round_dt<DT>(__builtin_fmaf(a.alpha_d, raw_elem<DT>(gr[i], k), round_dt<DT>(o[k] * a.beta)));
        }
        store_idx8(idxp + e0, ix);
        store8<DT>(out + e0, o);
    }
}

// NEST: Nesterov output, fixed per launch so the output loop has no branch
// and its codebook reads issue together.
template <int DT, bool SR, bool NEST>
__global__ void __launch_bounds__(kT) k_mom_emit_fast(MomArgs a, MomBatch bt) {
    __shared__ EmitLds<DT, SR> lds;
    const MomItem& it = bt.it[blockIdx.y];
    if (((int64_t)blockIdx.x + 1) * (kT * kMomCpt) <= a.N / kChunk) mom_emit_body<DT, SR, NEST, true>(a, it, lds);
    else mom_emit_body<DT, SR, NEST, false>(a, it, lds);
}

// ==================================================================
// NT GEMM on bf16 MFMA: D = bf16(alpha * (A B^T) + beta * Cin), optionally
// also Dt = D^T.  A: M x K, B: N x K, both row-major (K contiguous);
// Cin, D: M x N; Dt: N x M.  grid (ceil(N/128), ceil(M/128), batch).
// ==================================================================
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));


struct GemmArgs {
    const uint16_t* A; int64_t lda, sA;   // sA: elements between batch items
    const uint16_t* B; int64_t ldb, sB;
    const uint16_t* C; int64_t ldc, sC;   // epilogue input (nullptr: none)
    uint16_t* D; int64_t ldd, sD;        // nullptr: only the transposed copy is stored
    uint16_t* Dt; int64_t lddt, sDt;      // transposed copy of D (nullptr: none)
    int64_t M, N, K;
    float alpha, beta;
    int vec;                              // 16-byte loads allowed (K, lda, ldb % 8 == 0, aligned)
    int tri;                              // D symmetric (A = B, C symmetric): lower-triangle tiles only,
                                          // each off-diagonal tile also stores its mirror through Dt = D
    int64_t nt_m, nt_n, batch;            // tile grid of the launch (set by gemm_nt)
};

// Workgroup -> (batch item, tile row, tile column), XCD-aware.  The hardware
// deals consecutive workgroups round-robin to the 8 XCDs, each with its own
// L2; renumber them so that every XCD runs one contiguous range of logical
// tiles, and order the tiles of a matrix in bands of kGroupM tile rows,
// column by column inside a band.  The ~32 tiles an XCD holds at once then
// read kGroupM A panels and ~32/kGroupM B panels per K step, instead of
// tiles scattered over the whole grid.  Returns false for the upper-triangle
// tiles of a symmetric product (their values are the lower tiles' mirrors).
constexpr int64_t kXcds = 8;
constexpr int64_t kGroupM = 4;

__device__ __forceinline__ bool gemm_tile(const GemmArgs& g, int64_t& bz, int64_t& tm, int64_t& tn) {
    const int64_t T = g.nt_m * g.nt_n * g.batch;
    const int64_t wid = blockIdx.x;
    const int64_t q = T / kXcds, r = T % kXcds;
    const int64_t x = wid % kXcds;
    const int64_t L = x * q + (x < r ? x : r) + wid / kXcds;
    const int64_t per = g.nt_m * g.nt_n;
    bz = L / per;
    const int64_t t = L - bz * per;
    const int64_t band = g.nt_n * kGroupM;
    const int64_t m0 = (t / band) * kGroupM;
    const int64_t gm = g.nt_m - m0 < kGroupM ? g.nt_m - m0 : kGroupM;
    const int64_t tin = t - (t / band) * band;
    tm = m0 + tin % gm;
    tn = tin / gm;
    return !(g.tri && tn > tm);
}

__device__ __forceinline__ float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t f2bf(float x) { return (uint16_t)f32_to_bf16(x); }

// Load a ROWS x BK tile (rows r0.., k k0..) of a row-major bf16 matrix into
// ROWS*BK/2048 16-byte registers per thread; rows >= R or k >= K read as zero.
template <int ROWS, int BK, bool VEC>
__device__ __forceinline__ void gemm_load_tile(const uint16_t* __restrict__ base, int64_t ld, int64_t R,
                                               int64_t K, int64_t r0, int64_t k0, u32x4* v) {
    constexpr int kCpr = BK / 8;  // 16-byte chunks per row
#pragma unroll
    for (int i = 0; i < ROWS * kCpr / kT; ++i) {
        const int c = threadIdx.x + i * kT;
        const int row = c / kCpr;
        const int kc = (c % kCpr) * 8;
        const int64_t gr = r0 + row;
        const int64_t gk = k0 + kc;
        if constexpr (VEC) {
            // no branch around the load (out-of-range lanes read element 0 and
            // are zeroed after), so the wait counters stay exact
            const bool ok = gr < R && gk < K;
            const u32x4 t = *gbl(reinterpret_cast<const u32x4*>(base + (ok ? gr * ld + gk : 0)));
            v[i] = ok ? t : u32x4{0u, 0u, 0u, 0u};
        } else {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t lo = (gr < R && gk + 2 * j < K) ? *gbl(base + gr * ld + gk + 2 * j) : 0u;
                const uint32_t hi = (gr < R && gk + 2 * j + 1 < K) ? *gbl(base + gr * ld + gk + 2 * j + 1) : 0u;
                w[j] = lo | (hi << 16);
            }
            v[i] = u32x4{w[0], w[1], w[2], w[3]};
        }
    }
}

template <int ROWS, int BK>
__device__ __forceinline__ void gemm_store_tile(uint16_t* __restrict__ s, const u32x4* v) {
    constexpr int kCpr = BK / 8;
    constexpr int kPitch = BK + 8;  // bf16 per LDS row: the pad spreads 16-byte operand reads over banks
#pragma unroll
    for (int i = 0; i < ROWS * kCpr / kT; ++i) {
        const int c = threadIdx.x + i * kT;
        const int row = c / kCpr;
        const int kc = (c % kCpr) * 8;
        *reinterpret_cast<u32x4*>(s + row * kPitch + kc) = v[i];
    }
}

// Epilogue of a (64*WM) x (64*WN) tile through LDS, one 64-row slab at a
// time (wave (wm, wn) holds rows wm*32*WM + 32i .. +32, block i of slab
// wm*WM/2 + i/2): accumulators -> fp32 slab; every thread then forms
// bf16(alpha*acc + beta*C) for 8 consecutive columns (16-byte C loads and D
// stores) and writes the rounded value back; the transposed copy reads the
// slab by columns and stores rows of Dt as 16-byte vectors -- the same bf16
// values as D.
template <int WM, int WN>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& g, const f32x16 (&acc)[WM][WN], float* sOut,
                                              int64_t bz, bool diag, int64_t m0, int64_t n0, int wm, int wn,
                                              int l32, int lhi) {
    constexpr int BN = 64 * WN;
    constexpr int kOutPitch = BN + 1;  // odd: conflict-free column reads
    constexpr int kVecD = 64 * BN / 8 / kT;  // D vectors per thread and slab
    const uint16_t* C = g.C ? g.C + bz * g.sC : nullptr;
    uint16_t* D = g.D ? g.D + bz * g.sD : nullptr;
    uint16_t* Dt = (g.Dt && !(g.tri && diag)) ? g.Dt + bz * g.sDt : nullptr;
    const int tid = threadIdx.x;
#pragma unroll
    for (int h = 0; h < WM; ++h) {
        if (wm == h / (WM / 2)) {
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
                const int i = 2 * (h % (WM / 2)) + ii;
#pragma unroll
                for (int j = 0; j < WN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = ii * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
                        const int col = wn * (32 * WN) + j * 32 + l32;
                        sOut[row * kOutPitch + col] = acc[i][j][r];
                    }
            }
        }
        __syncthreads();
        const int64_t R0 = m0 + h * 64;
#pragma unroll
        for (int k = 0; k < kVecD; ++k) {
            const int v = tid + k * kT;
            const int row = v / (BN / 8), c8 = (v % (BN / 8)) * 8;
            const int64_t gr = R0 + row, gc = n0 + c8;
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = g.alpha * sOut[row * kOutPitch + c8 + e];
            const bool full = gr < g.M && gc + 8 <= g.N;
            if (C != nullptr) {
                const uint16_t* cp = C + gr * g.ldc + gc;
                if (full && (reinterpret_cast<uintptr_t>(cp) & 15) == 0) {
                    const u32x4 cv = *gbl(reinterpret_cast<const u32x4*>(cp));
                    const uint32_t cw[4] = {cv.x, cv.y, cv.z, cv.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        x[e] = __builtin_fmaf(g.beta, bf16f((uint16_t)(cw[e >> 1] >> (16 * (e & 1)))), x[e]);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (gr < g.M && gc + e < g.N) x[e] = __builtin_fmaf(g.beta, bf16f(*gbl(cp + e)), x[e]);
                }
            }
            uint16_t hv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                hv[e] = f2bf(x[e]);
                sOut[row * kOutPitch + c8 + e] = bf16f(hv[e]);
            }
            if (D == nullptr) continue;
            uint16_t* dp = D + gr * g.ldd + gc;
            if (full && (reinterpret_cast<uintptr_t>(dp) & 15) == 0) {
                const u32x4 dv = {(uint32_t)hv[0] | ((uint32_t)hv[1] << 16), (uint32_t)hv[2] | ((uint32_t)hv[3] << 16),
                                  (uint32_t)hv[4] | ((uint32_t)hv[5] << 16), (uint32_t)hv[6] | ((uint32_t)hv[7] << 16)};
                *gbl(reinterpret_cast<u32x4*>(dp)) = dv;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (gr < g.M && gc + e < g.N) *gbl(dp + e) = hv[e];
            }
        }
        if (Dt != nullptr) {
            __syncthreads();
#pragma unroll
            for (int k = 0; k < kVecD; ++k) {
                const int v = tid + k * kT;
                const int cc = v >> 3, r8 = (v & 7) * 8;
                const int64_t gc = n0 + cc, gr = R0 + r8;
                if (gc >= g.N) continue;
                uint16_t hv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) hv[e] = f2bf(sOut[(r8 + e) * kOutPitch + cc]);
                uint16_t* tp = Dt + gc * g.lddt + gr;
                if (gr + 8 <= g.M && (reinterpret_cast<uintptr_t>(tp) & 15) == 0) {
                    const u32x4 tv = {(uint32_t)hv[0] | ((uint32_t)hv[1] << 16), (uint32_t)hv[2] | ((uint32_t)hv[3] << 16),
                                      (uint32_t)hv[4] | ((uint32_t)hv[5] << 16), (uint32_t)hv[6] | ((uint32_t)hv[7] << 16)};
                    *gbl(reinterpret_cast<u32x4*>(tp)) = tv;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (gr + e < g.M) *gbl(tp + e) = hv[e];
                }
            }
        }
        __syncthreads();
    }
}

// Epilogue of a full (64*WM)^2 tile (every row and column in range, C, D and
// Dt 16-byte aligned with leading dimensions and batch strides multiples of 8):
// the same arithmetic as gemm_epilogue, with every global access unconditional
// and the next slab's C rows loaded before this slab's barrier.  The fp32 slab
// has rows of 64*WM floats whose 16-byte groups are XOR-swizzled by
// (row >> 3) & 7: the accumulator writes (16 or 32 consecutive columns per
// lane group), the row pass (a thread takes 16-byte groups q and q + 8*WM of
// a row, 4 + 4 columns, with 8-byte C loads and D stores) and the transposed
// copy's column reads (8 rows per thread) each spread over the banks.
// put(h) stores the calling wave's accumulators of 64-row slab h at
// sOut[epi_at(row - 64 h, col)] (the MFMA shape fixes which lane holds what).
template <int WM>
__device__ __forceinline__ int epi_at(int row, int col) {
    return row * (64 * WM) + 4 * ((col >> 2) ^ ((row >> 3) & 7)) + (col & 3);
}

// Slab h of a (64*WM)^2 tile held as 32 x 32 mfma blocks: wave (wm, wn) holds
// rows wm*32*WM + 32i.., columns wn*32*WM + 32j..; lane (l32, lhi) element r
// of a block sits at row (r >> 2) * 8 + lhi * 4 + (r & 3), column l32.
template <int WM>
__device__ __forceinline__ void put_acc32(const f32x16 (&acc)[WM][WM], float* sOut, int h, int wm, int wn, int l32,
                                          int lhi) {
    if (wm != h / (WM / 2)) return;
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int i = 2 * (h % (WM / 2)) + ii;
#pragma unroll
        for (int j = 0; j < WM; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = ii * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
                const int col = wn * (32 * WM) + j * 32 + l32;
                sOut[epi_at<WM>(row, col)] = acc[i][j][r];
            }
    }
}

template <int WM, typename Put>
__device__ __forceinline__ void gemm_epilogue_full(const GemmArgs& g, Put&& put, float* sOut, int64_t bz, bool diag,
                                                   int64_t m0, int64_t n0) {
    constexpr int BN = 64 * WM;
    constexpr int kHalfG = BN / 8;            // 16-byte groups per half row
    constexpr int kVecD = 64 * BN / 8 / kT;   // 8-element pieces per thread and slab
    const uint16_t* C = g.C ? g.C + bz * g.sC : nullptr;
    uint16_t* D = g.D ? g.D + bz * g.sD : nullptr;
    uint16_t* Dt = (g.Dt && !(g.tri && diag)) ? g.Dt + bz * g.sDt : nullptr;
    const int tid = threadIdx.x;
    u32x2 cpf[2][kVecD][2];
    auto fetch = [&](int h, u32x2 (&dst)[kVecD][2]) {
#pragma unroll
        for (int k = 0; k < kVecD; ++k) {
            const int v = tid + k * kT;
            const int row = v / kHalfG, q = v % kHalfG;
            const uint16_t* cp = C + (m0 + h * 64 + row) * g.ldc + n0 + 4 * q;
            dst[k][0] = __builtin_nontemporal_load(gbl(reinterpret_cast<const u32x2*>(cp)));
            dst[k][1] = __builtin_nontemporal_load(gbl(reinterpret_cast<const u32x2*>(cp + BN / 2)));
        }
    };
    if (C != nullptr) fetch(0, cpf[0]);
#pragma unroll
    for (int h = 0; h < WM; ++h) {
        put(h);
        if (C != nullptr && h + 1 < WM) fetch(h + 1, cpf[(h + 1) & 1]);
        __syncthreads();
        const int64_t R0 = m0 + h * 64;
#pragma unroll
        for (int k = 0; k < kVecD; ++k) {
            const int v = tid + k * kT;
            const int row = v / kHalfG, q = v % kHalfG;
            f32x4* s0 = reinterpret_cast<f32x4*>(sOut + epi_at<WM>(row, 4 * q));
            f32x4* s1 = reinterpret_cast<f32x4*>(sOut + epi_at<WM>(row, 4 * q + BN / 2));
            const f32x4 a0 = *s0, a1 = *s1;
            float x[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = g.alpha * x[e];
            if (C != nullptr) {
                const uint32_t cw[4] = {cpf[h & 1][k][0].x, cpf[h & 1][k][0].y, cpf[h & 1][k][1].x,
                                        cpf[h & 1][k][1].y};
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    x[e] = __builtin_fmaf(g.beta, bf16f((uint16_t)(cw[e >> 1] >> (16 * (e & 1)))), x[e]);
            }
            uint16_t hv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[e] = f2bf(x[e]);
            *s0 = f32x4{bf16f(hv[0]), bf16f(hv[1]), bf16f(hv[2]), bf16f(hv[3])};
            *s1 = f32x4{bf16f(hv[4]), bf16f(hv[5]), bf16f(hv[6]), bf16f(hv[7])};
            if (D != nullptr) {
                uint16_t* dp = D + (R0 + row) * g.ldd + n0 + 4 * q;
                const u32x2 d0 = {(uint32_t)hv[0] | ((uint32_t)hv[1] << 16), (uint32_t)hv[2] | ((uint32_t)hv[3] << 16)};
                const u32x2 d1 = {(uint32_t)hv[4] | ((uint32_t)hv[5] << 16), (uint32_t)hv[6] | ((uint32_t)hv[7] << 16)};
                *gbl(reinterpret_cast<u32x2*>(dp)) = d0;
                *gbl(reinterpret_cast<u32x2*>(dp + BN / 2)) = d1;
            }
        }
        if (Dt != nullptr) {
            __syncthreads();
#pragma unroll
            for (int k = 0; k < kVecD; ++k) {
                const int v = tid + k * kT;
                const int cc = v >> 3, r8 = (v & 7) * 8;
                uint16_t hv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) hv[e] = f2bf(sOut[epi_at<WM>(r8 + e, cc)]);
                const u32x4 tv = {(uint32_t)hv[0] | ((uint32_t)hv[1] << 16), (uint32_t)hv[2] | ((uint32_t)hv[3] << 16),
                                  (uint32_t)hv[4] | ((uint32_t)hv[5] << 16), (uint32_t)hv[6] | ((uint32_t)hv[7] << 16)};
                *gbl(reinterpret_cast<u32x4*>(Dt + (n0 + cc) * g.lddt + R0 + r8)) = tv;
            }
        }
        __syncthreads();
    }
}

__host__ __device__ inline bool epi_aligned(const void* p, int64_t ld, int64_t s) {
    return p == nullptr || ((reinterpret_cast<uintptr_t>(p) | (uintptr_t)(ld * 2) | (uintptr_t)(s * 2)) & 15) == 0;
}

// D = alpha * A B^T + beta * C (A [M x K], B [N x K], C and D [M x N], all
// row-major bf16, fp32 accumulation; optional transposed copy Dt = D^T).
// Workgroup tile (64*WM) x (64*WN): 2 x 2 waves, each (32*WM) x (32*WN) as
// WM x WN blocks of mfma_f32_32x32x16_bf16, so each wave reads WM + WN
// operand fragments from LDS per WM*WN MFMAs.  K in steps of BK, LDS double
// buffered, the next step's global loads in flight during this step's MFMAs.
template <int WM, int WN, int BK, bool VEC>
__global__ void __launch_bounds__(kT) k_gemm_nt(GemmArgs g) {
    constexpr int BM = 64 * WM, BN = 64 * WN;
    constexpr int kPitch = BK + 8;
    constexpr int kOutPitch = BN + 1;  // fp32 epilogue tile: odd pitch, conflict-free column reads
    constexpr size_t kLoopBytes = sizeof(uint16_t) * 2 * (size_t)(BM + BN) * kPitch;
    constexpr size_t kOutBytes = sizeof(float) * 64 * (size_t)kOutPitch;
    __shared__ __attribute__((aligned(16))) unsigned char smem[kLoopBytes > kOutBytes ? kLoopBytes : kOutBytes];
    uint16_t (*sA)[BM * kPitch] = reinterpret_cast<uint16_t (*)[BM * kPitch]>(smem);
    uint16_t (*sB)[BN * kPitch] = reinterpret_cast<uint16_t (*)[BN * kPitch]>(smem + sizeof(uint16_t) * 2 * BM * kPitch);
    float* sOut = reinterpret_cast<float*>(smem);
    int64_t bz, tm, tn;
    if (!gemm_tile(g, bz, tm, tn)) return;  // upper triangle: the mirror of a lower tile
    const uint16_t* A = g.A + bz * g.sA;
    const uint16_t* B = g.B + bz * g.sB;
    const int64_t m0 = tm * BM;
    const int64_t n0 = tn * BN;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, lhi = lane >> 5;

    f32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int64_t nk = cdiv(g.K, BK);
    constexpr int kRa = BM * BK / 8 / kT, kRb = BN * BK / 8 / kT;
    auto mma_step = [&](const uint16_t* a_s, const uint16_t* b_s) {
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            bf16x8 av[WM], bv[WN];
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                const int row = wm * (32 * WM) + i * 32 + l32;
                av[i] = *reinterpret_cast<const bf16x8*>(a_s + row * kPitch + ks * 16 + lhi * 8);
            }
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const int col = wn * (32 * WN) + j * 32 + l32;
                bv[j] = *reinterpret_cast<const bf16x8*>(b_s + col * kPitch + ks * 16 + lhi * 8);
            }
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
    };
    // one register stage: step kt+1's loads fly during step kt's MFMAs
    u32x4 ra[kRa], rb[kRb];
    gemm_load_tile<BM, BK, VEC>(A, g.lda, g.M, g.K, m0, 0, ra);
    gemm_load_tile<BN, BK, VEC>(B, g.ldb, g.N, g.K, n0, 0, rb);
    gemm_store_tile<BM, BK>(sA[0], ra);
    gemm_store_tile<BN, BK>(sB[0], rb);
    __syncthreads();
    for (int64_t kt = 0; kt < nk; ++kt) {
        const int cur = (int)(kt & 1);
        if (kt + 1 < nk) {
            gemm_load_tile<BM, BK, VEC>(A, g.lda, g.M, g.K, m0, (kt + 1) * BK, ra);
            gemm_load_tile<BN, BK, VEC>(B, g.ldb, g.N, g.K, n0, (kt + 1) * BK, rb);
        }
        mma_step(sA[cur], sB[cur]);
        if (kt + 1 < nk) {
            gemm_store_tile<BM, BK>(sA[cur ^ 1], ra);
            gemm_store_tile<BN, BK>(sB[cur ^ 1], rb);
        }
        __syncthreads();
    }

    gemm_epilogue<WM, WN>(g, acc, sOut, bz, tm == tn, m0, n0, wm, wn, l32, lhi);
}

// Direct-to-LDS variant (K a multiple of BK, 16-byte aligned rows): the
// operand tiles go from HBM straight into LDS (global_load_lds_dwordx4, no
// staging registers, no LDS store instructions).  Tile 128 x 128, K steps of
// BK, an S-stage LDS ring: step kt+S-1's loads are issued as step kt's MFMAs
// start, and a step waits only for its own loads.  A tile row (BK bf16 =
// BK/8 chunks of 16 bytes) keeps chunk c in slot c ^ f(row), f(row) =
// (row >> 1) & 7 (BK 64) or (row >> 2) & 3 (BK 32): the 32 rows one MFMA
// operand read touches then spread over all 64 banks.  Each load instruction
// fills 1 KB of LDS; its lanes fetch the global chunks their slots hold.
// Rows past M / N read a clamped valid row (their outputs are not stored).
template <int BK>
__device__ __forceinline__ int dl_slot(int row, int c) {
    if constexpr (BK == 64) return c ^ ((row >> 1) & 7);
    else return c ^ ((row >> 2) & 3);
}

template <int TILE, int BK>
__device__ __forceinline__ void dl_load_stage(const uint16_t* __restrict__ A, int64_t lda, int64_t M,
                                              const uint16_t* __restrict__ B, int64_t ldb, int64_t N,
                                              int64_t m0, int64_t n0, int64_t k0, uint16_t* stage) {
    constexpr int kCpr = BK / 8;             // chunks per row
    constexpr int kRpi = 64 / kCpr;          // rows per 1 KB instruction
    constexpr int kIpt = TILE / kRpi;        // instructions per operand tile
    constexpr int kIpw = 2 * kIpt / (kT / 64);  // instructions per wave
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int q = 0; q < kIpw; ++q) {
        const int inst = wave * kIpw + q;
        const bool is_b = inst >= kIpt;
        const int ti = is_b ? inst - kIpt : inst;
        const int row = ti * kRpi + lane / kCpr;  // tile row
        const int slot = lane % kCpr;
        const int chunk = dl_slot<BK>(row, slot);  // the swizzle is an involution
        const uint16_t* base = is_b ? B : A;
        const int64_t ld = is_b ? ldb : lda;
        const int64_t lim = is_b ? N : M;
        int64_t gr = (is_b ? n0 : m0) + row;
        gr = gr < lim ? gr : lim - 1;
        const uint16_t* src = base + gr * ld + k0 + chunk * 8;
        uint16_t* dst = stage + (is_b ? TILE * BK : 0) + ti * kRpi * BK;  // wave-uniform
        __builtin_amdgcn_global_load_lds((const GX_GLOBAL void*)src, (__attribute__((address_space(3))) void*)dst, 16,
                                         0, 0);
    }
}

// WM x WM blocks of 32 x 32 per wave, 2 x 2 waves: tile (64*WM)^2.
template <int WM, int BK, int S>
__global__ void __launch_bounds__(kT) k_gemm_dl(GemmArgs g) {
    static_assert(S == 2, "two-stage ring: the loop waits for every load in flight at each step");
    int64_t bz, tm, tn;
    if (!gemm_tile(g, bz, tm, tn)) return;  // upper triangle: the mirror of a lower tile
    constexpr int TILE = 64 * WM;
    constexpr int kStage = 2 * TILE * BK;                        // bf16 per stage: A then B
    constexpr int kEpi = 2 * 64 * (TILE + 1);                    // the epilogue's fp32 slab, in bf16 units
    constexpr int kSmem = S * kStage > kEpi ? S * kStage : kEpi;
    __shared__ __attribute__((aligned(16))) uint16_t smem[kSmem];
    const uint16_t* A = g.A + bz * g.sA;
    const uint16_t* B = g.B + bz * g.sB;
    const int64_t m0 = tm * TILE;
    const int64_t n0 = tn * TILE;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, lhi = lane >> 5;
    f32x16 acc[WM][WM];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WM; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    const int64_t nk = g.K / BK;
#pragma unroll
    for (int st = 0; st < S - 1; ++st)
        if (st < nk) dl_load_stage<TILE, BK>(A, g.lda, g.M, B, g.ldb, g.N, m0, n0, st * BK, smem + st * kStage);
    for (int64_t kt = 0; kt < nk; ++kt) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): step kt's loads, the only ones in flight
        __syncthreads();  // every wave's loads of step kt landed; step kt-1's buffer is free
        if (kt + S - 1 < nk)
            dl_load_stage<TILE, BK>(A, g.lda, g.M, B, g.ldb, g.N, m0, n0, (kt + S - 1) * BK,
                                    smem + ((kt + S - 1) % S) * kStage);
        const uint16_t* a_s = smem + (kt % S) * kStage;
        const uint16_t* b_s = a_s + TILE * BK;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int c = ks * 2 + lhi;
            bf16x8 av[WM], bv[WM];
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                const int row = wm * (32 * WM) + i * 32 + l32;
                av[i] = *reinterpret_cast<const bf16x8*>(a_s + row * BK + dl_slot<BK>(row, c) * 8);
            }
#pragma unroll
            for (int j = 0; j < WM; ++j) {
                const int row = wn * (32 * WM) + j * 32 + l32;
                bv[j] = *reinterpret_cast<const bf16x8*>(b_s + row * BK + dl_slot<BK>(row, c) * 8);
            }
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
    }
    __syncthreads();
    if (m0 + TILE <= g.M && n0 + TILE <= g.N && epi_aligned(g.C, g.ldc, g.sC) && epi_aligned(g.D, g.ldd, g.sD) &&
        epi_aligned(g.Dt, g.lddt, g.sDt)) {
        float* sOut = reinterpret_cast<float*>(smem);
        gemm_epilogue_full<WM>(g, [&](int h) { put_acc32<WM>(acc, sOut, h, wm, wn, l32, lhi); }, sOut, bz, tm == tn,
                               m0, n0);
    } else
        gemm_epilogue<WM, WM>(g, acc, reinterpret_cast<float*>(smem), bz, tm == tn, m0, n0, wm, wn, l32, lhi);
}

// One 1 KB direct-to-LDS load instruction (number q of this wave's share of
// a stage) of the same layout as dl_load_stage.
template <int TILE, int BK>
__device__ __forceinline__ void dl_load_one(const uint16_t* __restrict__ A, int64_t lda, int64_t M,
                                            const uint16_t* __restrict__ B, int64_t ldb, int64_t N,
                                            int64_t m0, int64_t n0, int64_t k0, uint16_t* stage, int q) {
    constexpr int kCpr = BK / 8;
    constexpr int kRpi = 64 / kCpr;
    constexpr int kIpt = TILE / kRpi;
    constexpr int kIpw = 2 * kIpt / (kT / 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int inst = wave * kIpw + q;
    const bool is_b = inst >= kIpt;
    const int ti = is_b ? inst - kIpt : inst;
    const int row = ti * kRpi + lane / kCpr;
    const int chunk = dl_slot<BK>(row, lane % kCpr);
    const uint16_t* base = is_b ? B : A;
    const int64_t ld = is_b ? ldb : lda;
    const int64_t lim = is_b ? N : M;
    int64_t gr = (is_b ? n0 : m0) + row;
    gr = gr < lim ? gr : lim - 1;
    const uint16_t* src = base + gr * ld + k0 + chunk * 8;
    uint16_t* dst = stage + (is_b ? TILE * BK : 0) + ti * kRpi * BK;  // wave-uniform
    __builtin_amdgcn_global_load_lds((const GX_GLOBAL void*)src, (__attribute__((address_space(3))) void*)dst, 16,
                                     0, 0);
}

// 256 x 256 tile for large grids whose tiles are not all full (full tiles
// take k_gemm_big16; one workgroup per CU: 128 KB of LDS, 256 fp32
// accumulators per lane), K steps of 64 in a two-stage LDS ring.  Each
// wave owns 128 x 128 as 4 x 4 blocks of mfma_f32_32x32x16_bf16: per 16-wide
// K sub-step, 16 MFMAs against 8 operand fragments, so the LDS reads per MFMA
// are half those of the 128 x 128 tile.  The instruction order inside a step
// is fixed with scheduling fences, one MFMA at a time: between consecutive
// MFMAs go the next sub-step's operand reads (fragments double-buffered in
// registers; B fragments first, since the next sub-step's first row needs
// all four, then A in row order) and, in the first two sub-steps, the next
// stage's 16 direct-to-LDS tile loads (one after the first and one after
// the last MFMA of each row), so reads and loads issue in the gaps between
// MFMAs instead of in blocks ahead of them.  The last step reloads its own K range into the idle
// buffer (never read) so every step issues the same loads without a branch.

__global__ void __launch_bounds__(kT) k_gemm_big(GemmArgs g) {
    constexpr int WM = 4, TILE = 256, BK = 64, KS = BK / 16;
    int64_t bz, tm, tn;
    if (!gemm_tile(g, bz, tm, tn)) return;  // upper triangle: the mirror of a lower tile
    constexpr int kStage = 2 * TILE * BK;
    constexpr int kIpw = 2 * (TILE * BK * 2 / 1024) / (kT / 64);  // 16 load instructions per wave and stage
    constexpr int kLoadKs = 2;
    constexpr int kLpr = kIpw / (4 * kLoadKs);
    static_assert(kLpr * 4 * kLoadKs == kIpw, "the loads spread evenly over the MFMA rows");
    constexpr int kEpi = 2 * 64 * (TILE + 1);
    constexpr int kSmem = 2 * kStage > kEpi ? 2 * kStage : kEpi;
    __shared__ __attribute__((aligned(16))) uint16_t smem[kSmem];
    const uint16_t* A = g.A + bz * g.sA;
    const uint16_t* B = g.B + bz * g.sB;
    const int64_t m0 = tm * TILE;
    const int64_t n0 = tn * TILE;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, lhi = lane >> 5;
    f32x16 acc[WM][WM];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WM; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    const int64_t nk = g.K / BK;
#pragma unroll
    for (int q = 0; q < kIpw; ++q) dl_load_one<TILE, BK>(A, g.lda, g.M, B, g.ldb, g.N, m0, n0, 0, smem, q);
    auto rd = [&](const uint16_t* t, int half, int idx, int ks) {
        const int row = half * (32 * WM) + idx * 32 + l32;
        return *reinterpret_cast<const bf16x8*>(t + row * BK + dl_slot<BK>(row, ks * 2 + lhi) * 8);
    };
    for (int64_t kt = 0; kt < nk; ++kt) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this step's loads, the only ones in flight
        __syncthreads();                     // ... landed for every wave; the other buffer is idle
        const uint16_t* a_s = smem + (kt & 1) * kStage;
        const uint16_t* b_s = a_s + TILE * BK;
        uint16_t* nxt = smem + ((kt + 1) & 1) * kStage;
        const int64_t kn = (kt + 1 < nk ? kt + 1 : kt) * BK;
        bf16x8 av[2][WM], bv[2][WM];
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            av[0][i] = rd(a_s, wm, i, 0);
            bv[0][i] = rd(b_s, wn, i, 0);
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
            for (int i = 0; i < WM; ++i) {
#pragma unroll
                for (int j = 0; j < WM; ++j) {
                    __builtin_amdgcn_sched_barrier(0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[ks & 1][i], bv[ks & 1][j], acc[i][j], 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    if (ks < kLoadKs) {
                        if (j == 0 || j == 3)
                            dl_load_one<TILE, BK>(A, g.lda, g.M, B, g.ldb, g.N, m0, n0, kn, nxt,
                                                  (ks * 4 + i) * kLpr + (j == 3));
                    }
                    // next sub-step's fragments: B first (row 0 needs all of them), then A in row order
                    const int slot = ks < kLoadKs ? j - 1 : j;  // reads in slots 1, 2 (0, 1 without loads)
                    if (ks + 1 < KS && slot >= 0 && slot < 2) {
                        const int f = 2 * i + slot;  // 0..7
                        if (f < 4) bv[(ks + 1) & 1][f] = rd(b_s, wn, f, ks + 1);
                        else av[(ks + 1) & 1][f - 4] = rd(a_s, wm, f - 4, ks + 1);
                    }
                }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // the last (discarded) reload lands before the epilogue reuses LDS
    __syncthreads();
    const bool full = m0 + TILE <= g.M && n0 + TILE <= g.N && epi_aligned(g.C, g.ldc, g.sC) &&
                      epi_aligned(g.D, g.ldd, g.sD) && epi_aligned(g.Dt, g.lddt, g.sDt);
    if (full) {
        float* sOut = reinterpret_cast<float*>(smem);
        gemm_epilogue_full<WM>(g, [&](int h) { put_acc32<WM>(acc, sOut, h, wm, wn, l32, lhi); }, sOut, bz, tm == tn,
                               m0, n0);
    } else
        gemm_epilogue<WM, WM>(g, acc, reinterpret_cast<float*>(smem), bz, tm == tn, m0, n0, wm, wn, l32, lhi);
}

// One 1 KB direct-to-LDS load of a full tile (every row in range, no clamp),
// the layout of dl_load_one: the instruction's first row at column k0 is a
// wave-uniform address, each lane adds its offset (its row within the
// instruction and the chunk its slot holds).
template <int TILE, int BK>
__device__ __forceinline__ void dl_load_full(const uint16_t* __restrict__ A, int64_t lda,
                                             const uint16_t* __restrict__ B, int64_t ldb, int64_t m0, int64_t n0,
                                             int64_t k0, uint16_t* stage, int wave, int q) {
    constexpr int kCpr = BK / 8;
    constexpr int kRpi = 64 / kCpr;
    constexpr int kIpt = TILE / kRpi;
    constexpr int kIpw = 2 * kIpt / (kT / 64);
    const int lane = threadIdx.x & 63;
    const int inst = wave * kIpw + q;
    const bool is_b = inst >= kIpt;
    const int ti = is_b ? inst - kIpt : inst;
    const int64_t ld = is_b ? ldb : lda;
    const unsigned char* ubase =
        reinterpret_cast<const unsigned char*>((is_b ? B : A) + ((is_b ? n0 : m0) + ti * kRpi) * ld + k0);
    const int rr = lane / kCpr;
    const int64_t voff = (int64_t)rr * ld * 2 + (int64_t)dl_slot<BK>(ti * kRpi + rr, lane % kCpr) * 16;
    uint16_t* dst = stage + (is_b ? TILE * BK : 0) + ti * kRpi * BK;  // wave-uniform
    __builtin_amdgcn_global_load_lds((const GX_GLOBAL void*)(ubase + voff),
                                     (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}

// Slab h of a 256 x 256 tile held as 16 x 16 mfma blocks: wave (wm, wn) holds
// rows wm*128 + 16i.., columns wn*128 + 16j..; block (i, j) is floats
// 4(j & 3) .. +3 of acc4[i][j >> 2], lane l's element r at row 4(l >> 4) + r,
// column l & 15.
__device__ __forceinline__ void put_acc16(const f32x16 (&acc4)[8][2], float* sOut, int h, int wm, int wn,
                                          int lane) {
    if (wm != h / 2) return;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
        const int i = 4 * (h % 2) + ii;
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = ii * 16 + (lane >> 4) * 4 + r;
                const int col = wn * 128 + j * 16 + (lane & 15);
                sOut[epi_at<4>(row, col)] = acc4[i][j >> 2][4 * (j & 3) + r];
            }
    }
}

// 256 x 256 full tiles (M and N multiples of 256, epilogue operands aligned
// as gemm_epilogue_full needs) on mfma_f32_16x16x32_bf16, which runs at a
// higher clock than the 32x32x16 form for the same work (measured: ~2.05
// against ~1.81 GHz with the MFMA pipes ~94% busy).  One workgroup per CU, K
// steps of 64 in a two-stage direct-to-LDS ring.  Each wave's 128 x 128 is
// 8 x 8 blocks of 16 x 16; a 32-wide K sub-step is 64 MFMAs against 16
// operand fragments, two sub-steps per K step.  The step's barrier sits
// between its sub-steps: sub-step 0 reads sub-step 1's fragments (the last
// reads of this stage); after the barrier (every wave's reads of this stage
// returned, the next stage landed) sub-step 1 issues the stage-after-next's
// loads into this stage's buffer and reads the next stage's sub-step 0
// fragments, so no step opens with an operand wait and the loads still lead
// by one K step.  The accumulators live as four 16 x 16 blocks per 16-float
// vector: held as 64 separate 4-float values the compiler's register
// allocation spilled.
__global__ void __launch_bounds__(kT) k_gemm_big16(GemmArgs g) {
    constexpr int TILE = 256, BK = 64;
    int64_t bz, tm, tn;
    if (!gemm_tile(g, bz, tm, tn)) return;  // upper triangle: the mirror of a lower tile
    constexpr int kStage = 2 * TILE * BK;
    constexpr int kIpw = 2 * (TILE * BK * 2 / 1024) / (kT / 64);  // 16 load instructions per wave and stage
    constexpr int kEpi = 2 * 64 * (TILE + 1);
    constexpr int kSmem = 2 * kStage > kEpi ? 2 * kStage : kEpi;
    __shared__ __attribute__((aligned(16))) uint16_t smem[kSmem];
    const uint16_t* A = g.A + bz * g.sA;
    const uint16_t* B = g.B + bz * g.sB;
    const int64_t m0 = tm * TILE;
    const int64_t n0 = tn * TILE;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int l16 = lane & 15, lq = lane >> 4;
    f32x16 acc4[8][2];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc4[i][j][r] = 0.0f;
    const int64_t nk = g.K / BK;
#pragma unroll
    for (int q = 0; q < kIpw; ++q) dl_load_full<TILE, BK>(A, g.lda, B, g.ldb, m0, n0, 0, smem, wave, q);
    // fragment idx (16 rows) of a wave half at 16-byte chunk c of the K row
    auto rd = [&](const uint16_t* t, int half, int idx, int c) {
        const int row = half * 128 + idx * 16 + l16;
        return *reinterpret_cast<const bf16x8*>(t + row * BK + dl_slot<BK>(row, c) * 8);
    };
    auto mma = [&](int i, int j, const bf16x8& a, const bf16x8& b) {
        f32x4 c;
#pragma unroll
        for (int r = 0; r < 4; ++r) c[r] = acc4[i][j >> 2][4 * (j & 3) + r];
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc4[i][j >> 2][4 * (j & 3) + r] = c[r];
    };
    // stage 0 landed for every wave; stage 1 (a reload of stage 0 when nk is
    // 1, never read) in flight; sub-step 0 fragments of stage 0 read
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    {
        const int64_t k1 = (nk > 1 ? 1 : 0) * BK;
#pragma unroll
        for (int q = 0; q < kIpw; ++q) dl_load_full<TILE, BK>(A, g.lda, B, g.ldb, m0, n0, k1, smem + kStage, wave, q);
    }
    bf16x8 f0a[8], f0b[8], f1a[8], f1b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        f0b[i] = rd(smem + TILE * BK, wn, i, lq);
        f0a[i] = rd(smem, wm, i, lq);
    }
#pragma unroll 1
    for (int64_t kt = 0; kt < nk; ++kt) {
        const uint16_t* a_s = smem + (kt & 1) * kStage;
        const uint16_t* b_s = a_s + TILE * BK;
        const uint16_t* a_n = smem + ((kt + 1) & 1) * kStage;
        const uint16_t* b_n = a_n + TILE * BK;
        uint16_t* nxt = smem + (kt & 1) * kStage;
        const int64_t k2 = (kt + 2 < nk ? kt + 2 : nk - 1) * BK;  // past the end: a reload, never read
        // sub-step 0: MFMAs on f0; sub-step 1's fragments (B first) read in rows 0-5
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                __builtin_amdgcn_sched_barrier(0);
                mma(i, j, f0a[i], f0b[j]);
                __builtin_amdgcn_sched_barrier(0);
                const int f = 3 * i + (j == 1 ? 0 : j == 3 ? 1 : 2);
                if ((j == 1 || j == 3 || j == 5) && f < 16) {
                    if (f < 8) f1b[f] = rd(b_s, wn, f, 4 + lq);
                    else f1a[f - 8] = rd(a_s, wm, f - 8, 4 + lq);
                }
            }
        }
        __syncthreads();  // every wave's reads of stage kt returned; stage kt+1 landed (vmcnt(0))
        // sub-step 1: MFMAs on f1; the stage-after-next's loads into stage kt's
        // buffer (two per row) and the next stage's sub-step 0 fragments (rows 0-5)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                __builtin_amdgcn_sched_barrier(0);
                mma(i, j, f1a[i], f1b[j]);
                __builtin_amdgcn_sched_barrier(0);
                if (j == 0 || j == 4) dl_load_full<TILE, BK>(A, g.lda, B, g.ldb, m0, n0, k2, nxt, wave, 2 * i + (j == 4));
                const int f = 3 * i + (j == 1 ? 0 : j == 3 ? 1 : 2);
                if ((j == 1 || j == 3 || j == 5) && f < 16) {
                    if (f < 8) f0b[f] = rd(b_n, wn, f, lq);
                    else f0a[f - 8] = rd(a_n, wm, f - 8, lq);
                }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // the last (discarded) loads land before the epilogue reuses LDS
    __syncthreads();
    float* sOut = reinterpret_cast<float*>(smem);
    gemm_epilogue_full<4>(g, [&](int h) { put_acc16(acc4, sOut, h, wm, wn, lane); }, sOut, bz, tm == tn, m0, n0);
}

static int gemm_nt(const GemmArgs& g, int64_t batch, hipStream_t s) {
    if (g.M <= 0 || g.N <= 0 || batch <= 0) return GEFENX_OK;
    if (g.K <= 0) return set_error(GEFENX_EINVAL, "newton-schulz gemm: K must be positive");
    GemmArgs a = g;
    const auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    a.vec = (g.K % 8 == 0) && (g.lda % 8 == 0) && (g.ldb % 8 == 0) && (g.sA % 8 == 0) && (g.sB % 8 == 0) &&
            al(g.A) && al(g.B);
    if (g.tri && (g.M != g.N || g.Dt != g.D || g.lddt != g.ldd || g.sDt != g.sD))
        return set_error(GEFENX_EINVAL, "newton-schulz gemm: symmetric mode needs a square D mirrored into itself");
    // direct-to-LDS when K is a multiple of 64 and the operands are 16-byte
    // aligned (every Newton-Schulz product of 64-multiple shapes), the
    // register-staged kernel otherwise.  Direct-to-LDS products whose 256 x
    // 256 tiles (lower triangle only when symmetric) fill the 256 CUs at least
    // once take a 256 x 256 kernel (16x16x32 MFMAs when every tile is full,
    // the 32x32x16 kernel with its clamped loads and guarded epilogue
    // otherwise); smaller grids keep 128 x 128 tiles (four times the
    // workgroups).
    const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool dl = a.vec && g.K % 64 == 0 && al16(g.A) && al16(g.B);
    constexpr int bm = 128, bn = 128;
    if (cdiv(g.M, bm) * cdiv(g.N, bn) * batch > 2147483647LL)
        return set_error(GEFENX_EINVAL, "newton-schulz gemm: %lld x %lld x batch %lld exceeds the launch grid",
                         (long long)g.M, (long long)g.N, (long long)batch);
    a.batch = batch;
    const int64_t t256m = cdiv(g.M, 256), t256n = cdiv(g.N, 256);
    const int64_t big_tiles = (g.tri ? t256m * (t256m + 1) / 2 : t256m * t256n) * batch;
    if (dl && big_tiles >= 256) {
        a.nt_m = t256m;
        a.nt_n = t256n;
        const bool full = g.M % 256 == 0 && g.N % 256 == 0 && epi_aligned(g.C, g.ldc, g.sC) &&
                          epi_aligned(g.D, g.ldd, g.sD) && epi_aligned(g.Dt, g.lddt, g.sDt);
        if (full) hipLaunchKernelGGL(k_gemm_big16, dim3((unsigned)(t256m * t256n * batch)), dim3(kT), 0, s, a);
        else hipLaunchKernelGGL(k_gemm_big, dim3((unsigned)(t256m * t256n * batch)), dim3(kT), 0, s, a);
        return launch_check("newton-schulz gemm");
    }
    a.nt_m = cdiv(g.M, bm);
    a.nt_n = cdiv(g.N, bn);
    const dim3 grid((unsigned)(a.nt_m * a.nt_n * batch));
    if (dl)
        hipLaunchKernelGGL((k_gemm_dl<2, 64, 2>), grid, dim3(kT), 0, s, a);
    else if (a.vec)
        hipLaunchKernelGGL((k_gemm_nt<2, 2, 64, true>), grid, dim3(kT), 0, s, a);
    else
        hipLaunchKernelGGL((k_gemm_nt<2, 2, 64, false>), grid, dim3(kT), 0, s, a);
    return launch_check("newton-schulz gemm");
}

// ==================================================================
// Newton-Schulz driver kernels
// ==================================================================
// Partial sums of squares (float64) of bf16(in), one per workgroup: the
// Frobenius norm of X = in.bfloat16() read straight from the input.
// grid (kParts, batch).  VEC: N % 8 == 0 and the input 16-byte aligned.
template <int DT, bool VEC>
__global__ void __launch_bounds__(kT) k_ns_sumsq(const void* in, int64_t N, double* part) {
    using T = typename Elem<DT>::T;
    __shared__ double s_w[kT / 64];
    const int64_t bz = blockIdx.y;
    const T* x = static_cast<const T*>(in) + bz * N;
    double acc = 0.0;
    if constexpr (VEC) {
        const int64_t n8 = N / 8;
#pragma unroll 2
        for (int64_t c = (int64_t)blockIdx.x * kT + threadIdx.x; c < n8; c += (int64_t)gridDim.x * kT) {
            Raw8<DT> r;
            load_raw8<DT>(x + c * 8, r);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float v = bf16f(f2bf(raw_elem<DT>(r, k)));
                acc += (double)(v * v);
            }
        }
    } else {
        for (int64_t e = (int64_t)blockIdx.x * kT + threadIdx.x; e < N; e += (int64_t)gridDim.x * kT) {
            const float v = bf16f(f2bf(to_f32<DT>(*gbl(x + e))));
            acc += (double)(v * v);
        }
    }
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < kT / 64; ++w) t += s_w[w];
        part[bz * gridDim.x + blockIdx.x] = t;
    }
}

// den = max(bf16(||X||), eps) per matrix (Tensor.norm of bf16 returns bf16).
__global__ void k_ns_norm(const double* part, int nparts, int64_t batch, float eps, float* den) {
    const int64_t bz = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (bz >= batch) return;
    double t = 0.0;
    for (int i = 0; i < nparts; ++i) t += part[bz * nparts + i];
    const float nb = bf16f(f2bf((float)sqrt(t)));
    den[bz] = nb < eps ? bf16f(f2bf(eps)) : nb;
}

// X (m x n) and Xt (n x m) from the input [R x C] of any grad dtype:
// bf16(bf16(in) / den), tall inputs (R > C) transposed (m = min(R, C),
// n = max(R, C)).  A workgroup moves one 64 x 64 tile: rows of 8 elements
// from the input to the same-layout output (16-byte stores), and through LDS
// (pitch 66 bf16, so the column reads below spread over the banks) to the
// transposed output, whose rows leave as 8-row 16-byte vectors, 8 lanes per
// 128-byte row segment.  grid (ceil(C/64), ceil(R/64), batch).  VEC: C % 8
// == 0 and the input, X and Xt 16-byte aligned (then every 8-element row
// piece is in bounds or entirely out).
constexpr int kTilePitch = 66;

template <int DT, bool VEC>
__global__ void __launch_bounds__(kT) k_ns_load(const void* in, int64_t R, int64_t Cc, uint16_t* X, uint16_t* Xt,
                                                const float* den_p) {
    using T = typename Elem<DT>::T;
    __shared__ uint16_t tile[64 * kTilePitch];
    const int64_t bz = blockIdx.z;
    const int64_t N = R * Cc;
    const T* src = static_cast<const T*>(in) + bz * N;
    const bool tall = R > Cc;
    uint16_t* same = (tall ? Xt : X) + bz * N;   // [R x C]
    uint16_t* trans = (tall ? X : Xt) + bz * N;  // [C x R]
    const float den = den_p[bz];
    const float yden = block_recip(den);  // RN(1/den), or 0 when den or 1/den is not normal
    const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
    // both chunks' loads before any store (the output may alias the input as
    // far as the compiler knows, so a load after a store could not move up)
    Raw8<DT> raws[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int v = threadIdx.x + k * kT;
        const int64_t r = r0 + (v >> 3), c = c0 + (v & 7) * 8;
        if (VEC && r < R && c < Cc) load_raw8<DT>(src + r * Cc + c, raws[k]);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int v = threadIdx.x + k * kT;
        const int row = v >> 3, c8 = (v & 7) * 8;
        const int64_t r = r0 + row, c = c0 + c8;
        uint32_t h[8];
        if (VEC && r < R && c < Cc) {
            const Raw8<DT>& raw = raws[k];
            // x / den through the reciprocal with one Markstein correction
            // (correctly rounded while x, the first quotient and 1/den stay
            // clear of the subnormal range); a wave with any lane outside
            // that (zero, tiny or NaN x) takes the guarded division instead
            float xs[8], qs[8];
            bool bad = yden == 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                xs[e] = bf16f(f2bf(raw_elem<DT>(raw, e)));
                const float q0 = xs[e] * yden;
                qs[e] = __builtin_fmaf(__builtin_fmaf(-q0, den, xs[e]), yden, q0);
                bad = bad || !(fabsf(xs[e]) >= 0x1p-100f) || !(fabsf(q0) >= 0x1p-100f);
            }
            if (__builtin_expect(__any(bad), 0)) {
#pragma unroll
                for (int e = 0; e < 8; ++e) qs[e] = div_by_block(xs[e], den, yden);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = f2bf(qs[e]);
            const u32x4 pk = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
            *gbl(reinterpret_cast<u32x4*>(same + r * Cc + c)) = pk;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                h[e] = 0u;
                if (r < R && c + e < Cc) {
                    h[e] = f2bf(bf16f(f2bf(to_f32<DT>(*gbl(src + r * Cc + c + e)))) / den);
                    *gbl(same + r * Cc + c + e) = (uint16_t)h[e];
                }
            }
        }
        uint32_t* trow = reinterpret_cast<uint32_t*>(tile + row * kTilePitch + c8);
#pragma unroll
        for (int q = 0; q < 4; ++q) trow[q] = h[2 * q] | (h[2 * q + 1] << 16);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int v = threadIdx.x + k * kT;
        const int cc = v >> 3, r8 = (v & 7) * 8;  // output row (input column), first output column
        const int64_t c = c0 + cc, r = r0 + r8;
        if (c >= Cc) continue;
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = tile[(r8 + e) * kTilePitch + cc];
        uint16_t* tp = trans + c * R + r;
        if (VEC && r + 8 <= R && (R & 7) == 0) {
            const u32x4 pk = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
            *gbl(reinterpret_cast<u32x4*>(tp)) = pk;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (r + e < R) *gbl(tp + e) = (uint16_t)h[e];
        }
    }
}

// out [R x C] (bf16) from the normalised X / Xt (a schedule of no steps).
__global__ void __launch_bounds__(kT) k_ns_store(const uint16_t* src, int64_t N, int64_t sX, uint16_t* out, int64_t s_out) {
    const int64_t bz = blockIdx.y;
    for (int64_t e = (int64_t)blockIdx.x * kT + threadIdx.x; e < N; e += (int64_t)gridDim.x * kT)
        *gbl(out + bz * s_out + e) = *gbl(src + bz * sX + e);
}

struct NsWs {
    size_t off_x, off_xt0, off_xt1, off_g, off_b, off_part, off_den, total;
    static constexpr int kParts = 256;
    static NsWs make(int64_t batch, int64_t R, int64_t C) {
        const int64_t m = std::min(R, C), n = std::max(R, C);
        NsWs w;
        size_t o = 0;
        const size_t mn = align256(sizeof(uint16_t) * (size_t)(batch * m * n));
        const size_t mm = align256(sizeof(uint16_t) * (size_t)(batch * m * m));
        w.off_x = o; o += mn;
        w.off_xt0 = o; o += mn;
        w.off_xt1 = o; o += mn;
        w.off_g = o; o += mm;
        w.off_b = o; o += mm;
        w.off_part = o; o += align256(sizeof(double) * (size_t)(batch * kParts));
        w.off_den = o; o += align256(sizeof(float) * (size_t)batch);
        w.total = o;
        return w;
    }
};

// ==================================================================
// NorMuon and the Muon apply
// ==================================================================
// The update stack U [n, R, C] (bf16, contiguous) from Newton-Schulz; matrix
// i of a launch is blockIdx.y (row norms, apply) or blockIdx.x (NorMuon
// scale).  Parameters may be strided views (logical row-major order).
struct ApplyItem {
    void* p;
    int64_t ps0, ps1;       // parameter strides in elements
    const float* scalars;   // capturable scalar row (fp32[4]) or nullptr
    float* v;               // normuon_v [R]
    const float* step_dev;  // capturable NorMuon step counter or nullptr
    float bc;               // 1 - beta2^step (host step)
    const void* g;          // cautious: the raw gradient view (parameter dtype)
    int64_t gs0, gs1;
    const unsigned long long* count;  // cautious: agreeing elements of the matrix
};
struct ApplyBatch {
    ApplyItem it[kMaxBatch];
};

// row_norm[i][r] = sqrt(sum_c u[r][c]^2) in fp32 from float64 sums
// (torch.linalg.vector_norm(..., dtype=float32)); one wave per row, 16-byte
// loads when C % 8 == 0 and U is 16-byte aligned.
template <bool VEC>
__global__ void __launch_bounds__(kT) k_row_norm(const uint16_t* U, int64_t R, int64_t C, float* row_norm) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * (kT / 64) + (threadIdx.x >> 6);
    const int64_t bz = blockIdx.y;
    if (r >= R) return;
    const uint16_t* row = U + (bz * R + r) * C;
    double acc = 0.0;
    if constexpr (VEC) {
#pragma unroll 4
        for (int64_t c8 = lane; c8 < C / 8; c8 += 64) {
            const u32x4 v = __builtin_nontemporal_load(gbl(reinterpret_cast<const u32x4*>(row + c8 * 8)));
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float f = bf16f((uint16_t)(w[e >> 1] >> (16 * (e & 1))));
                acc += (double)(f * f);
            }
        }
    } else {
        for (int64_t c = lane; c < C; c += 64) {
            const float v = bf16f(*gbl(row + c));
            acc += (double)(v * v);
        }
    }
    acc = wave_sum_d(acc);
    if (lane == 0) row_norm[bz * R + r] = (float)sqrt(acc);
}

// v <- v*beta2 + row_sq * ((1-beta2)/C); denom = sqrt(v/bc) + eps;
// frob_scale = sqrt(sum row_sq) / max(||row_norm / denom||, tiny);
// scale[r] = bf16(frob_scale / denom[r]).  One workgroup per matrix.
__global__ void __launch_bounds__(kT) k_normuon_scale(const float* row_norm, int64_t R, float beta2, float alpha,
                                                      float eps, float* denom, uint16_t* scale, double beta2_d,
                                                      ApplyBatch bt) {
    const ApplyItem& it = bt.it[blockIdx.x];
    __shared__ double s_a[kT / 64], s_b[kT / 64];
    const int64_t off = (int64_t)blockIdx.x * R;
    row_norm += off;
    denom += off;
    scale += off;
    float* v = it.v;
    // device step counter (capturable): the same float64 bias correction
    float bc = it.bc;
    if (it.step_dev != nullptr) bc = (float)(1.0 - pow(beta2_d, (double)*gbl(it.step_dev)));
    double sa = 0.0, sb = 0.0;
    for (int64_t r = threadIdx.x; r < R; r += kT) {
        const float rn = row_norm[r];
        const float rs = rn * rn;
        const float nv = __builtin_fmaf(rs, alpha, v[r] * beta2);
        v[r] = nv;
        const float d = sqrtf(nv / bc) + eps;
        denom[r] = d;
        const float q = rn / d;
        sa += (double)rs;
        sb += (double)(q * q);
    }
    sa = wave_sum_d(sa);
    sb = wave_sum_d(sb);
    if ((threadIdx.x & 63) == 0) { s_a[threadIdx.x >> 6] = sa; s_b[threadIdx.x >> 6] = sb; }
    __syncthreads();
    double ta = 0.0, tb = 0.0;
    for (int w = 0; w < kT / 64; ++w) { ta += s_a[w]; tb += s_b[w]; }
    const float num = sqrtf((float)ta);
    float den = sqrtf((float)tb);
    den = den < kTiny ? kTiny : den;
    const float fs = num / den;
    for (int64_t r = threadIdx.x; r < R; r += kT) scale[r] = f2bf(fs / denom[r]);
}

struct MuonApplyArgs {
    const uint16_t* U;      // [n, R, C]
    const uint16_t* scale;  // [n, R] NorMuon row scales, or nullptr
    int64_t R, C;
    double invC, lr_ratio;
    float wdf, alpha;
    int wd;
};

// Cautious masking (gefen_muon.py:396-405): an element keeps its update when
// update * grad, in torch's promoted dtype (bf16 for a bf16 grad, else fp32),
// is > 0; the kept ones are scaled by bf16(fp32(numel) / fp32(max(agree, 1))),
// the others become a zero of their own sign.
template <int DT>
__device__ __forceinline__ bool cautious_agree(float u, float g) {
    float prod = u * g;
    if constexpr (DT == BF16) prod = bf16f(f2bf(prod));
    return prod > 0.0f;
}

__device__ __forceinline__ float cautious_scale(int64_t numel, unsigned long long agree) {
    return bf16f(f2bf((float)numel / (float)(agree > 0ull ? agree : 1ull)));
}

// The 8 grad elements of row r, columns c .. c+7 of a strided view.
template <int DT>
__device__ __forceinline__ void load_grad8(const void* gp, int64_t gs0, int64_t gs1, int64_t r, int64_t c,
                                           float out[8]) {
    using T = typename Elem<DT>::T;
    const T* g = static_cast<const T*>(gp) + r * gs0;
    if (gs1 == 1 && (reinterpret_cast<uintptr_t>(g + c) & 15) == 0) {
        Raw8<DT> raw;
        load_raw8<DT>(g + c, raw);
#pragma unroll
        for (int k = 0; k < 8; ++k) out[k] = raw_elem<DT>(raw, k);
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) out[k] = to_f32<DT>(*gbl(g + (c + k) * gs1));
    }
}

// One element: u' = bf16(u * scale[row]) with a NorMuon scale, else u; with
// CAUT the cautious mask (gv the grad element, cs the matrix's scale); then
// p = D(p * wdf) (when wd), then p = D(fma(u', alpha, p)).
template <int DT, bool CAUT>
__device__ __forceinline__ float muon_elem(float u, float sc, bool has_scale, float pv, float wdf, bool wd,
                                           float alpha, float gv = 0.0f, float cs = 1.0f) {
    if (has_scale) u = bf16f(f2bf(u * sc));
    if constexpr (CAUT) u = cautious_agree<DT>(u, gv) ? bf16f(f2bf(u * cs)) : u * 0.0f;
    if (wd) pv = round_dt<DT>(pv * wdf);
    return __builtin_fmaf(u, alpha, pv);
}

// FAST: contiguous 16-byte aligned parameter, C % 8 == 0: each thread takes
// kApplyCpt chunks of 8 elements (one row each), all loads first.  Else any
// strides, one element at a time.
constexpr int kApplyCpt = 4;

template <int DT, bool FAST, bool CAUT>
__global__ void __launch_bounds__(kT) k_muon_apply(MuonApplyArgs a, ApplyBatch bt) {
    using T = typename Elem<DT>::T;
    const ApplyItem& it = bt.it[blockIdx.y];
    T* pp = static_cast<T*>(it.p);
    float wdf = a.wdf, alpha = a.alpha;
    if (it.scalars != nullptr) {  // capturable: lr and 1 - lr*wd from the device scalar row
        wdf = *gbl(it.scalars + 3);
        alpha = round_dt<DT>((float)(-((double)*gbl(it.scalars) * a.lr_ratio)));
    }
    const bool wd = a.wd != 0, has_scale = a.scale != nullptr;
    const int64_t N = a.R * a.C;
    const uint16_t* U = a.U + (int64_t)blockIdx.y * N;
    const uint16_t* S = has_scale ? a.scale + (int64_t)blockIdx.y * a.R : nullptr;
    float cs = 1.0f;
    if constexpr (CAUT) cs = cautious_scale(N, *gbl(it.count));
    if constexpr (FAST) {
        const int64_t nch = N / 8;
        const int64_t first = (int64_t)blockIdx.x * (kT * kApplyCpt) + threadIdx.x;
        u32x4 uv[kApplyCpt];
        Raw8<DT> pr[kApplyCpt];
        float sc[kApplyCpt];
#pragma unroll
        for (int i = 0; i < kApplyCpt; ++i) {
            const int64_t ch = first + (int64_t)i * kT;
            if (ch < nch) {
                uv[i] = __builtin_nontemporal_load(gbl(reinterpret_cast<const u32x4*>(U + ch * 8)));
                load_raw8<DT>(pp + ch * 8, pr[i]);
                sc[i] = has_scale ? bf16f(*gbl(S + div_floor(ch * 8, a.C, a.invC))) : 1.0f;
            }
        }
#pragma unroll
        for (int i = 0; i < kApplyCpt; ++i) {
            const int64_t ch = first + (int64_t)i * kT;
            if (ch >= nch) break;
            const uint32_t w[4] = {uv[i].x, uv[i].y, uv[i].z, uv[i].w};
            float gv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if constexpr (CAUT) {
                const int64_t r = div_floor(ch * 8, a.C, a.invC);
                load_grad8<DT>(it.g, it.gs0, it.gs1, r, ch * 8 - r * a.C, gv);
            }
            float o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                o[e] = muon_elem<DT, CAUT>(bf16f((uint16_t)(w[e >> 1] >> (16 * (e & 1)))), sc[i], has_scale,
                                           raw_elem<DT>(pr[i], e), wdf, wd, alpha, gv[e], cs);
            store8<DT>(pp + ch * 8, o);
        }
    } else {
        for (int64_t e = (int64_t)blockIdx.x * kT + threadIdx.x; e < N; e += (int64_t)gridDim.x * kT) {
            const int64_t r = div_floor(e, a.C, a.invC);
            T* q = pp + r * it.ps0 + (e - r * a.C) * it.ps1;
            float gv = 0.0f;
            if constexpr (CAUT) gv = to_f32<DT>(*gbl(static_cast<const T*>(it.g) + r * it.gs0 + (e - r * a.C) * it.gs1));
            const float o = muon_elem<DT, CAUT>(bf16f(*gbl(U + e)), has_scale ? bf16f(*gbl(S + r)) : 1.0f, has_scale,
                                                to_f32<DT>(*gbl(q)), wdf, wd, alpha, gv, cs);
            *gbl(q) = from_f32<DT>(o);
        }
    }
}

// Cautious agreement counts of n matrices (grid (parts, n)): the update u'
// as the apply forms it (NorMuon row scale included) against the raw grad;
// one atomic per wave into the matrix's 64-bit counter (a count is exact in
// any order).  C % 8 == 0: chunks of 8 along a row, else element by element.
struct CautItem {
    const void* g;
    int64_t gs0, gs1;
    unsigned long long* count;
};
struct CautBatch {
    CautItem it[kMaxBatch];
};

__global__ void k_cautious_zero(CautBatch bt, int n) {
    if ((int)threadIdx.x < n) *gbl(bt.it[threadIdx.x].count) = 0ull;
}

template <int DT>
__global__ void __launch_bounds__(kT) k_cautious_count(const uint16_t* U, const uint16_t* S, int64_t R, int64_t C,
                                                        double invC, CautBatch bt) {
    const CautItem& it = bt.it[blockIdx.y];
    const int64_t N = R * C;
    const uint16_t* u = U + (int64_t)blockIdx.y * N;
    const uint16_t* s = S ? S + (int64_t)blockIdx.y * R : nullptr;
    uint32_t cnt = 0u;
    if (C % 8 == 0) {
        for (int64_t ch = (int64_t)blockIdx.x * kT + threadIdx.x; ch < N / 8; ch += (int64_t)gridDim.x * kT) {
            const int64_t r = div_floor(ch * 8, C, invC);
            const u32x4 uv = __builtin_nontemporal_load(gbl(reinterpret_cast<const u32x4*>(u + ch * 8)));
            float gv[8];
            load_grad8<DT>(it.g, it.gs0, it.gs1, r, ch * 8 - r * C, gv);
            const float sc = s ? bf16f(*gbl(s + r)) : 1.0f;
            const uint32_t w[4] = {uv.x, uv.y, uv.z, uv.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float x = bf16f((uint16_t)(w[e >> 1] >> (16 * (e & 1))));
                if (s) x = bf16f(f2bf(x * sc));
                cnt += cautious_agree<DT>(x, gv[e]) ? 1u : 0u;
            }
        }
    } else {
        using T = typename Elem<DT>::T;
        for (int64_t e = (int64_t)blockIdx.x * kT + threadIdx.x; e < N; e += (int64_t)gridDim.x * kT) {
            const int64_t r = div_floor(e, C, invC);
            float x = bf16f(*gbl(u + e));
            if (s) x = bf16f(f2bf(x * bf16f(*gbl(s + r))));
            const float gv = to_f32<DT>(*gbl(static_cast<const T*>(it.g) + r * it.gs0 + (e - r * C) * it.gs1));
            cnt += cautious_agree<DT>(x, gv) ? 1u : 0u;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) cnt += (uint32_t)__shfl_xor((int)cnt, off, 64);
    if ((threadIdx.x & 63) == 0 && cnt != 0u)
        (void)__hip_atomic_fetch_add(gbl(it.count), (unsigned long long)cnt, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
}

static unsigned grid_for(int64_t n, int64_t cap = 8192) {
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(cap, cdiv(n, kT)));
}

static int check_dt(int dtype, const char* fn) {
    if (dtype == F64) return set_error(GEFENX_EDTYPE, "%s: not implemented for 'Double'", fn);
    if (dtype != F32 && dtype != F16 && dtype != BF16) return set_error(GEFENX_EINVAL, "%s: unknown dtype %d", fn, dtype);
    return GEFENX_OK;
}

// ------------------------------------------------------------ host side
static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// One launch set (block max, finalize, requantise + emit) for n matrices of
// one kind: FAST (the chunked kernels; every item qualifies) or general.
static void mom_launch(const MomArgs& a, const MomBatch& bt, int n, int dtype, bool fast, bool sr, hipStream_t s) {
    int64_t max_nb = 1;
    for (int i = 0; i < n; ++i) max_nb = std::max(max_nb, bt.it[i].nb);
    const dim3 gfin(grid_for(max_nb, 4096), (unsigned)n);
    if (fast) {
        const dim3 gf((unsigned)cdiv(a.N / kChunk, (int64_t)kT * kMomCpt), (unsigned)n);
        switch (dtype) {
            case F32: hipLaunchKernelGGL(k_mom_max_fast<F32>, gf, dim3(kT), 0, s, a, bt); break;
            case F16: hipLaunchKernelGGL(k_mom_max_fast<F16>, gf, dim3(kT), 0, s, a, bt); break;
            default: hipLaunchKernelGGL(k_mom_max_fast<BF16>, gf, dim3(kT), 0, s, a, bt); break;
        }
        hipLaunchKernelGGL(k_mom_finalize, gfin, dim3(kT), 0, s, bt);
#define GX_EMIT_FAST(SRV, NV)                                                                              \
    switch (dtype) {                                                                                       \
        case F32: hipLaunchKernelGGL((k_mom_emit_fast<F32, SRV, NV>), gf, dim3(kT), 0, s, a, bt); break;   \
        case F16: hipLaunchKernelGGL((k_mom_emit_fast<F16, SRV, NV>), gf, dim3(kT), 0, s, a, bt); break;   \
        default: hipLaunchKernelGGL((k_mom_emit_fast<BF16, SRV, NV>), gf, dim3(kT), 0, s, a, bt); break;   \
    }
        if (sr) {
            if (a.nesterov) { GX_EMIT_FAST(true, true) } else { GX_EMIT_FAST(true, false) }
        } else {
            if (a.nesterov) { GX_EMIT_FAST(false, true) } else { GX_EMIT_FAST(false, false) }
        }
#undef GX_EMIT_FAST
        return;
    }
    const dim3 g(grid_for(a.N, 16384), (unsigned)n);
    switch (dtype) {
        case F32: hipLaunchKernelGGL(k_mom_max<F32>, g, dim3(kT), 0, s, a, bt); break;
        case F16: hipLaunchKernelGGL(k_mom_max<F16>, g, dim3(kT), 0, s, a, bt); break;
        default: hipLaunchKernelGGL(k_mom_max<BF16>, g, dim3(kT), 0, s, a, bt); break;
    }
    hipLaunchKernelGGL(k_mom_finalize, gfin, dim3(kT), 0, s, bt);
#define GX_EMIT(SRV)                                                                                       \
    switch (dtype) {                                                                                       \
        case F32: hipLaunchKernelGGL((k_mom_emit<F32, SRV>), g, dim3(kT), 0, s, a, bt); break;             \
        case F16: hipLaunchKernelGGL((k_mom_emit<F16, SRV>), g, dim3(kT), 0, s, a, bt); break;             \
        default: hipLaunchKernelGGL((k_mom_emit<BF16, SRV>), g, dim3(kT), 0, s, a, bt); break;             \
    }
    if (sr) { GX_EMIT(true) } else { GX_EMIT(false) }
#undef GX_EMIT
}

// Validate one matrix of a momentum batch and describe it.
static int mom_item(const char* fn, const gefenx_muon_item& in, int64_t rows, int64_t cols, MomItem& it) {
    const int64_t numel = rows * cols;
    if (in.period <= 0 || numel % in.period != 0)
        return set_error(GEFENX_EINVAL, "%s: period %lld does not divide numel %lld", fn, (long long)in.period,
                         (long long)numel);
    if (!in.grad || !in.m_codebook || !in.m_magnitude || !in.workspace)
        return set_error(GEFENX_EINVAL, "%s: null pointer argument", fn);
    const int64_t nb = numel / in.period;
    const MomentumWs L = MomentumWs::make(nb);
    if (in.workspace_bytes < L.total)
        return set_error(GEFENX_EINVAL, "%s: workspace %zu bytes < required %zu", fn, in.workspace_bytes, L.total);
    char* ws = static_cast<char*>(in.workspace);
    it.g = in.grad;
    it.gs0 = in.grad_stride0;
    it.gs1 = in.grad_stride1;
    it.idx = in.m_codebook;
    it.mag = in.m_magnitude;
    it.magbits = reinterpret_cast<uint32_t*>(ws + L.off_magbits);
    it.mag_old = reinterpret_cast<float*>(ws + L.off_magold);
    it.minv = reinterpret_cast<float*>(ws + L.off_minv);
    it.P = in.period;
    it.nb = nb;
    it.shards = mag_shards(nb);
    it.invP = 1.0 / (double)in.period;
    return GEFENX_OK;
}

// The momentum of n matrices [rows, cols]: runs of consecutive matrices of
// one kind (chunked / general), at most kMaxBatch per launch set; matrix i
// writes momentum_out + i * rows * cols.
static int momentum_batch(const char* fn, const gefenx_muon_item* items, int n, int dtype, int64_t rows,
                          int64_t cols, const void* qtable_dev, void* momentum_out, double beta1,
                          int stochastic_round, int64_t rng_seed, const int64_t* seed_dev, int nesterov,
                          hipStream_t s) {
    int rc = check_dt(dtype, fn);
    if (rc) return rc;
    if (n < 0 || rows < 0 || cols < 0) return set_error(GEFENX_EINVAL, "%s: negative size", fn);
    if (n == 0 || rows == 0 || cols == 0) return GEFENX_OK;
    if (!items || !qtable_dev || !momentum_out) return set_error(GEFENX_EINVAL, "%s: null pointer argument", fn);
    const int64_t numel = rows * cols;
    if (cdiv(numel / kChunk, (int64_t)kT * kMomCpt) > 2147483647LL)
        return set_error(GEFENX_EINVAL, "%s: %lld elements per matrix exceed the launch grid", fn, (long long)numel);
    const size_t es = dtype == F32 ? 4 : 2;
    std::vector<MomItem> its((size_t)n);
    std::vector<char> fast((size_t)n);
    for (int i = 0; i < n; ++i) {
        rc = mom_item(fn, items[i], rows, cols, its[(size_t)i]);
        if (rc) return rc;
        const MomItem& it = its[(size_t)i];
        fast[(size_t)i] = it.gs1 == 1 && it.gs0 == cols && it.P % kChunk == 0 && numel % kChunk == 0 &&
                          al16(it.g) && (reinterpret_cast<uintptr_t>(it.idx) & 7) == 0 &&
                          al16(static_cast<char*>(momentum_out) + (size_t)i * (size_t)numel * es);
    }
    MomArgs a;
    std::memset(&a, 0, sizeof(a));
    a.qt = static_cast<const QTable*>(qtable_dev);
    a.seed_dev = seed_dev;
    a.N = numel;
    a.C = cols;
    a.invC = 1.0 / (double)cols;
    a.seed = (uint64_t)rng_seed;
    a.w = (float)(1.0 - beta1);
    a.beta = (float)beta1;
    a.alpha_d = dtype == BF16 ? round_bf16(a.w) : dtype == F16 ? round_f16(a.w) : a.w;
    a.nesterov = nesterov ? 1 : 0;
    // algorithmic bytes: grad read, indices read + write, momentum written
    int ph = prof_begin(GEFENX_K_MOMENTUM, (double)n * (double)numel * (2.0 * (double)es + 2.0), 0.0, s);
    for (int i0 = 0; i0 < n;) {
        int i1 = i0 + 1;
        while (i1 < n && i1 - i0 < kMaxBatch && fast[(size_t)i1] == fast[(size_t)i0]) ++i1;
        MomBatch bt;
        std::memset(&bt, 0, sizeof(bt));
        for (int i = i0; i < i1; ++i) bt.it[i - i0] = its[(size_t)i];
        a.out = static_cast<char*>(momentum_out) + (size_t)i0 * (size_t)numel * es;
        mom_launch(a, bt, i1 - i0, dtype, fast[(size_t)i0] != 0, stochastic_round != 0, s);
        i0 = i1;
    }
    prof_end(ph, s);
    return launch_check(fn);
}

static int normuon_batch(const char* fn, const gefenx_muon_item* items, int n, const void* update, int64_t rows,
                         int64_t cols, double beta2, double eps, void* scale_out, void* workspace,
                         size_t workspace_bytes, hipStream_t s) {
    if (n < 0) return set_error(GEFENX_EINVAL, "%s: negative batch", fn);
    if (n == 0 || rows <= 0 || cols <= 0) return GEFENX_OK;
    if (!items || !update || !scale_out || !workspace) return set_error(GEFENX_EINVAL, "%s: bad argument", fn);
    const size_t slab = align256(sizeof(float) * (size_t)n * (size_t)rows);
    if (workspace_bytes < 2 * slab)
        return set_error(GEFENX_EINVAL, "%s: workspace %zu bytes < required %zu", fn, workspace_bytes, 2 * slab);
    if (cdiv(rows, kT / 64) > 2147483647LL) return set_error(GEFENX_EINVAL, "%s: too many rows", fn);
    float* row_norm = static_cast<float*>(workspace);
    float* denom = reinterpret_cast<float*>(static_cast<char*>(workspace) + slab);
    const uint16_t* U = static_cast<const uint16_t*>(update);
    const bool vec = cols % 8 == 0 && al16(U);
    const float alpha = (float)((1.0 - beta2) / (double)cols);
    for (int i0 = 0; i0 < n; i0 += kMaxBatch) {
        const int m = std::min(kMaxBatch, n - i0);
        ApplyBatch bt;
        std::memset(&bt, 0, sizeof(bt));
        for (int i = 0; i < m; ++i) {
            const gefenx_muon_item& in = items[i0 + i];
            if (!in.normuon_v || (in.normuon_step < 1 && !in.normuon_step_dev))
                return set_error(GEFENX_EINVAL, "%s: item %d has no NorMuon state or step", fn, i0 + i);
            bt.it[i].v = in.normuon_v;
            bt.it[i].step_dev = in.normuon_step_dev;
            bt.it[i].bc = in.normuon_step_dev ? 1.0f : (float)(1.0 - std::pow(beta2, (double)in.normuon_step));
        }
        const uint16_t* Ui = U + (size_t)i0 * (size_t)rows * (size_t)cols;
        float* rn = row_norm + (size_t)i0 * (size_t)rows;
        const dim3 gr((unsigned)cdiv(rows, kT / 64), (unsigned)m);
        if (vec) hipLaunchKernelGGL(k_row_norm<true>, gr, dim3(kT), 0, s, Ui, rows, cols, rn);
        else hipLaunchKernelGGL(k_row_norm<false>, gr, dim3(kT), 0, s, Ui, rows, cols, rn);
        hipLaunchKernelGGL(k_normuon_scale, dim3((unsigned)m), dim3(kT), 0, s, rn, rows, (float)beta2, alpha,
                           (float)eps, denom + (size_t)i0 * (size_t)rows,
                           static_cast<uint16_t*>(scale_out) + (size_t)i0 * (size_t)rows, beta2, bt);
    }
    return launch_check(fn);
}

static int apply_batch(const char* fn, const gefenx_muon_item* items, int n, int dtype, const void* update,
                       const void* row_scale, int64_t rows, int64_t cols, double lr, double weight_decay,
                       double adjusted_lr, double lr_ratio, const uint64_t* cautious_counts, hipStream_t s) {
    int rc = check_dt(dtype, fn);
    if (rc) return rc;
    if (n < 0) return set_error(GEFENX_EINVAL, "%s: negative batch", fn);
    if (n == 0 || rows <= 0 || cols <= 0) return GEFENX_OK;
    if (!items || !update) return set_error(GEFENX_EINVAL, "%s: null pointer argument", fn);
    const int64_t N = rows * cols;
    MuonApplyArgs a;
    a.R = rows;
    a.C = cols;
    a.invC = 1.0 / (double)cols;
    a.lr_ratio = lr_ratio;
    a.wdf = (float)(1.0 - lr * weight_decay);
    a.wd = weight_decay > 0.0 ? 1 : 0;
    float alpha = (float)(-adjusted_lr);
    a.alpha = dtype == BF16 ? round_bf16(alpha) : dtype == F16 ? round_f16(alpha) : alpha;
    const uint16_t* U = static_cast<const uint16_t*>(update);
    const uint16_t* S = static_cast<const uint16_t*>(row_scale);
    const int64_t fwgs = cdiv(N / 8, (int64_t)kT * kApplyCpt);
    if (fwgs > 2147483647LL) return set_error(GEFENX_EINVAL, "%s: too large", fn);
    std::vector<char> fast((size_t)n);
    for (int i = 0; i < n; ++i) {
        const gefenx_muon_item& in = items[i];
        if (!in.param) return set_error(GEFENX_EINVAL, "%s: item %d has no parameter", fn, i);
        if (cautious_counts && !in.grad) return set_error(GEFENX_EINVAL, "%s: cautious item %d has no grad", fn, i);
        fast[(size_t)i] = in.param_stride1 == 1 && in.param_stride0 == cols && cols % 8 == 0 && al16(in.param) &&
                          al16(U + (size_t)i * (size_t)N);
    }
    for (int i0 = 0; i0 < n;) {
        int i1 = i0 + 1;
        while (i1 < n && i1 - i0 < kMaxBatch && fast[(size_t)i1] == fast[(size_t)i0]) ++i1;
        ApplyBatch bt;
        std::memset(&bt, 0, sizeof(bt));
        for (int i = i0; i < i1; ++i) {
            bt.it[i - i0].p = items[i].param;
            bt.it[i - i0].ps0 = items[i].param_stride0;
            bt.it[i - i0].ps1 = items[i].param_stride1;
            bt.it[i - i0].scalars = items[i].step_scalars;
            if (cautious_counts) {
                bt.it[i - i0].g = items[i].grad;
                bt.it[i - i0].gs0 = items[i].grad_stride0;
                bt.it[i - i0].gs1 = items[i].grad_stride1;
                bt.it[i - i0].count = reinterpret_cast<const unsigned long long*>(cautious_counts + i);
            }
        }
        a.U = U + (size_t)i0 * (size_t)N;
        a.scale = S ? S + (size_t)i0 * (size_t)rows : nullptr;
        const unsigned m = (unsigned)(i1 - i0);
#define GX_APPLY(FASTV, CAUTV)                                                                         \
    switch (dtype) {                                                                                   \
        case F32: hipLaunchKernelGGL((k_muon_apply<F32, FASTV, CAUTV>), g, dim3(kT), 0, s, a, bt); break; \
        case F16: hipLaunchKernelGGL((k_muon_apply<F16, FASTV, CAUTV>), g, dim3(kT), 0, s, a, bt); break; \
        default: hipLaunchKernelGGL((k_muon_apply<BF16, FASTV, CAUTV>), g, dim3(kT), 0, s, a, bt); break; \
    }
        if (fast[(size_t)i0]) {
            const dim3 g((unsigned)fwgs, m);
            if (cautious_counts) { GX_APPLY(true, true) } else { GX_APPLY(true, false) }
        } else {
            const dim3 g(grid_for(N, 16384), m);
            if (cautious_counts) { GX_APPLY(false, true) } else { GX_APPLY(false, false) }
        }
#undef GX_APPLY
        i0 = i1;
    }
    return launch_check(fn);
}

static int cautious_count_batch(const char* fn, const gefenx_muon_item* items, int n, int dtype, const void* update,
                                const void* row_scale, int64_t rows, int64_t cols, uint64_t* counts,
                                hipStream_t s) {
    int rc = check_dt(dtype, fn);
    if (rc) return rc;
    if (n < 0) return set_error(GEFENX_EINVAL, "%s: negative batch", fn);
    if (n == 0) return GEFENX_OK;
    if (!items || !update || !counts) return set_error(GEFENX_EINVAL, "%s: null pointer argument", fn);
    if (rows < 0 || cols < 0) return set_error(GEFENX_EINVAL, "%s: negative shape", fn);
    for (int i = 0; i < n; ++i)
        if (!items[i].grad) return set_error(GEFENX_EINVAL, "%s: item %d has no grad", fn, i);
    const int64_t N = rows * cols;
    if (N > 0 && cols % 8 == 0 && !al16(update)) return set_error(GEFENX_EINVAL, "%s: update not 16-byte aligned", fn);
    const uint16_t* U = static_cast<const uint16_t*>(update);
    const uint16_t* S = static_cast<const uint16_t*>(row_scale);
    for (int i0 = 0; i0 < n; i0 += kMaxBatch) {
        const int m = std::min(n - i0, kMaxBatch);
        CautBatch bt;
        std::memset(&bt, 0, sizeof(bt));
        for (int i = 0; i < m; ++i) {
            bt.it[i].g = items[i0 + i].grad;
            bt.it[i].gs0 = items[i0 + i].grad_stride0;
            bt.it[i].gs1 = items[i0 + i].grad_stride1;
            bt.it[i].count = reinterpret_cast<unsigned long long*>(counts + i0 + i);
        }
        // counters cleared by a kernel (no memset node under graph capture)
        hipLaunchKernelGGL(k_cautious_zero, dim3(1), dim3(kMaxBatch), 0, s, bt, m);
        if (N == 0) continue;
        const dim3 g(grid_for(cols % 8 == 0 ? N / 8 : N, 2048), (unsigned)m);
        const uint16_t* Ui = U + (size_t)i0 * (size_t)N;
        const uint16_t* Si = S ? S + (size_t)i0 * (size_t)rows : nullptr;
        const double invC = 1.0 / (double)cols;
        switch (dtype) {
            case F32: hipLaunchKernelGGL(k_cautious_count<F32>, g, dim3(kT), 0, s, Ui, Si, rows, cols, invC, bt); break;
            case F16: hipLaunchKernelGGL(k_cautious_count<F16>, g, dim3(kT), 0, s, Ui, Si, rows, cols, invC, bt); break;
            default: hipLaunchKernelGGL(k_cautious_count<BF16>, g, dim3(kT), 0, s, Ui, Si, rows, cols, invC, bt); break;
        }
    }
    return launch_check(fn);
}

}  // namespace muon
}  // namespace gx

using namespace gx;
using namespace gx::muon;

extern "C" {

int gefenx_quantized_momentum_update(const void* grad, int dtype, int64_t numel, int64_t period,
                                     uint8_t* m_codebook, float* m_magnitude, const void* qtable_dev,
                                     void* momentum_out, double beta1, int stochastic_round, int64_t rng_seed,
                                     const int64_t* seed_dev, int nesterov, void* workspace,
                                     size_t workspace_bytes, void* stream) {
    const char* fn = "gefenx_quantized_momentum_update";
    int rc = check_dt(dtype, fn);
    if (rc) return rc;
    if (numel < 0) return set_error(GEFENX_EINVAL, "%s: negative numel", fn);
    if (numel == 0) return GEFENX_OK;
    gefenx_muon_item it;
    std::memset(&it, 0, sizeof(it));
    it.grad = grad;
    it.grad_stride0 = numel;
    it.grad_stride1 = 1;
    it.m_codebook = m_codebook;
    it.m_magnitude = m_magnitude;
    it.period = period;
    it.workspace = workspace;
    it.workspace_bytes = workspace_bytes;
    return momentum_batch(fn, &it, 1, dtype, 1, numel, qtable_dev, momentum_out, beta1, stochastic_round, rng_seed,
                          seed_dev, nesterov, static_cast<hipStream_t>(stream));
}

int gefenx_muon_momentum_batch(const gefenx_muon_item* items, int n, int dtype, int64_t rows, int64_t cols,
                               const void* qtable_dev, void* momentum_out, double beta1, int stochastic_round,
                               int64_t rng_seed, const int64_t* seed_dev, int nesterov, void* stream) {
    return momentum_batch("gefenx_muon_momentum_batch", items, n, dtype, rows, cols, qtable_dev, momentum_out,
                          beta1, stochastic_round, rng_seed, seed_dev, nesterov, static_cast<hipStream_t>(stream));
}

size_t gefenx_ns_workspace_bytes(int64_t batch, int64_t rows, int64_t cols) {
    if (batch <= 0 || rows <= 0 || cols <= 0) return 256;
    return NsWs::make(batch, rows, cols).total;
}

int gefenx_newton_schulz(const void* in, int in_dtype, void* out, int64_t batch, int64_t rows, int64_t cols,
                         const double* abc, int steps, double eps, void* workspace, size_t workspace_bytes,
                         void* stream) {
    int rc = check_dt(in_dtype, "gefenx_newton_schulz");
    if (rc) return rc;
    if (batch < 0 || rows < 0 || cols < 0 || steps < 0 || (steps > 0 && !abc))
        return set_error(GEFENX_EINVAL, "gefenx_newton_schulz: bad shape or schedule");
    if (batch == 0 || rows == 0 || cols == 0) return GEFENX_OK;
    if (!in || !out || !workspace) return set_error(GEFENX_EINVAL, "gefenx_newton_schulz: null pointer argument");
    const NsWs L = NsWs::make(batch, rows, cols);
    if (workspace_bytes < L.total)
        return set_error(GEFENX_EINVAL, "gefenx_newton_schulz: workspace %zu bytes < required %zu", workspace_bytes,
                         L.total);
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);
    uint16_t* X = reinterpret_cast<uint16_t*>(ws + L.off_x);
    uint16_t* Xt[2] = {reinterpret_cast<uint16_t*>(ws + L.off_xt0), reinterpret_cast<uint16_t*>(ws + L.off_xt1)};
    uint16_t* G = reinterpret_cast<uint16_t*>(ws + L.off_g);
    uint16_t* Bm = reinterpret_cast<uint16_t*>(ws + L.off_b);
    double* part = reinterpret_cast<double*>(ws + L.off_part);
    float* den = reinterpret_cast<float*>(ws + L.off_den);
    uint16_t* o16 = static_cast<uint16_t*>(out);
    const int64_t m = std::min(rows, cols), n = std::max(rows, cols);
    const int64_t N = m * n;
    const bool tall = rows > cols;
    const dim3 gt((unsigned)cdiv(cols, 64), (unsigned)cdiv(rows, 64), (unsigned)batch);
    if (cdiv(rows, 64) > 65535 || batch > 65535)
        return set_error(GEFENX_EINVAL, "gefenx_newton_schulz: %lld rows x batch %lld exceed the launch grid",
                         (long long)rows, (long long)batch);
    // X = bf16(in) / max(bf16(||bf16(in)||), eps): the norm straight from the
    // input, the division fused into the load that lays out X and X^T
    const bool vin = N % 8 == 0 && al16(in);
    const dim3 gp(NsWs::kParts, (unsigned)batch);
#define GX_NS_SUMSQ(DTV)                                                                                   \
    if (vin) hipLaunchKernelGGL((k_ns_sumsq<DTV, true>), gp, dim3(kT), 0, s, in, N, part);                \
    else hipLaunchKernelGGL((k_ns_sumsq<DTV, false>), gp, dim3(kT), 0, s, in, N, part);
    switch (in_dtype) {
        case F32: GX_NS_SUMSQ(F32) break;
        case F16: GX_NS_SUMSQ(F16) break;
        default: GX_NS_SUMSQ(BF16) break;
    }
#undef GX_NS_SUMSQ
    hipLaunchKernelGGL(k_ns_norm, dim3((unsigned)cdiv(batch, 64)), dim3(64), 0, s, part, NsWs::kParts, batch,
                       (float)eps, den);
    const bool vload = cols % 8 == 0 && al16(in);
#define GX_NS_LOAD(DTV)                                                                                    \
    if (vload) hipLaunchKernelGGL((k_ns_load<DTV, true>), gt, dim3(kT), 0, s, in, rows, cols, X, Xt[0], den); \
    else hipLaunchKernelGGL((k_ns_load<DTV, false>), gt, dim3(kT), 0, s, in, rows, cols, X, Xt[0], den);
    switch (in_dtype) {
        case F32: GX_NS_LOAD(F32) break;
        case F16: GX_NS_LOAD(F16) break;
        default: GX_NS_LOAD(BF16) break;
    }
#undef GX_NS_LOAD
    rc = launch_check("newton-schulz prologue");
    if (rc) return rc;
    if (steps == 0) {
        const dim3 g2(grid_for(N, 4096), (unsigned)batch);
        hipLaunchKernelGGL(k_ns_store, g2, dim3(kT), 0, s, tall ? Xt[0] : X, N, N, o16, N);
        return launch_check("newton-schulz epilogue");
    }
    int cur = 0;
    // algorithmic FLOPs of the iteration (three full products), as quoted for
    // the reference; the symmetric products execute about half of theirs
    const double flops_iter = 2.0 * (double)batch * ((double)m * m * n * 2.0 + (double)m * m * m);
    for (int it = 0; it < steps; ++it) {
        const float a = (float)abc[3 * it], b = (float)abc[3 * it + 1], c = (float)abc[3 * it + 2];
        const bool last = it + 1 == steps;
        int ph = prof_begin(GEFENX_K_NS_GEMM, 0.0, flops_iter, s);
        // G = X X^T (symmetric: lower tiles, mirrored)
        GemmArgs g1{X, n, N, X, n, N, nullptr, 0, 0, G, m, m * m, G, m, m * m, m, m, n, 1.0f, 0.0f, 0, 1};
        rc = gemm_nt(g1, batch, s);
        // B = b G + c G G^T (symmetric: lower tiles, mirrored)
        GemmArgs gg{G, m, m * m, G, m, m * m, G, m, m * m, Bm, m, m * m, Bm, m, m * m, m, m, m, c, b, 0, 1};
        if (!rc) rc = gemm_nt(gg, batch, s);
        // X = a X + B X  (B operand X^T), X^T of the result into the other
        // buffer; the last iteration writes the result straight to out in the
        // input's orientation (X when wide, X^T when tall) and nothing else
        uint16_t* D = last ? (tall ? nullptr : o16) : X;
        uint16_t* Dt = last ? (tall ? o16 : nullptr) : Xt[cur ^ 1];
        GemmArgs gx{Bm, m, m * m, Xt[cur], m, N, X, n, N, D, n, N, Dt, m, N, m, n, m, 1.0f, a, 0};
        if (!rc) rc = gemm_nt(gx, batch, s);
        prof_end(ph, s);
        if (rc) return rc;
        cur ^= 1;
    }
    return GEFENX_OK;
}

int gefenx_normuon_scale(const void* update, int64_t rows, int64_t cols, float* normuon_v, double beta2,
                         int64_t step, double eps, void* scale_out, void* workspace, size_t workspace_bytes,
                         const float* step_dev, void* stream) {
    if (rows <= 0 || cols <= 0) return GEFENX_OK;
    if (!update || !normuon_v || !scale_out || !workspace || (step < 1 && !step_dev))
        return set_error(GEFENX_EINVAL, "gefenx_normuon_scale: bad argument");
    gefenx_muon_item it;
    std::memset(&it, 0, sizeof(it));
    it.normuon_v = normuon_v;
    it.normuon_step = step;
    it.normuon_step_dev = step_dev;
    return normuon_batch("gefenx_normuon_scale", &it, 1, update, rows, cols, beta2, eps, scale_out, workspace,
                         workspace_bytes, static_cast<hipStream_t>(stream));
}

size_t gefenx_normuon_workspace_bytes(int64_t rows) {
    return 2 * align256(sizeof(float) * (size_t)(rows > 0 ? rows : 1));
}

size_t gefenx_normuon_batch_workspace_bytes(int n, int64_t rows) {
    return 2 * align256(sizeof(float) * (size_t)(n > 0 ? n : 1) * (size_t)(rows > 0 ? rows : 1));
}

int gefenx_normuon_scale_batch(const gefenx_muon_item* items, int n, const void* update, int64_t rows, int64_t cols,
                               double beta2, double eps, void* scale_out, void* workspace, size_t workspace_bytes,
                               void* stream) {
    return normuon_batch("gefenx_normuon_scale_batch", items, n, update, rows, cols, beta2, eps, scale_out, workspace,
                         workspace_bytes, static_cast<hipStream_t>(stream));
}

int gefenx_muon_apply(void* p, int dtype, const void* update, const void* row_scale, int64_t rows, int64_t cols,
                      double lr, double weight_decay, double adjusted_lr, const float* step_scalars,
                      double lr_ratio, void* stream) {
    gefenx_muon_item it;
    std::memset(&it, 0, sizeof(it));
    it.param = p;
    it.param_stride0 = cols;
    it.param_stride1 = 1;
    it.step_scalars = step_scalars;
    return apply_batch("gefenx_muon_apply", &it, 1, dtype, update, row_scale, rows, cols, lr, weight_decay,
                       adjusted_lr, lr_ratio, nullptr, static_cast<hipStream_t>(stream));
}

int gefenx_muon_apply_batch(const gefenx_muon_item* items, int n, int dtype, const void* update,
                            const void* row_scale, int64_t rows, int64_t cols, double lr, double weight_decay,
                            double adjusted_lr, double lr_ratio, const uint64_t* cautious_counts, void* stream) {
    return apply_batch("gefenx_muon_apply_batch", items, n, dtype, update, row_scale, rows, cols, lr, weight_decay,
                       adjusted_lr, lr_ratio, cautious_counts, static_cast<hipStream_t>(stream));
}

int gefenx_muon_cautious_count_batch(const gefenx_muon_item* items, int n, int dtype, const void* update,
                                     const void* row_scale, int64_t rows, int64_t cols, uint64_t* counts,
                                     void* stream) {
    return cautious_count_batch("gefenx_muon_cautious_count_batch", items, n, dtype, update, row_scale, rows, cols,
                                counts, static_cast<hipStream_t>(stream));
}

int gefenx_gemm_nt_bf16(const void* A, const void* B, const void* C, void* D, int64_t M, int64_t N, int64_t K,
                        float alpha, float beta, void* stream) {
    if (M < 0 || N < 0 || K < 0) return set_error(GEFENX_EINVAL, "gefenx_gemm_nt_bf16: negative shape");
    if (M == 0 || N == 0) return GEFENX_OK;
    // every kernel reads the first K step of A and B before its loop
    if (K == 0) return set_error(GEFENX_EINVAL, "gefenx_gemm_nt_bf16: K must be positive");
    if (!A || !B || !D) return set_error(GEFENX_EINVAL, "gefenx_gemm_nt_bf16: null pointer argument");
    GemmArgs g{static_cast<const uint16_t*>(A), K, 0, static_cast<const uint16_t*>(B), K, 0,
               static_cast<const uint16_t*>(C), N, 0, static_cast<uint16_t*>(D), N, 0, nullptr, 0, 0,
               M, N, K, alpha, beta, 0};
    return gemm_nt(g, 1, static_cast<hipStream_t>(stream));
}

}  // extern "C"
