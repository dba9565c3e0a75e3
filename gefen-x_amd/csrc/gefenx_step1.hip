// gefenx_step1.hip -- first-step kernels: block-period search statistics and
// the block-absmax-normalised histogram the exact-DP codebook is learned from,
// plus the standalone second-moment EMAs.
#include "gefenx_device.h"
#include "gefenx_dp.h"
#include "gefenx_internal.h"
#include "gefenx.h"

#include <algorithm>
#include <cmath>
#include <limits>
#include <vector>

namespace gx {

constexpr int kT = 256;

template <int DT>
__device__ __forceinline__ float load_elem(const void* base, int64_t i) {
    return to_f32<DT>(static_cast<const typename Elem<DT>::T*>(base)[i]);
}

// -------------------------------------------------------- period variance
// err(p) = sqrt(mean_b var_b(x)), x = fp32(g)^2 widened to float64
// (partitioning.py:62-84 via gefen.py:2639-2655).

// Small periods: numpy's two-pass variance (mean, then mean squared
// deviation) per block in float64 (k_var_tile).  Every workgroup reduces its blocks'
// variances in LDS and writes one partial (no shared-address atomics); the
// partials of a period are summed in a fixed order by k_var_sum.
// x of one element: fp32(g)^2 widened to float64, or fp32(g) itself when the
// input already holds squares (the reference's input_is_squared).
template <bool SQ>
__device__ __forceinline__ double var_x(float v) { return SQ ? (double)(v * v) : (double)v; }

constexpr int64_t kWavePeriod = 4096;
constexpr int64_t kThreadPeriod = 64;   // below: a thread per block
constexpr int64_t kGroupPeriod = 512;   // below: 8 lanes per block; from here a wave per block
constexpr int64_t kSeg = 65536;  // elements per workgroup segment of a large block
constexpr int kVarGrid = 2048;   // workgroups (and partials) per small-period pass

__device__ __forceinline__ void var_partial(double acc, double* part) {
    __shared__ double sh[kT / 64];
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < kT / 64; ++w) t += sh[w];
        part[blockIdx.x] = t;
    }
}

// One kernel for every P <= kWavePeriod: a workgroup takes tiles of whole
// blocks (about kVarTile elements) and stages their raw elements in LDS --
// 16-byte loads from the 16-byte boundary below the tile, lanes outside it
// dropped, the next tile's loads in flight during this tile's math -- then
// runs the two passes from LDS on x = fp32(g)^2: a thread per block when
// P < 64 (rows padded to an odd pitch, so the threads' strided reads fall in
// distinct banks), 8 lanes per block when P < 512, a wave per block otherwise.
constexpr int kVarTile = 8192;

template <int DT>
struct VarTile {
    using T = typename Elem<DT>::T;
    static constexpr int kPerVec = 16 / (int)sizeof(T);                      // elements per 16-byte load
    static constexpr int kVecs = (kVarTile + 2 * kPerVec) / kPerVec;          // covers any alignment
    static constexpr int kVecPerThread = (kVecs + kT - 1) / kT;
};

template <int DT, bool SQ = true>
__global__ void __launch_bounds__(kT) k_var_tile(const void* g, int64_t nb, int64_t P, double* part) {
    using T = typename Elem<DT>::T;
    using VT = VarTile<DT>;
    __shared__ T sx[kVarTile + kVarTile / 2];
    const T* gt = static_cast<const T*>(g);
    const int Pi = (int)P;
    const bool thread_blocks = P < kThreadPeriod;
    const int pitch = thread_blocks ? (Pi | 1) : Pi;
    const int nbt = kVarTile / Pi;                                            // blocks per tile
    const uint32_t magic = ((1u << 19) + (uint32_t)Pi - 1u) / (uint32_t)Pi;  // e / P for e < 2^13, P < 64
    const int64_t ntiles = (nb + nbt - 1) / nbt;
    const int64_t total = nb * P;
    const double fP = (double)P;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t misalign = (int64_t)((((uintptr_t)gt) & 15) / sizeof(T));  // base pointer offset in elements
    double acc = 0.0;

    u32x4 cur[VT::kVecPerThread], nxt[VT::kVecPerThread];
    int64_t a_cur = 0, a_nxt = 0;  // element index (relative to gt) of vector 0
    auto fetch = [&](int64_t tile, u32x4* v, int64_t& a0) {
        const int64_t base = tile * nbt * P;
        const int64_t hi = std::min<int64_t>(base + (int64_t)nbt * P, total);
        a0 = ((base + misalign) & ~(int64_t)(VT::kPerVec - 1)) - misalign;  // 16-byte aligned address
#pragma unroll
        for (int q = 0; q < VT::kVecPerThread; ++q) {
            const int64_t e0 = a0 + (int64_t)(tid + q * kT) * VT::kPerVec;
            v[q] = u32x4{0u, 0u, 0u, 0u};
            if (e0 + VT::kPerVec > base && e0 < hi) {
                if (e0 >= 0 && e0 + VT::kPerVec <= total) {
                    v[q] = *gbl(reinterpret_cast<const u32x4*>(gt + e0));
                } else {  // a vector straddling the tensor's ends: element loads
                    T tmp[VT::kPerVec];
#pragma unroll
                    for (int k = 0; k < VT::kPerVec; ++k) {
                        const int64_t e = e0 + k;
                        tmp[k] = (e >= 0 && e < total) ? gt[e] : T(0);
                    }
                    __builtin_memcpy(&v[q], tmp, sizeof(tmp));
                }
            }
        }
    };

    int64_t tile = blockIdx.x;
    if (tile < ntiles) fetch(tile, cur, a_cur);
    for (; tile < ntiles; tile += gridDim.x) {
        const int64_t b0 = tile * nbt;
        const int nbl = (int)std::min<int64_t>(nbt, nb - b0);
        const int elems = nbl * Pi;
        const int64_t base = b0 * P;
        // stage this tile's elements
#pragma unroll
        for (int q = 0; q < VT::kVecPerThread; ++q) {
            const T* el = reinterpret_cast<const T*>(&cur[q]);
            const int64_t e0 = a_cur + (int64_t)(tid + q * kT) * VT::kPerVec - base;
#pragma unroll
            for (int k = 0; k < VT::kPerVec; ++k) {
                const int64_t e = e0 + k;
                if (e >= 0 && e < elems) {
                    const int ei = (int)e;
                    const int at = thread_blocks ? ei + (pitch - Pi) * (int)(((uint32_t)ei * magic) >> 19) : ei;
                    sx[at] = el[k];
                }
            }
        }
        __syncthreads();
        if (tile + gridDim.x < ntiles) fetch(tile + gridDim.x, nxt, a_nxt);
        if (thread_blocks) {
            for (int bl = tid; bl < nbl; bl += kT) {
                const T* x = sx + bl * pitch;
                double s = 0.0;
                for (int j = 0; j < Pi; ++j) {
                    const float v = to_f32<DT>(x[j]);
                    s += var_x<SQ>(v);
                }
                const double mean = s / fP;
                double d2 = 0.0;
                for (int j = 0; j < Pi; ++j) {
                    const float v = to_f32<DT>(x[j]);
                    const double d = var_x<SQ>(v) - mean;
                    d2 += d * d;
                }
                acc += d2 / fP;
            }
        } else if (P < kGroupPeriod) {
            const int gl = lane & 7;
            for (int bl = wave * 8 + (lane >> 3); bl < nbl; bl += kT / 8) {
                const T* x = sx + bl * pitch;
                double s = 0.0;
                for (int j = gl; j < Pi; j += 8) {
                    const float v = to_f32<DT>(x[j]);
                    s += var_x<SQ>(v);
                }
                const double mean = group8_sum_d(s) / fP;
                double d2 = 0.0;
                for (int j = gl; j < Pi; j += 8) {
                    const float v = to_f32<DT>(x[j]);
                    const double d = var_x<SQ>(v) - mean;
                    d2 += d * d;
                }
                d2 = group8_sum_d(d2);
                if (gl == 0) acc += d2 / fP;
            }
        } else {
            for (int bl = wave; bl < nbl; bl += kT / 64) {
                const T* x = sx + bl * pitch;
                double s = 0.0;
                for (int j = lane; j < Pi; j += 64) {
                    const float v = to_f32<DT>(x[j]);
                    s += var_x<SQ>(v);
                }
                const double mean = wave_allsum_d(s) / fP;
                double d2 = 0.0;
                for (int j = lane; j < Pi; j += 64) {
                    const float v = to_f32<DT>(x[j]);
                    const double d = var_x<SQ>(v) - mean;
                    d2 += d * d;
                }
                d2 = wave_sum_d63(d2);
                if (lane == 63) acc += d2 / fP;
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < VT::kVecPerThread; ++q) cur[q] = nxt[q];
        a_cur = a_nxt;
    }
    var_partial(acc, part);
}

// totals[i] = sum of the n partials of period i, in index order (one wave per period).
__global__ void __launch_bounds__(64) k_var_sum(const double* part, int n, double* totals) {
    const double* q = part + (int64_t)blockIdx.x * kVarGrid;
    double t = 0.0;
    for (int k = threadIdx.x; k < n; k += 64) t += q[k];
    t = wave_sum_d(t);
    if (threadIdx.x == 0) totals[blockIdx.x] += t;
}

// Large periods: one workgroup per kSeg-element segment of a block; float64
// (sum, sum of squares) per segment, combined per block with two atomics.
// Segments whose start is 16-byte aligned and whose length is a multiple of
// 8 read 8 elements per load (two loads in flight per thread).
template <int DT, bool SQ = true>
__global__ void __launch_bounds__(kT) k_var_seg(const void* g, int64_t P, int64_t segs_per_block,
                                               double* s1, double* s2) {
    using T = typename Elem<DT>::T;
    __shared__ double sh[2][kT / 64];
    const int64_t b = (int64_t)blockIdx.x / segs_per_block;
    const int64_t sg = (int64_t)blockIdx.x - b * segs_per_block;
    const int64_t lo = b * P + sg * kSeg;
    const int64_t hi = std::min<int64_t>(lo + kSeg, (b + 1) * P);
    double a1 = 0.0, a2 = 0.0, c1 = 0.0, c2 = 0.0;
    const T* gt = static_cast<const T*>(g);
    if ((((uintptr_t)(gt + lo)) & 15) == 0 && ((hi - lo) & 7) == 0) {
        const int64_t nch = (hi - lo) >> 3;
        int64_t c = threadIdx.x;
        for (; c + kT < nch; c += 2 * kT) {
            float x[8], y[8];
            load8<DT>(gt + lo + c * 8, x);
            load8<DT>(gt + lo + (c + kT) * 8, y);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const double p = var_x<SQ>(x[k]);
                const double q = var_x<SQ>(y[k]);
                a1 += p; a2 += p * p;
                c1 += q; c2 += q * q;
            }
        }
        if (c < nch) {
            float x[8];
            load8<DT>(gt + lo + c * 8, x);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const double p = var_x<SQ>(x[k]);
                a1 += p; a2 += p * p;
            }
        }
    } else {
        for (int64_t i = lo + threadIdx.x; i < hi; i += kT) {
            const float v = load_elem<DT>(g, i);
            const double x = var_x<SQ>(v);
            a1 += x;
            a2 += x * x;
        }
    }
    a1 = wave_sum_d(a1 + c1);
    a2 = wave_sum_d(a2 + c2);
    if ((threadIdx.x & 63) == 0) { sh[0][threadIdx.x >> 6] = a1; sh[1][threadIdx.x >> 6] = a2; }
    __syncthreads();
    if (threadIdx.x == 0) {
        double t1 = 0.0, t2 = 0.0;
        for (int w = 0; w < kT / 64; ++w) { t1 += sh[0][w]; t2 += sh[1][w]; }
        atomicAdd(s1 + b, t1);
        atomicAdd(s2 + b, t2);
    }
}

__global__ void __launch_bounds__(kT) k_var_finish(double* s1, double* s2, int64_t nb, int64_t P,
                                                  double* total) {
    double acc = 0.0;
    const double fP = (double)P;
    for (int64_t b = (int64_t)blockIdx.x * kT + threadIdx.x; b < nb; b += (int64_t)gridDim.x * kT) {
        const double m = s1[b] / fP;
        double v = s2[b] / fP - m * m;
        if (v < 0.0) v = 0.0;
        acc += v;
        s1[b] = 0.0;
        s2[b] = 0.0;
    }
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0 && acc != 0.0) atomicAdd(total, acc);
}

__global__ void k_zero_f64(double* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0.0;
}

__global__ void k_zero_u32(uint32_t* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// ---------------------------------------------------------------- histogram
// gefen.py:455-469: absmax per block, x = g / absmax (0 when absmax is not
// > 0), bin = clamp(floor((x + 1) * (bins / 2)), 0, bins - 1), the scaling of
// the reference's histogram kernel (kernels/exact_histogram_fused_kernel.cu:
// 66-76); for the optimizer's 4096 bins it equals the torch path's division
// by 2 / bins exactly.  The absmax is carried as ordered uint bits of |g|
// (NaN > inf > finite), so a NaN block bins every element at x = 0 as the
// reference's torch.where does.

__device__ __forceinline__ int bin_of(float v, float amax, bool nz, float scale, int bins) {
    const float x = nz ? v / amax : 0.0f;
    const float t = floorf((x + 1.0f) * scale);
    if (!(t >= 0.0f)) return 0;
    if (t > (float)(bins - 1)) return bins - 1;
    return (int)t;
}

// Small periods: one wave per block, max then binning over the same block.
template <int DT>
__global__ void __launch_bounds__(kT) k_hist_wave(const void* g, int64_t nb, int64_t P, int bins,
                                                 unsigned long long* counts) {
    __shared__ uint32_t s_cnt[4096];
    for (int i = threadIdx.x; i < bins; i += kT) s_cnt[i] = 0u;
    __syncthreads();
    const float scale = 0.5f * (float)bins;
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * kT + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * kT) >> 6;
    for (int64_t b = wave; b < nb; b += nwaves) {
        const int64_t base = b * P;
        uint32_t m = 0u;
        for (int64_t j = lane; j < P; j += 64) {
            const uint32_t ub = __float_as_uint(load_elem<DT>(g, base + j)) & 0x7fffffffu;
            m = ub > m ? ub : m;
        }
        m = wave_max_u(m);
        const float amax = __uint_as_float(m);
        const bool nz = amax > 0.0f;
        for (int64_t j = lane; j < P; j += 64)
            atomicAdd(&s_cnt[bin_of(load_elem<DT>(g, base + j), amax, nz, scale, bins)], 1u);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < bins; i += kT)
        if (s_cnt[i]) atomicAdd(counts + i, (unsigned long long)s_cnt[i]);
}

// Large periods: segment max, then segment binning.
template <int DT>
__global__ void __launch_bounds__(kT) k_absmax_seg(const void* g, int64_t P, int64_t segs_per_block,
                                                  uint32_t* bits) {
    const int64_t b = (int64_t)blockIdx.x / segs_per_block;
    const int64_t sg = (int64_t)blockIdx.x - b * segs_per_block;
    const int64_t lo = b * P + sg * kSeg;
    const int64_t hi = std::min<int64_t>(lo + kSeg, (b + 1) * P);
    uint32_t m = 0u;
    for (int64_t i = lo + threadIdx.x; i < hi; i += kT) {
        const uint32_t ub = __float_as_uint(load_elem<DT>(g, i)) & 0x7fffffffu;
        m = ub > m ? ub : m;
    }
    m = wave_max_u(m);
    if ((threadIdx.x & 63) == 0 && m) atomicMax(bits + b, m);
}

template <int DT>
__global__ void __launch_bounds__(kT) k_hist_seg(const void* g, int64_t P, int64_t segs_per_block,
                                                const uint32_t* bits, int bins,
                                                unsigned long long* counts) {
    __shared__ uint32_t s_cnt[4096];
    for (int i = threadIdx.x; i < bins; i += kT) s_cnt[i] = 0u;
    __syncthreads();
    const float scale = 0.5f * (float)bins;
    const int64_t b = (int64_t)blockIdx.x / segs_per_block;
    const int64_t sg = (int64_t)blockIdx.x - b * segs_per_block;
    const int64_t lo = b * P + sg * kSeg;
    const int64_t hi = std::min<int64_t>(lo + kSeg, (b + 1) * P);
    const float amax = __uint_as_float(bits[b]);
    const bool nz = amax > 0.0f;
    for (int64_t i = lo + threadIdx.x; i < hi; i += kT)
        atomicAdd(&s_cnt[bin_of(load_elem<DT>(g, i), amax, nz, scale, bins)], 1u);
    __syncthreads();
    for (int i = threadIdx.x; i < bins; i += kT)
        if (s_cnt[i]) atomicAdd(counts + i, (unsigned long long)s_cnt[i]);
}

// --------------------------------------------------------------- EMAs

__global__ void k_v_ema(float* v, const float* sq, int64_t n, float inv_count, float beta2,
                        float alpha2, int divide, float count) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float ms = divide ? sq[i] / count : sq[i] * inv_count;
        v[i] = __builtin_fmaf(ms, alpha2, v[i] * beta2);
    }
}

template <int DT>
__global__ void __launch_bounds__(kT) k_vmean(float* vmean, const void* g, int64_t nb, int64_t P,
                                             float beta2, float alpha2) {
    // one wave per block: float64 partial sums, one mean per block
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * kT + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * kT) >> 6;
    for (int64_t b = wave; b < nb; b += nwaves) {
        double s = 0.0;
        for (int64_t j = lane; j < P; j += 64) {
            const float v = load_elem<DT>(g, b * P + j);
            float sq = v * v;
            if constexpr (DT == BF16) sq = round_dt<BF16>(sq);
            s += (double)sq;
        }
        s = wave_sum_d(s);
        if (lane == 0) {
            float mean = (float)s / (float)P;
            if constexpr (DT == BF16) mean = round_dt<BF16>(mean);
            vmean[b] = __builtin_fmaf(mean, alpha2, vmean[b] * beta2);
        }
    }
}

// ---------------------------------------------------------- exact DP
// Level c of the exact-DP codebook solver (quantization.py:75-139) for every
// segment end at once: one wave per end, lanes over the segment starts s,
// each lane keeping its first strict minimum of prev[s-1] + cost(s, end); the
// wave then takes the (value, start) lexicographic minimum, which is the
// sequential scan's first minimum.  Costs are the host solver's operations
// in the same order (dp_cost), so values and choices are bit-identical.
__global__ void __launch_bounds__(kT) k_dp_level(const double* __restrict__ pw, const double* __restrict__ pwx,
                                                const double* __restrict__ pwx2, const double* __restrict__ prev,
                                                double* __restrict__ cur, int32_t* __restrict__ bt_row, int c, int n,
                                                int endpoint, double fc) {
    const int lane = threadIdx.x & 63;
    const int64_t w = ((int64_t)blockIdx.x * kT + threadIdx.x) >> 6;
    const int end = c + (int)w;
    if (end > n) return;  // whole waves
    double best = __builtin_huge_val();
    int best_s = -1;
    for (int s = c + lane; s <= end; s += 64) {
        const double cand = prev[s - 1] + dp_cost(pw, pwx, pwx2, s, end, endpoint != 0, fc);
        if (cand < best) { best = cand; best_s = s; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const double ob = __shfl_xor(best, off, 64);
        const int os = __shfl_xor(best_s, off, 64);
        if (ob < best || (ob == best && os >= 0 && (best_s < 0 || os < best_s))) {
            best = ob;
            best_s = os;
        }
    }
    if (lane == 0) {
        cur[end] = best;
        bt_row[end] = best_s;
    }
}

static int grid_cap(int64_t items, int per, int cap) {
    int64_t g = (items + per - 1) / per;
    return (int)std::max<int64_t>(1, std::min<int64_t>(g, cap));
}

static int check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GEFENX_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
    return GEFENX_OK;
}

#define GX_DISPATCH(dtype, KERNEL, grid, block, stream, ...)                                       \
    do {                                                                                            \
        if ((dtype) == F32) hipLaunchKernelGGL(KERNEL<F32>, grid, block, 0, stream, __VA_ARGS__);   \
        else if ((dtype) == F16) hipLaunchKernelGGL(KERNEL<F16>, grid, block, 0, stream, __VA_ARGS__); \
        else hipLaunchKernelGGL(KERNEL<BF16>, grid, block, 0, stream, __VA_ARGS__);                 \
    } while (0)

// The same for inputs that already hold squares.
#define GX_DISPATCH_SQ(dtype, KERNEL, grid, block, stream, ...)                                          \
    do {                                                                                                  \
        if ((dtype) == F32) hipLaunchKernelGGL((KERNEL<F32, false>), grid, block, 0, stream, __VA_ARGS__);   \
        else if ((dtype) == F16) hipLaunchKernelGGL((KERNEL<F16, false>), grid, block, 0, stream, __VA_ARGS__); \
        else hipLaunchKernelGGL((KERNEL<BF16, false>), grid, block, 0, stream, __VA_ARGS__);                 \
    } while (0)

static int dtype_ok(int dtype, const char* fn) {
    if (dtype == F64) return set_error(GEFENX_EDTYPE, "%s: not implemented for 'Double'", fn);
    if (dtype != F32 && dtype != F16 && dtype != BF16) return set_error(GEFENX_EINVAL, "%s: bad dtype %d", fn, dtype);
    return GEFENX_OK;
}


}  // namespace gx

using namespace gx;

extern "C" {

int gefenx_block_variance_errors(const void* grad, int dtype, int64_t numel, const int64_t* periods,
                                 int n_periods, double* err_host, void* stream) {
    return gefenx_block_variance_errors_ex(grad, dtype, numel, periods, n_periods, 0, err_host, stream);
}

int gefenx_block_variance_errors_ex(const void* grad, int dtype, int64_t numel, const int64_t* periods,
                                    int n_periods, int input_is_squared, double* err_host, void* stream) {
    int rc = dtype_ok(dtype, "gefenx_block_variance_errors");
    if (rc) return rc;
    if (!grad || !periods || !err_host || numel <= 0 || n_periods < 0)
        return set_error(GEFENX_EINVAL, "gefenx_block_variance_errors: bad arguments");
    hipStream_t s = static_cast<hipStream_t>(stream);
    int64_t max_nb = 0;
    for (int i = 0; i < n_periods; ++i) {
        const int64_t P = periods[i];
        if (P <= 0 || numel % P != 0)
            return set_error(GEFENX_EINVAL, "period %lld does not divide numel %lld", (long long)P, (long long)numel);
        if (P > kWavePeriod) max_nb = std::max<int64_t>(max_nb, numel / P);
    }
    // [n_periods] totals, [n_periods][kVarGrid] small-period partials (zero
    // where a pass uses fewer workgroups), then 2 * max_nb block sums
    double* dev = nullptr;
    const int64_t n_part = (int64_t)n_periods * kVarGrid;
    const size_t bytes = sizeof(double) * ((size_t)n_periods + (size_t)n_part + 2 * (size_t)max_nb + 1);
    if (hipMalloc(&dev, bytes) != hipSuccess)
        return set_error(GEFENX_ENOMEM, "gefenx_block_variance_errors: hipMalloc(%zu) failed", bytes);
    double* totals = dev;
    double* part = dev + n_periods;
    double* s1 = part + n_part;
    double* s2 = s1 + max_nb;
    const int64_t fill = (int64_t)n_periods + n_part + 2 * max_nb;
    hipLaunchKernelGGL(k_zero_f64, dim3(grid_cap(fill, kT, 4096)), dim3(kT), 0, s, dev, fill);
    bool any_small = false;
    for (int i = 0; i < n_periods && rc == GEFENX_OK; ++i) {
        const int64_t P = periods[i];
        const int64_t nb = numel / P;
        if (P == 1) continue;  // single-element blocks have zero variance
        double* pi = part + (int64_t)i * kVarGrid;
        if (P <= kWavePeriod) {
            const int64_t tiles = (nb + kVarTile / P - 1) / (kVarTile / P);
            if (input_is_squared)
                GX_DISPATCH_SQ(dtype, k_var_tile, dim3(grid_cap(tiles, 1, kVarGrid)), dim3(kT), s, grad, nb, P, pi);
            else
                GX_DISPATCH(dtype, k_var_tile, dim3(grid_cap(tiles, 1, kVarGrid)), dim3(kT), s, grad, nb, P, pi);
            any_small = true;
        } else {
            const int64_t spb = (P + kSeg - 1) / kSeg;
            if (input_is_squared)
                GX_DISPATCH_SQ(dtype, k_var_seg, dim3((unsigned)(nb * spb)), dim3(kT), s, grad, P, spb, s1, s2);
            else
                GX_DISPATCH(dtype, k_var_seg, dim3((unsigned)(nb * spb)), dim3(kT), s, grad, P, spb, s1, s2);
            hipLaunchKernelGGL(k_var_finish, dim3(grid_cap(nb, kT, 4096)), dim3(kT), 0, s, s1, s2, nb, P, totals + i);
        }
        rc = check("block variance");
    }
    if (rc == GEFENX_OK && any_small && n_periods > 0) {
        hipLaunchKernelGGL(k_var_sum, dim3((unsigned)n_periods), dim3(64), 0, s, part, kVarGrid, totals);
        rc = check("block variance sum");
    }
    std::vector<double> host((size_t)std::max(n_periods, 1));
    if (rc == GEFENX_OK && n_periods > 0) {
        if (hipMemcpyAsync(host.data(), totals, sizeof(double) * (size_t)n_periods, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            rc = set_error(GEFENX_ELAUNCH, "gefenx_block_variance_errors: copy-back failed");
    }
    hipStreamSynchronize(s);
    hipFree(dev);
    if (rc) return rc;
    for (int i = 0; i < n_periods; ++i) {
        const double nb = (double)(numel / periods[i]);
        err_host[i] = std::sqrt(host[(size_t)i] / nb);
    }
    return GEFENX_OK;
}

int gefenx_exact_histogram(const void* grad, int dtype, int64_t numel, int64_t period,
                           int64_t* bin_counts, int bins, void* stream) {
    int rc = dtype_ok(dtype, "gefenx_exact_histogram");
    if (rc) return rc;
    if (!grad || !bin_counts || bins <= 0 || bins > 4096)
        return set_error(GEFENX_EINVAL, "Expected histogram bins in [1, 4096], got %d", bins);
    if (numel == 0) return GEFENX_OK;
    if (period <= 0 || numel % period != 0)
        return set_error(GEFENX_EINVAL, "Expected grad_flat.numel()=%lld to be divisible by period=%lld.",
                         (long long)numel, (long long)period);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t nb = numel / period;
    unsigned long long* cnt = reinterpret_cast<unsigned long long*>(bin_counts);
    if (period <= kWavePeriod) {
        GX_DISPATCH(dtype, k_hist_wave, dim3(grid_cap(nb * 64, kT, 8192)), dim3(kT), s, grad, nb, period, bins, cnt);
        return check("exact histogram");
    }
    uint32_t* bits = nullptr;
    if (hipMallocAsync((void**)&bits, sizeof(uint32_t) * (size_t)nb, s) != hipSuccess)
        return set_error(GEFENX_ENOMEM, "gefenx_exact_histogram: allocation failed");
    hipLaunchKernelGGL(k_zero_u32, dim3(grid_cap(nb, kT, 1024)), dim3(kT), 0, s, bits, nb);
    const int64_t spb = (period + kSeg - 1) / kSeg;
    GX_DISPATCH(dtype, k_absmax_seg, dim3((unsigned)(nb * spb)), dim3(kT), s, grad, period, spb, bits);
    GX_DISPATCH(dtype, k_hist_seg, dim3((unsigned)(nb * spb)), dim3(kT), s, grad, period, spb, bits, bins, cnt);
    rc = check("exact histogram");
    hipFreeAsync(bits, s);
    return rc;
}

int gefenx_factored_v_ema(float* v_row, float* v_col, const float* row_sq, const float* col_sq,
                          int64_t rows, int64_t cols, double beta2, void* stream) {
    if (rows == 0 && cols == 0) return GEFENX_OK;
    if (rows <= 0 || cols <= 0)
        return set_error(GEFENX_EINVAL, "gefenx_factored_v_ema: expected both v_row and v_col to be non-empty");
    if (!v_row || !v_col || !row_sq || !col_sq)
        return set_error(GEFENX_EINVAL, "gefenx_factored_v_ema: null pointer argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const float b2 = (float)beta2, a2 = (float)(1.0 - beta2);
    // the aten chain v.mul_(beta2).add_(sq.div_(n), alpha=1-beta2) on the GPU
    // (kernels/automatic_gefen_fused_kernel.cu:2010-2020): the scalar divide
    // is a multiply by the fp32 reciprocal of n, then fma(1-beta2, t, v*beta2)
    if (rows) hipLaunchKernelGGL(k_v_ema, dim3(grid_cap(rows, kT, 1024)), dim3(kT), 0, s, v_row, row_sq, rows,
                                 1.0f / (float)cols, b2, a2, 0, (float)cols);
    if (cols) hipLaunchKernelGGL(k_v_ema, dim3(grid_cap(cols, kT, 1024)), dim3(kT), 0, s, v_col, col_sq, cols,
                                 1.0f / (float)rows, b2, a2, 0, (float)rows);
    return check("gefenx_factored_v_ema");
}

int gefenx_vmean_update(float* vmean, const void* grad, int dtype, int64_t numel, int64_t period,
                        double beta2, void* stream) {
    int rc = dtype_ok(dtype, "gefenx_vmean_update");
    if (rc) return rc;
    if (!vmean || !grad || period <= 0 || numel < 0 || numel % period != 0)
        return set_error(GEFENX_EINVAL, "gefenx_vmean_update: bad arguments");
    if (numel == 0) return GEFENX_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t nb = numel / period;
    GX_DISPATCH(dtype, k_vmean, dim3(grid_cap(nb * 64, kT, 8192)), dim3(kT), s, vmean, grad, nb, period,
                (float)beta2, (float)(1.0 - beta2));
    return check("gefenx_vmean_update");
}

int gefenx_exact_dp_device(const float* active_centers, const float* active_counts, int n_points, int k,
                           int force_endpoints, float* codebook_out, void* stream) {
    if (!active_centers || !active_counts || !codebook_out || n_points < 1 || k < 1)
        return set_error(GEFENX_EINVAL, "gefenx_exact_dp_device: bad arguments (n=%d k=%d)", n_points, k);
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
    hipStream_t s = static_cast<hipStream_t>(stream);
    // device: pw, pwx, pwx2, prev, cur (double [W] each), bt (int32 [k+1][W])
    const size_t dbytes = sizeof(double) * 5 * W;
    const size_t btbytes = sizeof(int32_t) * (size_t)(k + 1) * W;
    char* dev = nullptr;
    if (hipMalloc((void**)&dev, dbytes + btbytes) != hipSuccess)
        return set_error(GEFENX_ENOMEM, "gefenx_exact_dp_device: hipMalloc(%zu) failed", dbytes + btbytes);
    double* d_pw = reinterpret_cast<double*>(dev);
    double* d_pwx = d_pw + W;
    double* d_pwx2 = d_pwx + W;
    double* d_prev = d_pwx2 + W;
    double* d_cur = d_prev + W;
    int32_t* d_bt = reinterpret_cast<int32_t*>(dev + dbytes);
    std::vector<double> prev0(W, std::numeric_limits<double>::infinity());
    prev0[0] = 0.0;
    std::vector<int32_t> bt((size_t)(k + 1) * W, -1);
    int rc = GEFENX_OK;
    if (hipMemcpyAsync(d_pw, pre.pw.data(), sizeof(double) * W, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(d_pwx, pre.pwx.data(), sizeof(double) * W, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(d_pwx2, pre.pwx2.data(), sizeof(double) * W, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(d_prev, prev0.data(), sizeof(double) * W, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(d_bt, bt.data(), btbytes, hipMemcpyHostToDevice, s) != hipSuccess)
        rc = set_error(GEFENX_ELAUNCH, "gefenx_exact_dp_device: upload failed");
    for (int c = 1; c <= k && rc == GEFENX_OK; ++c) {
        const int ends = n - c + 1;
        if (ends > 0) {
            const bool endpoint = force_endpoints && (c == 1 || c == k);
            const double fc = (c == 1) ? -1.0 : 1.0;
            hipLaunchKernelGGL(k_dp_level, dim3((unsigned)(((int64_t)ends * 64 + kT - 1) / kT)), dim3(kT), 0, s,
                               d_pw, d_pwx, d_pwx2, d_prev, d_cur, d_bt + (size_t)c * W, c, n, endpoint ? 1 : 0, fc);
            rc = check("exact DP level");
        }
        std::swap(d_prev, d_cur);
    }
    if (rc == GEFENX_OK && (hipMemcpyAsync(bt.data(), d_bt, btbytes, hipMemcpyDeviceToHost, s) != hipSuccess ||
                            hipStreamSynchronize(s) != hipSuccess))
        rc = set_error(GEFENX_ELAUNCH, "gefenx_exact_dp_device: download failed");
    hipStreamSynchronize(s);
    hipFree(dev);
    if (rc) return rc;
    if (!dp_backtrack(pre, bt.data(), W, n, k, force_endpoints, codebook_out))
        return set_error(GEFENX_EINVAL, "gefenx_exact_dp_device: infeasible segmentation");
    return GEFENX_OK;
}

}  // extern "C"
