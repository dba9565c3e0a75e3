// gefenx_device.h -- device helpers for the MI355X Gefen kernels (gfx950).
//
// Compiled with -ffp-contract=off: every fused multiply-add below is an
// explicit __builtin_fmaf, so the momentum recurrence is bit-identical to the
// reference's decomposed CPU step (Tensor.lerp is fma(w, end-self, self)).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "gefenx_common.h"

namespace gx {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Global-address-space views of generic pointers.  Pointers read from a
// descriptor in memory are generic; loads through them would be FLAT
// instructions, which count against lgkmcnt together with LDS reads, so every
// wait for an LDS gather would also wait for the HBM loads in flight.
#define GX_GLOBAL __attribute__((address_space(1)))
template <class T> __device__ __forceinline__ GX_GLOBAL T* gbl(T* p) { return (GX_GLOBAL T*)p; }
template <class T> __device__ __forceinline__ const GX_GLOBAL T* gbl(const T* p) {
    return (const GX_GLOBAL T*)p;
}

// Wave-uniform read of device memory that no kernel writes while this one
// runs, through the scalar cache (an s_load: it waits on lgkmcnt, not on the
// vector-memory counter, and takes no vector-memory issue slot).  p must be
// the same for every lane.
template <class T>
__device__ __forceinline__ T sload(const T* p) {
    return *(const __attribute__((address_space(4))) T*)p;
}

// Atomics on device memory through the global address space: they become
// global_atomic_* instructions, which the compiler's wait-counter tracking
// orders with the other vector memory operations (a flat atomic makes every
// later wait drain all outstanding loads).
__device__ __forceinline__ void gatomic_max(uint32_t* p, uint32_t v) {
    (void)__hip_atomic_fetch_max(gbl(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void gatomic_add(double* p, double v) {
    (void)__hip_atomic_fetch_add(gbl(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int DT> struct Elem { using T = uint16_t; };
template <> struct Elem<F32> { using T = float; };

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round-to-nearest-even fp32 -> bf16 (gfx950 v_cvt_pk_bf16_f32; NaN stays NaN).
__device__ __forceinline__ uint32_t f32_to_bf16(float x) {
    return (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)x);
}

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)h));
}
// The fp32 value reaches the conversion through an empty asm, so the compiler
// cannot fold the fp32 op that produced it into a mixed-precision instruction
// with a 16-bit result (v_fma_mixlo_f16 rounds once; the reference's torch ops
// round to fp32, then to fp16, and the two differ on some inputs).
__device__ __forceinline__ uint32_t f32_to_f16(float x) {
    asm volatile("" : "+v"(x));
    return (uint32_t)__half_as_ushort(__float2half_rn(x));
}

template <int DT> __device__ __forceinline__ float to_f32(typename Elem<DT>::T v) {
    if constexpr (DT == F32) return v;
    else if constexpr (DT == BF16) return bf16_to_f32(v);
    else return f16_to_f32(v);
}
template <int DT> __device__ __forceinline__ typename Elem<DT>::T from_f32(float v) {
    if constexpr (DT == F32) return v;
    else if constexpr (DT == BF16) return (uint16_t)f32_to_bf16(v);
    else return (uint16_t)f32_to_f16(v);
}
template <int DT> __device__ __forceinline__ float round_dt(float v) {
    if constexpr (DT == F32) return v;
    else return to_f32<DT>(from_f32<DT>(v));
}

// ---------------------------------------------------------- 8-element I/O
// A "chunk" is 8 consecutive logical elements starting at a multiple of 8.

template <int DT>
__device__ __forceinline__ void load8(const typename Elem<DT>::T* __restrict__ base, float v[8]) {
    if constexpr (DT == F32) {
        const GX_GLOBAL f32x4* q = gbl(reinterpret_cast<const f32x4*>(base));
        f32x4 a = q[0];
        f32x4 b = q[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        u32x4 a = *gbl(reinterpret_cast<const u32x4*>(base));
        uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = to_f32<DT>((uint16_t)(w[i] & 0xffffu));
            v[2 * i + 1] = to_f32<DT>((uint16_t)(w[i] >> 16));
        }
    }
}

template <int DT>
__device__ __forceinline__ void store8(typename Elem<DT>::T* __restrict__ base, const float v[8]) {
    if constexpr (DT == F32) {
        GX_GLOBAL f32x4* q = gbl(reinterpret_cast<f32x4*>(base));
        f32x4 a = {v[0], v[1], v[2], v[3]};
        f32x4 b = {v[4], v[5], v[6], v[7]};
        __builtin_nontemporal_store(a, q);
        __builtin_nontemporal_store(b, q + 1);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = (uint32_t)from_f32<DT>(v[2 * i]) | ((uint32_t)from_f32<DT>(v[2 * i + 1]) << 16);
        u32x4 a = {w[0], w[1], w[2], w[3]};
        __builtin_nontemporal_store(a, gbl(reinterpret_cast<u32x4*>(base)));
    }
}

__device__ __forceinline__ void load_idx8(const uint8_t* __restrict__ base, uint32_t ix[8]) {
    u32x2 a = *gbl(reinterpret_cast<const u32x2*>(base));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ix[i] = (a.x >> (8 * i)) & 0xffu;
        ix[4 + i] = (a.y >> (8 * i)) & 0xffu;
    }
}

// Workgroup barrier for data exchanged through LDS only: waits for this
// wave's LDS operations, not for its global loads and stores in flight
// (__syncthreads()'s workgroup fence makes the compiler drain those too, so a
// prefetch issued before it would be waited for at once).  No global memory
// written by one wave may be read by another across this barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ void store_idx8(uint8_t* __restrict__ base, const uint32_t ix[8]) {
    u32x2 a;
    a.x = ix[0] | (ix[1] << 8) | (ix[2] << 16) | (ix[3] << 24);
    a.y = ix[4] | (ix[5] << 8) | (ix[6] << 16) | (ix[7] << 24);
    __builtin_nontemporal_store(a, gbl(reinterpret_cast<u32x2*>(base)));
}

// Packed (as-loaded) 8-element chunks: loads stay packed while in flight and
// are unpacked element by element at use (k is a compile-time index).
template <int DT> struct Raw8 { uint32_t w[4]; };
template <> struct Raw8<F32> { float f[8]; };

// Streamed data (grads, parameters, indices) is read once per pass: the loads
// are non-temporal, so they do not displace the per-row / per-block values
// the kernels reuse (measured on MI355X: +7% on an apply-shaped stream, +10%
// on a stats-shaped one).
template <int DT>
__device__ __forceinline__ void load_raw8(const typename Elem<DT>::T* __restrict__ base, Raw8<DT>& r) {
    if constexpr (DT == F32) {
        const GX_GLOBAL f32x4* q = gbl(reinterpret_cast<const f32x4*>(base));
        const f32x4 a = __builtin_nontemporal_load(q);
        const f32x4 b = __builtin_nontemporal_load(q + 1);
        r.f[0] = a.x; r.f[1] = a.y; r.f[2] = a.z; r.f[3] = a.w;
        r.f[4] = b.x; r.f[5] = b.y; r.f[6] = b.z; r.f[7] = b.w;
    } else {
        const u32x4 v = __builtin_nontemporal_load(gbl(reinterpret_cast<const u32x4*>(base)));
        r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
    }
}

template <int DT>
__device__ __forceinline__ float raw_elem(const Raw8<DT>& r, int k) {
    if constexpr (DT == F32) return r.f[k];
    else return to_f32<DT>((uint16_t)((k & 1) ? (r.w[k >> 1] >> 16) : (r.w[k >> 1] & 0xffffu)));
}

// The same 8 elements through element loads, for a base that is not
// 16-byte aligned (any element offset); packed as load_raw8 packs them.
template <int DT>
__device__ __forceinline__ void load_raw8_elems(const typename Elem<DT>::T* __restrict__ base, Raw8<DT>& r) {
    if constexpr (DT == F32) {
#pragma unroll
        for (int k = 0; k < 8; ++k) r.f[k] = *gbl(base + k);
    } else {
        const uint16_t* b = reinterpret_cast<const uint16_t*>(base);
#pragma unroll
        for (int j = 0; j < 4; ++j) r.w[j] = (uint32_t)*gbl(b + 2 * j) | ((uint32_t)*gbl(b + 2 * j + 1) << 16);
    }
}

// Squared-gradient accumulation.  The reference's decomposed step squares in
// fp32 and sums in float64 (gefen.py:2959-2996, 129-191).  A double
// accumulator does the same; a float one keeps 8-element fp32 partials, which
// is exact per term for 16-bit grads (g*g fits in fp32) and within 1e-6
// after the sum.
__device__ __forceinline__ void sq_add(float& a, float g) { a = __builtin_fmaf(g, g, a); }
__device__ __forceinline__ void sq_add(double& a, float g) { a += (double)(g * g); }

struct RawIdx8 { uint32_t lo, hi; };

__device__ __forceinline__ RawIdx8 load_raw_idx8(const uint8_t* __restrict__ base) {
    const u32x2 v = __builtin_nontemporal_load(gbl(reinterpret_cast<const u32x2*>(base)));
    return RawIdx8{v.x, v.y};
}

// The same through an ordinary load, for a wave that reads half of each
// 128-byte line and the other half later: a non-temporal load does not keep
// the line in L2, so the second half would be fetched from HBM again
// (measured: one extra pass over the indices, 1 B per element).
__device__ __forceinline__ RawIdx8 load_raw_idx8_cached(const uint8_t* __restrict__ base) {
    const u32x2 v = *gbl(reinterpret_cast<const u32x2*>(base));
    return RawIdx8{v.x, v.y};
}

__device__ __forceinline__ RawIdx8 load_raw_idx8_elems(const uint8_t* __restrict__ base) {
    RawIdx8 r{0u, 0u};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t v = (uint32_t)*gbl(base + k);
        if (k < 4) r.lo |= v << (8 * k);
        else r.hi |= v << (8 * (k - 4));
    }
    return r;
}

__device__ __forceinline__ uint32_t raw_idx(const RawIdx8& r, int k) {
    return ((k < 4 ? r.lo : r.hi) >> (8 * (k & 3))) & 0xffu;
}

// --------------------------------------------------------- momentum math

struct MomentumCoef {
    float w;      // (float)(1 - beta1): Tensor.lerp weight
    float wm1;    // w - 1 (lerp's large-weight form)
    int small;    // |w| < 0.5 selects fma(w, g - cm, cm)
};

// u = lerp(cr * mag_old, g, w): gefen.py:3465-3470 / ATen lerp kernel.
// LF picks lerp's form at compile time: 1 small weight (fma(w, g - cm, cm)),
// 2 large weight (fma(w - 1, g - cm, g)), 0 decided per call from mc.small.
// Hot loops take 1 or 2 (the choice is uniform over a launch), so the
// compiler does not evaluate both forms and select.
constexpr int kLerpRuntime = 0;
constexpr int kLerpSmall = 1;
constexpr int kLerpLarge = 2;

template <int LF = kLerpRuntime>
__device__ __forceinline__ float momentum_value(float cr, float mag_old, float g,
                                                const MomentumCoef& mc) {
    const float cm = cr * mag_old;
    const float d = g - cm;
    if constexpr (LF == kLerpSmall) return __builtin_fmaf(mc.w, d, cm);
    else if constexpr (LF == kLerpLarge) return __builtin_fmaf(mc.wm1, d, g);
    else return mc.small ? __builtin_fmaf(mc.w, d, cm) : __builtin_fmaf(mc.wm1, d, g);
}

// Nearest-codeword index through the exact threshold table (see gefenx_host.cpp).
__device__ __forceinline__ uint32_t quant_nearest(float x, const uint32_t* __restrict__ s_bkt,
                                                  const float* __restrict__ s_thr, uint32_t kmax) {
    if (x != x) return kmax;  // NaN: searchsorted returns k -> index k-1
    const float s = (x + 1.0f) * (float)(kBuckets / 2);
    int b = (int)floorf(s);
    b = b < 0 ? 0 : (b > kBuckets - 1 ? kBuckets - 1 : b);
    const uint32_t e = s_bkt[b];
    const uint32_t base = e & 0xffffu;
    const uint32_t cnt = e >> 16;
    uint32_t idx = base;
    for (uint32_t j = 0; j < cnt; ++j) idx += (s_thr[base + j] < x) ? 1u : 0u;
    return idx;
}

// SplitMix64 finalizer over seed + golden_gamma * (idx + 1), top 24 bits.
__device__ __forceinline__ float sr_uniform(uint64_t seed, int64_t idx) {
    uint64_t z = seed + 0x9E3779B97F4A7C15ULL * ((uint64_t)idx + 1ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    z = z ^ (z >> 31);
    return (float)(z >> 40) * (1.0f / 16777216.0f);
}

// Unbiased stochastic rounding between the bracketing codewords.
__device__ __forceinline__ uint32_t quant_stochastic(float x, const float* __restrict__ s_cb,
                                                     const int16_t* __restrict__ s_lut, int k,
                                                     uint64_t seed, int64_t elem) {
    int b = (int)floorf((x + 1.0f) * (float)(kBuckets / 2));
    b = b < 0 ? 0 : (b > kBuckets - 1 ? kBuckets - 1 : b);
    int lo = s_lut[b], hi = s_lut[b + 1];
    lo = lo < 0 ? 0 : (lo > k ? k : lo);
    hi = hi < lo ? lo : (hi > k ? k : hi);
    while (lo < hi) {
        const int mid = lo + ((hi - lo) >> 1);
        if (s_cb[mid] < x) lo = mid + 1; else hi = mid;
    }
    const int r = lo > k - 1 ? k - 1 : lo;
    const int l = r - 1 < 0 ? 0 : r - 1;
    if (l == r) return (uint32_t)r;
    const float lv = s_cb[l], hv = s_cb[r];
    const float span = hv - lv;
    float v = x;
    v = v < lv ? lv : (v > hv ? hv : v);
    const float p_up = span > 0.0f ? (v - lv) / span : 0.0f;
    return sr_uniform(seed, elem) < p_up ? (uint32_t)r : (uint32_t)l;
}

// ------------------------------------------------------------- utilities

// Correctly rounded u / b given y = RN(1 / b) (y == 0 marks blocks where the
// reciprocal is not usable).  q0 = RN(u*y) is within 1 ulp of u/b, r = u - b*q0
// is exact in one fma, and RN(q0 + r*y) is RN(u/b) (Markstein's theorem) when
// nothing underflows; tiny |u| or an unusable y take the IEEE divide.
__device__ __forceinline__ float div_by_block(float u, float b, float y) {
    if (y != 0.0f && fabsf(u) >= 0x1p-100f) {
        const float q0 = u * y;
        if (fabsf(q0) >= 0x1p-100f) {
            const float r = __builtin_fmaf(-q0, b, u);
            return __builtin_fmaf(r, y, q0);
        }
    }
    return u / b;
}

// RN(u/d) for a divisor shared by many elements, with y = block_recip(d):
// div_by_block's Markstein step wherever nothing under- or overflows (u zero
// or 2^-100 <= |u|, |u*y| <= 2^100), the IEEE divide elsewhere.
__device__ __forceinline__ float div_by_const(float u, float d, float y) {
    const float q0 = u * y;
    const float aq = fabsf(q0);
    if (y != 0.0f && fabsf(u) >= 0x1p-100f && fabsf(u) <= 0x1p100f && aq >= 0x1p-100f && aq <= 0x1p100f) {
        const float r = __builtin_fmaf(-q0, d, u);
        return __builtin_fmaf(r, y, q0);
    }
    return u == 0.0f && y != 0.0f ? q0 : u / d;
}

// Reciprocal for div_by_block: RN(1/b) when b and 1/b are normal and finite.
__device__ __forceinline__ float block_recip(float b) {
    if (!(b >= 0x1p-125f) || !(b <= 0x1p125f)) return 0.0f;
    return 1.0f / b;
}

// floor(n / d) for 0 <= n < 2^53, d >= 1, with inv = 1.0 / d.
__device__ __forceinline__ int64_t div_floor(int64_t n, int64_t d, double inv) {
    int64_t q = (int64_t)((double)n * inv);
    const int64_t r = n - q * d;
    if (r < 0) q -= 1;
    else if (r >= d) q += 1;
    return q;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

// ---------------------------------------------------- DPP wave reductions
// GFX9 full-wave sequence (quad_perm 1032, quad_perm 2301, row_half_mirror,
// row_mirror, row_bcast:15 into rows 1/3, row_bcast:31 into rows 2/3): the
// total ends in lane 63.  No LDS traffic, unlike a shuffle.
template <int CTRL, int RMASK>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, RMASK, 0xf, false);
}
template <int CTRL, int RMASK>
__device__ __forceinline__ double dpp64(double v) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = dpp32<CTRL, RMASK>((uint32_t)b);
    const uint32_t hi = dpp32<CTRL, RMASK>((uint32_t)(b >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// sum over the wave, valid in lane 63
__device__ __forceinline__ double wave_sum_d63(double v) {
    v += dpp64<0xB1, 0xf>(v);
    v += dpp64<0x4E, 0xf>(v);
    v += dpp64<0x141, 0xf>(v);
    v += dpp64<0x140, 0xf>(v);
    v += dpp64<0x142, 0xa>(v);
    v += dpp64<0x143, 0xc>(v);
    return v;
}
// sum over each aligned group of 8 lanes, in all 8 (every lane adds the same
// two operands at each step, so the 8 results are bitwise equal)
__device__ __forceinline__ double group8_sum_d(double v) {
    v += dpp64<0xB1, 0xf>(v);
    v += dpp64<0x4E, 0xf>(v);
    v += dpp64<0x141, 0xf>(v);
    return v;
}
// sum over the wave, in every lane (lane 63's DPP total, read as a scalar)
__device__ __forceinline__ double wave_allsum_d(double v) {
    const uint64_t b = (uint64_t)__double_as_longlong(wave_sum_d63(v));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), 63);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// max over the wave, valid in lane 63
__device__ __forceinline__ uint32_t wave_max_u63(uint32_t v) {
    uint32_t o;
    o = dpp32<0xB1, 0xf>(v); v = o > v ? o : v;
    o = dpp32<0x4E, 0xf>(v); v = o > v ? o : v;
    o = dpp32<0x141, 0xf>(v); v = o > v ? o : v;
    o = dpp32<0x140, 0xf>(v); v = o > v ? o : v;
    o = dpp32<0x142, 0xa>(v); v = o > v ? o : v;
    o = dpp32<0x143, 0xc>(v); v = o > v ? o : v;
    return v;
}

// Stage the quantisation table parts a kernel needs into LDS.  thr is padded
// with +inf and bkt with a copy of its last bucket so the fast quantiser needs
// no bounds checks (x = 1 lands in bucket 4096).
struct SharedTables {
    float cbr[kCodebookMax];
    float thr[kCodebookMax + 4];
    uint32_t bkt[kBuckets + 4];
};

__device__ __forceinline__ void stage_tables(SharedTables& s, const QTable* __restrict__ t) {
    const int tid = threadIdx.x;
    const int nt = blockDim.x;
    const uint4* src = reinterpret_cast<const uint4*>(t->bucket);
    uint4* dst = reinterpret_cast<uint4*>(s.bkt);
    for (int i = tid; i < kBuckets / 4; i += nt) dst[i] = src[i];
    for (int i = tid; i < kCodebookMax; i += nt) {
        s.cbr[i] = t->cbr[i];
        s.thr[i] = t->thr[i];
    }
    if (tid < 4) {
        s.thr[kCodebookMax + tid] = __builtin_inff();
        s.bkt[kBuckets + tid] = t->bucket[kBuckets - 1];
    }
}

// Nearest index for x in [-1, 1] (never NaN).  Thresholds in later buckets
// are > x, so the first two slots from the bucket's base can be compared
// unconditionally; buckets holding more than two thresholds (`dense` tables
// only) continue with the remaining ones.
__device__ __forceinline__ uint32_t quant_fast(float x, const SharedTables& s, bool dense) {
    const int b = (int)__builtin_fmaf(x, (float)(kBuckets / 2), (float)(kBuckets / 2));
    const uint32_t e = s.bkt[b];
    const uint32_t base = e & 0xffffu;
    uint32_t idx = base + (s.thr[base] < x ? 1u : 0u) + (s.thr[base + 1] < x ? 1u : 0u);
    if (dense) {
        const uint32_t cnt = e >> 16;
        for (uint32_t j = 2; j < cnt; ++j) idx += (s.thr[base + j] < x) ? 1u : 0u;
    }
    return idx;
}

struct SharedSR {
    float cb[kCodebookMax];
    int16_t lut[kLutEntries + 7];
};

__device__ __forceinline__ void stage_sr(SharedSR& s, const QTable* __restrict__ t) {
    for (int i = threadIdx.x; i < kCodebookMax; i += blockDim.x) s.cb[i] = t->cb[i];
    for (int i = threadIdx.x; i < kLutEntries + 7; i += blockDim.x) s.lut[i] = t->lut[i];
}

// Hands block b's shard values base[sh * nb + b] to f in shard order, then
// zeroes them: every load is issued before any store (a store between them
// would make each load wait for the previous one, as the compiler cannot
// tell the addresses apart), eight at a time.
template <typename T, typename F>
__device__ __forceinline__ void drain_shards(T* base, int64_t shards, int64_t nb, int64_t b, F&& f) {
    int64_t sh = 0;
    for (; sh + 8 <= shards; sh += 8) {
        T v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = base[(sh + k) * nb + b];
#pragma unroll
        for (int k = 0; k < 8; ++k) f(v[k]);
    }
    for (; sh < shards; ++sh) f(base[sh * nb + b]);
    for (sh = 0; sh < shards; ++sh) base[sh * nb + b] = T(0);
}

}  // namespace gx
