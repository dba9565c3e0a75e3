// gefenx_common.h -- shared host/device definitions of the MI355X Gefen step.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace gx {

enum DType : int { F32 = 0, F16 = 1, BF16 = 2, F64 = 3 };

constexpr int kCodebookMax = 256;
constexpr int kBuckets = 4096;        // bucket index over [-1, 1] (2^12)
constexpr int kLutEntries = kBuckets + 1;

// Byte image of the quantisation table (gefenx_qtable_build).  Plain data,
// copied verbatim to device memory; kernels stage the parts they need in LDS.
struct QTable {
    int32_t k;                       // codebook size (1..256)
    int32_t dtype;                   // grad dtype the dequant table rounds through
    int32_t n_thr;                   // k - 1 decision thresholds
    int32_t pad0;
    float cb[kCodebookMax];          // raw fp32 codebook (padded with its last entry)
    float cbr[kCodebookMax];         // codebook rounded through the grad dtype
    float thr[kCodebookMax];         // thr[i] = largest x in [-1,1] with nearest(x) <= i
    uint32_t bucket[kBuckets];       // base | (count << 16) of thresholds per bucket
    int16_t lut[kLutEntries + 7];    // reference search LUT (stochastic rounding)
};

static_assert(sizeof(QTable) % 16 == 0, "QTable must stay 16-byte aligned in size");

// Workspace layouts (all sub-arrays 256-byte aligned).  Accumulators are
// zero on entry and left zero on exit by the finalize kernels.
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct FactoredWs {
    // double row_sq[rows], double col_sq[cols], uint32 magbits[nb],
    // float mag_old[nb], float scalars[4] (mean_r, ...)
    size_t off_row, off_col, off_magbits, off_magold, off_scal, total;
    static FactoredWs make(int64_t rows, int64_t cols, int64_t nb) {
        FactoredWs w;
        size_t o = 0;
        w.off_row = o;     o += align256(sizeof(double) * (size_t)rows);
        w.off_col = o;     o += align256(sizeof(double) * (size_t)cols);
        w.off_magbits = o; o += align256(sizeof(uint32_t) * (size_t)nb);
        w.off_magold = o;  o += align256(sizeof(float) * (size_t)nb);
        w.off_scal = o;    o += 256;
        w.total = o;
        return w;
    }
};

struct BlockWs {
    // double blk_sq[nb], uint32 magbits[nb], float mag_old[nb], float step[nb]
    size_t off_sq, off_magbits, off_magold, off_step, total;
    static BlockWs make(int64_t nb) {
        BlockWs w;
        size_t o = 0;
        w.off_sq = o;      o += align256(sizeof(double) * (size_t)nb);
        w.off_magbits = o; o += align256(sizeof(uint32_t) * (size_t)nb);
        w.off_magold = o;  o += align256(sizeof(float) * (size_t)nb);
        w.off_step = o;    o += align256(sizeof(float) * (size_t)nb);
        w.total = o;
        return w;
    }
};

struct MomentumWs {
    size_t off_magbits, off_magold, total;
    static MomentumWs make(int64_t nb) {
        MomentumWs w;
        size_t o = 0;
        w.off_magbits = o; o += align256(sizeof(uint32_t) * (size_t)nb);
        w.off_magold = o;  o += align256(sizeof(float) * (size_t)nb);
        w.total = o;
        return w;
    }
};

}  // namespace gx
