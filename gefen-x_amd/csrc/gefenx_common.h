// gefenx_common.h -- shared host/device definitions of the MI355X Gefen step.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace gx {

enum DType : int { F32 = 0, F16 = 1, BF16 = 2, F64 = 3 };

constexpr int kCodebookMax = 256;
constexpr int kBuckets = 4096;        // bucket index over [-1, 1] (2^12)
constexpr int kLutEntries = kBuckets + 1;
constexpr int kFqEntries = kBuckets + 8;  // fast-quantiser entries incl. padding (x = 1 lands in 4096)

// Byte image of the quantisation table (gefenx_qtable_build).  Plain data,
// copied verbatim to device memory; kernels stage the parts they need in LDS.
struct QTable {
    int32_t k;                       // codebook size (1..256)
    int32_t dtype;                   // grad dtype the dequant table rounds through
    int32_t n_thr;                   // k - 1 decision thresholds
    int32_t max_cnt;                 // most thresholds falling in one bucket
    float cb[kCodebookMax];          // raw fp32 codebook (padded with its last entry)
    float cbr[kCodebookMax];         // codebook rounded through the grad dtype
    float thr[kCodebookMax];         // thr[i] = largest x in [-1,1] with nearest(x) <= i
    uint32_t bucket[kBuckets];       // base | (count << 16) of thresholds per bucket
    int16_t lut[kLutEntries + 7];    // reference search LUT (stochastic rounding)
    // Fast quantiser, one 8-byte entry per bucket: {bits of thr[base], base}.
    // When no bucket holds more than one threshold (max_cnt <= 1) the nearest
    // index of x in bucket b is base + (thr[base] < x).
    uint32_t fq[2 * kFqEntries];
};

static_assert(sizeof(QTable) % 16 == 0, "QTable must stay 16-byte aligned in size");

// Workspace layouts (all sub-arrays 256-byte aligned).  Accumulators are
// zero on entry and left zero on exit by the finalize kernels.
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Factored stats tiling: a workgroup covers kFactTileCols columns (64 lanes x
// two 8-column chunks) of `tile_rows` consecutive rows.  Tiles hold about
// N/32 elements, between 64K (16K-element tiles spend a third of the pass on
// per-workgroup set-up and flushes) and 1M.  The multi-tensor launch puts
// every parameter's tiles in one grid, largest tiles first, so fewer, larger
// tiles cost no occupancy until the last round of workgroups, one of the
// smallest tiles, runs part-empty.  Measured (stats kernel on the Llama-3-8B
// set, tiles ordered by size): caps of 256K / 512K / 768K / 1M / 1.5M / 2M
// 4.29-4.31 / 4.08 / 4.01-4.04 / 3.96-3.99 / 4.05-4.07 / 3.95-3.96 ms (1.5M
// and 2M leave 4096-row tensors a short last row tile; 1M splits the common
// shapes evenly).  The tiling is per tensor, so a tensor's float64 partials
// do not depend on the other tensors of its launch.
constexpr int64_t kFactTileCols = 1024;
constexpr int64_t kFactTileMinElems = 1 << 16;
constexpr int64_t kFactTileMaxElems = 1 << 20;

// Transposed-view stats (strides (1, ld)) use the same column tiles but row
// tiles of whole 64-row bands, at most kTvStatsMaxRows rows.
constexpr int64_t kTvStatsMaxRows = 256;

struct FactTiles {
    int64_t ct, rt, tile_rows;
    int64_t rt_tv, tv_rows;  // row tiles of the transposed-view stats kernel
    static FactTiles make(int64_t rows, int64_t cols) {
        FactTiles t;
        t.ct = (cols + kFactTileCols - 1) / kFactTileCols;
        if (t.ct < 1) t.ct = 1;
        const int64_t tc = cols < kFactTileCols ? (cols < 1 ? 1 : cols) : kFactTileCols;
        int64_t elems = rows * cols / 32;
        elems = elems < kFactTileMinElems ? kFactTileMinElems : (elems > kFactTileMaxElems ? kFactTileMaxElems : elems);
        int64_t tr = (elems + tc - 1) / tc;
        tr = (tr + 7) & ~int64_t(7);  // whole two-row steps for each of the 4 waves
        if (tr > rows) tr = rows;
        if (tr < 1) tr = 1;
        t.tile_rows = tr;
        t.rt = (rows + tr - 1) / tr;
        if (t.rt < 1) t.rt = 1;
        int64_t tv = (tr + 63) & ~int64_t(63);
        if (tv > kTvStatsMaxRows) tv = kTvStatsMaxRows;
        if (tv > rows) tv = rows < 1 ? 1 : rows;
        t.tv_rows = tv;
        t.rt_tv = (rows + tv - 1) / tv;
        if (t.rt_tv < 1) t.rt_tv = 1;
        return t;
    }
};

// Block-max (and block-path sum-of-squares) accumulators are sharded when
// there are few blocks: workgroup w folds into shard (w % shards), so one huge
// block is not a single atomic hot spot; the finalize kernels reduce the
// shards in a fixed order.
constexpr int64_t kMagShardMaxBlocks = 4096;
constexpr int64_t kMagShards = 32;
inline int64_t mag_shards(int64_t nb) { return nb <= kMagShardMaxBlocks ? kMagShards : 1; }

// Rows of v_row handled per finalize workgroup (one float64 partial of
// sum(v_row) each; the apply kernel adds the partials in a fixed order).
constexpr int64_t kFinRowsPerWg = 256;

struct FactoredWs {
    // double row_part[ct][rows], double col_part[max(rt, rt_tv)][cols] (per-tile partial
    // sums, fully rewritten every step), uint32 magbits[shards][nb] (zero
    // between steps), float mag_old[nb], float minv[nb],
    // double vrow_sum[ceil(rows/256)] (partials of sum(v_row)), float vcs[cols] (sqrt(v_col)),
    // {uint32 finalize counter (zero between steps), float mean(v_row)}
    size_t off_rowp, off_colp, off_magbits, off_magold, off_minv, off_vsum, off_vcs, off_fin, total;
    static FactoredWs make(int64_t rows, int64_t cols, int64_t nb) {
        FactoredWs w;
        const FactTiles t = FactTiles::make(rows, cols);
        size_t o = 0;
        w.off_rowp = o;    o += align256(sizeof(double) * (size_t)(t.ct * rows));
        const int64_t rt = t.rt > t.rt_tv ? t.rt : t.rt_tv;  // either stats layout fits
        w.off_colp = o;    o += align256(sizeof(double) * (size_t)(rt * cols));
        w.off_magbits = o; o += align256(sizeof(uint32_t) * (size_t)(nb * mag_shards(nb)));
        w.off_magold = o;  o += align256(sizeof(float) * (size_t)nb);
        w.off_minv = o;    o += align256(sizeof(float) * (size_t)nb);
        w.off_vsum = o;    o += align256(sizeof(double) * (size_t)((rows + kFinRowsPerWg - 1) / kFinRowsPerWg));
        w.off_vcs = o;     o += align256(sizeof(float) * (size_t)cols);
        w.off_fin = o;     o += 256;
        w.total = o;
        return w;
    }
};

// Block stats record of one workgroup: the sums of squares of its first and
// last block (key -1: none), which may continue in neighbouring workgroups.
struct DetRec {
    int64_t kf;
    double sf;
    int64_t kl;
    double sl;
};

// Elements per workgroup of the block stats with one element per item (the
// smallest geometry, so it bounds the record count).
constexpr int64_t kBlockStatsMinElems = 8 * 256;

struct BlockWs {
    // double blk_sq[shards][nb] (zero between steps), uint32
    // magbits[shards][nb] (zero between steps), float mag_old[nb], float
    // step[nb], float minv[nb], DetRec rec[ceil(numel / kBlockStatsMinElems)]
    size_t off_sq, off_magbits, off_magold, off_step, off_minv, off_rec, total;
    static BlockWs make(int64_t nb, int64_t numel) {
        BlockWs w;
        size_t o = 0;
        w.off_sq = o;      o += align256(sizeof(double) * (size_t)(nb * mag_shards(nb)));
        w.off_magbits = o; o += align256(sizeof(uint32_t) * (size_t)(nb * mag_shards(nb)));
        w.off_magold = o;  o += align256(sizeof(float) * (size_t)nb);
        w.off_step = o;    o += align256(sizeof(float) * (size_t)nb);
        w.off_minv = o;    o += align256(sizeof(float) * (size_t)nb);
        w.off_rec = o;     o += align256(sizeof(DetRec) * (size_t)((numel + kBlockStatsMinElems - 1) /
                                                                   kBlockStatsMinElems));
        w.total = o;
        return w;
    }
};

struct MomentumWs {
    size_t off_magbits, off_magold, off_minv, total;
    static MomentumWs make(int64_t nb) {
        MomentumWs w;
        size_t o = 0;
        w.off_magbits = o; o += align256(sizeof(uint32_t) * (size_t)(nb * mag_shards(nb)));
        w.off_magold = o;  o += align256(sizeof(float) * (size_t)nb);
        w.off_minv = o;    o += align256(sizeof(float) * (size_t)nb);
        w.total = o;
        return w;
    }
};

}  // namespace gx
