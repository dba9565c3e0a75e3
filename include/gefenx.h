/*
 * gefenx.h -- C ABI of the MI355X-native Gefen optimizer step.
 *
 * Plain pointers, sizes and scalars only: no torch types cross this boundary.
 * Every device pointer must be a HIP device allocation on the current device;
 * kernels are enqueued on `stream` (hipStream_t passed as void*) and no call
 * synchronises the host except where stated.  Return value: GEFENX_OK (0) or a
 * negative status; gefenx_last_error() returns the thread-local message.
 * Status -> Python exception mapping used by the bindings:
 *   GEFENX_EINVAL -> ValueError, GEFENX_EDTYPE -> NotImplementedError,
 *   GEFENX_ELAUNCH / GEFENX_ENOMEM -> RuntimeError.
 *
 * Each entry point replaces one reference interface (paths relative to the
 * reference repo root, src/gefen/ omitted); the cited pybind function has the
 * same argument order except that tensors become (pointer, sizes) and the
 * launcher's internal `at::zeros` scratch becomes the caller-provided
 * workspace.
 */
#ifndef GEFENX_H_
#define GEFENX_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: the block-path workspace (GEFENX_WS_BLOCK) grew by one fixed-order
 * partial record per stats workgroup, sized from numel, so a block workspace
 * sized by a version-1 header is too small for the multi-tensor launcher.
 * 3: gefenx_tensor_desc gained the trailing field bc2_div.
 * Bindings compare gefenx_abi_version() with the version they were written
 * against and refuse a mismatch. */
#define GEFENX_ABI_VERSION 3

enum gefenx_status {
    GEFENX_OK = 0,
    GEFENX_EINVAL = -1,  /* bad shape/size/pointer/argument  -> ValueError          */
    GEFENX_EDTYPE = -2,  /* unsupported dtype (fp64)          -> NotImplementedError */
    GEFENX_ELAUNCH = -3, /* HIP launch/runtime failure        -> RuntimeError        */
    GEFENX_ENOMEM = -4   /* host allocation failure           -> RuntimeError        */
};

/* Parameter / gradient element type. */
enum gefenx_dtype { GEFENX_F32 = 0, GEFENX_F16 = 1, GEFENX_BF16 = 2, GEFENX_F64 = 3 };

/* Version of this ABI (GEFENX_ABI_VERSION of the built library). */
int gefenx_abi_version(void);

/* Thread-local message describing the last non-OK status of this thread. */
const char* gefenx_last_error(void);

/* ------------------------------------------------------------------------
 * Quantisation table.  The fused kernels never binary-search the codebook:
 * the host derives, once per (codebook, dtype), the exact fp32 decision
 * thresholds of the reference's nearest-codeword rule (searchsorted + "ties to
 * the lower index", gefen.py:288-334) plus a 4096-bucket index over them, the
 * reference's own search LUT (kernels/automatic_gefen_fused.py:81-121, used by
 * stochastic rounding) and the codebook rounded through the grad dtype (the
 * dequantisation of gefen.py:337-373).  The table is a flat byte image that
 * the caller copies to device memory unchanged.
 * ---------------------------------------------------------------------- */

/* Size in bytes of a table image. */
size_t gefenx_qtable_bytes(void);

/* Build the table image for `codebook` (k fp32 values, sorted ascending,
 * 1 <= k <= 256) and the grad dtype into host memory `table_out`.
 * Replaces _codebook_search_lut (kernels/automatic_gefen_fused.py:81-121). */
int gefenx_qtable_build(const float* codebook, int k, int dtype, void* table_out);

/* The reference's int16 search LUT (buckets+1 entries) on the host:
 * kernels/automatic_gefen_fused.py:81-121. */
int gefenx_search_lut(const float* codebook, int k, int buckets, int16_t* lut_out);

/* ------------------------------------------------------------------------
 * Workspace.  Every update entry point takes a device workspace whose size is
 * given by gefenx_workspace_bytes(kind, ...).  It must be zero-filled before
 * its first use; each call returns its accumulators and counters to zero (the
 * rest is scratch rewritten by every call), so one workspace per parameter can
 * be reused across steps (and inside a captured graph) without clearing.
 * ---------------------------------------------------------------------- */
enum gefenx_ws_kind { GEFENX_WS_FACTORED = 0, GEFENX_WS_BLOCK = 1, GEFENX_WS_MOMENTUM = 2 };
/* FACTORED: the parameter's [rows, cols] and block count.  BLOCK: rows * cols
 * = the parameter's numel (e.g. rows = 1, cols = numel) and its block count;
 * the block sums need per-workgroup records sized from numel.  MOMENTUM:
 * rows and cols unused. */
size_t gefenx_workspace_bytes(int kind, int64_t rows, int64_t cols, int64_t num_blocks);

/* ------------------------------------------------------------------------
 * Factored (row/column) second-moment step for one 2D parameter [rows, cols]
 * with the 8-bit quantised momentum over blocks of `period` elements in
 * logical row-major order.  Replaces gefen_factored_update_cuda:
 * kernels/automatic_gefen_fused_kernel.cu:2534-2790 (binding
 * kernels/automatic_gefen_fused_binding.cpp:89-110).
 *   p, grad : [rows, cols] of `dtype`, element strides (ps0, ps1) / (gs0, gs1)
 *             (transposed or otherwise strided views need no copy);
 *   m_codebook : uint8 [numel] (contiguous); m_magnitude : fp32 [numel/period];
 *   v_row fp32 [rows]; v_col fp32 [cols]; all mutated in place.
 *   step_scalars: NULL, or a device fp32[4] = [lr, 1/bc2, 1/bc1, wd_factor]
 *   overriding the host scalars (capturable mode);
 *   seed_dev: NULL or a device int64 overriding rng_seed.
 * ---------------------------------------------------------------------- */
int gefenx_factored_update(
    void* p, const void* grad, int dtype, int64_t rows, int64_t cols,
    int64_t ps0, int64_t ps1, int64_t gs0, int64_t gs1,
    uint8_t* m_codebook, float* m_magnitude, float* v_row, float* v_col,
    int64_t period, const void* qtable_dev,
    double beta1, double beta2, double lr, double eps,
    double inv_bias_correction_2, double inv_bias_correction_1,
    double weight_decay_factor, int stochastic_round, int64_t rng_seed,
    const float* step_scalars, const int64_t* seed_dev,
    void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * The factored step without a workspace argument and without allocating:
 * no counterpart in the reference.  For callers that cannot allocate device
 * memory at step time (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as
 * gefenx_factored_update minus (workspace, workspace_bytes): the kernels use
 * a static device array of GEFENX_NOALLOC_SCRATCH_BYTES per GPU (held until
 * the process ends), so shapes whose gefenx_workspace_bytes(GEFENX_WS_FACTORED,
 * ...) exceeds it are rejected with GEFENX_EINVAL (every Llama-3-8B and
 * Qwen3-4B tensor fits; the embedding needs 21 MiB).  The first call on a
 * device resolves the array's address there (make it outside a capture).
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (two streams, two threads) race.  The call clears what must start at zero
 * with a kernel, so it may be recorded into a graph.
 * ---------------------------------------------------------------------- */
#define GEFENX_NOALLOC_SCRATCH_BYTES (32u << 20)
int gefenx_factored_update_noalloc(
    void* p, const void* grad, int dtype, int64_t rows, int64_t cols,
    int64_t ps0, int64_t ps1, int64_t gs0, int64_t gs1,
    uint8_t* m_codebook, float* m_magnitude, float* v_row, float* v_col,
    int64_t period, const void* qtable_dev,
    double beta1, double beta2, double lr, double eps,
    double inv_bias_correction_2, double inv_bias_correction_1,
    double weight_decay_factor, int stochastic_round, int64_t rng_seed,
    const float* step_scalars, const int64_t* seed_dev, void* stream);

/* ------------------------------------------------------------------------
 * Block-vmean step (1D params, and 2D params with factored_v_2d=False).
 * Replaces automatic_gefen_fused_full_update_cuda
 * (kernels/automatic_gefen_fused_kernel.cu:2233-2409) and
 * automatic_gefen_fused_update_v2_full_cuda (:3029-3242); both reference
 * kernels compute the same step, and so does this single entry point.
 *   p, grad: numel elements, contiguous; vmean fp32 [numel/period].
 *   step_scalars: NULL or device fp32[4] = [lr, 1/sqrt(bc2), 1/bc1, wd_factor].
 * ---------------------------------------------------------------------- */
int gefenx_block_update(
    void* p, const void* grad, int dtype, int64_t numel, int64_t period,
    uint8_t* m_codebook, float* m_magnitude, float* vmean, const void* qtable_dev,
    double beta1, double beta2, double lr, double eps,
    double inv_sqrt_bias_correction_2, double inv_bias_correction_1,
    double weight_decay_factor, int stochastic_round, int64_t rng_seed,
    const float* step_scalars, const int64_t* seed_dev,
    void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Muon momentum: advance the quantised momentum by one EMA step and emit the
 * dense momentum (optionally Nesterov) in grad dtype.  Replaces
 * gefen_quantized_momentum_update_cuda
 * (kernels/automatic_gefen_fused_kernel.cu:2852-3027, binding :75-87).
 * Arithmetic of the reference's decomposed Muon momentum
 * (gefen_muon.py:1136-1144, 948-974): every intermediate rounds to the grad
 * dtype D; Nesterov out = D(fma(D(1-beta), g, D(out*beta))).
 * workspace: gefenx_workspace_bytes(GEFENX_WS_MOMENTUM, 0, 0, numel/period).
 * ---------------------------------------------------------------------- */
int gefenx_quantized_momentum_update(
    const void* grad, int dtype, int64_t numel, int64_t period,
    uint8_t* m_codebook, float* m_magnitude, const void* qtable_dev,
    void* momentum_out, double beta1, int stochastic_round, int64_t rng_seed,
    const int64_t* seed_dev, int nesterov,
    void* workspace, size_t workspace_bytes, void* stream);

/* Factored EMA alone, for row and column sums of squares:
 * v <- fma(1-beta2, sq * RN(1/n), RN(v*beta2)) with n = cols for v_row and
 * rows for v_col -- the GPU aten chain v.mul_(beta2).add_(sq.div_(n), 1-beta2)
 * that the reference's standalone kernel reproduces bit for bit (the fused
 * step's own EMA divides, as the reference's CPU step does).  rows == cols ==
 * 0 is a no-op; exactly one of them zero is GEFENX_EINVAL.  Replaces
 * gefen_factored_v_ema_cuda (kernels/automatic_gefen_fused_kernel.cu:1990-2042,
 * 2792-2850; binding kernels/automatic_gefen_fused_binding.cpp:114-120). */
int gefenx_factored_v_ema(float* v_row, float* v_col, const float* row_sq,
                          const float* col_sq, int64_t rows, int64_t cols,
                          double beta2, void* stream);

/* ------------------------------------------------------------------------
 * Momentum requantisation and apply with a per-block stepsize the caller
 * computed (the legacy partial update; no second moment, no weight decay):
 * the quantised momentum advances as in gefenx_block_update, then
 * p <- D(p - c[idx'] * mag' * stepsize[b] * lr) (lr == 0: p untouched).
 * stepsize: device fp32 [numel/period].  workspace:
 * gefenx_workspace_bytes(GEFENX_WS_BLOCK, 1, numel, numel/period).
 * Replaces automatic_gefen_fused_update_cuda and
 * automatic_gefen_fused_update_v2_cuda (kernels/automatic_gefen_fused_kernel.cu:
 * 331-415, 2102-2231, 2411-2532; binding
 * kernels/automatic_gefen_fused_binding.cpp:9-31); both compute this step.
 * ---------------------------------------------------------------------- */
int gefenx_momentum_apply(
    void* p, const void* grad, int dtype, int64_t numel, int64_t period,
    uint8_t* m_codebook, float* m_magnitude, const float* stepsize, const void* qtable_dev,
    double beta1, double lr, void* workspace, size_t workspace_bytes, void* stream);

/* Block vmean EMA alone.  Replaces automatic_vmean_update_cuda
 * (kernels/automatic_vmean_kernel.cu:122-214); bf16 squares/means round
 * through bf16 as the reference's decomposed path does (gefen.py:129-191). */
int gefenx_vmean_update(float* vmean, const void* grad, int dtype, int64_t numel,
                        int64_t period, double beta2, void* stream);

/* ------------------------------------------------------------------------
 * Step-1 helpers.
 * ---------------------------------------------------------------------- */

/* Block-absmax-normalised histogram accumulated into int64 bin_counts[bins]
 * (bins <= 4096).  Replaces gefen_exact_histogram_cuda
 * (kernels/exact_histogram_fused_kernel.cu:144-180). */
int gefenx_exact_histogram(const void* grad, int dtype, int64_t numel, int64_t period,
                           int64_t* bin_counts, int bins, void* stream);

/* Within-block variance error for every divisor period in `periods[n]` at
 * once: err[i] = sqrt(mean over blocks of var(x)), x = grad^2 (fp32 square,
 * float64 arithmetic, two-pass variance as numpy's var).  Replaces the
 * per-divisor average_within_block_variance_cuda
 * (kernels/period_variance_kernel.cu:82-164) and the CPU backend
 * (partitioning.py:62-84).  err_dev: device double[n].  Synchronous. */
int gefenx_block_variance_errors(const void* grad, int dtype, int64_t numel,
                                 const int64_t* periods, int n_periods,
                                 double* err_host, void* stream);

/* The same with the reference kernel's input_is_squared switch
 * (kernels/period_variance_kernel.cu:15-80, 82-164; binding
 * kernels/period_variance_binding.cpp): nonzero takes x = fp32(value) (the
 * caller already squared), zero squares as above.  Backs
 * average_within_block_variance_cuda_kernel (kernels/period_variance.py:62-85)
 * and the gefen::average_within_block_variance_cuda custom op. */
int gefenx_block_variance_errors_ex(const void* grad, int dtype, int64_t numel,
                                    const int64_t* periods, int n_periods,
                                    int input_is_squared, double* err_host, void* stream);

/* Exact optimal 1-D weighted k-means codebook (host, float64 DP with forced
 * +-1 endpoints), from active histogram bins.  Replaces quantization.exact_dp
 * (quantization.py:197-253).  codebook_out receives k sorted fp32 values. */
int gefenx_exact_dp(const float* active_centers, const float* active_counts,
                    int n_points, int k, int force_endpoints, float* codebook_out);

/* The same solver with each DP level on the device (one launch per centre,
 * every segment end in parallel), bit-identical to gefenx_exact_dp; host
 * inputs and output, synchronous on `stream`.  Replaces the same
 * quantization.exact_dp (quantization.py:197-253). */
int gefenx_exact_dp_device(const float* active_centers, const float* active_counts,
                           int n_points, int k, int force_endpoints, float* codebook_out,
                           void* stream);

/* ------------------------------------------------------------------------
 * Multi-tensor step: one launch sequence for many parameters.  No
 * counterpart in the reference (its fused path is one call per parameter,
 * gefen.py:5760-5761); it replaces the per-parameter loop of Gefen.step
 * (gefen.py:5783-5820) for the fused path.
 * ---------------------------------------------------------------------- */
typedef struct gefenx_tensor_desc {
    void* p;                /* param data */
    const void* grad;       /* grad data */
    uint8_t* m_codebook;    /* uint8 [numel] */
    float* m_magnitude;     /* fp32 [numel/period] */
    float* v0;              /* factored: v_row [rows];  block: vmean [nb] */
    float* v1;              /* factored: v_col [cols];  block: unused (NULL) */
    void* workspace;        /* zero-filled, gefenx_workspace_bytes(...) bytes */
    int64_t rows, cols;     /* logical 2D shape (1D: rows=1, cols=numel) */
    int64_t ps0, ps1;       /* param element strides */
    int64_t gs0, gs1;       /* grad element strides.  Factored: any strides
                             * (logical row-major order; transposed views,
                             * strides (1, ld), take tiled kernels when rows,
                             * cols and period are multiples of 8).  Block:
                             * contiguous, or a grad that is contiguous or such
                             * a transposed view (GEFENX_EINVAL otherwise). */
    int64_t period;
    int32_t dtype;          /* gefenx_dtype of p and grad */
    int32_t factored;       /* 1: factored second moment; 0: block vmean */
    float lr, eps, inv_bc2, inv_bc1, wd_factor;
    /* inv_bc2: factored 1/bc2, block 1/sqrt(bc2) */
    float lerp_w;           /* (float)(1 - beta1): momentum lerp weight */
    float beta2;            /* (float)beta2 */
    float alpha2;           /* (float)(1 - beta2), rounded from double */
    float bc2_div;          /* the divisor of the reference's CPU step, or 0:
                             * factored (float)bc2, block (float)sqrt(bc2).
                             * Given (and no step_scalars row), the step size
                             * rounds as the reference's decomposed step does
                             * (gefen.py:2996-3006, 3794-3805): the block path
                             * h = sqrt(vmean) / bc2_div + eps for every dtype,
                             * the factored path vh = (v_row * v_col) / mean,
                             * h = sqrt(vh / bc2_div) + eps for fp32
                             * parameters.  0: the kernels multiply by inv_bc2
                             * (within 1e-6 of that). */
} gefenx_tensor_desc;

/* Step every tensor in descs[n] (host array; copied to the device inside the
 * call).  All tensors share the codebook table `qtable_dev` of their dtype:
 * qtables_dev[dtype] (array of 3 device pointers, indexed by gefenx_dtype).
 * rng_seed / stochastic_round apply to all. */
int gefenx_multi_tensor_step(const gefenx_tensor_desc* descs, int n,
                             const void* const* qtables_dev, int stochastic_round,
                             int64_t rng_seed, void* desc_scratch_dev,
                             size_t desc_scratch_bytes, void* stream);

/* Bytes of device scratch gefenx_multi_tensor_step needs for n tensors
 * (descriptors and the workgroup -> tensor segment tables). */
size_t gefenx_multi_tensor_scratch_bytes(int n);

/* ------------------------------------------------------------------------
 * Capturable step (graph capture / replay).  Replaces the reference's
 * capturable machinery: the per-parameter device scalar buffer refresh
 * (_refresh_capturable_step_scalars, gefen.py:1929-2005, and its batched
 * cohort form _capt_batched_refresh, gefen.py:2006-2465), the device global
 * step and stochastic-rounding seed (_advance_gefen_global_step /
 * _advance_sr_seeds, gefen.py:1842-1853, 1872-1885) and the kernels' device
 * scalar / seed pointers (resolve_step_scalars_ptr / resolve_seed_dev_ptr,
 * kernels/automatic_gefen_fused_kernel.cu:2044-2098).
 *
 * A plan is built once on the host for a fixed set of tensors (pointers,
 * shapes, periods, hyperparameters) and launched every step.  A launch
 * enqueues kernels only -- no host synchronisation, copy node or memset -- so
 * it can be recorded into a graph and replayed:
 *   1. the plan's descriptor image is copied into its device buffer by a
 *      kernel that reads the plan's pinned host image (only on the first
 *      launch into a buffer, and on every launch recorded by a capture);
 *   2. the prologue kernel advances every parameter's device step counters
 *      and writes its fp32[4] scalar row, and advances the global step /
 *      seed counter;
 *   3. the multi-tensor stats / finalize / apply launches, each tensor
 *      reading its scalars and the stochastic-rounding seed from the device.
 * ---------------------------------------------------------------------- */
typedef struct gefenx_capt_desc {
    float* step;            /* device fp32 0-dim: state["step"] (+= 1) */
    float* bc2_step;        /* device fp32 0-dim: factored_step or vmean_step (+= 1);
                             * NULL: none (bc2 then uses `step`) */
    float* scalars;         /* device fp32[4] written: lr, 1/bc2 (factored) or
                             * 1/sqrt(bc2) (block), 1/bc1, weight-decay factor */
    const void* lr_dev;     /* NULL: the host `lr` below; else a device 0-dim lr */
    double lr;              /* host lr (used when lr_dev is NULL) */
    double weight_decay;
    double beta1, beta2;
    int32_t lr_dtype;       /* dtype of *lr_dev: GEFENX_F32 or GEFENX_F64 */
    int32_t sqrt_bc2;       /* 1: block path (1/sqrt(bc2)); 0: factored (1/bc2) */
} gefenx_capt_desc;

typedef struct gefenx_mt_plan gefenx_mt_plan;

/* Build a plan.  descs[n]: as gefenx_multi_tensor_step (their lr / inv_bc2 /
 * inv_bc1 / wd_factor fields are ignored when step_scalars[i] is set).
 * step_scalars: NULL, or n device fp32[4] rows (NULL entries allowed) that
 * the tensors read their per-step scalars from.  capt[n_capt]: counters and
 * scalar rows the prologue refreshes (any tensors, also ones stepped by the
 * single-tensor entry points with the same scalar rows).  counter_dev: NULL,
 * or a device int64[3] = {global step, next seed, seed of the running step}:
 * each launch sets [2] = [1], then increments [0] and [1]; with
 * stochastic_round the tensors take their rounding seed from [2] instead of
 * rng_seed.  Host work only (validation, layout, pinned image); allowed
 * while a stream is being captured.  The arrays are copied. */
int gefenx_mt_plan_create(const gefenx_tensor_desc* descs, int n, const float* const* step_scalars,
                          const void* const* qtables_dev, int stochastic_round, int64_t rng_seed,
                          const gefenx_capt_desc* capt, int n_capt, int64_t* counter_dev,
                          gefenx_mt_plan** plan_out);

/* Bytes of the device buffer a launch of `plan` needs. */
size_t gefenx_mt_plan_device_bytes(const gefenx_mt_plan* plan);

/* Enqueue one step of `plan` on `stream` (see above).  dev_buf: a device
 * buffer of gefenx_mt_plan_device_bytes(plan) bytes owned by the caller for
 * the plan's lifetime; once a launch has uploaded into it outside a capture,
 * later launches on the same stream skip the copy.  Launches of one plan on
 * several streams at once race. */
int gefenx_mt_plan_launch(gefenx_mt_plan* plan, void* dev_buf, size_t dev_bytes, void* stream);

/* Free a plan (synchronises the device before its pinned image is freed).
 * Never call it while a graph that recorded a launch of the plan may still
 * be replayed. */
void gefenx_mt_plan_destroy(gefenx_mt_plan* plan);

/* ------------------------------------------------------------------------
 * Newton-Schulz orthogonalisation of a batch of matrices on bf16 MFMA.
 * Replaces _zeropower_via_newtonschulz / _zeropower_via_newtonschulz_batched
 * (gefen_muon.py:236-291, 353-393).  in: [batch, rows, cols] contiguous of
 * in_dtype (the dense momentum); it is rounded to bf16, transposed when
 * rows > cols, divided by max(bf16(||X||_F), eps), then for i < steps:
 * G = XX^T, B = b_i G + c_i G G, X = a_i X + B X, each product rounded to
 * bf16 (fp32 accumulation).  out: bf16 [batch, rows, cols] in the input's
 * orientation.  abc: steps x (a, b, c) doubles.  workspace:
 * gefenx_ns_workspace_bytes(batch, rows, cols) bytes (any contents).
 * ---------------------------------------------------------------------- */
size_t gefenx_ns_workspace_bytes(int64_t batch, int64_t rows, int64_t cols);
int gefenx_newton_schulz(const void* in, int in_dtype, void* out, int64_t batch, int64_t rows,
                         int64_t cols, const double* abc, int steps, double eps, void* workspace,
                         size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Batched Muon launches over matrices of one shape [rows, cols] (one launch
 * set per up to 16 matrices instead of one per matrix; the reference steps
 * them one at a time, gefen_muon.py:1064-1146, 1192-1300).  Each matrix is
 * described by one gefenx_muon_item; the fields a call does not read may be
 * left zero.  Grads and parameters may be strided views (logical row-major
 * order), as in gefenx_tensor_desc.
 * ---------------------------------------------------------------------- */
typedef struct gefenx_muon_item {
    const void* grad;            /* momentum: grad [rows, cols] of the batch dtype */
    int64_t grad_stride0, grad_stride1;
    uint8_t* m_codebook;         /* momentum: indices [numel] */
    float* m_magnitude;          /* momentum: fp32 [numel/period] */
    int64_t period;
    void* workspace;             /* momentum: GEFENX_WS_MOMENTUM workspace of this matrix */
    size_t workspace_bytes;
    void* param;                 /* apply: parameter [rows, cols] */
    int64_t param_stride0, param_stride1;
    float* normuon_v;            /* NorMuon: fp32 [rows], mutated */
    const float* normuon_step_dev; /* NorMuon: device fp32 step counter (capturable) or NULL */
    int64_t normuon_step;        /* NorMuon: host step (>= 1) when normuon_step_dev is NULL */
    const float* step_scalars;   /* apply: capturable scalar row fp32[4] or NULL */
} gefenx_muon_item;

/* gefenx_quantized_momentum_update for n matrices; matrix i emits its dense
 * momentum to momentum_out + i * rows * cols (elements of the grad dtype). */
int gefenx_muon_momentum_batch(const gefenx_muon_item* items, int n, int dtype, int64_t rows,
                               int64_t cols, const void* qtable_dev, void* momentum_out, double beta1,
                               int stochastic_round, int64_t rng_seed, const int64_t* seed_dev,
                               int nesterov, void* stream);

/* gefenx_normuon_scale for n matrices: update [n, rows, cols] bf16, scale_out
 * [n, rows] bf16; workspace: gefenx_normuon_batch_workspace_bytes(n, rows). */
size_t gefenx_normuon_batch_workspace_bytes(int n, int64_t rows);
int gefenx_normuon_scale_batch(const gefenx_muon_item* items, int n, const void* update,
                               int64_t rows, int64_t cols, double beta2, double eps, void* scale_out,
                               void* workspace, size_t workspace_bytes, void* stream);

/* gefenx_muon_apply for n matrices: update [n, rows, cols] bf16, row_scale
 * [n, rows] bf16 or NULL; each item's param, strides and step_scalars.
 * cautious_counts: NULL, or the agreement counts of
 * gefenx_muon_cautious_count_batch for the same items and update: then each
 * update element is cautiously masked (gefen_muon.py:396-405, 1148-1162)
 * against the item's grad after the NorMuon row scale. */
int gefenx_muon_apply_batch(const gefenx_muon_item* items, int n, int dtype, const void* update,
                            const void* row_scale, int64_t rows, int64_t cols, double lr,
                            double weight_decay, double adjusted_lr, double lr_ratio,
                            const uint64_t* cautious_counts, void* stream);

/* Cautious-mask agreement counts (gefen_muon.py:396-405): counts[i] (device
 * uint64) = #elements of matrix i where u' * grad > 0, u' the bf16 update
 * [n, rows, cols] (times row_scale [n, rows] bf16 when not NULL, rounded to
 * bf16) and grad the item's gradient view of dtype `dtype`, the product
 * taken in torch's promoted dtype (bf16 for bf16 grads, else fp32).  The
 * counters are cleared by the call (a kernel, so it can be captured). */
int gefenx_muon_cautious_count_batch(const gefenx_muon_item* items, int n, int dtype, const void* update,
                                     const void* row_scale, int64_t rows, int64_t cols, uint64_t* counts,
                                     void* stream);

/* NorMuon row scale of a bf16 update [rows, cols] (gefen_muon.py:1192-1230):
 * normuon_v (fp32 [rows], mutated) <- v*beta2 + row_sq*((1-beta2)/cols);
 * scale_out (bf16 [rows]) = bf16(frob_scale / (sqrt(v/(1-beta2^step)) + eps)).
 * step_dev: NULL, or a device fp32 0-dim step counter read instead of `step`
 * (capturable mode; the counter is advanced by the capturable prologue).
 * workspace: gefenx_normuon_workspace_bytes(rows) bytes. */
size_t gefenx_normuon_workspace_bytes(int64_t rows);
int gefenx_normuon_scale(const void* update, int64_t rows, int64_t cols, float* normuon_v,
                         double beta2, int64_t step, double eps, void* scale_out,
                         void* workspace, size_t workspace_bytes, const float* step_dev,
                         void* stream);

/* Muon parameter update (gefen_muon.py:1286-1300): p = D(p*(1-lr*wd)) when
 * weight_decay > 0, then p = D(fma(u, D(-adjusted_lr), p)) with u the bf16
 * update [rows, cols], multiplied first by row_scale (bf16 [rows], NorMuon)
 * and rounded to bf16 when row_scale is not NULL.  step_scalars: NULL, or a
 * device fp32[4] scalar row of the capturable prologue (gefenx_capt_desc):
 * then 1-lr*wd is its [3] and adjusted_lr = (double)[0] * lr_ratio
 * (capturable mode, gefen_muon.py:1243-1270). */
int gefenx_muon_apply(void* p, int dtype, const void* update, const void* row_scale,
                      int64_t rows, int64_t cols, double lr, double weight_decay,
                      double adjusted_lr, const float* step_scalars, double lr_ratio,
                      void* stream);

/* The Newton-Schulz GEMM alone: D = bf16(alpha * A B^T + beta * C) for bf16
 * row-major A [M, K], B [N, K], C / D [M, N] (C may be NULL; K >= 1, K == 0
 * is GEFENX_EINVAL; M or N == 0 is a no-op).  No counterpart
 * in the reference (its Newton-Schulz calls torch.matmul / addmm); exposed
 * for testing and measuring the MFMA kernel. */
int gefenx_gemm_nt_bf16(const void* A, const void* B, const void* C, void* D, int64_t M,
                        int64_t N, int64_t K, float alpha, float beta, void* stream);

/* ------------------------------------------------------------------------
 * Kernel timing.  When enabled, every update-kernel launch is bracketed by
 * HIP events on its own stream and tagged with its kind and algorithmic
 * bytes (compulsory traffic of the step it belongs to); gefenx_profile_read
 * synchronises those events and returns the totals of one kind.  No
 * counterpart in the reference (its benches time with CUDA events from
 * Python, benchmarks/microbench/microbench_v1v2.py:36-47).
 * kinds: 0 stats and 2 apply of the factored (2D) path, 1 finalize (both
 * paths, incl. the mean(v_row) launch), 5 stats and 6 apply of the block
 * path, 3 momentum, 4 newton-schulz gemm.
 * ---------------------------------------------------------------------- */
enum gefenx_kernel_kind {
    GEFENX_K_STATS = 0, GEFENX_K_FINALIZE = 1, GEFENX_K_APPLY = 2,
    GEFENX_K_MOMENTUM = 3, GEFENX_K_NS_GEMM = 4, GEFENX_K_BLOCK_STATS = 5,
    GEFENX_K_BLOCK_APPLY = 6, GEFENX_K_COUNT = 7
};
int gefenx_profile_enable(int on);
int gefenx_profile_read(int kind, double* total_ms, int64_t* launches, double* algo_bytes,
                        double* algo_flops);
int gefenx_profile_reset(void);

#ifdef __cplusplus
}
#endif
#endif /* GEFENX_H_ */
