/*
 * credit.h -- C-ABI of libcredit_hip.so, the MI355X (gfx950) wide-row kernels.
 *
 * In the reference (zhengxiongli08/CREDIT) the native code sits behind a
 * process boundary: dsmem_eval/runner.py:280-310 spawns one CUDA executable
 * per workload (`build/<workload> --csv --rows R --n-values ... --cluster-size P`)
 * and parses its `RESULT,...` stdout line (src/workloads/layernorm_backward.cu:
 * 730-765, parsed at dsmem_eval/runner.py:258-277); the in-process operator
 * form of the same workloads is the Triton launcher table
 * `launcher(inputs, outputs, block_size, num_warps)` of
 * dsmem_eval/triton_kernels.py:300-400.  This library replaces both with
 * in-process calls: plain device pointers and sizes, no torch types.
 *
 * Contract shared by every compute entry point:
 *  - Ownership: the caller owns every buffer.  Pointers are device pointers,
 *    borrowed for the duration of the (asynchronous) call.
 *  - Layout: row-major, contiguous, rows x cols.  bf16 tensors are passed as
 *    uint16_t bit patterns.  Vectorised paths need 16-byte aligned rows; other
 *    shapes take a scalar path, they are never rejected for alignment alone.
 *  - Errors: every function returns 0 (CREDIT_OK) or a negative CREDIT_ERR_*
 *    code; credit_last_error() gives the message (thread-local).  Nothing
 *    exits or throws across the ABI.  Arguments are validated on the host
 *    before any HIP call, so a bad call never reaches the GPU.
 *  - Streams: work is enqueued on cfg->stream (a hipStream_t; NULL means the
 *    null stream).  cfg itself may be NULL (= all defaults).
 *  - Workspace: split-row variants exchange partial results through a device
 *    buffer: a 256-byte header (the watchdog word, the exchange-tag sequence
 *    and an exit count), a 1 MiB counter area (ticket dispensers, arrival
 *    counters), a 4 MiB area of tagged exchange slots, then per-call scratch
 *    (dweight partials, the FFN's hidden activation, ...).
 *    - cfg->workspace == NULL: the library keeps one buffer per (device,
 *      stream) and grows it on demand.  Calls on one stream run in order,
 *      calls on different streams get different buffers, so concurrent
 *      streams never share partials.  The first call on a stream (and any
 *      call that needs a larger buffer) allocates with hipMalloc, so such a
 *      call cannot be captured into a HIP graph; a grown-out buffer is
 *      retired, not freed, while work queued earlier may still use it.
 *    - cfg->workspace set: it must hold credit_workspace_bytes(...) bytes,
 *      be 256-byte aligned, and its first 5 MiB + 256 bytes (header,
 *      counters, slots) must read zero before its first use.  Calls keep
 *      those bytes in that state, so no clearing is needed between calls;
 *      the scratch part is overwritten freely.  Calls that share one caller
 *      workspace must not run concurrently (on different streams).
 *    - Exchange tags come from the header's sequence word, which each split
 *      launch reads as it starts and its last workgroup advances on the
 *      device; the launch that takes it past 3 * 2^30 returns the slot area
 *      to zero and restarts it.  Nothing about the tags is fixed at enqueue
 *      time, so a split call captured into a HIP graph (on a stream whose
 *      workspace exists, a caller workspace, or the allocation-free entry
 *      point) computes correct results on every replay.
 *  - Split launches and co-residency: the SPLIT kernels (and AUTO when it
 *    splits a row) size their grid to the workgroups the device holds at
 *    once and wait inside a group for all of its members.  They need the
 *    device's CUs to themselves: a kernel on another stream that occupies
 *    CUs meanwhile can delay members until the bounded wait (about 2^21
 *    polls, 1-2 s) expires.  The launch then finishes with wrong outputs
 *    and raises the workspace's watchdog word and a host-mapped word of the
 *    device; the call itself returned CREDIT_OK when it was enqueued.  The
 *    host word makes it sticky without a synchronisation: once the failed
 *    launch has run, every later split call on that device refuses with
 *    CREDIT_ERR_WATCHDOG, until credit_check_watchdog() (which synchronises,
 *    reports CREDIT_ERR_WATCHDOG and clears both words) is called.
 */
#ifndef CREDIT_H_
#define CREDIT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ status ---- */
#define CREDIT_OK 0
#define CREDIT_ERR_NULL_POINTER (-1)
#define CREDIT_ERR_BAD_SHAPE (-2)
#define CREDIT_ERR_ALIGNMENT (-3)
#define CREDIT_ERR_UNSUPPORTED (-4)
#define CREDIT_ERR_WORKSPACE (-5)
#define CREDIT_ERR_HIP (-6)
#define CREDIT_ERR_WATCHDOG (-7)
#define CREDIT_ERR_BAD_CONFIG (-8)

/* ----------------------------------------------------------- variants ---
 * The reference times three kernel variants per workload
 * (src/workloads/layernorm_backward.cu:470-593): block_read (one CTA per row,
 * re-reading HBM on every pass), block_smem (one CTA per row, row staged on
 * chip) and cluster_smem (row split over a P-CTA cluster, partials exchanged
 * through DSMEM).  Their gfx950 counterparts: */
#define CREDIT_VARIANT_AUTO 0     /* library picks                          */
#define CREDIT_VARIANT_READ 1     /* one workgroup per row, streams HBM     */
#define CREDIT_VARIANT_STAGED 2   /* one workgroup per row, row in VGPRs/LDS */
#define CREDIT_VARIANT_SPLIT 3    /* P workgroups per row, L2 exchange      */

typedef struct credit_cfg {
  void* stream;           /* hipStream_t or NULL                            */
  int32_t variant;        /* CREDIT_VARIANT_*                               */
  int32_t split;          /* P for CREDIT_VARIANT_SPLIT; 0 = library choice */
  void* workspace;        /* optional caller scratch, see contract above    */
  size_t workspace_bytes; /* its size                                       */
} credit_cfg;

/* Operation ids for credit_workspace_bytes(). */
#define CREDIT_OP_ROW_SUM_MAX 1
#define CREDIT_OP_LAYERNORM_FWD 2
#define CREDIT_OP_LAYERNORM_BWD 3
#define CREDIT_OP_RMSNORM_FWD 4
#define CREDIT_OP_RMSNORM_BWD 5
#define CREDIT_OP_SOFTMAX_FWD 6
#define CREDIT_OP_SOFTMAX_BWD 7
#define CREDIT_OP_SOFTMAX_LOGITS_BWD 8
#define CREDIT_OP_FFN 9
#define CREDIT_OP_LAYERNORM_BWD_BF16 10
#define CREDIT_OP_ROWWISE_QUANT 11
#define CREDIT_OP_LARS_MOMENTUM 12
#define CREDIT_OP_WEIGHTED_VAR_BWD 13
#define CREDIT_OP_PEARSON_BWD 14
#define CREDIT_OP_RMSNORM_FWD_BWD 15

/* ------------------------------------------------------------ library --- */

/* Library version string, e.g. "credit-hip 0.1.0 gfx950". */
const char* credit_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* credit_last_error(void);

/* Static name of a status code. */
const char* credit_status_string(int status);

/* Replaces query_device_info (src/workloads/layernorm_backward.cu:440-468),
 * which reported opt-in shared memory and cluster support. */
typedef struct credit_device_info {
  char name[128];
  char arch[64];
  int32_t device;
  int32_t cu_count;
  int32_t xcd_count;
  int32_t wave_size;
  int32_t max_threads_per_block;
  int32_t cooperative_launch;
  int64_t lds_bytes_per_block;
  int64_t lds_bytes_per_cu;
  int64_t l2_bytes;
  int64_t hbm_bytes;
  int32_t clock_khz;
  int32_t mem_clock_khz;
  int32_t mem_bus_width_bits;
  int32_t reserved;
} credit_device_info;
int credit_query_device(int32_t device, credit_device_info* info);

/* Bytes of workspace a call needs (0 when the chosen variant needs none).
 * The reference has no counterpart: its DSMEM exchange lives in the
 * cluster's shared memory (cost_model.py:47-52 sizes that). */
size_t credit_workspace_bytes(int32_t op, int64_t rows, int64_t cols,
                              int32_t variant, int32_t split);

/* Waits for cfg->stream, then reports CREDIT_ERR_WATCHDOG (and clears the
 * flags) if a split-row barrier of an earlier call on this workspace -- or
 * any split launch on this device -- gave up waiting.  The reference's
 * cluster.sync() cannot time out; this is the host-visible form of the
 * bounded spin that replaces it. */
int credit_check_watchdog(const credit_cfg* cfg);

/* Polls a split launch's bounded wait makes before it gives up (default
 * 2^21, about 1-2 s of polling); applies to launches enqueued afterwards,
 * process-wide.  0 gives up at the first poll that finds a member's partial
 * missing: the failure path (wrong outputs, CREDIT_ERR_WATCHDOG) on demand,
 * for tests and for callers that prefer a fast error to a long wait.
 * *previous (if not NULL) receives the old value.  No counterpart in the
 * reference, whose cluster barriers cannot time out. */
int credit_set_spin_limit(uint32_t polls, uint32_t* previous);

/* ------------------------------------------------ C1: row sum and max ---
 * sum[r] = sum_j x[r, j] (accumulated in fp64, rounded once to fp32) and
 * max[r] = max_j x[r, j] (NaN-propagating, bit-exact with torch.amax).
 * Generalises the max-abs row reduction of
 * src/workloads/rowwise_quant.cu:260-363 (launched per runner.py:280-310);
 * the reference has no standalone sum/max workload.  cols >= 1. */
int credit_row_sum_max_f32(const float* x, float* sum, float* max,
                           int64_t rows, int64_t cols, const credit_cfg* cfg);

/* --------------------------------------------- C2: LayerNorm forward -----
 * y = (x - mean) * rstd * gamma + beta over each row, bf16 in/out, fp32
 * statistics: mean and the mean squared deviation about it, formed from
 * one pass of sum(x) and sum(x^2) (fp64 across lanes) when mean^2 <= var/4,
 * else from a second pass of squared deviations (rows with a large offset).
 * No forward kernel exists in the reference; its statistics follow
 * src/workloads/layernorm_backward.cu:286-295 and the eps of
 * dsmem_eval/workloads.py:55.  Variants: STAGED (row in one workgroup's
 * VGPRs, cols <= 65536), SPLIT (P workgroups per row of at most 32768
 * columns each, at most 32 members, exchanging (sum, sum of squares) once,
 * plus squared deviations for offset rows: one read of x; the split form of
 * src/workloads/layernorm_backward.cu:376-438), READ (vectorised streaming
 * passes; any shape).  AUTO: the persistent two-row pipeline for tall
 * matrices of 16385..32768 columns, STAGED up to 65536 columns, SPLIT with
 * the fewest members beyond, READ for cols % 8 != 0 or unaligned buffers. */
int credit_layernorm_fwd_bf16(const uint16_t* x, const uint16_t* gamma,
                              const uint16_t* beta, uint16_t* y, float* mean,
                              float* rstd, int64_t rows, int64_t cols,
                              float eps, const credit_cfg* cfg);

/* -------------------------------- LayerNorm backward (reference) -------
 * dx = (g - mean(g) - xhat * mean(g * xhat)) * rstd with g = dy * gamma and
 * the row's two-pass statistics (xhat = (x - mean) * rstd): the reference
 * workload layernorm_backward (dsmem_eval/workloads.py:53-61, kernels
 * src/workloads/layernorm_backward.cu:274-438, launched per
 * dsmem_eval/runner.py:280-310).  fp32 and bf16 (fp32 arithmetic).
 * Variants: STAGED (x and dy of the row in one workgroup's VGPRs: 32768 fp32
 * / 32768 bf16 columns), SPLIT (two exchanges per row, as the reference's
 * two cluster stages), READ (three streaming passes; any shape). */
int credit_layernorm_bwd_f32(const float* x, const float* dy, const float* gamma, float* dx,
                             int64_t rows, int64_t cols, float eps, const credit_cfg* cfg);
int credit_layernorm_bwd_bf16(const uint16_t* x, const uint16_t* dy, const uint16_t* gamma,
                              uint16_t* dx, int64_t rows, int64_t cols, float eps,
                              const credit_cfg* cfg);

/* ------------------------------------------ C3: RMSNorm forward ---------
 * rstd[r] = 1/sqrt(mean_j x[r,j]^2 + eps) (fp32), y = x * rstd * w (bf16).
 * No RMSNorm exists in the reference; the row sum of squares is the LARS
 * norm of src/workloads/lars_momentum.cu:283-319 (dsmem_eval/workloads.py:
 * 139-140).  Variants: STAGED (row in one workgroup's VGPRs, cols <= 65536),
 * SPLIT (cfg->split workgroups per row exchanging one partial; at most 32
 * members of 8193-16384 columns each run a barrier-free pipeline of rows,
 * whose row groups take rows from a launch-wide ticket counter in the
 * workspace's counter area, so faster groups take more rows; other splits
 * a slice kernel of at most 65536 columns per member), READ
 * (two streaming passes; any shape).  AUTO: STAGED when the row fits, else
 * the pipeline when at most 8 members of <= 16384 columns cover the row
 * (C3: 8 members), else the smallest slice SPLIT that holds it; READ for
 * cols % 8 != 0 or unaligned buffers. */
int credit_rmsnorm_fwd_bf16(const uint16_t* x, const uint16_t* w, uint16_t* y, float* rstd,
                            int64_t rows, int64_t cols, float eps, const credit_cfg* cfg);

/* ------------------------------------------ C3: RMSNorm backward --------
 * Given the forward's rstd: g = dy*w, xhat = x*rstd, c = mean_j(g*xhat),
 * dx = rstd*(g - xhat*c) (bf16), dw[j] = sum_r dy[r,j]*xhat[r,j] (fp32,
 * accumulated in fp64, summed over row blocks in a fixed order, so it is
 * deterministic).  Needs cols % 8 == 0 and 16-byte aligned x, w, dy, dx, dw.
 * Variants: STAGED (cols <= 8192), SPLIT (P >= cols/8192 members per row
 * block, one exchange per row), READ (a streaming row-dot pre-pass, then
 * column tiles).  rows == 0 writes dw = 0.  Always uses the workspace (dw
 * partials). */
int credit_rmsnorm_bwd_bf16(const uint16_t* x, const uint16_t* w, const uint16_t* dy,
                            const float* rstd, uint16_t* dx, float* dw, int64_t rows,
                            int64_t cols, const credit_cfg* cfg);

/* --------------------------------- C3: RMSNorm forward + backward fused --
 * The forward and the backward in one pass over x and dy: y = x * rstd * w,
 * rstd (fp32), dx and dw as credit_rmsnorm_bwd_bf16 -- 2 reads and 2 writes
 * per element instead of the separate calls' 1 + 1 and 2 + 1 (C3: 1.07 GB
 * against 1.34 GB).  The row's sum of squares travels in the same exchange
 * as sum(dy*w*x).  AUTO / SPLIT: the group kernel, cfg->split or the fewest
 * power-of-two members with slices of at most 8192 columns (at most 32
 * members; one member for rows of at most 8192 columns); READ (and AUTO on
 * shapes without cols % 8 == 0 and 16-byte aligned buffers): the forward
 * then the backward.  STAGED is refused.  No counterpart in the reference
 * (it has no RMSNorm); the fusion BASELINE's C3 names. */
int credit_rmsnorm_fwd_bwd_bf16(const uint16_t* x, const uint16_t* w, const uint16_t* dy,
                                uint16_t* y, float* rstd, uint16_t* dx, float* dw, int64_t rows,
                                int64_t cols, float eps, const credit_cfg* cfg);

/* The same backward, allocating nothing: no counterpart in the reference.
 * It is for callers that cannot allocate device memory -- code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.  The
 * workspace (header, counters, exchange slots, dweight partials) lives in a
 * fixed 40 MiB device array the library holds on every GPU it runs on until
 * the process ends; shapes that need more (more than 40 MiB of workspace by
 * credit_workspace_bytes, e.g. beyond 1024 x 262144 under AUTO) return
 * CREDIT_ERR_WORKSPACE, and a cfg->workspace is refused (CREDIT_ERR_BAD_CONFIG).
 * Outputs equal credit_rmsnorm_bwd_bf16's bit for bit.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams,
 * other threads) race and must not be issued.  A split-barrier timeout
 * (outputs then wrong, as with the allocating call) raises the array's own
 * watchdog word, which credit_check_watchdog reads, reports and clears;
 * the device's sticky host-mapped word (later split calls refuse) is raised
 * too only if an allocating split call created it earlier -- this call
 * creates none. */
int credit_rmsnorm_bwd_bf16_noalloc(const uint16_t* x, const uint16_t* w, const uint16_t* dy,
                                    const float* rstd, uint16_t* dx, float* dw, int64_t rows,
                                    int64_t cols, const credit_cfg* cfg);

/* ------------------------------------- C4: online softmax forward -------
 * m = max_j x, s = sum_j e^(x - m): p = e^(x - m)/s, rowmax = m (NaN-
 * propagating, bit-exact with torch.amax), lse = m + ln s; fp32.  The
 * reference fuses softmax into its backward (src/workloads/
 * softmax_logits_backward.cu:314-476) and emits no p, max or lse.
 * Variants: STAGED (row <= 65536 columns in one workgroup's VGPRs), SPLIT
 * (P workgroups per row merging (max, sum) pairs once: one read, one write),
 * READ (online streaming pass + output pass; any shape).  AUTO: the fewest
 * members that hold the row; READ for cols % 4 != 0 or unaligned buffers. */
int credit_softmax_fwd_f32(const float* x, float* p, float* rowmax, float* lse, int64_t rows,
                           int64_t cols, const credit_cfg* cfg);

/* ------------------------------------- C4: softmax backward -------------
 * dx = p * (dy - sum_j p*dy), fp32, given the forward's p.  Variants as the
 * forward; STAGED holds p and dy for rows <= 32768 columns. */
int credit_softmax_bwd_f32(const float* p, const float* dy, float* dx, int64_t rows,
                           int64_t cols, const credit_cfg* cfg);

/* ------------------------------- softmax-logits backward (reference) ----
 * p = softmax(logits), dx = p * (dy - sum_j p*dy): the reference workload
 * softmax_logits_backward (dsmem_eval/workloads.py:122-125, kernels
 * src/workloads/softmax_logits_backward.cu:314-476, launched per
 * dsmem_eval/runner.py:280-310), fp32.  SPLIT exchanges twice per row
 * ((max, sum), then sum p*dy); READ streams three passes. */
int credit_softmax_logits_bwd_f32(const float* logits, const float* dy, float* dx,
                                  int64_t rows, int64_t cols, const credit_cfg* cfg);

/* --------------------------------------- rowwise_quant (reference) -----
 * q = int8(clamp(rint(x * inv), -127, 127)), inv = (1 / max_j |x_j|) * 127
 * (0 for an all-zero row), scale = max_j |x_j| / 127, fp32 in: the reference
 * workload rowwise_quant (dsmem_eval/workloads.py:150-154; kernels
 * src/workloads/rowwise_quant.cu:260-363, launched per
 * dsmem_eval/runner.py:280-310).  Bit-exact against the reference's torch
 * function for finite x (inv rounds the reciprocal first, as torch
 * evaluates 127.0 / max_abs).  x and q [rows, cols], scale [rows].
 * Variants: STAGED holds rows <= 65536 columns; SPLIT exchanges the partial
 * maximum once per row; READ reads x twice and takes any width and
 * alignment (STAGED/SPLIT need cols % 4 == 0, x 16-byte and q 4-byte
 * aligned). */
int credit_rowwise_quant_f32(const float* x, int8_t* q, float* scale, int64_t rows,
                             int64_t cols, const credit_cfg* cfg);

/* --------------------------------------- lars_momentum (reference) -----
 * u = 0.9 m + g + 0.01 w (fp32, torch's operation order: bit-exact),
 * trust = 0.02 ||w|| / (||u|| + 1e-6) per row, w' = w - 1e-3 trust u: the
 * reference workload lars_momentum (dsmem_eval/workloads.py:136-143; kernels
 * src/workloads/lars_momentum.cu:283-416, launched per
 * dsmem_eval/runner.py:280-310).  weight, grad, momentum in; weight_out
 * (w') and update_out (u) out, all fp32 [rows, cols].  Variants: STAGED
 * holds w and u for rows <= 32768 columns; SPLIT exchanges the two sums of
 * squares once per row; READ streams the inputs twice, any width. */
int credit_lars_momentum_f32(const float* weight, const float* grad, const float* momentum,
                             float* weight_out, float* update_out, int64_t rows, int64_t cols,
                             const credit_cfg* cfg);

/* ------------------------------- weighted_var_backward (reference) -----
 * dx of y = (x - mean_w) / sqrt(var_w + eps) with row weights w (the
 * weighted mean and variance normalised by sum w + eps): the reference
 * workload weighted_var_backward (dsmem_eval/workloads.py:72-85; kernels
 * src/workloads/weighted_var_backward.cu:303-506, launched per
 * dsmem_eval/runner.py:280-310).  x, weight, dy, dx fp32 [rows, cols]; eps
 * > 0 (the reference's torch function uses 1e-5).  One exchange of five
 * sums per row (SPLIT: at most 12 members of at most 32768 columns each);
 * STAGED holds x, w and dy for rows <= 16384 columns; READ streams the
 * inputs twice, any width.  AUTO splits into members of at most 16384
 * columns and takes READ where that needs more than 12. */
int credit_weighted_var_bwd_f32(const float* x, const float* weight, const float* dy,
                                float* dx, int64_t rows, int64_t cols, float eps,
                                const credit_cfg* cfg);

/* ------------------------------------ pearson_backward (reference) -----
 * Gradients of the row-wise Pearson correlation of x and y, scaled by the
 * row's upstream grad: the reference workload pearson_backward
 * (dsmem_eval/workloads.py:96-112; kernels
 * src/workloads/pearson_backward.cu:311-482, launched per
 * dsmem_eval/runner.py:280-310).  x, y, dx, dy fp32 [rows, cols]; grad fp32
 * [rows]; eps > 0 (the torch function uses 1e-6).  One exchange of five
 * sums per row (SPLIT: at most 12 members); STAGED holds x and y for rows
 * <= 32768 columns; READ streams the inputs twice, any width. */
int credit_pearson_bwd_f32(const float* x, const float* y, const float* grad, float* dx,
                           float* dy, int64_t rows, int64_t cols, float eps,
                           const credit_cfg* cfg);

/* ------------------------------------------ C5: norm-fused FFN ----------
 * out = bf16(x + h @ W2^T), h = bf16(GELU_tanh(rstd * (x @ W1^T))) with
 * rstd = 1/sqrt(mean_j x^2 + eps) per row (RMSNorm with unit weight), fp32
 * accumulation on bf16 MFMA.  (Shapes that take the 128 x 128 tile GEMM --
 * d or f not a multiple of 256 -- form h = bf16(GELU_tanh(bf16(x * rstd) @
 * W1^T)): the normalised input rounded to bf16 before the product.)  Weights in the nn.Linear layout:
 * w1 [f, d] and w2 [d, f] (K contiguous).  x, out [rows, d].  rows, d and
 * f must be multiples of 128; buffers 16-byte aligned.  The hidden
 * activation h [rows, f] lives in the workspace (query with
 * credit_workspace_bytes(CREDIT_OP_FFN, rows, f, ...)).  No FFN exists in
 * the reference. */
int credit_ffn_rmsnorm_gelu_bf16(const uint16_t* x, const uint16_t* w1, const uint16_t* w2,
                                 uint16_t* out, int64_t rows, int64_t d, int64_t f, float eps,
                                 const credit_cfg* cfg);
/* The same FFN with the weights in the [in_features, out_features] layout
 * the BASELINE gives them: w1 [d, f], w2 [f, d] (out = x + GELU(RMSNorm(x)
 * w1) w2), read as they are -- the GEMMs take B as [K, N] tiles and gather
 * its MFMA fragments with transposing LDS reads, so no transpose runs.
 * Outputs are bit-identical to credit_ffn_rmsnorm_gelu_bf16 on the
 * transposed weights.  Same shape, alignment and workspace rules. */
int credit_ffn_rmsnorm_gelu_kn_bf16(const uint16_t* x, const uint16_t* w1, const uint16_t* w2,
                                    uint16_t* out, int64_t rows, int64_t d, int64_t f, float eps,
                                    const credit_cfg* cfg);
/* The forward of a training step: credit_ffn_rmsnorm_gelu_bf16 (nn.Linear
 * weights) that also hands back what its backward needs, so that
 * credit_ffn_rmsnorm_gelu_bwd_saved_bf16 need not recompute it: rstd
 * [rows] fp32, u [rows, f] = bf16(rstd * (x @ W1^T)) and h [rows, f] =
 * bf16(GELU_tanh(rstd * (x @ W1^T))), both bf16 row-major (h is the hidden
 * activation GEMM2 reads).  out is bit-identical to
 * credit_ffn_rmsnorm_gelu_bf16.  No workspace.  Same shape and alignment
 * rules (u and h 16-byte aligned too).  No counterpart in the reference. */
int credit_ffn_rmsnorm_gelu_fwd_train_bf16(const uint16_t* x, const uint16_t* w1,
                                           const uint16_t* w2, uint16_t* out, float* rstd,
                                           uint16_t* u, uint16_t* h, int64_t rows, int64_t d,
                                           int64_t f, float eps, const credit_cfg* cfg);
/* The same training forward on the [in, out] weights (w1 [d, f], w2 [f, d]),
 * as credit_ffn_rmsnorm_gelu_kn_bf16 takes them: out, rstd, u and h
 * bit-identical to the nn.Linear form on transposed weights.  Feeds
 * credit_ffn_rmsnorm_gelu_bwd_saved_kn_bf16.  No counterpart in the
 * reference. */
int credit_ffn_rmsnorm_gelu_fwd_train_kn_bf16(const uint16_t* x, const uint16_t* w1,
                                              const uint16_t* w2, uint16_t* out, float* rstd,
                                              uint16_t* u, uint16_t* h, int64_t rows, int64_t d,
                                              int64_t f, float eps, const credit_cfg* cfg);

/* ----------------------------------- FFN backward (next row of C5) -------
 * The gradients of out = x + GELU_tanh(RMSNorm(x) @ W1^T) @ W2^T (unit
 * RMSNorm weight, eps as the forward) for the upstream gradient dout:
 *   dx  [rows, d] = dout + RMSNorm backward of (du @ W1), bf16;
 *   dw1 [f, d]    = du^T a,  dw2 [d, f] = dout^T h   (the weights' own
 *                                                     nn.Linear layouts), bf16;
 * with a = bf16(x rstd), u = bf16(a W1^T) (recomputed), h = bf16(GELU(u)),
 * du = bf16((dout W2) * GELU'(u)); fp32 accumulation on MFMA.  Five GEMMs
 * (one recompute, four gradients; w1 and w2 are read in place, as [K, N]
 * operands where the product needs them so) plus transposes of dout and a
 * into the K-contiguous layout the weight-gradient GEMMs' A operand takes.  No FFN exists in the reference; this is
 * the "backward of the fused FFN" next row.  Same shape and alignment rules
 * as the forward.  Needs credit_ffn_bwd_workspace_bytes(rows, d, f) bytes of
 * workspace (cfg->workspace, or the library's cached buffer). */
int credit_ffn_rmsnorm_gelu_bwd_bf16(const uint16_t* x, const uint16_t* w1, const uint16_t* w2,
                                     const uint16_t* dout, uint16_t* dx, uint16_t* dw1,
                                     uint16_t* dw2, int64_t rows, int64_t d, int64_t f, float eps,
                                     const credit_cfg* cfg);
/* The same gradients from the saved rstd, u and h of
 * credit_ffn_rmsnorm_gelu_fwd_train_bf16 on the same x, w1, w2: four GEMMs
 * instead of five (no recompute of u; h is read as the dW2 GEMM's [K, N]
 * operand, so it needs no transpose either).  dx, dw1 and dw2 are
 * bit-identical to credit_ffn_rmsnorm_gelu_bwd_bf16's.  eps is the
 * forward's (already in rstd).  Same shape, alignment and workspace rules as
 * credit_ffn_rmsnorm_gelu_bwd_bf16.  No counterpart in the reference: the
 * training-step form of the FFN backward, for callers that keep the
 * forward's activations. */
int credit_ffn_rmsnorm_gelu_bwd_saved_bf16(const uint16_t* x, const uint16_t* w1,
                                           const uint16_t* w2, const uint16_t* dout,
                                           const float* rstd, const uint16_t* u,
                                           const uint16_t* h, uint16_t* dx, uint16_t* dw1,
                                           uint16_t* dw2, int64_t rows, int64_t d, int64_t f,
                                           const credit_cfg* cfg);
/* Both backward forms on the [in, out] weights (w1 [d, f], w2 [f, d], BASELINE
 * C5's own layout), returning the gradients in that layout too: dw1 [d, f],
 * dw2 [f, d].  The weights, dout and the activations are read in place; the
 * weight-gradient GEMMs take their operands the other way round (dw1 = a^T
 * du with du read as [K, N], dw2 = h^T dout with dout read as [K, N]), so
 * neither dout^T nor du^T is formed (the saved form's dw2, from h [rows, f],
 * is (dout^T h)^T stored transposed).  The gradients are bit-identical to the
 * nn.Linear entry points' on transposed weights, transposed.  Same shape,
 * alignment and workspace rules.  No counterpart in the reference. */
int credit_ffn_rmsnorm_gelu_bwd_kn_bf16(const uint16_t* x, const uint16_t* w1,
                                        const uint16_t* w2, const uint16_t* dout, uint16_t* dx,
                                        uint16_t* dw1, uint16_t* dw2, int64_t rows, int64_t d,
                                        int64_t f, float eps, const credit_cfg* cfg);
int credit_ffn_rmsnorm_gelu_bwd_saved_kn_bf16(const uint16_t* x, const uint16_t* w1,
                                              const uint16_t* w2, const uint16_t* dout,
                                              const float* rstd, const uint16_t* u,
                                              const uint16_t* h, uint16_t* dx, uint16_t* dw1,
                                              uint16_t* dw2, int64_t rows, int64_t d, int64_t f,
                                              const credit_cfg* cfg);
/* Workspace bytes the FFN backward (either form) needs at (rows, d, f); 0
 * for an empty shape.  Plumbing of this ABI, no counterpart in the
 * reference. */
size_t credit_ffn_bwd_workspace_bytes(int64_t rows, int64_t d, int64_t f);

/* dst[c, r] = src[r, c] for a rows x cols bf16 matrix: converts a [d, f]
 * weight to the [f, d] layout credit_ffn_rmsnorm_gelu_bf16 takes.  No
 * counterpart in the reference. */
int credit_transpose_bf16(const uint16_t* src, uint16_t* dst, int64_t rows, int64_t cols,
                          const credit_cfg* cfg);

/* ------------------------------------------- calibration (gfx950) -------
 * Replaces the reference's build/primitive_benchmark executable
 * (src/primitive_benchmark.cu:605-993, its stdout parsed by
 * dsmem_eval/profile.py:27-103).  Allocates its own buffers and runs on the
 * null stream of the current device.  results[] layout per benchmark:
 *   HBM_READ/WRITE/COPY : [0] best GB/s, [1..] GB/s of each kernel shape
 *                         tried (bytes = buffer size, default 1 GiB,
 *                         three rotating buffer sets)
 *   CLOCK               : [0] shader clock in MHz (s_memtime vs the 100 MHz
 *                         s_memrealtime)
 *   LATENCY             : [0..3] cycles per dependent load with working sets
 *                         of 16 KiB, 2 MiB, 64 MiB and 1 GiB (L1, L2, MALL,
 *                         HBM); iters = chain steps
 *   LDS_READ/WRITE      : [0] bytes per cycle per CU (one workgroup per CU)
 *   EXCHANGE_ROUNDTRIP  : [0] cycles per device-scope atomic round trip
 *                         between two workgroups on one XCD, [1] on two
 *                         XCDs (iters = rounds); the gfx950 stand-in for
 *                         the reference's DSMEM latency/visibility tests
 *   CACHE_READ          : [0] bytes per cycle per CU read from its vector
 *                         L1 (16 KiB working set), [1] bytes per cycle per
 *                         XCD read from L2 (2 MiB working set), [2] that L2
 *                         rate as device GB/s (iters = passes); replaces
 *                         l1_bandwidth_kernel / l2_bandwidth_kernel of
 *                         src/primitive_benchmark.cu:118-158
 *   EXCHANGE_THROUGHPUT : [0] bytes per cycle per workgroup of device-scope
 *                         64-bit slot stores (the split exchange's publish)
 *                         with one workgroup per CU, [1] the same as device
 *                         GB/s, [2] cycles per ticket draw (device-scope
 *                         fetch-add with return) on a private line, [3] on
 *                         one line shared by one workgroup per CU (iters =
 *                         store rounds); replaces the DSMEM store/load
 *                         throughput of src/primitive_benchmark.cu:433-503
 *   MFMA_BF16           : [0] dense bf16 MFMA TFLOP/s (v_mfma_f32_32x32x16_bf16
 *                         chains, no memory traffic, one workgroup per CU,
 *                         best of 4 and 8 waves per workgroup), [1] the mean
 *                         shader clock of its waves during the loop (MHz),
 *                         [2] flops per shader cycle per CU, [3] waves per
 *                         SIMD of the best, [4] TFLOP/s at 4 waves, [5] at 8
 *                         (iters = rounds of 8 MFMAs per wave); the
 *                         reference has no counterpart (its workloads have
 *                         no GEMM): the attainable rate the FFN GEMMs are
 *                         measured against, beside the 2.5 PFLOP/s datasheet
 *                         peak
 *  HBM_READ/WRITE/COPY run the mixed-stream kernels of credit_stream_ceiling
 *  (mixes 1:0, 0:1, 1:1). */
#define CREDIT_MB_HBM_READ 1
#define CREDIT_MB_HBM_WRITE 2
#define CREDIT_MB_HBM_COPY 3
#define CREDIT_MB_CLOCK 4
#define CREDIT_MB_LATENCY 5
#define CREDIT_MB_LDS_READ 6
#define CREDIT_MB_LDS_WRITE 7
#define CREDIT_MB_EXCHANGE_ROUNDTRIP 8
#define CREDIT_MB_CACHE_READ 9
#define CREDIT_MB_EXCHANGE_THROUGHPUT 10
#define CREDIT_MB_MFMA_BF16 11
/*  XCC_MAP                the XCC (hardware register XCC_ID) each workgroup
 *                         of an n_results-workgroup grid ran on, results[b]
 *                         for workgroup b: the round-robin dispatch the
 *                         split launches' ticket subsets assume.  No
 *                         counterpart in the reference (one die per GPU). */
#define CREDIT_MB_XCC_MAP 12
/*  RUNTIME_COPY           the runtime's device-to-device hipMemcpyAsync of
 *                         `bytes` (default 128 MiB) per call, settled and
 *                         timed as credit_stream_ceiling times its kernels
 *                         (three rotating buffer sets): [0] GB/s counting
 *                         read and write bytes, [1] ms per call.  An
 *                         independent 1:1 ceiling; the DRAM copy of
 *                         primitive_benchmark.cu:160-171 in the reference. */
#define CREDIT_MB_RUNTIME_COPY 13
int credit_microbench(int32_t which, int64_t bytes, int32_t iters, double* results,
                      int32_t n_results);

/* Settled HBM stream ceiling of a read:write byte mix: `reads` source and
 * `writes` destination streams of call_bytes / (reads + writes) bytes each
 * (rounded down to 64 KiB), three rotating buffer sets (so the 256 MB MALL
 * cannot serve a repeated set), every launch shape of the library's stream
 * kernel with nontemporal and with plain stores.  Each shape runs
 * back-to-back for settle_ms, then `trials` blocks of `iters` launches;
 * its time is the median block's per-launch time.  Mixes built: 1:0 0:1
 * 1:1 2:1 3:1 4:1 3:2 2:2 1:2.  results: [0] best GB/s, [1] its ms per
 * call, [2] lanes per workgroup, [3] 16-byte vectors per lane and stream,
 * [4] workgroups per CU, [5] 1 if nontemporal stores, [6] bytes moved per
 * call, then the GB/s of every (store policy, shape) tried.  The
 * reference's dram_bandwidth_kernel (src/primitive_benchmark.cu:160-171)
 * measures the 1:1 mix once; this is the ceiling each wide-row kernel's
 * HBM rate is compared with at its own mix and size.  Runs on the null
 * stream of the current device and allocates its own buffers. */
int credit_stream_ceiling(int32_t reads, int32_t writes, int64_t call_bytes, int32_t trials,
                          int32_t iters, double settle_ms, double* results, int32_t n_results);

/* Replaces build/cluster_control (src/cluster_control.cu:114-180, read at
 * dsmem_eval/runner.py:313-347): time of a grid of `rows` groups of `split`
 * workgroups that meet at `barriers` split-row barriers (the ticketed
 * exchange of the split kernels), against a plain launch of the same grid
 * that does nothing.  The barrier workgroups have `threads` lanes (0: 256)
 * and `lds_bytes` of dynamic LDS, as the reference's cluster kernel has
 * --shared-bytes of dynamic shared memory (cluster_control.cu:76-88,135,149):
 * the split launch being priced gives both (credit_last_split_shape), so the
 * barrier grid holds as many workgroups per CU as that launch.  cooperative
 * != 0 launches the barrier grid with hipLaunchCooperativeKernel instead
 * (capped at what fits the device), to expose that launch path's fixed
 * cost. */
int credit_control_overhead(int64_t rows, int32_t split, int32_t barriers, int32_t lds_bytes,
                            int32_t threads, int32_t warmup, int32_t iters, int32_t cooperative,
                            double* plain_ms, double* split_ms);

/* Measurement aid, no counterpart in the reference: while `sums` (a device
 * buffer of two uint64 the caller zeroes) is set, every workgroup of the
 * FFN's 256-tile GEMM kernels adds its shader cycles (s_memtime) to sums[0]
 * and its 100 MHz constant-clock ticks (s_memrealtime) to sums[1], start to
 * end; 100 * sums[0] / sums[1] is the mean shader clock (MHz) the GEMM tiles
 * ran at.  NULL switches it off (the default).  Process-wide; the GEMMs
 * launched meanwhile on any stream add to the same sums. */
int credit_set_clock_probe(uint64_t* sums);

/* Host-mapped watchdog words this process has allocated (at most one per
 * device; the first allocating split call on a device makes it).  Lets a
 * caller check that the allocation-free entry point allocated nothing.  No
 * counterpart in the reference. */
int credit_host_watchdog_words(int32_t* count);

/* Shape of the last co-resident split launch this thread made: block size
 * (data lanes plus any communication wave), LDS per workgroup (static and
 * dynamic), workgroups resident per CU, and its ticket subsets.  What the
 * reference's runner passes to cluster_control as --shared-bytes for each
 * sweep point (dsmem_eval/runner.py:714-723); CREDIT_ERR_UNSUPPORTED before
 * any split launch on this thread. */
int credit_last_split_shape(int32_t* threads, int32_t* lds_bytes, int32_t* per_cu,
                            int32_t* dispensers);

#ifdef __cplusplus
}
#endif

#endif /* CREDIT_H_ */
