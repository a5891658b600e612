/*
 * memfast_hip.h -- C ABI of the MI355X (gfx950) sliced analog matrix engine.
 *
 * This library replaces the reference's accelerator backend, memfast/cuda.py
 * (NVRTC-compiled memfast/kernels.cu loaded through ctypes).  The reference
 * binds its backend with ctypes from Python; the drop-in binding of these
 * entry points is memfast_amd/hip.py (also ctypes), see INTEGRATION.md.
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless stated otherwise;
 *     the caller (PyTorch's caching allocator) owns all memory.  Entry points
 *     never allocate device memory.
 *   - `stream` is a hipStream_t passed as void* (PyTorch's current stream).
 *     Launches are asynchronous; nothing synchronizes the device.
 *   - Return value: 0 on success, otherwise an MF_E_* status.  The message of
 *     the last failure on the calling thread is available from mf_last_error().
 *   - All physical constants travel in one POD descriptor, mf_config, built by
 *     memfast_amd/hip.py from a memfast Config (the reference instead bakes
 *     them into the CUDA source as #defines, memfast/cuda.py:67-127).
 */
#ifndef MEMFAST_HIP_H
#define MEMFAST_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MF_ABI_VERSION 9
#define MF_MAX_SLICES 32

enum {
    MF_OK = 0,
    MF_E_INVALID = 1,      /* bad argument, shape or descriptor      -> ValueError */
    MF_E_UNSUPPORTED = 2,  /* configuration not implemented on HIP  -> NotImplementedError */
    MF_E_RESOURCE = 3,     /* launch exceeds a device/kernel limit   -> ResourceError */
    MF_E_HIP = 4           /* HIP runtime error                      -> RuntimeError */
};

enum { MF_READ_SHARED = 0, MF_READ_SLICE_PAIR = 1, MF_READ_OUTPUT = 2 };

/* Bits kernels OR into a caller-owned device status word (uint32) instead of
 * synchronizing: the caller reads it once per product and raises the matching
 * error (memfast/functional.py:49-53, quantization.py:25-26,
 * simulator.py:614-615 and :643-644 check the same conditions on the host). */
enum {
    MF_STATUS_INPUT = 1,   /* non-finite activation value */
    MF_STATUS_WEIGHT = 2,  /* non-finite weight value */
    MF_STATUS_OUTPUT = 4,  /* non-finite FP32 output of mf_mm */
    MF_STATUS_RANGE = 16   /* mf_mm_from_float and the wide dynamic quantizers: a group
                            * scale above the bound that keeps every FP32 output (for
                            * wide reads, the FP32 cast of the FP64 output) finite;
                            * MF_STATUS_OUTPUT is then known only once the read has
                            * finished */
};
/* Set in a mailbox word (mf_mm_from_float) beside the status bits it carries. */
#define MF_STATUS_PUBLISHED 0x80000000u

/* Physical configuration (memfast/config.py:21-224), derived on the host.
 * f_* members are the FP32 values the reference's torch CPU ops use (Python
 * scalars are rounded to FP32 before they meet an FP32 tensor); d_* are the
 * FP64 values used when precise_currents is set. */
typedef struct mf_config {
    int32_t abi_version;          /* MF_ABI_VERSION */
    int32_t rows, cols;           /* array_size R, C */
    int32_t read_rows, reads;     /* P = rows_per_read or R; Gr = ceil(R/P) */
    int32_t activation_bits, weight_bits;
    int32_t weight_signed;
    int32_t n_in, n_w;            /* number of input / weight slices (A, W) */
    int32_t in_shift[MF_MAX_SLICES], in_mask[MF_MAX_SLICES];
    int64_t in_factor[MF_MAX_SLICES];
    int32_t w_shift[MF_MAX_SLICES], w_mask[MF_MAX_SLICES];
    int64_t w_factor[MF_MAX_SLICES];
    int32_t adc_max[MF_MAX_SLICES];   /* LSB-first ADC maxima 2^bits-1 */
    int32_t precise;              /* FP64 conductances and currents */
    int32_t read_mode;            /* MF_READ_* */
    int32_t has_write, has_read, has_vnoise, has_nonlinear, has_saf, has_drift;
    /* FP32 constants */
    float f_high, f_low, f_voltage, f_span;   /* fp32(H), fp32(L), fp32(V), fp32(H-L) */
    float f_inv_unit;                         /* fp32(1/((H-L)V)) */
    float f_write, f_read, f_vnoise;          /* noise sigmas */
    float f_drift;                            /* fp32(drift factor) */
    float f_saf_low, f_saf_band;              /* fp32(p_low), fp32(p_low+p_high) */
    float f_out_mean, f_out_var;              /* fp32(expm1(s^2/2)), fp32(exp(s^2)expm1(s^2)) */
    float f_two_pi;                           /* fp32(2*pi) */
    float f_alpha_over_max[MF_MAX_SLICES];    /* fp32(alpha / adc_max[w]) */
    /* FP64 constants (precise currents) */
    double d_high, d_low, d_voltage, d_span, d_inv_unit, d_drift;
    double d_alpha_over_max[MF_MAX_SLICES];
    /* Wide configurations (memfast/config.py:213-215 `wide`): precision above 8
     * bits or block floating point.  Codes are 32-bit (uint32_t), scales and
     * outputs FP64; the *_wide entry points take them. */
    int32_t wide;
    int32_t bw_e;                 /* BFP exponent bits, 0 for INT quantization */
} mf_config;

/* Identity of a device for the tuning-cache key (replaces memfast/cuda.py:376-389). */
typedef struct mf_identity {
    char arch[64];                /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    char name[256];
    int32_t compute_units;
    int32_t driver_version;
    int32_t runtime_version;
    int64_t memory_bytes;
} mf_identity;

/* Per-kernel resource figures (replaces Program.resources, memfast/cuda.py:239-273). */
typedef struct mf_resources {
    int32_t threads;              /* threads per block */
    int32_t shared_bytes;         /* LDS per block */
    int32_t registers;            /* VGPRs per thread */
    int32_t local_bytes;          /* private (spill) bytes per thread */
    int32_t max_blocks_per_cu;    /* occupancy */
} mf_resources;

/* ---- library ------------------------------------------------------------ */
int32_t mf_abi_version(void);
const char *mf_last_error(void);
/* Hash of the kernel sources compiled into this library (tuning-cache key;
 * replaces the source_hash of memfast/simulator.py:48-54 for the native part). */
const char *mf_source_hash(void);
int mf_device_identity(int device, mf_identity *out);

/* ---- quantization and programming --------------------------------------- */
/* Fixed-scale input tiles (memfast/quantization.py:115-137 with fixed_scale, the
 * set_input_scale path): codes q [n, m*R] (uint8, two's complement masked to
 * activation_bits, zero padded) and per-read scales xscale [n, m*Gr] from a
 * per-feature scale row `scale` [k]. */
int mf_input_tiles(const mf_config *cfg, const float *x, int64_t n, int64_t k, int64_t ld,
                   const float *scale, uint8_t *q, float *xscale, void *stream);

/* Dynamic grouped quantization of activations, whole (memfast/quantization.py:9-44
 * followed by input_tiles :115-137): group-scale grid scale [ceil(n/gr), ceil(k/gc)],
 * codes q [n, m*R] and per-read scales xscale [n, m*Gr] in one call.  Row-local
 * groups (gr == 1) run one fused pass; other shapes need `work` (uint32, grid
 * sized).  status (may be NULL) receives MF_STATUS_INPUT for a non-finite x.
 * `scale` may equal `xscale` when every group is one read (gr == 1, gc ==
 * read_rows, k == m*R): the grid is then the per-read table and no gather runs;
 * any other aliasing is MF_E_INVALID. */
int mf_quantize_inputs(const mf_config *cfg, const float *x, int64_t n, int64_t k, int64_t ld,
                       int64_t gr, int64_t gc, uint32_t *work, float *scale, uint8_t *q,
                       float *xscale, uint32_t *status, void *stream);

/* Dynamic grouped quantization and programming of a logical [k, o] weight
 * matrix (memfast/quantization.py:9-44 followed by weight_tiles :82-112):
 * scale grid, packed [m, p, R, C], packed_t [p*C, m*R] (may be NULL) and
 * wscale [m*Gr, p*C].  Column-local groups (gc == 1, gr <= 256) run one fused
 * pass; other shapes need `work`.  status receives MF_STATUS_WEIGHT.  `scale`
 * may equal `wscale` when every group is one read of one column (gc == 1, gr
 * == read_rows, k == m*R, o == p*C); any other aliasing is MF_E_INVALID. */
int mf_quantize_weights(const mf_config *cfg, const float *b, int64_t k, int64_t o, int64_t ld,
                        int64_t gr, int64_t gc, uint32_t *work, float *scale, uint8_t *packed,
                        uint8_t *packed_t, float *wscale, uint32_t *status, void *stream);

/* packed [m, p, R, C] -> packed_t [p*C, m*R] (for checkpoints loaded from disk). */
int mf_transpose_packed(const mf_config *cfg, const uint8_t *packed, int64_t m, int64_t p,
                        uint8_t *packed_t, void *stream);

/* ---- conductances ------------------------------------------------------- */
/* Programmed and read conductances (memfast/reference.py:10-51, kernels.cu:43-69)
 * for tiles [begin, end): g [planes][m][end-begin][W][R][C] in FP32 (FP64 when
 * cfg->precise), planes = n_in for read_mode slice_pair with read noise, else 1. */
int mf_restore(const mf_config *cfg, const uint8_t *packed, int64_t m, int64_t p,
               int64_t begin, int64_t end, uint32_t seed, uint64_t event, void *g,
               void *stream);

/* ---- array reads --------------------------------------------------------- */
/* Reference-compatible partial (memfast/cuda.py:322-373 / memfast/reference.py:63-117):
 * integer slice totals T [n, m*Gr, end-begin, C] as FP32 (all integer valued).
 * g: conductances as written by mf_restore for the same [begin, end), or an
 * injected tensor of that layout.  NULL g means ideal devices (closed form).
 * codes (optional, may be NULL): per-pair ADC counts int32
 * [n, m*Gr, n_in, n_w, end-begin, C] for code-level parity. */
int mf_partial(const mf_config *cfg, const uint8_t *q, int64_t n, int64_t m,
               const uint8_t *packed, int64_t p, int64_t begin, int64_t end, const void *g,
               uint32_t seed, uint64_t event, float *totals, int32_t *codes, void *stream);

/* mf_mm `variant` flag (no reference counterpart): the workspace still holds the
 * conductance terms that a previous mf_mm call of the same program (codes,
 * seed, descriptor, workspace) sampled for every column, so the noisy-device
 * MFMA read skips sampling them again.  Honoured only when the terms do not
 * depend on the read event (no read variation); otherwise ignored. */
#define MF_MM_REUSE_TERMS 0x100

/* Schedule fields of the `variant` word of mf_mm, mf_mm_static and mf_mm_wide (the
 * tuned mode's grid; memfast/simulator.py:27-45 holds the reference's).  Results
 * never depend on them; a field the selected kernel does not have is ignored.
 *   bits 0-7   ideal-device read tiling: 0 default (32 vectors per wave),
 *              1: 64 vectors per wave (32-row reads), 2: 32 vectors per wave.
 *   bits 12-15 noisy-device read: read chunks per output block.  0 automatic
 *              (grids under 512 blocks are split), 1 never, s >= 2 that many
 *              chunks (each writes integer totals to the workspace; one pass
 *              restores and sums them); MF_E_RESOURCE when the workspace cannot
 *              hold the chunks' totals (mf_mm_workspace prices them).
 *   bits 16-19 wide noisy-device read: LDS capacity per read, 0 automatic (the
 *              smallest holding a read's conductance terms), 1..3: 24, 36 or 72
 *              fragments; MF_E_RESOURCE when it cannot hold them. */
#define MF_MM_SPLIT_SHIFT 12
#define MF_MM_TIER_SHIFT 16

/* Fused read + scale restore (memfast/simulator.py:561-586 without the bias):
 * out [n, ldo] FP32 receives columns [0, p*C) of
 *   sum over reads g in torch's CPU order of (float(T[n,g,o]) * xscale[n,g]) * wscale[g,o].
 * g as for mf_partial over all tiles (begin=0, end=p); NULL means ideal devices.
 * For ideal devices with packed_t != NULL and a workspace of at least
 * mf_mm_workspace() bytes (256-byte aligned) the MFMA kernel is used;
 * `variant` holds the schedule fields above (the tuned mode's grid) and
 * MF_MM_REUSE_TERMS.  Results do not depend on the schedule fields.
 * out_cols (1..p*C) and k_rows (1..m*R) are the matrix's logical output columns
 * and input rows: the MFMA kernels compute only columns [0, out_cols) (the
 * reference slices the rest away before any check, :586) and skip the reads
 * that lie wholly in the zero padding past row k_rows, whose counts are 0
 * (leaving out those +0 terms does not change torch's sum).  Pass p*C and m*R
 * for every column and read.
 * status (may be NULL) receives MF_STATUS_OUTPUT when an output is non-finite. */
int mf_mm(const mf_config *cfg, const uint8_t *q, const float *xscale, int64_t n, int64_t m,
          const uint8_t *packed, const uint8_t *packed_t, const float *wscale, int64_t p,
          int64_t out_cols, int64_t k_rows, const void *g, uint32_t seed, uint64_t event,
          float *out, int64_t ldo, void *workspace, int64_t workspace_bytes, int32_t variant,
          uint32_t *status, void *stream);

/* Both quantizations and the ideal read in two launches (memfast/functional.py:130-136:
 * the RHS program of Simulator._matrix_for, memfast/simulator.py:133-171 with
 * quantization.py:82-137, read by AnalogMatrix.forward, :618-646): x [n, k] FP32 (leading
 * dimension ldx) and b [k, o] FP32 (ldb) are quantized exactly as mf_quantize_inputs
 * (groups x_gr x x_gc) and mf_quantize_weights (groups w_gr x w_gc) would, into q
 * [n, m, R], xscale [n, m*Gr], packed [m, p, R, C], packed_t [p*C, m*R] and wscale
 * [m*Gr, p, C]; the quantizing workgroups also reduce the digit sums of the codes they
 * wrote into the workspace's clamp-proof masks; then out [n, ldo] receives mf_mm's
 * result for all o columns.  Status bits as those three calls set them.  Applies to ideal
 * devices with 32 rows per read, groups of one read on both sides ((1, 32) and (32, 1)),
 * R % 128 == 0, C % 64 == 0, k == m*R, o == p*C, 16-byte aligned x, q, packed,
 * packed_t and out, and a workspace of mf_mm_workspace() bytes; otherwise it launches
 * nothing and returns MF_E_UNSUPPORTED (the caller takes the three calls).
 * The quantizers set MF_STATUS_RANGE when a group scale exceeds
 * sqrt(FLT_MAX / (2 * G * Tmax)) (G reads, Tmax the largest |count total| of one read):
 * below it no product, restore or sum of the read can overflow, so MF_STATUS_OUTPUT
 * cannot be set.  mailbox (may be NULL): a host word of pinned memory (hipHostMalloc),
 * cleared by the call before it launches, that the read's first workgroup sets when it
 * ends to MF_STATUS_PUBLISHED | the status bits (the quantizers' are final by then, as
 * they finished before the read began); mf_status_wait reads it.  A caller that finds no
 * bit but MF_STATUS_PUBLISHED there has every status bit of the call without waiting for
 * the rest of the read, which then overlaps the caller's next work on the stream. */
int mf_mm_from_float(const mf_config *cfg, const float *x, int64_t n, int64_t k, int64_t ldx,
                     const float *b, int64_t o, int64_t ldb, int64_t x_gr, int64_t x_gc,
                     int64_t w_gr, int64_t w_gc, uint8_t *q, float *xscale, uint8_t *packed,
                     uint8_t *packed_t, float *wscale, float *out, int64_t ldo, void *workspace,
                     int64_t workspace_bytes, int32_t variant, uint32_t *status,
                     uint32_t *mailbox, void *stream);

/* No counterpart in the reference (which checks its operands with host scans that
 * synchronize).  Queues, on `stream`, a copy of the device status word into the mailbox
 * (pinned host memory; cleared here first), marked MF_STATUS_PUBLISHED: what the kernels
 * queued before it have set.  A caller that launches it between a quantizer and the read
 * learns the quantizer's bits without waiting for the read. */
int mf_status_publish(const uint32_t *status, uint32_t *mailbox, void *stream);

/* No counterpart in the reference (which checks its operands with host scans that
 * synchronize).  Waits until the mailbox word of mf_mm_from_float or mf_status_publish
 * holds MF_STATUS_PUBLISHED or timeout_us microseconds have passed (spinning, then
 * sleeping in short steps); *flags receives the word without that bit and *published
 * whether it was set.  A caller that times out reads the device status word instead. */
int mf_status_wait(const uint32_t *mailbox, int64_t timeout_us, uint32_t *flags,
                   int32_t *published);

/* No counterpart in the reference.  mf_mm for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): the same read, arguments and results, with the scratch that mf_mm
 * takes as `workspace` drawn from a static device array of MF_STATIC_SCRATCH_BYTES
 * that the library holds on each GPU it runs on until the process ends.  The call
 * allocates nothing (no hipMalloc/hipFree; benchmark timing is off for it); its
 * first call on a device looks the array's address up on that device.
 *  - Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 *    (other streams or host threads) race.  Serialize them.
 *  - Noisy reads sample their conductance terms on every call (MF_MM_REUSE_TERMS
 *    is ignored) and run in column chunks that fit the array.
 *  - A read whose least scratch exceeds the array (the ideal-device read's digit
 *    masks, ceil(n/64)*G*8 + ceil(p*C/32)*G*8 bytes rounded up to 256; or one
 *    64-column chunk of noisy conductance terms, 256*W*m*R bytes) fails with
 *    MF_E_RESOURCE before launching anything. */
#define MF_STATIC_SCRATCH_BYTES (64ll << 20)
int mf_mm_static(const mf_config *cfg, const uint8_t *q, const float *xscale, int64_t n,
                 int64_t m, const uint8_t *packed, const uint8_t *packed_t, const float *wscale,
                 int64_t p, int64_t out_cols, int64_t k_rows, const void *g, uint32_t seed,
                 uint64_t event, float *out, int64_t ldo, int32_t variant, uint32_t *status,
                 void *stream);

/* The cast of a wide read's FP64 output to FP32 inputs' dtype and its finiteness check
 * (memfast/simulator.py:642-644, `.to(x.dtype)` then a host `isfinite` scan):
 * out[v * cols + c] = (float) in[v * ld + c] for c < cols (round to nearest even), and a
 * non-finite result sets MF_STATUS_OUTPUT in status (may be NULL), so the call's one
 * status read also answers the scan. */
int mf_narrow_output(const double *in, int64_t n, int64_t cols, int64_t ld, float *out,
                     uint32_t *status, void *stream);

/* Bias of an FP32 read (memfast/simulator.py:612-613, `out + bias`): out[v, c]
 * += bias[c] for c < o, one FP32 add each; a non-finite sum sets
 * MF_STATUS_OUTPUT in status (may be NULL), which replaces the host-side
 * finiteness scan that decides the FP64 retry (:614-615). */
int mf_bias_add(float *out, int64_t n, int64_t o, int64_t ldo, const float *bias,
                uint32_t *status, void *stream);

/* Geometry of one convolution group for mf_conv_input_tiles: NCHW input
 * [n, channels, height, width], this group's channels [c0, c0 + group_channels),
 * output [out_height, out_width] and the kernel's size, stride, zero padding
 * and dilation (as nn.Conv2d holds them). */
typedef struct mf_conv_geometry {
    int64_t n, channels, height, width;
    int64_t c0, group_channels;
    int64_t out_height, out_width;
    int32_t kh, kw, sh, sw, ph, pw, dh, dw;
} mf_conv_geometry;

/* Implicit im2col: the input tiles that mf_input_tiles (fixed_scale != NULL,
 * [K] per-column scales) or mf_quantize_inputs (fixed_scale == NULL, groups of
 * gr rows and gc columns; `work` uint32 [ceil(rows/gr), ceil(K/gc)] scratch and
 * `scale` FP32 of that shape) produce from the patch matrix that F.unfold
 * builds for one convolution group (memfast/nn/convolution.py:49-54: row
 * b*L + oh*out_width + ow, column (c*kh + i)*kw + j, K = group_channels*kh*kw),
 * read straight from the FP32 NCHW input.  q [rows, m, R], xscale
 * [rows, m*Gr]; a non-finite gathered value sets MF_STATUS_INPUT in status
 * (may be NULL). */
int mf_conv_input_tiles(const mf_config *cfg, const float *x, const mf_conv_geometry *geom,
                        const float *fixed_scale, int64_t gr, int64_t gc, uint32_t *work,
                        float *scale, uint8_t *q, float *xscale, uint32_t *status, void *stream);

/* GRU gates over the two projections of one step (memfast/nn/recurrent.py
 * `AnalogGRUCell`, PyTorch's gate equations): with inputs and hidden [n, 3H]
 * (chunks r, z, n) and hx [n, H],
 *   out = (1 - z) * tanh(in + r * hn) + z * hx,  r|z = sigmoid(i + h),
 * every operation rounded to FP32 as PyTorch's separate elementwise ops are.
 * Leading dimensions in elements. */
int mf_gru_gates(const float *inputs, int64_t ldi, const float *hidden, int64_t ldh,
                 const float *hx, int64_t ldx, float *out, int64_t ldo, int64_t n, int64_t width,
                 void *stream);

/* One direction of a GRU layer after its input projections (memfast/nn/recurrent.py:204-210,
 * the per-step `AnalogGRUCell.forward` of :101-116, replacing its hidden read, bias add and
 * gate ops with one call).  For i = 0 .. steps-1, t = reverse ? steps-1-i : i, and
 * h_{-1} = h0 ([batch, width], leading dimension ld_h0):
 *   hidden = mf_mm(mf_quantize_inputs(h_{i-1}), hidden program) read at event event0 + i,
 *   h_i    = gates(projected + t*proj_step, hidden + bias, h_{i-1})   (as mf_gru_gates),
 * written to out + t*out_step (rows out_row apart).  projected holds each step's input
 * projection [batch, 3*width] (rows proj_row apart), bias (may be NULL) the hidden bias [3*width].
 * gr, gc, work, scale, q, xscale: the dynamic input groups and scratch of mf_quantize_inputs;
 * packed .. p, seed, workspace, variant: the hidden program's arguments of mf_mm (out_cols
 * 3*width, k_rows width), with `hidden` [batch, ld_hidden] its output scratch.  Reads after
 * the first reuse the first read's conductance terms where they do not depend on the event.
 * Non-finite values set bits of *status as the separate calls do; nothing is read back, so
 * the caller checks *status once after the call. */
int mf_gru_sequence(const mf_config *cfg, int64_t steps, int32_t reverse, int64_t batch,
                    int64_t width, const float *projected, int64_t proj_step, int64_t proj_row,
                    const float *h0, int64_t ld_h0, int64_t gr, int64_t gc, uint32_t *work,
                    float *scale, uint8_t *q, float *xscale, const uint8_t *packed,
                    const uint8_t *packed_t, const float *wscale, int64_t m, int64_t p,
                    const float *bias, uint32_t seed, uint64_t event0, float *hidden,
                    int64_t ld_hidden, void *workspace, int64_t workspace_bytes, int32_t variant,
                    float *out, int64_t out_step, int64_t out_row, uint32_t *status,
                    void *stream);

/* Overflow-safe FP64 restore and read sum of one chunk of `width` tiles
 * (memfast/simulator.py:57-66 restore_scales and :578-585, the wide/retry path
 * taken when the FP32 restore is non-finite, :614-615): totals [n, G, width*C]
 * from mf_partial, xscale [n, G], wscale [G, ldws]; writes the FP64 sums to
 * out[v * ldo + col0 + c] for c < width*C, in torch's CPU summation order. */
int mf_stable_sum(const mf_config *cfg, const float *totals, int64_t n, int64_t G, int64_t width,
                  const float *xscale, const float *wscale, int64_t ldws, int64_t col0, double *out,
                  int64_t ldo, void *stream);

/* ---- wide configurations ------------------------------------------------
 * Precision above 8 bits or BFP (cfg->wide): codes are uint32_t (the
 * reference's int64 codes masked to the precision), scales and outputs FP64,
 * as memfast/quantization.py:9-137 and memfast/simulator.py:561-585 compute
 * them there.  The u8 entry points above reject wide descriptors and these
 * reject narrow ones. */
/* Dynamic grouped INT/BFP quantization of activations in FP64 (`work`: uint64
 * grid scratch); BFP exponents follow floor(log2(max)) of a correctly rounded
 * log2. */
int mf_quantize_inputs_wide(const mf_config *cfg, const double *x, int64_t n, int64_t k,
                            int64_t ld, int64_t gr, int64_t gc, uint64_t *work, double *scale,
                            uint32_t *q, double *xscale, uint32_t *status, void *stream);
/* The same quantization of FP32 activations (memfast/quantization.py:9-31 takes them in
 * FP64): each value is widened exactly as it is read, so the codes and scales are those
 * of the FP64 copy, which the caller need not make. */
int mf_quantize_inputs_wide_f32(const mf_config *cfg, const float *x, int64_t n, int64_t k,
                                int64_t ld, int64_t gr, int64_t gc, uint64_t *work, double *scale,
                                uint32_t *q, double *xscale, uint32_t *status, void *stream);
/* Fixed-scale input tiles (scale [k]). */
int mf_input_tiles_wide(const mf_config *cfg, const double *x, int64_t n, int64_t k, int64_t ld,
                        const double *scale, uint32_t *q, double *xscale, void *stream);

/* Implicit im2col for wide configurations: the tiles mf_input_tiles_wide (fixed_scale
 * != NULL, [K] FP64 per-column scales) or mf_quantize_inputs_wide (fixed_scale == NULL:
 * groups of gr rows and gc columns, `work` uint64 and `scale` FP64 scratch of
 * [ceil(rows/gr), ceil(K/gc)]) produce from a convolution group's patch matrix
 * (memfast/nn/convolution.py:49-54, the same order as mf_conv_input_tiles), gathered
 * from the FP64 NCHW input x.  q [rows, m, R] uint32 codes, xscale [rows, m*Gr] FP64; a
 * non-finite gathered value sets MF_STATUS_INPUT in status (may be NULL). */
int mf_conv_input_tiles_wide(const mf_config *cfg, const double *x, const mf_conv_geometry *geom,
                             const double *fixed_scale, int64_t gr, int64_t gc, uint64_t *work,
                             double *scale, uint32_t *q, double *xscale, uint32_t *status,
                             void *stream);
/* Weight programming: packed [m, p, R, C] as int64 (the reference's checkpoint
 * dtype) and the same codes as uint32_t for the read kernels. */
int mf_quantize_weights_wide(const mf_config *cfg, const double *b, int64_t k, int64_t o,
                             int64_t ld, int64_t gr, int64_t gc, uint64_t *work, double *scale,
                             int64_t *packed, uint32_t *packed32, double *wscale, uint32_t *status,
                             void *stream);
/* The same programming of FP32 weights, widened exactly as they are read. */
int mf_quantize_weights_wide_f32(const mf_config *cfg, const float *b, int64_t k, int64_t o,
                                 int64_t ld, int64_t gr, int64_t gc, uint64_t *work, double *scale,
                                 int64_t *packed, uint32_t *packed32, double *wscale,
                                 uint32_t *status, void *stream);
/* mf_restore, mf_partial and mf_mm for wide codes (totals and outputs FP64;
 * the fused read restores with restore_scales in FP64 and sums in torch's
 * FP64 order).  mf_mm_wide uses the noisy-device fp16 MFMA read (conductance
 * terms split into fp16 hi + lo) when the
 * configuration allows it (mf_mm_kernel reports 3) and `workspace` holds at
 * least the 64-column minimum of mf_mm_workspace (smaller than its full
 * figure: column chunks); otherwise the general read. */
int mf_restore_wide(const mf_config *cfg, const uint32_t *packed, int64_t m, int64_t p,
                    int64_t begin, int64_t end, uint32_t seed, uint64_t event, void *g,
                    void *stream);
int mf_partial_wide(const mf_config *cfg, const uint32_t *q, int64_t n, int64_t m,
                    const uint32_t *packed, int64_t p, int64_t begin, int64_t end, const void *g,
                    uint32_t seed, uint64_t event, double *totals, int32_t *codes, void *stream);
int mf_mm_wide(const mf_config *cfg, const uint32_t *q, const double *xscale, int64_t n, int64_t m,
               const uint32_t *packed, const double *wscale, int64_t p, const void *g,
               uint32_t seed, uint64_t event, double *out, int64_t ldo, void *workspace,
               int64_t workspace_bytes, int32_t variant, uint32_t *status, void *stream);
/* Integer slice totals T [n, m*Gr, p*C] (FP64) of the wide noisy-device MFMA
 * read (mf_mm_kernel 3), for parity tests: the values mf_partial_wide returns
 * for tiles [0, p).  g NULL samples conductances from packed (seed, event), or
 * g is an injected FP32 [m][p][W][R][C] tensor.  MF_E_UNSUPPORTED when
 * mf_mm_wide would not use that kernel. */
int mf_mm_totals_wide(const mf_config *cfg, const uint32_t *q, int64_t n, int64_t m,
                      const uint32_t *packed, int64_t p, const float *g, uint32_t seed,
                      uint64_t event, double *totals, void *workspace, int64_t workspace_bytes,
                      void *stream);

/* Benchmark timing of mf_mm's main read kernel (no reference counterpart; the
 * reference times whole candidate calls with CUDA events, memfast/simulator.py:306-316):
 * while enabled, each mf_mm call records a HIP event pair on its stream around
 * the read-kernel launch only.  mf_profile_collect waits for the recorded pairs
 * and returns their count and summed milliseconds, then forgets them. */
int mf_profile_kernels(int32_t enable);
int mf_profile_collect(int64_t *launches, double *milliseconds);

/* Workspace bytes mf_mm (mf_mm_wide) needs for its MFMA kernels under the
 * schedule fields of `variant`: per-read digit-sum maxima (ideal devices), or
 * the conductance terms of every column plus a split read's integer totals
 * (noisy devices; a smaller workspace of at least 64 columns' worth makes mf_mm
 * work in column chunks, unsplit), or 16-bit input codes and terms (wide
 * codes).  0 when the general kernel is used. */
int mf_mm_workspace(const mf_config *cfg, int64_t n, int64_t m, int64_t p, int32_t variant,
                    int64_t *bytes);

/* Integer slice totals T [n, m*Gr, p*C] (FP32) of the noisy-device MFMA read,
 * the values memfast/cuda.py:322-373 partial returns for tiles [0, p), for
 * parity tests of that kernel: g NULL restores conductances from packed_t
 * (seed, event) like mf_restore, or g is an injected FP32 [m][p][W][R][C]
 * tensor.  MF_E_UNSUPPORTED when mf_mm would not use that kernel. */
int mf_mm_totals(const mf_config *cfg, const uint8_t *q, int64_t n, int64_t m,
                 const uint8_t *packed_t, int64_t p, const float *g, uint32_t seed, uint64_t event,
                 float *totals, void *workspace, int64_t workspace_bytes, void *stream);

/* Kernel selected by mf_mm (mf_mm_wide) for this shape: 0 = general (FP64 currents,
 * precise_currents, run on FP64 MFMA unless voltage variation or output-mode read
 * noise needs the FMA kernel; so do mf_partial's totals without per-pair codes),
 * 1 = MFMA ideal, 2 = MFMA noisy (fp16 hi + lo conductance terms), 3 = MFMA noisy
 * for wide codes. */
int mf_mm_kernel(const mf_config *cfg, int64_t n, int64_t m, int64_t p, int32_t has_packed_t,
                 int32_t *kernel_id);

/* Resource figures (registers, scratch spill, LDS, resident blocks per CU) of the
 * read kernel instance mf_mm (mf_mm_wide) launches as `kernel_id` (mf_mm_kernel: 0
 * general, 1 ideal MFMA, 2 noisy MFMA, 3 wide noisy MFMA) for `n` input vectors (n <= 0:
 * the instances of batches above 32) under the schedule `variant` (mf_mm's variant word:
 * the ideal read's tile, the noisy read's split, the wide read's LDS tier).  A noisy read
 * of at most 32 vectors is taken as split (the automatic schedule splits reads of fewer
 * than 32768 output columns), the split the small-batch kernel k_noisy_pairs serves.
 * Replaces the per-candidate compiled-kernel attributes memfast/simulator.py:230-236
 * reads (memfast/cuda.py:376-389). */
int mf_resources_query(const mf_config *cfg, int32_t kernel_id, int64_t n, int32_t variant,
                       mf_resources *out);

/* ---- counter-based RNG (memfast/random.py:8-33), for parity tests -------- */
/* out[i] = uniform(address[i], seed, stream) (FP32) */
int mf_rng_uniform(const uint64_t *address, int64_t count, uint64_t seed, uint32_t stream,
                   float *out, void *stream_handle);
/* out[i] = normal(address[i], seed, stream) (FP32, Box-Muller with OCML) */
int mf_rng_normal(const uint64_t *address, int64_t count, uint64_t seed, uint32_t stream,
                  float *out, void *stream_handle);

#ifdef __cplusplus
}
#endif
#endif /* MEMFAST_HIP_H */
