// Kernel argument structs and kernel declarations shared by the translation
// units of libmemfast_hip.so (one definition each).
#pragma once

#include "mf_physics.h"

namespace mf {

// ---- general read (general.hip) -------------------------------------------
enum { OUT_FUSED = 0, OUT_TOTALS = 1 };

// Code and scale types follow the configuration: u8 codes with FP32 scales
// and output, or (wide) u32 codes with FP64 scales and output.
struct GeneralArgs {
    const void *q;        // [n, m*R] input codes
    const void *packed;   // [m, p, R, C] (used when g == nullptr)
    const void *g;        // [planes][m][width][W][R][C] or nullptr
    const void *xscale;   // [n, G]
    const void *wscale;   // [G, ldws]
    void *out;            // fused: [n, ldo]; totals: [n, G, width, C]
    int32_t *codes;       // optional [n, G, A, W, width*C]
    u32 *status;          // optional: MF_STATUS_OUTPUT for a non-finite fused output
    i64 n, m, p, begin, width, ldo, ldws;
    u32 seed;
    u64 event;
    int planes;
    int lp_cascade, lp_interleaved;   // level powers of torch's cascade
};

template <typename Phys, int WG, bool OUTPUT_NOISE, bool WIDE>
__global__ void k_general(const mf_config cfg, const GeneralArgs args, int out_kind);
// The read of precise currents on FP64 MFMA (no voltage variation, no output-mode read
// noise), fused or to totals as k_general.
template <bool WIDE, bool STAGED>
__global__ void k_general_mfma64(const mf_config cfg, const GeneralArgs args, int out_kind);
constexpr int MFMA64_STAGED_MAX_W = 8;   // weight slices of the LDS-staged variant

// ---- ideal MFMA read (ideal_mfma.hip) -------------------------------------
constexpr int IDEAL_MAX_CA = 8;     // input slices with at least one clamped pair
constexpr int IDEAL_MAX_CW = 8;     // weight slices with at least one clamped pair

// The linear part of every slice pair, sum_aw fa*fw*S_aw, is the plain int8
// product of the codes.  Pairs that can exceed their ADC limit form a
// (clamp-w x clamp-a) grid of slots s = cw * 8 + ca.  Per read and wave a slot
// is *proven clamp-free* when a digit-sum bound shows S <= max: max_n sum_r da
// <= floor(max_w / Mw) (input side) or max_c sum_r dw <= floor(max_w / Ma)
// (weight side).  The pre-pass k_digit_bits evaluates these tests and stores
// one 64-bit slot mask per (block, read).  Other candidates are recomputed on
// "natural" operand forms (masked two's complement bytes whose int8 value is
// factor*digit), Y = fa*fw*S, and corrected to min(Y, fa*fw*max_w) (max for
// negative pairs) where needed.
struct IdealPlan {
    int n_ca, n_cw;
    u32 ca_xnat[IDEAL_MAX_CA];
    int ca_factor[IDEAL_MAX_CA];                      // fa
    u32 cw_wnat[IDEAL_MAX_CW];
    int cw_limit[IDEAL_MAX_CW];                       // fw * max_w
    u32 cw_negative_ca[IDEAL_MAX_CW];                 // bit ca: fa * fw < 0
    uint64_t exists;                                  // slots holding a clamp candidate
};

// Tests evaluated by k_digit_bits for one side: slot s passes when the block's
// maximum digit sum of slice[s] is at most thr[s].
struct SlotTests {
    uint64_t exists;
    int slice[64];
    int thr[64];
};

struct IdealArgs {
    const u8 *q;            // [n, kp] input codes
    const u8 *wt;           // [ncols, kp] weight codes, column-major (packed_t)
    const float *xscale;    // [n, G]
    const float *wscale;    // [G, ldws]
    const uint64_t *xbits;  // [ceil(n/64), G] input-side proven slots per 64 vectors
    const uint64_t *wbits;  // [ceil(ncols/32), G] weight-side proven slots per 32 columns
    float *out;             // [n, ldo]
    u32 *status;            // optional: MF_STATUS_OUTPUT for a non-finite output
    u32 *mailbox;           // optional: pinned host word; the first workgroup copies the
                            // status bits there (with MF_STATUS_PUBLISHED) when it ends
    i64 n, kp, G, ldo, ldws, ncols;
    i64 G_run;              // reads executed: [0, G_run) (the rest is zero padding)
    int Gr, R, P;
    int a_bits, w_bits;     // code widths (< 8: sign-extend bytes on load)
};

template <int TN, int KS>
__global__ void k_ideal(const IdealPlan plan, const IdealArgs args);

struct SliceLayout {
    int count;
    int shift[MF_MAX_SLICES];
    int mask[MF_MAX_SLICES];
};

// Per-read digit sums of every slice, maximized over blocks of `block` rows,
// turned into the slot mask of `tests`: out[rb][g].  One launch serves both
// sides: grid rows [0, first_blocks) take job `a` (the inputs), the rest job `b`
// (the weight columns).
constexpr int DIGIT_WAVES = 16;   // waves per k_digit_bits workgroup
struct DigitJob {
    const u8 *codes;   // [rows, kp]
    i64 rows;
    int block;         // rows per maximum (32 or 64)
    SliceLayout layout;
    SlotTests tests;
    uint64_t *out;     // [ceil(rows / block), G]
};
template <int P>
__global__ void k_digit_bits(const DigitJob a, const DigitJob b, i64 first_blocks, i64 kp, i64 G);

// The same masks produced by the quantizers that wrote the codes (k_read_groups).
struct TileDigits {
    SliceLayout layout;
    SlotTests tests;
    uint64_t *bits;    // [blocks, G]
    i64 G;
    float scale_bound; // group scales above it set MF_STATUS_RANGE
};

// k_read_groups: B [k, o] (ld ldb) programmed in 32-row column groups into packed,
// packed_t and the per-read scale table wscale [G, o]; A [n, k] (ld ldx) quantized in
// groups of one read into q [n, k] and xscale [n, G]; both sides' digit-sum masks.
// Requires rows per read 32, k == m*R and o == p*C.
struct ReadGroupArgs {
    const float *b;
    i64 k, o, ldb;
    int R, C;
    i64 m, p;
    float wlower, wupper;
    u32 wmask;
    u8 *packed, *packed_t;
    float *wscale;
    i64 wgrid_x, wblocks;     // tile grid width (o / 64) and tile workgroups
    const float *x;
    i64 n, ldx;
    float xupper;
    u32 xmask;
    u8 *q;
    float *xscale;
    i64 G;
    TileDigits wdigits, xdigits;
    u32 *status;
};
__global__ void k_read_groups(const ReadGroupArgs a);

// ---- conductances (restore.hip) -------------------------------------------
template <typename Phys, typename Code>
__global__ void k_restore(const mf_config cfg, const Code *packed, i64 m, i64 p, i64 begin,
                          i64 width, u32 seed, u64 event, int planes, Phys *g);

// ---- noisy-device MFMA read (noisy_mfma.hip) -------------------------------
constexpr int NOISY_TERMS = 2;   // fp16 terms per conductance (hi, lo)

// Per-slice constants of the fused ADC: z = k1[w] * sum_r da * (g - L),
// S-curve z / (1 + |alpha[w] * z|), code = round(clamp(z, 0, top[w])),
// T += fa[a] * fw[w] * code.
struct NoisyPlan {
    int n_in, n_w;
    int planes;        // planes of terms per weight slice: n_in (slice_pair), 2 (output), else 1
    int out_noise;     // output-mode read noise: plane 1 holds (k1*g/Mw)^2
    float kl[8];       // k1 * L: the current of a digit at the low conductance (output mode)
    float qk[8];       // k1 / Mw (output mode)
    float out_var[8];  // Mw^2 * fp32(exp(s^2) * expm1(s^2)) (output mode)
    float out_mean;    // fp32(expm1(s^2 / 2)) (output mode)
    float two_pi;
    float k1[8], top[8], alpha[8], fa[8], fw[8];
    int in_shift[8];
    u32 in_mask4[8];   // input slice mask replicated into four bytes
    u32 bias;          // -0x400000 * sum(fa*fw) modulo 2^32
    u32 f24[8][8];     // fa*fw as the 24-bit signed operand of v_mad_i32_i24, per (a, w)
    float top_magic[8];  // 1.5 * 2^23 + adc_max[w] (exact in FP32)
};

struct NoisyArgs {
    const u8 *q;          // [n, kp] input codes
    const uint4 *gs;      // conductance terms of columns [c_begin, c_begin + 32*CB), fragment order
    const float *xscale;  // [n, G]
    const float *wscale;  // [G, ldws]
    float *out;           // fused: [n, ldo]; totals: [n, G, ldo]
    u32 *status;          // optional: MF_STATUS_OUTPUT for a non-finite fused output
    i64 n, kp, G, ldo, ldws, ncols, c_begin, CB;
    i64 g_begin, g_end;   // reads of this launch (blockIdx.z adds g_step)
    i64 g_step;
    int totals;
    // Voltage variation: input operands [2][A][ceil(n/32)][kp/8][32] uint4 of 8 fp16 (hi,
    // lo) of digit * (1 + vv*z) from k_voltage_terms, read instead of the digits of q.
    const uint4 *volt;
    u64 read_seed;        // output-mode read noise: event_seed(seed, event)
    i64 C;                // array columns (output-mode noise addresses)
    int restored;         // k_noisy_pairs: write (float(T) * xs) * ws instead of float(T)
};

// Terms are k1[w] * (g - L), so the read's MFMA output is in ADC counts.
template <int KS>
__global__ void k_split_conductances(const mf_config cfg, const u8 *packed_t, const float *g_in,
                                     i64 m, i64 p, i64 ncols, u32 seed, u64 event, i64 c_begin,
                                     i64 CB, const NoisyPlan plan, uint4 *gs);
template <int KS, int NA, bool NONLINEAR, bool VNOISE, bool SLICE, bool OUTN>
__global__ void k_noisy(const NoisyPlan plan, const NoisyArgs args);
// Split read of batches of at most 32 vectors: block = one wave per weight slice on 32
// vectors x 32 columns and one read (grid: column blocks, vector blocks, reads); writes
// slice totals [n, G, ldo], or with args.restored the restored (float(T) * xs) * ws
// (plain and S-curve reads).
template <int KS, int NA, bool NONLINEAR>
__global__ void k_noisy_pairs(const NoisyPlan plan, const NoisyArgs args);
// Input operands of a read with voltage variation (memfast/reference.py:77-82): per
// input slice a, vector v and physical row k, x = digit * (1 + vv * z(address)) split into
// fp16 hi + lo (terms 0, 1), and with `squares` (output-mode read noise) RN(x * x) split
// the same way (terms 2, 3).  Layout [terms][A][ceil(n/32)][kp/8][32] of uint4 (8 rows
// each): the 32 vectors of a block are innermost, so one MFMA operand of a wave (32
// vectors, two 8-row units) is 1 KiB contiguous.  Vectors past n hold zeros.
// Code: u8 (narrow codes) or u32 (wide codes, digits up to 255).
template <typename Code>
__global__ void k_voltage_terms(const mf_config cfg, const Code *q, i64 n, i64 m, u32 seed,
                                u64 event, int squares, uint4 *volt);
// (float(T) * xs) * ws summed over reads in torch's cascade order, from slice
// totals [n, G, ldt]: the epilogue of a read split across blocks.
// With `restored` the values are already (float(T) * xs) * ws and are only summed.
__global__ void k_restore_sum_f32(const float *totals, i64 n, i64 G, i64 g_run, i64 ldt,
                                  i64 ncols, const float *xscale, const float *wscale, i64 ldws,
                                  float *out, i64 ldo, int lp, int restored, u32 *status);

// ---- noisy-device MFMA read, wide configurations (noisy_wide.hip) ----------
// Same ADC model as NoisyPlan; integer totals accumulate modulo 2^32 as
// fa*fw*(0x400000 + code) and `bias` = -0x400000 * sum(fa*fw) restores them.
constexpr int WIDE_MFMA_MAX_A = 16;
constexpr int WIDE_MFMA_MAX_W = 8;
struct NoisyWidePlan {
    int n_in, n_w;
    int planes;        // planes of terms per weight slice: n_in (slice_pair read noise), else 1
    float k1[WIDE_MFMA_MAX_W], top[WIDE_MFMA_MAX_W], alpha[WIDE_MFMA_MAX_W];
    int fw[WIDE_MFMA_MAX_W];
    int fa[WIDE_MFMA_MAX_A];
    int in_shift[WIDE_MFMA_MAX_A];
    u32 in_mask2[WIDE_MFMA_MAX_A];   // input slice mask in both 16-bit halves
    u32 bias;
};

struct NoisyWideArgs {
    const uint16_t *q16;   // [n, kp] input codes, 16 bits
    const uint4 *gs;       // conductance terms [CB][G][W*planes][2][KS][64 lanes] of the chunk
    const double *xscale;  // [n, G]
    const double *wscale;  // [G, ldws]
    double *out;           // fused: [n, ldo]; totals: [n, G, ldo]
    u32 *status;           // optional: MF_STATUS_OUTPUT for a non-finite fused output
    i64 n, kp, G, ldo, ldws, ncols, c_begin;
    int totals;
    // Voltage variation: input operands [2][A][ceil(n/32)][kp/8][32] uint4 of 8 fp16 (hi,
    // lo) of digit * (1 + vv*z) from k_voltage_terms<u32>, read instead of the digits.
    const uint4 *volt;
};

__global__ void k_codes16(const u32 *q, i64 count, uint16_t *q16);
template <int KS>
__global__ void k_split_wide(const mf_config cfg, const u32 *packed, const float *g_in, i64 m,
                             i64 p, i64 ncols, u32 seed, u64 event, i64 c_begin, i64 CB,
                             const NoisyWidePlan plan, uint4 *gs);
// LDS capacity of the wide read: fragments (1 KiB) per read and buffer.  24:
// two buffers in 48 KiB (three blocks per CU); 36: 72 KiB (two blocks per CU);
// 72: 144 KiB (one block per CU).
constexpr int WIDE_FRAGS_TINY = 24;
constexpr int WIDE_FRAGS_SMALL = 36;
constexpr int WIDE_FRAGS_LARGE = 72;
// Blocks per CU the wide read is compiled for: three (at most 168 VGPRs) where
// the LDS allows it and the linear converter leaves the registers to spare.  (Voltage
// operands on 64-row reads spill two VGPRs at three blocks; two blocks without the spill
// ran 4.6% slower at 4096^3.)
constexpr int wide_blocks_per_cu(int frmax, bool nonlinear) {
    return frmax <= WIDE_FRAGS_TINY && !nonlinear ? 3 : 2;
}
// VNOISE: voltage variation (real input operands from args.volt, one input slice a step).
// SLICE: slice_pair read noise (a plane of terms per (weight slice, input slice), staged in
// LDS one (read, input slice) unit at a time).
template <int KS, bool NONLINEAR, int FRMAX, bool VNOISE, bool SLICE>
__global__ void k_noisy_wide(const NoisyWidePlan plan, const NoisyWideArgs args);

// ---- FP64 restore and read sum (stable.hip) --------------------------------
__global__ void k_stable_sum(const float *totals, i64 n, i64 G, i64 wc, const float *xscale,
                             const float *wscale, i64 ldws, i64 col0, double *out, i64 ldo,
                             int lp_cascade, int lp_interleaved);

// ---- quantization (quantize.hip) ------------------------------------------
__global__ void k_fill_u32(u32 *p, i64 count, u32 value);
__global__ void k_gru_gates(const float *inputs, i64 ldi, const float *hidden, i64 ldh,
                            const float *hx, i64 ldx, float *out, i64 ldo, i64 n, i64 width,
                            const float *bias, u32 *status, u32 flag);
__global__ void k_bias_add(float *out, i64 n, i64 o, i64 ldo, const float *bias, u32 *status,
                           u32 flag);
__global__ void k_narrow_f64(const double *in, i64 n, i64 cols, i64 ld, float *out, u32 *status,
                             u32 flag);

// One GRU step after its hidden read (recurrent.hip): the read's restore and read-order sum
// from split totals (or its fused output), the gate equations of k_gru_gates, and the
// quantization of the new state for the next step's hidden read (row groups of the whole
// state, as k_row_groups_wave writes them).  One workgroup of 1024 threads per batch row,
// with 3H floats of dynamic LDS.
struct GruStepArgs {
    const float *inputs;        // projected inputs of the step [B, 3H] (row stride ldi)
    i64 ldi;
    const float *hidden;        // the hidden read's output [B, 3H] (when totals is null)
    i64 ldh;
    const float *totals;        // split read: integer totals [B, G, ldt], or with restored
    int restored;               // set, the values (float(T) * xs) * ws
    i64 G, g_run, ldt;
    int lp;                     // level power of the read-order cascade
    const float *xscale_in;     // [B, G] scales of the read's input codes
    const float *wscale;        // [G, ldws]
    i64 ldws;
    const float *bias;          // hidden projection bias [3H] or null
    const float *hx;            // previous state [B, H]
    i64 ldx;
    float *out;                 // new state [B, H]
    i64 ldo, width;
    int quantize;               // 0: last step (no next read)
    i64 kp;                     // code row length (>= H, zero past H)
    float upper;
    u32 mask;
    u8 *q;                      // next codes [B, kp]
    float *scale;               // group scale per row [B]
    float *xscale_out;          // [B, G] per-read scales of the next read (may be xscale_in)
    u32 *status;
};
__global__ void k_gru_step(const GruStepArgs a);
__global__ void k_group_max(const float *x, i64 rows, i64 cols, i64 ld, i64 gr, i64 gc, i64 ncg,
                            u32 *work, u32 *status, u32 flag);
template <bool VEC>
__global__ void k_row_groups(const float *x, i64 n, i64 k, i64 ld, i64 gc, i64 ncg, i64 kp,
                             float lower, float upper, u32 mask, u8 *q, float *scale,
                             u32 *status, u32 flag);
__global__ void k_row_groups_lanes(const float *x, i64 n, i64 k, i64 ld, int L, i64 ncg, i64 kp,
                                   float lower, float upper, u32 mask, u8 *q, float *scale,
                                   u32 *status, u32 flag);
// The per-read scale table a row-group quantizer may fill as it goes: xscale
// [n, G] (NULL: not filled) over reads of P rows, Gr per array of R rows.
struct ReadTable {
    float *xscale;
    i64 G;
    int R, P, Gr;
};
template <int V>
__global__ void k_row_groups_wave(const float *x, i64 n, i64 k, i64 ld, i64 ncg, i64 kp,
                                  float lower, float upper, u32 mask, u8 *q, float *scale,
                                  u32 *status, u32 flag, const ReadTable reads);
template <int GR, bool WORD>
__global__ void k_col_groups_reg(const float *b, i64 k, i64 o, i64 ld, int R, int C, i64 m,
                                 i64 p, float lower, float upper, u32 mask, u8 *packed,
                                 u8 *packed_t, float *scale, u32 *status, u32 flag);
template <int GR, bool GIVEN>
__global__ void k_col_groups_tile(const float *b, i64 k, i64 o, i64 ld, int R, int C, i64 m, i64 p,
                                  float lower, float upper, u32 mask, u8 *packed, u8 *packed_t,
                                  float *scale, i64 gr, u32 *status, u32 flag);
template <bool WORD>
__global__ void k_col_groups(const float *b, i64 k, i64 o, i64 ld, i64 gr, i64 span, int R,
                             int C, i64 m, i64 p, float lower, float upper, u32 mask,
                             u8 *packed, u8 *packed_t, float *scale, u32 *status, u32 flag);
__global__ void k_group_scale(const u32 *work, i64 groups, float upper, float *scale);
__global__ void k_input_codes(const float *x, i64 n, i64 k, i64 ld, i64 kp, const float *scale,
                              i64 gr, i64 gc, i64 ncg, int fixed, float lower, float upper,
                              u32 mask, u8 *q);
template <typename I>
__global__ void k_input_codes4(const float *x, i64 n, i64 k, i64 ld, i64 kp, const float *scale,
                               i64 gr, i64 gc, i64 ncg, int fixed, float lower, float upper,
                               u32 mask, u8 *q);
__global__ void k_conv_group_max_f64(const double *x, const mf_conv_geometry g, i64 K, i64 gr,
                                     i64 gc, i64 ncg, u64 *work, u32 *status, u32 flag);
__global__ void k_conv_codes_f64(const double *x, const mf_conv_geometry g, i64 K, i64 kp,
                                 const double *scale, i64 gr, i64 gc, i64 ncg, int fixed,
                                 double lower, double upper, u64 mask, int narrow, u32 *q,
                                 u32 *status, u32 flag);
constexpr int CONV_CHUNK_COLS = 128;   // patch columns per k_conv_codes block
__global__ void k_conv_codes(const float *x, const mf_conv_geometry g, i64 K, i64 kp,
                             const float *scale, i64 gr, i64 gc, i64 ncg, float lower, float upper,
                             u32 mask, u8 *q, int vec, u32 *status, u32 flag);
__global__ void k_conv_group_max(const float *x, const mf_conv_geometry g, i64 K, i64 gr, i64 gc,
                                 i64 ncg, u32 *work, u32 *status, u32 flag);
__global__ void k_input_scales(i64 n, i64 k, i64 groups, int R, int P, int Gr, const float *scale,
                               i64 gr, i64 gc, i64 ncg, int fixed, float *xscale);
__global__ void k_weight_codes(const float *b, i64 k, i64 o, i64 ld, int R, int C, i64 m, i64 p,
                               const float *scale, i64 gr, i64 gc, i64 ncg, float lower,
                               float upper, u32 mask, u8 *packed, u8 *packed_t);
__global__ void k_weight_scales(i64 k, i64 o, i64 groups, i64 op, int R, int P, int Gr,
                                const float *scale, i64 gr, i64 gc, i64 ncg, float *wscale);
template <bool WORD>
__global__ void k_col_codes(const float *b, i64 k, i64 o, i64 ld, i64 gr, i64 span, int R, int C,
                            i64 m, i64 p, const float *scale, float lower, float upper, u32 mask,
                            u8 *packed, u8 *packed_t);
__global__ void k_transpose_packed(const u8 *packed, int R, int C, i64 m, i64 p, u8 *packed_t);
template <typename S>
__global__ void k_group_max_f64(const S *x, i64 rows, i64 cols, i64 ld, i64 gr, i64 gc,
                                i64 ncg, u64 *work, u32 *status, u32 flag);
// Group maxima of |x| as bit patterns (U = u32 for float, unsigned long long for
// double): reduced along rows first (any gr, gc; V adjacent columns per lane),
// or along a row (gr == 1).  S is the stored type (float values widened to T = double).
template <typename T, typename U, int V, typename S = T>
__global__ void k_col_group_max(const S *x, i64 rows, i64 cols, i64 ld, i64 gr, i64 gc, i64 ncg,
                                i64 chunk, U *work, u32 *status, u32 flag);
constexpr int COL_CHUNK_ROWS = 256;   // rows per k_col_group_max block, one column per lane
constexpr int COL_CHUNK_ROWS_VEC = 64;  // rows per block, 16 bytes of columns per lane
template <typename T, typename U, typename S = T>
__global__ void k_row_group_max(const S *x, i64 rows, i64 cols, i64 ld, i64 gc, i64 ncg, U *work,
                                u32 *status, u32 flag);
constexpr int ROW_CHUNK_COLS = 1024;  // columns per k_row_group_max wave
// `narrow`: an INT operand of at most 8 bits in a wide configuration, quantized in FP32 as
// the reference does (its dtype follows the operand's own width).
__global__ void k_group_scale_f64(const u64 *work, i64 groups, int bits, int bw_e, double upper,
                                  int narrow, double *scale, double bound, u32 *status);
template <typename S>
__global__ void k_input_codes_f64(const S *x, i64 n, i64 k, i64 ld, i64 kp,
                                  const double *scale, i64 gr, i64 gc, i64 ncg, int fixed,
                                  double lower, double upper, u64 mask, int narrow, u32 *q);
template <typename S>
__global__ void k_weight_codes_f64(const S *b, i64 k, i64 o, i64 ld, int R, int C, i64 m,
                                   i64 p, const double *scale, i64 gr, i64 gc, i64 ncg,
                                   double lower, double upper, u64 mask, int narrow, i64 *packed,
                                   u32 *packed32);
__global__ void k_input_scales_f64(i64 n, i64 k, i64 groups, int R, int P, int Gr,
                                   const double *scale, i64 gr, i64 gc, i64 ncg, int fixed,
                                   double *xscale);
__global__ void k_weight_scales_f64(i64 k, i64 o, i64 groups, i64 op, int R, int P, int Gr,
                                    const double *scale, i64 gr, i64 gc, i64 ncg, double *wscale);

}  // namespace mf
