// Kernel argument structs and kernel declarations shared by the translation
// units of libmemfast_hip.so (one definition each).
#pragma once

#include "mf_physics.h"

namespace mf {

// ---- general read (general.hip) -------------------------------------------
enum { OUT_FUSED = 0, OUT_TOTALS = 1 };

struct GeneralArgs {
    const u8 *q;          // [n, m*R] input codes
    const u8 *packed;     // [m, p, R, C] (used when g == nullptr)
    const void *g;        // [planes][m][width][W][R][C] or nullptr
    const float *xscale;  // [n, G]
    const float *wscale;  // [G, ldws]
    float *out;           // fused: [n, ldo]; totals: [n, G, width, C]
    int32_t *codes;       // optional [n, G, A, W, width*C]
    i64 n, m, p, begin, width, ldo, ldws;
    u32 seed;
    u64 event;
    int planes;
    int lp_cascade, lp_interleaved;   // level powers of torch's cascade
};

template <typename Phys, int WG, bool OUTPUT_NOISE>
__global__ void k_general(const mf_config cfg, const GeneralArgs args, int out_kind);

// ---- ideal MFMA read (ideal_mfma.hip) -------------------------------------
constexpr int IDEAL_MAX_LIN = 16;
constexpr int IDEAL_MAX_CLAMP = 64;

struct IdealPlan {
    int n_lin, n_clamp;
    u32 lin_a[IDEAL_MAX_LIN], lin_b[IDEAL_MAX_LIN];
    u32 cl_a[IDEAL_MAX_CLAMP], cl_b[IDEAL_MAX_CLAMP];
    int cl_val[IDEAL_MAX_CLAMP];
    int cl_upper[IDEAL_MAX_CLAMP];   // 1: min(X, val); 0: max(X, val)
};

struct IdealArgs {
    const u8 *q;          // [n, kp] input codes
    const u8 *wt;         // [ncols, kp] weight codes, column-major (packed_t)
    const float *xscale;  // [n, G]
    const float *wscale;  // [G, ldws]
    float *out;           // [n, ldo]
    i64 n, kp, G, ldo, ldws, ncols;
    int Gr, R, P;
    int a_bits, w_bits;   // code widths (< 8: sign-extend bytes on load)
};

template <int TM, int TN, int KS>
__global__ void k_ideal(const IdealPlan plan, const IdealArgs args);

// ---- conductances (restore.hip) -------------------------------------------
template <typename Phys>
__global__ void k_restore(const mf_config cfg, const u8 *packed, i64 m, i64 p, i64 begin,
                          i64 width, u32 seed, u64 event, int planes, Phys *g);

// ---- quantization (quantize.hip) ------------------------------------------
__global__ void k_fill_u32(u32 *p, i64 count, u32 value);
__global__ void k_group_max(const float *x, i64 rows, i64 cols, i64 ld, i64 gr, i64 gc, i64 ncg,
                            u32 *work);
__global__ void k_group_scale(const u32 *work, i64 groups, float upper, float *scale);
__global__ void k_input_codes(const float *x, i64 n, i64 k, i64 ld, i64 kp, const float *scale,
                              i64 gr, i64 gc, i64 ncg, int fixed, float lower, float upper,
                              u32 mask, u8 *q);
__global__ void k_input_scales(i64 n, i64 k, i64 groups, int R, int P, int Gr, const float *scale,
                               i64 gr, i64 gc, i64 ncg, int fixed, float *xscale);
__global__ void k_weight_codes(const float *b, i64 k, i64 o, i64 ld, int R, int C, i64 m, i64 p,
                               const float *scale, i64 gr, i64 gc, i64 ncg, float lower,
                               float upper, u32 mask, u8 *packed, u8 *packed_t);
__global__ void k_weight_scales(i64 k, i64 o, i64 groups, i64 op, int R, int P, int Gr,
                                const float *scale, i64 gr, i64 gc, i64 ncg, float *wscale);
__global__ void k_transpose_packed(const u8 *packed, int R, int C, i64 m, i64 p, u8 *packed_t);

}  // namespace mf
