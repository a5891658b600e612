// Grouped INT quantization, slicing layout and per-read scale gathering on gfx950.
//
// Semantics follow memfast/quantization.py for INT codes of at most 8 bits
// (FP32 arithmetic): grouped_quantize (:9-44), read_starts (:76-79),
// pack_weight (:94-112) and input_tiles (:115-137).  Division is IEEE
// correctly rounded FP32 (as torch CPU's true division) and rounding is
// round-half-even (rintf), so codes and scales are bit-identical to the CPU
// reference.  All kernels are HBM-bound elementwise passes.
#include "mf_kernels.h"

namespace mf {

__global__ void k_fill_u32(u32 *p, i64 count, u32 value) {
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += i64(gridDim.x) * blockDim.x)
        p[i] = value;
}

// Per-group max |x| via an integer atomicMax on the FP32 bit pattern (|x| >= 0
// orders like its bits).  Each thread first folds a run of up to 8 elements
// of one row that lie in the same group, to cut atomic traffic.
__global__ void k_group_max(const float *x, i64 rows, i64 cols, i64 ld, i64 gr, i64 gc,
                            i64 ncg, u32 *work) {
    const i64 runs_per_row = (cols + 7) / 8;
    const i64 total = rows * runs_per_row;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 r = i / runs_per_row;
        const i64 c0 = (i % runs_per_row) * 8;
        const float *row = x + r * ld;
        u32 best = 0;
        i64 group = -1;
        for (int e = 0; e < 8; ++e) {
            const i64 c = c0 + e;
            if (c >= cols) break;
            const i64 g = c / gc;
            if (g != group) {
                if (group >= 0) atomicMax(&work[(r / gr) * ncg + group], best);
                group = g;
                best = 0;
            }
            const u32 bits = __float_as_uint(fabsf(row[c]));
            best = bits > best ? bits : best;
        }
        if (group >= 0) atomicMax(&work[(r / gr) * ncg + group], best);
    }
}

// scale = (max > 0 ? max : 1) / upper, clamped below by the smallest subnormal.
__global__ void k_group_scale(const u32 *work, i64 groups, float upper, float *scale) {
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < groups;
         i += i64(gridDim.x) * blockDim.x) {
        const float peak = __uint_as_float(work[i]);
        float s = (peak > 0.0f ? peak : 1.0f) / upper;
        const float tiny = __uint_as_float(1u);
        s = s < tiny ? tiny : s;
        scale[i] = s;
    }
}

__device__ __forceinline__ u8 quantize_code(float x, float s, float lower, float upper,
                                            u32 mask) {
    float c = rintf(x / s);
    c = c < lower ? lower : c;
    c = c > upper ? upper : c;
    return u8(u32(int(c)) & mask);
}

// q [n, kp] with kp = m*R; columns >= k are zero padding.
__global__ void k_input_codes(const float *x, i64 n, i64 k, i64 ld, i64 kp, const float *scale,
                              i64 gr, i64 gc, i64 ncg, int fixed, float lower, float upper,
                              u32 mask, u8 *q) {
    const i64 total = n * kp;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 row = i / kp, col = i % kp;
        u8 code = 0;
        if (col < k) {
            const float s = fixed ? scale[col] : scale[(row / gr) * ncg + col / gc];
            code = quantize_code(x[row * ld + col], s, lower, upper, mask);
        }
        q[i] = code;
    }
}

// xscale [n, m*Gr]: scale of the read's first physical row, replicate-padded.
__global__ void k_input_scales(i64 n, i64 k, i64 groups, int R, int P, int Gr,
                               const float *scale, i64 gr, i64 gc, i64 ncg, int fixed,
                               float *xscale) {
    const i64 total = n * groups;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 row = i / groups, g = i % groups;
        i64 col = (g / Gr) * R + (g % Gr) * P;
        col = col < k ? col : k - 1;
        xscale[i] = fixed ? scale[col] : scale[(row / gr) * ncg + col / gc];
    }
}

// packed [m, p, R, C] and packed_t [p*C, m*R] from logical [k, o] weights.
__global__ void k_weight_codes(const float *b, i64 k, i64 o, i64 ld, int R, int C, i64 m,
                               i64 p, const float *scale, i64 gr, i64 gc, i64 ncg,
                               float lower, float upper, u32 mask, u8 *packed, u8 *packed_t) {
    const i64 kp = m * R, op = p * C;
    const i64 total = kp * op;
    for (i64 idx = i64(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += i64(gridDim.x) * blockDim.x) {
        const i64 row = idx / op, col = idx % op;
        u8 code = 0;
        if (row < k && col < o) {
            const float s = scale[(row / gr) * ncg + col / gc];
            code = quantize_code(b[row * ld + col], s, lower, upper, mask);
        }
        const i64 i = row / R, r = row % R, t = col / C, c = col % C;
        packed[((i * p + t) * R + r) * C + c] = code;
        if (packed_t) packed_t[col * kp + row] = code;
    }
}

// wscale [m*Gr, p*C]: replicate-padded scale at each read's first row.
__global__ void k_weight_scales(i64 k, i64 o, i64 groups, i64 op, int R, int P, int Gr,
                                const float *scale, i64 gr, i64 gc, i64 ncg, float *wscale) {
    const i64 total = groups * op;
    for (i64 idx = i64(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += i64(gridDim.x) * blockDim.x) {
        const i64 g = idx / op, col = idx % op;
        i64 row = (g / Gr) * R + (g % Gr) * P;
        row = row < k ? row : k - 1;
        const i64 cc = col < o ? col : o - 1;
        wscale[idx] = scale[(row / gr) * ncg + cc / gc];
    }
}

__global__ void k_transpose_packed(const u8 *packed, int R, int C, i64 m, i64 p, u8 *packed_t) {
    const i64 kp = m * R, op = p * C;
    const i64 total = kp * op;
    for (i64 idx = i64(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += i64(gridDim.x) * blockDim.x) {
        const i64 col = idx / kp, row = idx % kp;  // coalesced writes along rows
        const i64 i = row / R, r = row % R, t = col / C, c = col % C;
        packed_t[idx] = packed[((i * p + t) * R + r) * C + c];
    }
}

}  // namespace mf
