// Noisy-device sliced array read for wide configurations (precision above 8
// bits or BFP inputs, memfast/config.py `wide`) on gfx950 fp16 MFMA, fused with
// the ADC, the signed shift-add, the FP64 scale restore and torch's FP64
// read-order summation.  Only `out` (FP64) is written.
//
// Model (memfast/reference.py:63-117, memfast/simulator.py:57-66, 578-585):
// per read group g, input slice a and weight slice w,
//   I = sum_r (V * da/Ma) * (g[r,c] - L),   z = I * Ma*Mw / unit,
//   z = z / (1 + |alpha/max_w * z|) (S-curve),  code = round(clamp(z, 0, max_w)),
//   T = sum_a sum_w fa*fw*code                 (exact integer)
//   out[n,c] = sum_g restore_scales(T, xs[n,g], ws[g,c])   (FP64, torch order)
// As in the narrow kernel, z = sum_r da * k1 * (g - L) with k1 = V*Mw/unit:
// input digits are exact in fp16 and k1 * (g - L) (at most Mw <= 255 times the
// conductance noise) is held as two fp16 terms hi = fp16(x), lo = fp16(x - hi),
// within 2^-23 of x relative to its magnitude, so two fp16 MFMAs with FP32
// accumulation give z to about FP32 accuracy.
//
// Integer totals: the S-curve uses the reference's FP32 roundings (scurve in
// mf_device.h); the rounded, clamped count is formed in the exponent-fixed
// domain y = z + 1.5*2^23 (one rounding, half-even), med3-clamped to
// [1.5*2^23, 1.5*2^23 + max_w]; the low 24 bits of y are 0x400000 + code, and
// v_mad_i32_i24 accumulates fa*fw*(0x400000 + code) modulo 2^32.  The constant
// 0x400000 * sum(fa*fw) is removed at the end; the host checks that every true
// total fits in int32, so the modular sum is exact.
//
// Layout: k_split_wide writes the conductance terms of each 32-column block
// and read as one contiguous run [w][term][ks] of 1 KiB fragments (MFMA lane
// order); with slice_pair read noise one such run per input slice.  Block = 4
// waves on the same 32 columns and 128 vectors (32 per wave); per read (or per
// read and input slice) the block copies the run into LDS with global_load_lds
// (double-buffered in two LDS objects, one barrier per run) and every wave
// reads it from there.  FRMAX bounds the fragments per run (W * 2 * KS); the
// smallest capacity is compiled for three blocks per CU.
// Input codes are repacked to 16 bits (k_codes16) so a lane's 8 rows of a
// 16-row step are one 16-byte load.  Bound: VALU (digit expansion + ADC per
// slice pair) with fp16 MFMA as co-bound.
#include <cfloat>

#include "mf_kernels.h"

namespace mf {

typedef _Float16 v8h_w __attribute__((ext_vector_type(8)));
typedef float v16f_w __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

namespace {

__device__ __forceinline__ __amdgpu_buffer_rsrc_t wide_buffer(const void *base, i64 bytes) {
    const int records = bytes > 0x7FFFFFFF ? 0x7FFFFFFF : int(bytes < 0 ? 0 : bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), short(0), records,
                                             0x00020000);
}

// Digits of slice (shift, mask2), any width up to 8 bits, of eight 16-bit codes as eight
// fp16: each field d is OR-ed into the mantissa of fp16 1024 (0x6400, mantissa step 1),
// and one packed fp16 subtraction of 1024 leaves d exactly (the same fp16 values as a
// conversion).  Three instructions per two digits: shift, and-or (one v_and_or_b32, the
// constant held in a VGPR: VOP3 takes no literal), packed subtract.
__device__ __forceinline__ v8h_w digits_magic(uint4 c, int shift, u32 mask2, u32 magic) {
    typedef _Float16 v2h_w __attribute__((ext_vector_type(2)));
    const v2h_w base = {_Float16(1024.0f), _Float16(1024.0f)};
    const u32 w[4] = {c.x, c.y, c.z, c.w};
    u32 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        u32 x;
        asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(x) : "v"(w[i] >> shift), "s"(mask2), "v"(magic));
        o[i] = __builtin_bit_cast(u32, __builtin_bit_cast(v2h_w, x) - base);
    }
    return __builtin_bit_cast(v8h_w, make_uint4(o[0], o[1], o[2], o[3]));
}

// One 1 KiB LDS DMA: lane l's 16 bytes at src go to lds_base + 16 * l.  Issued
// as inline assembly so that the compiler's wait-count analysis does not track
// it (it would otherwise wait for it at the next loop header); the kernel waits
// for it explicitly (s_waitcnt vmcnt(0) and a barrier) before reading the data.
__device__ __forceinline__ void lds_dma_16(const void *src, u32 lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 1\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(lds_base)
                 : "memory", "m0");
}

// After an explicit s_waitcnt vmcnt(0): re-define the loaded registers so the
// compiler's wait-count analysis no longer sees a load pending on them (it
// would otherwise flush vmcnt at the next loop header, where the next read's
// LDS DMA is in flight).
template <int N>
__device__ __forceinline__ void settle(uint4 (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i].x), "+v"(v[i].y), "+v"(v[i].z), "+v"(v[i].w));
}

template <typename T>
__device__ __forceinline__ void settle_one(T &v) {
    asm volatile("" : "+v"(v));
}

// Float value held by lane `i` (readlane moves 32-bit integers).
__device__ __forceinline__ float lane_float(float v, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

// restore_scales of one total: (T * xs) * ws when no intermediate leaves the
// normal FP64 range (then it equals the frexp/ldexp form exactly), else the
// frexp/ldexp form itself.
__device__ __forceinline__ double restore_fast(int total, double xs, double ws) {
    if (total == 0) return 0.0;
    const double v1 = double(total) * xs;
    const double v2 = v1 * ws;
    const double a1 = fabs(v1), a2 = fabs(v2);
    if (a1 >= DBL_MIN && a2 >= DBL_MIN && a2 <= DBL_MAX) return v2;
    return restore_f64(double(total), xs, ws);
}

}  // namespace

__global__ void k_codes16(const u32 *q, i64 count, uint16_t *q16) {
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += i64(gridDim.x) * blockDim.x)
        q16[i] = uint16_t(q[i]);
}

template <int KS>
__global__ __launch_bounds__(256) void k_split_wide(const mf_config cfg, const u32 *packed,
                                                    const float *g_in, i64 m, i64 p, i64 ncols,
                                                    u32 seed, u64 event, i64 c_begin, i64 CB,
                                                    const NoisyWidePlan plan, uint4 *gs) {
    constexpr int P = 16 * KS;
    const int R = cfg.rows, C = cfg.cols, W = cfg.n_w;
    const i64 G = m * R / P;
    const i64 total = CB * G * W * plan.planes * KS * 64;
    const u64 read_seed = event_seed(seed, event);
    for (i64 t = i64(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += i64(gridDim.x) * blockDim.x) {
        i64 rest = t;
        const int lane = int(rest & 63); rest >>= 6;
        const int ks = int(rest % KS); rest /= KS;
        const int vw = int(rest % (W * plan.planes)); rest /= W * plan.planes;
        const int plane = vw / W, w = vw - plane * W;   // planes outermost: [plane][w]
        const i64 g = rest % G;
        const i64 cb = rest / G;
        const int lr = lane & 31, h = lane >> 5;
        const i64 c = c_begin + cb * 32 + lr;
        const i64 k0 = g * P + ks * 16 + h * 8;
        u32 terms[2][4] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
        if (c < ncols) {
            const i64 i = k0 / R, r0 = k0 - i * R;
            const i64 tt = c / C, cc = c - tt * C;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const i64 r = r0 + j;
                const u64 cell = u64((((i * p + tt) * W + w) * R + r) * C + cc);
                float level;
                if (g_in) {
                    level = g_in[cell];
                } else {
                    const u32 code = packed[((i * p + tt) * R + r) * C + cc];
                    level = cell_conductance<float>(cfg, code, w, cell, seed, read_seed);
                }
                // slice_pair read noise (memfast/reference.py:86-90): a read factor per
                // (cell, input slice), one plane of terms per input slice.
                if (plan.planes > 1)
                    level = level * exp_small(cfg.f_read *
                                              normal_fast(cell * u64(cfg.n_in) + u64(plane),
                                                          read_seed, 20u));
                const float delta = (level - cfg.f_low) * plan.k1[w];   // ADC counts per digit
                const _Float16 hi = static_cast<_Float16>(delta);        // round to nearest even
                const _Float16 lo = static_cast<_Float16>(delta - static_cast<float>(hi));
                const int shift = 16 * (j & 1);
                terms[0][j >> 1] |= u32(__builtin_bit_cast(unsigned short, hi)) << shift;
                terms[1][j >> 1] |= u32(__builtin_bit_cast(unsigned short, lo)) << shift;
            }
        }
        uint4 *dst = gs + ((((cb * G + g) * W * plan.planes + vw) * NOISY_TERMS) * KS + ks) * 64 +
                     lane;
#pragma unroll
        for (int term = 0; term < NOISY_TERMS; ++term)
            dst[term * KS * 64] = make_uint4(terms[term][0], terms[term][1], terms[term][2],
                                             terms[term][3]);
    }
}

template __global__ void k_split_wide<2>(const mf_config, const u32 *, const float *, i64, i64,
                                         i64, u32, u64, i64, i64, const NoisyWidePlan, uint4 *);
template __global__ void k_split_wide<4>(const mf_config, const u32 *, const float *, i64, i64,
                                         i64, u32, u64, i64, i64, const NoisyWidePlan, uint4 *);

template <int KS, bool NONLINEAR, int FRMAX, bool VNOISE, bool SLICE>
__global__ __launch_bounds__(256, wide_blocks_per_cu(FRMAX, NONLINEAR)) void k_noisy_wide(
    const NoisyWidePlan plan,
                                                       const NoisyWideArgs args) {
    // Two LDS objects (read g in one, read g+1 arriving in the other) so that the
    // compiler can tell the in-flight LDS DMA from the LDS reads of the current
    // read and does not wait for the DMA before them.
    __shared__ __align__(16) uint4 sF0[FRMAX * 64], sF1[FRMAX * 64];
    constexpr int P = 16 * KS;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int A = plan.n_in, W = plan.n_w;
    const int G = int(args.G);
    // Fragments per LDS unit: one read's terms [w][term][ks], or with slice_pair read noise
    // one (read, input slice) plane set: a read is A units, each staged in turn.
    const int FR = W * NOISY_TERMS * KS;
    const int UNITS = SLICE ? A : 1;   // LDS units per read
    // Column blocks are the fast grid axis: the dispatcher deals neighbouring workgroups to
    // different XCDs, so each XCD holds every eighth column block's terms for the vector
    // blocks in flight, and the 16-bit codes of those vector blocks are shared by all of
    // them.  (Giving each XCD a contiguous run with vector blocks fastest cut FETCH_SIZE by
    // 19% at the q_proj shape but re-read the codes at 4096 vectors: 8% slower there.)
    const i64 cb = blockIdx.x;                    // chunk-relative 32-column block
    const i64 v0 = i64(blockIdx.y) * 128 + wave * 32;
    const i64 kp = args.kp;

    // Conductance terms of this column block: [g][unit][w][term][ks][lane].
    const uint4 *frag = args.gs + cb * i64(G) * UNITS * FR * 64 + lane;
    auto fetch = [&](int u, uint4 *dst) {   // unit u = g * UNITS + a
        const uint4 *src = frag + i64(u) * FR * 64;
        const u32 base = u32(reinterpret_cast<uintptr_t>((lds_void *)dst));
        for (int f = wave; f < FR; f += 4)
            lds_dma_16(src + f * 64, __builtin_amdgcn_readfirstlane(base + u32(f) * 1024u));
    };

    // Per-slice constants in a lane table (lane a: slice a), read with readlane.
    int slice_shift = lane < A ? plan.in_shift[lane] : 0;
    u32 slice_mask2 = lane < A ? plan.in_mask2[lane] : 0u;
    int slice_factor = lane < A ? plan.fa[lane] : 0;
    float w_top = lane < W ? plan.top[lane] : 0.0f;
    float w_alpha = lane < W ? plan.alpha[lane] : 0.0f;
    int w_factor = lane < W ? plan.fw[lane] : 0;
    // 16-bit input codes of this wave's 32 vectors (rows past n read as zero).
    const i64 vrows = (args.n - v0) < 32 ? (args.n - v0) : 32;
    const __amdgpu_buffer_rsrc_t qbuf =
        wide_buffer(args.q16 + (vrows > 0 ? v0 : 0) * kp, (vrows > 0 ? vrows : 0) * kp * 2);
    const int q_off = (lrow * int(kp) + lhalf * 8) * 2;
    uint4 qc[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
        qc[ks] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                               qbuf, q_off + ks * 32, 0, 0));

    const i64 n_out = v0 + lrow;
    const bool live_n = n_out < args.n;
    const bool live_block = v0 < args.n;   // wave-uniform: the wave holds some vector
    const i64 col_tile = args.c_begin + cb * 32;   // absolute first column of the block
    double acc0[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc0[r] = 0.0;

    fetch(0, sF0);
    __builtin_amdgcn_s_waitcnt(0);
    settle(qc);
    settle_one(slice_shift);
    settle_one(slice_mask2);
    settle_one(slice_factor);
    settle_one(w_top);
    settle_one(w_alpha);
    settle_one(w_factor);
    __syncthreads();

    u32 magic16 = 0x64006400u;   // fp16 1024 in both halves (digits_magic)
    settle_one(magic16);
    const float MAGIC = 12582912.0f;   // 1.5 * 2^23
    auto step = [&](int g, const uint4 *sCur, uint4 *sNext) {
        if (!SLICE && g + 1 < G) fetch(g + 1, sNext);
        u32 T[16];   // modulo 2^32, offset by 0x400000 * sum(fa*fw) (plan.bias undoes it)
#pragma unroll
        for (int r = 0; r < 16; ++r) T[r] = 0u;
        const uint4 *fl = sCur + lane;
        // ADC of one slice pair's count argument (the terms carry k1): per output
        // add into the exponent-fixed domain, med3 clamp, 24-bit multiply-accumulate
        // of fa*fw*(0x400000 + code).
        auto convert = [&](const v16f_w &I, int w, int a) {
            const float top = MAGIC + lane_float(w_top, w);
            const int f = __builtin_amdgcn_readlane(slice_factor, a) *
                          __builtin_amdgcn_readlane(w_factor, w);   // |fa*fw| < 2^23
            const u32 f24 = u32(int(u32(f) << 8) >> 8);
            float alpha = 0.0f;
            if (NONLINEAR) alpha = lane_float(w_alpha, w);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float y = (NONLINEAR ? scurve(I[r], alpha) : I[r]) + MAGIC;
                y = __builtin_amdgcn_fmed3f(y, MAGIC, top);
                // 0x400000 + code in the low 24 bits; v_mad_i32_i24 reads only those.
                asm("v_mad_i32_i24 %0, %1, %2, %0" : "+v"(T[r]) : "v"(y), "s"(f24));
            }
        };
        auto digits = [&](v8h_w (&B)[KS], int a) {
            const int shift = __builtin_amdgcn_readlane(slice_shift, a);
            const u32 mask2 = u32(__builtin_amdgcn_readlane(int(slice_mask2), a));
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                B[ks] = digits_magic(qc[ks], shift, mask2, magic16);
        };
        auto terms = [&](v8h_w (&F)[NOISY_TERMS][KS], int w) {
#pragma unroll
            for (int term = 0; term < NOISY_TERMS; ++term)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    F[term][ks] = __builtin_bit_cast(
                        v8h_w, fl[((w * NOISY_TERMS + term) * KS + ks) * 64]);
        };
        if (VNOISE || SLICE) {
            // One input slice a step.  Voltage variation (memfast/reference.py:77-82): every
            // input value carries its own factor, x = digit * (1 + vv*z), held as fp16 hi + lo
            // operands, and a pair takes 3*KS MFMAs (hi*hi + lo*hi + hi*lo, the narrow voltage
            // read's order).  slice_pair read noise (memfast/reference.py:86-90): each (weight
            // slice, input slice) pair reads its own plane of terms; input slice a's planes are
            // LDS unit g*A + a, in the buffer of its parity, the next unit's DMA in flight.
            const i64 vunits = kp / 8;
            const uint4 *vbase = args.volt + (v0 / 32) * vunits * 32 + lane;
            const i64 vplane = ((args.n + 31) / 32) * vunits * 32;
            for (int a = 0; a < A; ++a) {
                const int u = g * A + a;
                if (SLICE && u + 1 < G * A) fetch(u + 1, ((u + 1) & 1) ? sF1 : sF0);
                const uint4 *fu = (SLICE ? ((u & 1) ? sF1 : sF0) : sCur) + lane;
                v8h_w hi[KS], lo[KS];
                if (VNOISE) {
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        const i64 at = (g * (P / 8) + ks * 2) * 32;
                        hi[ks] = __builtin_bit_cast(v8h_w, live_block ? vbase[a * vplane + at]
                                                                      : uint4{});
                        lo[ks] = __builtin_bit_cast(v8h_w, live_block ? vbase[(A + a) * vplane + at]
                                                                      : uint4{});
                    }
                } else {
                    digits(hi, a);
                }
                for (int w = 0; w < W; ++w) {
                    v8h_w F[NOISY_TERMS][KS];
#pragma unroll
                    for (int term = 0; term < NOISY_TERMS; ++term)
#pragma unroll
                        for (int ks = 0; ks < KS; ++ks)
                            F[term][ks] = __builtin_bit_cast(
                                v8h_w, fu[((w * NOISY_TERMS + term) * KS + ks) * 64]);
                    v16f_w I = {};
                    if (VNOISE) {
#pragma unroll
                        for (int term = 0; term < NOISY_TERMS; ++term)
#pragma unroll
                            for (int ks = 0; ks < KS; ++ks)
                                I = __builtin_amdgcn_mfma_f32_32x32x16_f16(F[term][ks], hi[ks], I,
                                                                           0, 0, 0);
#pragma unroll
                        for (int ks = 0; ks < KS; ++ks)
                            I = __builtin_amdgcn_mfma_f32_32x32x16_f16(F[0][ks], lo[ks], I, 0, 0,
                                                                       0);
                    } else {
#pragma unroll
                        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                            for (int term = 0; term < NOISY_TERMS; ++term)
                                I = __builtin_amdgcn_mfma_f32_32x32x16_f16(F[term][ks], hi[ks], I,
                                                                           0, 0, 0);
                    }
                    convert(I, w, a);
                }
                // slice_pair: the next unit is in LDS and every wave is done with this one
                // (the read's last unit waits at the end of the step).
                if (SLICE && a + 1 < A) {
                    __builtin_amdgcn_s_waitcnt(0);
                    __syncthreads();
                }
            }
        }
        // Input slices in pairs: the digits of a slice are built once per read;
        // per weight slice the two currents are two interleaved MFMA chains.
        int a = 0;
        for (; !VNOISE && !SLICE && a + 1 < A; a += 2) {
            v8h_w B0[KS], B1[KS];
            digits(B0, a);
            digits(B1, a + 1);
            for (int w = 0; w < W; ++w) {
                v8h_w F[NOISY_TERMS][KS];
                terms(F, w);
                v16f_w I0 = {}, I1 = {};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                    for (int term = 0; term < NOISY_TERMS; ++term) {
                        I0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(F[term][ks], B0[ks], I0, 0, 0, 0);
                        I1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(F[term][ks], B1[ks], I1, 0, 0, 0);
                    }
                convert(I0, w, a);
                convert(I1, w, a + 1);
            }
        }
        if (!VNOISE && !SLICE && a < A) {
            v8h_w B0[KS];
            digits(B0, a);
            for (int w = 0; w < W; ++w) {
                v8h_w F[NOISY_TERMS][KS];
                terms(F, w);
                v16f_w I0 = {};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                    for (int term = 0; term < NOISY_TERMS; ++term)
                        I0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(F[term][ks], B0[ks], I0, 0, 0, 0);
                convert(I0, w, a);
            }
        }

        // FP64 restore and torch's cascade over reads (level step 16; level 1
        // is kept in `out`, reads < 256).
        if (args.totals) {
            if (live_n) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const i64 c = col_tile + (r >> 2) * 8 + lhalf * 4 + (r & 3);
                    if (c < args.ncols)
                        args.out[(n_out * G + g) * args.ldo + c] = double(int(T[r] + plan.bias));
                }
            }
        } else {
            const double xs = live_n ? args.xscale[n_out * G + g] : 0.0;
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const i64 c = col_tile + qd * 8 + lhalf * 4;
                double ws[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    ws[e] = (c + e < args.ncols) ? args.wscale[i64(g) * args.ldws + c + e] : 0.0;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc0[qd * 4 + e] = acc0[qd * 4 + e] + restore_fast(int(T[qd * 4 + e] + plan.bias),
                                                                       xs, ws[e]);
            }
            if (((g + 1) & 15) == 0) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const i64 c = col_tile + (r >> 2) * 8 + lhalf * 4 + (r & 3);
                    if (live_n && c < args.ncols) {
                        double *dst = args.out + n_out * args.ldo + c;
                        *dst = g + 1 == 16 ? acc0[r] : *dst + acc0[r];
                    }
                    acc0[r] = 0.0;
                }
            }
        }
        // The next read's codes arrive with its conductance terms, before the
        // barrier, so no load is outstanding inside the next step's compute.
        if (g + 1 < G) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                qc[ks] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                       qbuf, q_off + (g + 1) * P * 2 + ks * 32, 0, 0));
        }
        __builtin_amdgcn_s_waitcnt(0);
        settle(qc);
        __syncthreads();
    };
    for (int g = 0; g < G; g += 2) {
        step(g, sF0, sF1);
        if (g + 1 < G) step(g + 1, sF1, sF0);
    }
    if (args.totals || !live_n) return;

    bool finite = true;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const i64 c = col_tile + (r >> 2) * 8 + lhalf * 4 + (r & 3);
        if (c >= args.ncols) continue;
        double *dst = args.out + n_out * args.ldo + c;
        const double s = acc0[r] + (G >= 16 ? *dst : 0.0);
        *dst = s;
        finite = finite && fabs(s) <= DBL_MAX;
    }
    if (!finite && args.status) atomicOr(args.status, u32(MF_STATUS_OUTPUT));
}

#define MF_NOISY_WIDE_INST(KS, NL, FRMAX, VN, SL)                                             \
    template __global__ void k_noisy_wide<KS, NL, FRMAX, VN, SL>(const NoisyWidePlan,            \
                                                                 const NoisyWideArgs);
// Linear or S-curve ADC; digits or voltage operands; shared (one LDS unit per read) or
// slice_pair read noise (one LDS unit per read and input slice).
#define MF_NOISY_WIDE_INST4(KS, FRMAX)                  \
    MF_NOISY_WIDE_INST(KS, false, FRMAX, false, false)  \
    MF_NOISY_WIDE_INST(KS, true, FRMAX, false, false)   \
    MF_NOISY_WIDE_INST(KS, false, FRMAX, true, false)   \
    MF_NOISY_WIDE_INST(KS, true, FRMAX, true, false)    \
    MF_NOISY_WIDE_INST(KS, false, FRMAX, false, true)   \
    MF_NOISY_WIDE_INST(KS, true, FRMAX, false, true)    \
    MF_NOISY_WIDE_INST(KS, false, FRMAX, true, true)    \
    MF_NOISY_WIDE_INST(KS, true, FRMAX, true, true)
MF_NOISY_WIDE_INST4(2, WIDE_FRAGS_TINY)
MF_NOISY_WIDE_INST4(2, WIDE_FRAGS_SMALL)
MF_NOISY_WIDE_INST4(2, WIDE_FRAGS_LARGE)
MF_NOISY_WIDE_INST4(4, WIDE_FRAGS_TINY)
MF_NOISY_WIDE_INST4(4, WIDE_FRAGS_SMALL)
MF_NOISY_WIDE_INST4(4, WIDE_FRAGS_LARGE)

}  // namespace mf
