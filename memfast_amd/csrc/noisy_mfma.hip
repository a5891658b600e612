// Noisy-device sliced array read on gfx950 fp16 MFMA, fused with the ADC, the
// signed shift-add, the scale restore and torch's read-order summation.
//
// Model (memfast/reference.py:63-117): per read group, input slice a and
// weight slice w,
//   I = sum_r (V * da/Ma) * (g[r,c] - L),   z = I * Ma*Mw / unit,
//   z = z / (1 + |alpha/max_w * z|) (S-curve),  code = round(clamp(z, 0, max_w)),
//   T = sum_a sum_w fa*fw*code.
// Here z = sum_r da * k1 * (g - L) with k1 = V*Mw/unit: the input digits da are
// small integers (exact in fp16) and k1 * (g - L) (FP32, at most Mw <= 255 times
// the conductance noise) is held as two fp16 terms hi + lo, hi = fp16(x) and
// lo = fp16(x - hi): 22 significant bits, within 2^-23 |x| of x (or 2^-25
// absolute where lo is an fp16 subnormal; the FP32 value itself carries 24 bits).  Two fp16 MFMAs with FP32
// accumulation give z to about FP32 accuracy; codes may flip where z lies within
// that error of a rounding boundary (a few in 10^7 codes on the bench shapes),
// the same order as FP32 summation-order differences from the CPU reference.
// ADC: the S-curve in the reference's FP32 roundings (RN(alpha*z), RN(1 + |t|), a
// correctly rounded quotient: scurve in mf_device.h), then y + 1.5*2^23 rounds half-even,
// med3 clamps, and v_mad_i32_i24 accumulates fa*fw*(0x400000 + code) modulo 2^32;
// plan.bias removes the offset (|T| < 2^24, so float(T) is exact).
//
// k_split_conductances writes the conductances (programming, drift, stuck-at
// and shared read noise, as memfast/reference.py:10-51, or an injected
// tensor) as g - L terms in MFMA fragment order, so each wave loads its
// 32-column x 32-row operand with one contiguous 1 KiB access per term.
// k_noisy: block = 4 waves (2 column x 2 vector), wave tile 32 columns x 32
// vectors, A operand = conductance terms, B operand = input digits built in
// registers from the codes q.  Per read and pair: 2*KS MFMAs and the ADC.
// With voltage variation (VNOISE) every input digit carries its own factor
// (1 + vv*z), so the B operand is real too: k_voltage_terms splits digit*(1 + vv*z)
// into fp16 hi + lo, and a pair takes 3*KS MFMAs (hi*hi + lo*hi + hi*lo; the lo*lo
// term is below 2^-21 of the product).  With slice_pair read noise (SLICE) each
// (weight slice, input slice) pair reads its own conductances: k_split_conductances
// writes one plane of terms per input slice and a pair loads its plane.
#include <cfloat>

#include "mf_kernels.h"

namespace mf {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4fn __attribute__((ext_vector_type(4)));

template <int KS>
__global__ __launch_bounds__(256) void k_split_conductances(const mf_config cfg, const u8 *packed_t,
                                                            const float *g_in, i64 m, i64 p,
                                                            i64 ncols, u32 seed, u64 event,
                                                            i64 c_begin, i64 CB,
                                                            const NoisyPlan plan, uint4 *gs) {
    constexpr int P = 16 * KS;
    const int R = cfg.rows, C = cfg.cols, W = cfg.n_w;
    const i64 kp = m * R, G = kp / P;
    const i64 total = i64(W) * CB * G * KS * 64;
    const u64 read_seed = event_seed(seed, event);
    for (i64 t = i64(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += i64(gridDim.x) * blockDim.x) {
        i64 rest = t;
        const int lane = int(rest & 63); rest >>= 6;
        const int ks = int(rest % KS); rest /= KS;
        const i64 g = rest % G; rest /= G;
        const i64 cb = rest % CB;
        const int w = int(rest / CB);
        const int lr = lane & 31, h = lane >> 5;
        const i64 c = c_begin + cb * 32 + lr;
        const i64 k0 = g * P + ks * 16 + h * 8;
        float level[8] = {};
        u64 cells[8] = {};
        if (c < ncols) {
            const uint2 bytes = *reinterpret_cast<const uint2 *>(packed_t + c * kp + k0);
            const i64 i = k0 / R, r0 = k0 - i * R;
            const i64 tt = c / C, cc = c - tt * C;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const u8 code = u8(((j < 4 ? bytes.x : bytes.y) >> (8 * (j & 3))) & 0xFFu);
                cells[j] = u64((((i * p + tt) * W + w) * R + r0 + j) * C + cc);
                level[j] = g_in ? g_in[cells[j]]
                                : cell_conductance<float>(cfg, code, w, cells[j], seed, read_seed);
            }
        }
        // slice_pair read noise (memfast/reference.py:86-90): an independent read factor
        // per (cell, input slice), one plane of terms per input slice.
        // Output-mode read noise: plane 1 holds (k1 * g / Mw)^2 for the variance
        // sum_r d^2 * (k1 * g)^2 (memfast/reference.py:104-108).
        for (int plane = 0; plane < plan.planes; ++plane) {
            u32 terms[2][4] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
            if (c < ncols) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float g_read = level[j];
                    if (plan.out_noise && plane == 1) {
                        const float y = g_read * plan.qk[w];
                        const float q = y * y;
                        const _Float16 hi = static_cast<_Float16>(q);
                        const _Float16 lo = static_cast<_Float16>(q - static_cast<float>(hi));
                        const int shift = 16 * (j & 1);
                        terms[0][j >> 1] |= u32(__builtin_bit_cast(unsigned short, hi)) << shift;
                        terms[1][j >> 1] |= u32(__builtin_bit_cast(unsigned short, lo)) << shift;
                        continue;
                    }
                    if (plan.planes > 1 && !plan.out_noise) {
                        const u64 address = cells[j] * u64(cfg.n_in) + u64(plane);
                        g_read = g_read * exp_small(cfg.f_read * normal_fast(address, read_seed, 20u));
                    }
                    const float delta = (g_read - cfg.f_low) * plan.k1[w];   // ADC counts per digit
                    const _Float16 hi = static_cast<_Float16>(delta);         // round to nearest even
                    const _Float16 lo = static_cast<_Float16>(delta - static_cast<float>(hi));
                    const int shift = 16 * (j & 1);
                    terms[0][j >> 1] |= u32(__builtin_bit_cast(unsigned short, hi)) << shift;
                    terms[1][j >> 1] |= u32(__builtin_bit_cast(unsigned short, lo)) << shift;
                }
            }
            const i64 vw = i64(w) * plan.planes + plane;   // plane of (weight, input) slices
            uint4 *dst = gs + (((vw * CB + cb) * G + g) * NOISY_TERMS * KS + ks) * 64 + lane;
#pragma unroll
            for (int term = 0; term < NOISY_TERMS; ++term)
                dst[term * KS * 64] = make_uint4(terms[term][0], terms[term][1], terms[term][2],
                                                 terms[term][3]);
        }
    }
}

template __global__ void k_split_conductances<2>(const mf_config, const u8 *, const float *, i64,
                                                 i64, i64, u32, u64, i64, i64, const NoisyPlan,
                                                 uint4 *);
template __global__ void k_split_conductances<4>(const mf_config, const u8 *, const float *, i64,
                                                 i64, i64, u32, u64, i64, i64, const NoisyPlan,
                                                 uint4 *);

// Buffer resource over [base, base + bytes): loads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t noisy_buffer(const void *base, i64 bytes) {
    const int records = bytes > 0x7FFFFFFF ? 0x7FFFFFFF : int(bytes < 0 ? 0 : bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), short(0), records,
                                             0x00020000);
}

// Eight input digits (bytes of `word`, slice (shift, mask)) as eight fp16.  Each digit d
// (at most 8 bits) becomes the low byte of fp16 0x64dd = 1024 + d: one v_perm places two
// digits beside two 0x64 bytes, and one packed fp16 subtraction of 1024 leaves d exactly
// (the same fp16 values as a conversion).  Six instructions per four digits.
__device__ __forceinline__ v8h digits_f16(uint2 word, int shift, u32 mask4) {
    typedef _Float16 v2f16 __attribute__((ext_vector_type(2)));
    const v2f16 base = {_Float16(1024.0f), _Float16(1024.0f)};
    const u32 lo = (word.x >> shift) & mask4, hi = (word.y >> shift) & mask4;
    // Byte pool of v_perm(src0, src1, sel): src1 bytes 0-3 (0x64), src0 bytes 4-7.
    const u32 k64 = 0x64646464u;
    const u32 w[4] = {__builtin_amdgcn_perm(lo, k64, 0x00050004u), __builtin_amdgcn_perm(lo, k64, 0x00070006u),
                      __builtin_amdgcn_perm(hi, k64, 0x00050004u), __builtin_amdgcn_perm(hi, k64, 0x00070006u)};
    u32 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = __builtin_bit_cast(u32, __builtin_bit_cast(v2f16, w[i]) - base);
    return __builtin_bit_cast(v8h, make_uint4(o[0], o[1], o[2], o[3]));
}

// Eight consecutive input codes of one vector: bytes (narrow) or 32-bit words (wide).
__device__ __forceinline__ void codes8(const u8 *q, u32 (&c)[8]) {
    const uint2 bytes = *reinterpret_cast<const uint2 *>(q);
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = ((j < 4 ? bytes.x : bytes.y) >> (8 * (j & 3))) & 0xFFu;
}
__device__ __forceinline__ void codes8(const u32 *q, u32 (&c)[8]) {
    const uint4 a = *reinterpret_cast<const uint4 *>(q);
    const uint4 b = *reinterpret_cast<const uint4 *>(q + 4);
    c[0] = a.x; c[1] = a.y; c[2] = a.z; c[3] = a.w;
    c[4] = b.x; c[5] = b.y; c[6] = b.z; c[7] = b.w;
}

template <typename Code>
__global__ void k_voltage_terms(const mf_config cfg, const Code *q, i64 n, i64 m, u32 seed,
                                u64 event, int squares, uint4 *volt) {
    const int R = cfg.rows, A = cfg.n_in;
    const i64 kp = m * R, units = kp / 8, vblocks = (n + 31) / 32;
    const i64 total = i64(A) * vblocks * units * 32;
    const u64 read_seed = event_seed(seed, event);
    for (i64 t = i64(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += i64(gridDim.x) * blockDim.x) {
        // t is the operand's index in [A][vblocks][units][32].
        const i64 lr = t & 31, rest = t >> 5;
        const i64 u = rest % units, vb = (rest / units) % vblocks;
        const int a = int(rest / (units * vblocks));
        const i64 v = vb * 32 + lr;
        const i64 plane = i64(A) * vblocks * units * 32;   // one term of every slice
        if (v >= n) {
            for (int term = 0; term < (squares ? 4 : 2); ++term)
                volt[term * plane + t] = make_uint4(0u, 0u, 0u, 0u);
            continue;
        }
        const i64 k0 = u * 8;
        u32 codes[8];
        codes8(q + v * kp + k0, codes);
        const u32 shift = u32(cfg.in_shift[a]), mask = u32(cfg.in_mask[a]);
        // Terms 0, 1: hi and lo of x = digit * (1 + vv*z); with `squares` (output-mode read
        // noise) terms 2, 3: hi and lo of RN(x * x), the variance sum's operand.
        u32 w4[4][4] = {};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const u32 digit = (codes[j] >> shift) & mask;
            float x = 0.0f;   // a zero digit stays zero whatever its factor
            if (digit) {
                const i64 k = k0 + j, i = k / R, r = k - i * R;
                const u64 address = u64(((v * m + i) * A + a) * R + r);
                const float z = normal_fast(address, read_seed, 40u);
                x = float(digit) * (1.0f + cfg.f_vnoise * z);
            }
            const float sq = x * x;
            const float value[2] = {x, sq};
            const int half = 16 * (j & 1);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const _Float16 hi = static_cast<_Float16>(value[k]);
                const _Float16 lo = static_cast<_Float16>(value[k] - static_cast<float>(hi));
                w4[2 * k][j >> 1] |= u32(__builtin_bit_cast(unsigned short, hi)) << half;
                w4[2 * k + 1][j >> 1] |= u32(__builtin_bit_cast(unsigned short, lo)) << half;
            }
        }
        for (int term = 0; term < (squares ? 4 : 2); ++term)
            volt[term * plane + t] = make_uint4(w4[term][0], w4[term][1], w4[term][2], w4[term][3]);
    }
}

template __global__ void k_voltage_terms<u8>(const mf_config, const u8 *, i64, i64, u32, u64,
                                            int, uint4 *);
template __global__ void k_voltage_terms<u32>(const mf_config, const u32 *, i64, i64, u32, u64,
                                             int, uint4 *);

// normal_fast() at the addresses base + offset (offset < 2^31) for one stream pair: the
// high-word folds of both streams are computed once for base's high word, and again only in
// a lane whose low word carries.
struct NormalRun {
    u32 lo, hi, fold_u, fold_v;
    __device__ __forceinline__ NormalRun(u64 base, u64 seed, u32 stream)
        : lo(u32(base)), hi(u32(base >> 32)), fold_u(uniform_fold(hi, seed, stream)),
          fold_v(uniform_fold(hi, seed, stream + 1u)) {}
    __device__ __forceinline__ float at(u32 offset, u64 seed, u32 stream) const {
        const u32 low = lo + offset;
        u32 fu = fold_u, fv = fold_v;
        if (low < offset) {   // the low word carried into the high word
            fu = uniform_fold(hi + 1u, seed, stream);
            fv = uniform_fold(hi + 1u, seed, stream + 1u);
        }
        return box_muller(uniform_finish(low, fu), uniform_finish(low, fv));
    }
};

template <int KS, int NA, bool NONLINEAR, bool VNOISE, bool SLICE, bool OUTN>
__device__ __forceinline__ void noisy_read(const NoisyPlan &plan, const NoisyArgs &args) {
    const float MAGIC = 12582912.0f;   // 1.5 * 2^23
    constexpr int P = 16 * KS;
    constexpr int BC = 64, BV = 64;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wc = wave & 1, wv = wave >> 1;
    const int lrow = lane & 31, lhalf = lane >> 5;
    // Vector blocks are the fast tile axis and each XCD takes a contiguous run of tiles, so
    // the blocks in flight on an XCD share a column block's conductance terms in its L2
    // (FETCH_SIZE at config 2: -34%, slice_pair -77%).  Voltage operands are as large as the
    // terms and indexed by the vector block; there the plain order fetches 3.5 times less.
    u32 vtile = blockIdx.x, ctile = blockIdx.y;
    if (!VNOISE) xcd_tile(blockIdx.x + blockIdx.y * gridDim.x, gridDim.x, gridDim.y, vtile, ctile);
    const i64 c0 = i64(ctile) * BC;                   // chunk-relative first column
    const i64 v0 = i64(vtile) * BV;
    const int G = int(args.G);
    const int A = plan.n_in, W = plan.n_w;
    const i64 kp = args.kp;
    const i64 cbw = (c0 + wc * 32) / 32;
    const i64 vrows = (args.n - v0) < BV ? (args.n - v0) : BV;
    const __amdgpu_buffer_rsrc_t qbuf = noisy_buffer(args.q + v0 * kp, vrows * kp);
    const int q_off = (wv * 32 + lrow) * int(kp) + lhalf * 8;
    const uint4 *frag_base = args.gs + cbw * i64(G) * NOISY_TERMS * KS * 64 + lane;
    const i64 w_stride = args.CB * i64(G) * NOISY_TERMS * KS * 64;

    // This lane's output coordinates (MFMA 32x32 layout: reg r -> column
    // 8*(r/4) + 4*lhalf + r%4 of the wave tile, vector lrow).
    const i64 n_out = v0 + wv * 32 + lrow;
    const i64 col_tile = args.c_begin + c0 + wc * 32;   // absolute first column of the wave

    // Cascade levels 0 and 1 per output.  The 32-row reads keep them in LDS (each lane
    // only ever touches its own words), which leaves room for a fourth wave per SIMD
    // (not with voltage noise, whose operand loads run faster at three).
    constexpr bool LDS_SUMS = KS == 2 && !VNOISE;
    __shared__ float sums[LDS_SUMS ? 2 : 1][LDS_SUMS ? 4 : 1][16][64];
    float acc[2][LDS_SUMS ? 1 : 16];
    auto sum_get = [&](int level, int r) -> float {
        if constexpr (LDS_SUMS) return sums[level][wave][r][lane];
        else return acc[level][r];
    };
    auto sum_set = [&](int level, int r, float v) {
        if constexpr (LDS_SUMS) sums[level][wave][r][lane] = v;
        else acc[level][r] = v;
    };
#pragma unroll
    for (int r = 0; r < 16; ++r) { sum_set(0, r, 0.0f); sum_set(1, r, 0.0f); }

    // Reads of this block: [g0, g1) (a read split across blocks writes totals).
    const int g0 = int(args.g_begin + i64(blockIdx.z) * args.g_step);
    const int g1 = int((g0 + args.g_step) < args.g_end ? (g0 + args.g_step) : args.g_end);
    uint2 qw[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        qw[ks] = make_uint2(0u, 0u);
        if (VNOISE) continue;
        const u32 x = __builtin_amdgcn_raw_buffer_load_b32(qbuf, q_off + g0 * P + ks * 16, 0, 0);
        const u32 y = __builtin_amdgcn_raw_buffer_load_b32(qbuf, q_off + g0 * P + ks * 16 + 4, 0, 0);
        qw[ks] = make_uint2(x, y);
    }
    // Voltage-noise operands of this wave's 32 vectors: [term][a][vector block] runs of
    // kp/8 units of 32 uint4, so a wave's operand is 1 KiB contiguous.
    const i64 vunits = kp / 8, vblocks = (args.n + 31) / 32, vblock = (v0 + wv * 32) / 32;
    const bool vlive = vblock < vblocks;   // wave-uniform; padded vectors hold zeros
    const i64 vplane = vblocks * vunits * 32;   // one (term, a) plane, in uint4
    const uint4 *vbase = args.volt + vblock * vunits * 32 + lane;   // lane = lhalf * 32 + lrow
    auto volt_operand = [&](int term, int a, int g, int ks) -> v8h {
        if (!vlive) return v8h{};
        return __builtin_bit_cast(
            v8h, vbase[(term * A + a) * vplane + (g * (P / 8) + ks * 2) * 32]);
    };

    // Conductance terms of (read g, weight slice w), double-buffered in registers:
    // the next slice's terms are in flight while the current slice's MFMAs run.
    // `w` indexes planes of terms: the weight slice, or with SLICE (weight slice, input
    // slice) as w * A + a.
    auto load_terms = [&](v8h (&F)[NOISY_TERMS][KS], int g, int w) {
        const uint4 *frag = frag_base + i64(g) * NOISY_TERMS * KS * 64 + w * w_stride;
#pragma unroll
        for (int term = 0; term < NOISY_TERMS; ++term)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                F[term][ks] = __builtin_bit_cast(v8h, frag[(term * KS + ks) * 64]);
    };
    // (With KS == 2 a second buffer would cost the third wave per SIMD: 32-row reads
    // load each slice's terms where they are used.)
    v8h Fa[NOISY_TERMS][KS], Fb[NOISY_TERMS][KS];
    if (KS != 2 && !SLICE && !OUTN && g0 < g1) load_terms(Fa, g0, 0);

    for (int g = g0; g < g1; ++g) {
        // Input digits of this read for every slice (B operands).  With voltage
        // variation the operands come from k_voltage_terms where they are used.
        v8h B[(VNOISE || OUTN) ? 1 : NA][KS];
        // Output-mode noise builds each slice's digits where they are used, from the codes
        // of this read (kept past the next read's prefetch).
        uint2 qcur[OUTN ? KS : 1];
        if (OUTN) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) qcur[OUTN ? ks : 0] = qw[ks];
        }
        if (!VNOISE && !OUTN) {
#pragma unroll
            for (int a = 0; a < NA; ++a) {
                if (a >= A) break;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    B[(VNOISE || OUTN) ? 0 : a][ks] =
                        digits_f16(qw[ks], plan.in_shift[a], plan.in_mask4[a]);
            }
        }
        if (!VNOISE && g + 1 < g1) {
            const int next = (g + 1) * P;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const u32 x = __builtin_amdgcn_raw_buffer_load_b32(qbuf, q_off + next + ks * 16, 0, 0);
                const u32 y = __builtin_amdgcn_raw_buffer_load_b32(qbuf, q_off + next + ks * 16 + 4, 0, 0);
                qw[ks] = make_uint2(x, y);
            }
        }

        // Integer totals modulo 2^32.  Every conversion adds fa*fw*(0x400000 + code), so
        // they start at plan.bias = -0x400000 * sum(fa*fw) and end at the totals themselves.
        u32 Ti[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) Ti[r] = plan.bias;
        // The reads of weight slice w with input slices [a_lo, a_hi) from terms F.
        auto slice_reads = [&](const v8h (&F)[NOISY_TERMS][KS], int w, int a_lo, int a_hi) {
            const float top = plan.top_magic[w], alpha = plan.alpha[w];
            auto convert = [&](const v16f &I, int a) {
                // Sign-extended here so the compiler sees a 24-bit operand (v_mad_i32_i24).
                const u32 f24 = u32(int(plan.f24[a][w] << 8) >> 8);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    // The terms carry k1, so I is already z = I * Ma*Mw / unit.  The
                    // S-curve is the reference's rounded arithmetic (scurve); rounding to
                    // an integer (half-even) happens in the add to 1.5 * 2^23, then med3
                    // clamps in that domain; its low 24 bits are 0x400000 + code.
                    float y = (NONLINEAR ? scurve(I[r], alpha) : I[r]) + MAGIC;
                    y = __builtin_amdgcn_fmed3f(y, MAGIC, top);
                    const int low = int(__float_as_uint(y) << 8) >> 8;
                    Ti[r] += u32(low) * f24;
                }
            };
#pragma unroll
            for (int a = 0; a < NA; ++a) {
                if (a >= A) break;
                if (a < a_lo || a >= a_hi) continue;
                v16f I = {};
                if (VNOISE) {
                    v8h hi[KS], lo[KS];
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        hi[ks] = volt_operand(0, a, g, ks);
                        lo[ks] = volt_operand(1, a, g, ks);
                    }
#pragma unroll
                    for (int term = 0; term < NOISY_TERMS; ++term)
#pragma unroll
                        for (int ks = 0; ks < KS; ++ks)
                            I = __builtin_amdgcn_mfma_f32_32x32x16_f16(F[term][ks], hi[ks], I, 0, 0,
                                                                       0);
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks)
                        I = __builtin_amdgcn_mfma_f32_32x32x16_f16(F[0][ks], lo[ks], I, 0, 0, 0);
                } else {
#pragma unroll
                    for (int term = 0; term < NOISY_TERMS; ++term)
#pragma unroll
                        for (int ks = 0; ks < KS; ++ks)
                            I = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                                F[term][ks], B[(VNOISE || OUTN) ? 0 : a][ks], I, 0, 0, 0);
                }
                convert(I, a);
            }
        };
        // Output-mode read noise (memfast/reference.py:99-112), in ADC counts: the current
        // z = I (terms k1*(g - L)); the mean's sum k1*sum d*g = I + k1*L*sum d; the
        // variance's sum Mw^2 * Q with Q = sum d^2 * (k1*g/Mw)^2 (plane 1, digits squared
        // exactly in fp16); then z += mean + sqrt(variance) * normal(address) with the
        // reference's per-(vector, read, tile, a, w, column) address, and the ADC.
        auto output_reads = [&](const v8h (&Fg)[NOISY_TERMS][KS], const v8h (&Fq)[NOISY_TERMS][KS],
                                int w) {
            const float top = plan.top_magic[w], alpha = plan.alpha[w];
            const float var_scale = plan.out_var[w];
            const i64 C = args.C;
            const i64 tile = col_tile / C, cc0 = col_tile - tile * C;
            const i64 p_tiles = args.ldws / C;
            // One input slice at a time (not unrolled): the 16 in-kernel normals per slice
            // need the registers.
#pragma unroll 1
            for (int a = 0; a < A; ++a) {
                v16f I = {}, Q = {};
                float rowsum;   // this lane's vector's input sum over the read's rows
                if (VNOISE) {
                    // Voltage variation: real operands x = digit * (1 + vv*z) and RN(x*x), each
                    // as fp16 hi + lo (3*KS MFMAs each, as the voltage read takes them); the sum
                    // of x in FP32 from its hi and lo terms.
                    v8h hi[KS], lo[KS];
                    float part = 0.0f;
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        hi[ks] = volt_operand(0, a, g, ks);
                        lo[ks] = volt_operand(1, a, g, ks);
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            part = part + (float(hi[ks][j]) + float(lo[ks][j]));
                    }
                    rowsum = part + __shfl_xor(part, 32);
#pragma unroll
                    for (int term = 0; term < NOISY_TERMS; ++term)
#pragma unroll
                        for (int ks = 0; ks < KS; ++ks)
                            I = __builtin_amdgcn_mfma_f32_32x32x16_f16(Fg[term][ks], hi[ks], I, 0,
                                                                       0, 0);
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks)
                        I = __builtin_amdgcn_mfma_f32_32x32x16_f16(Fg[0][ks], lo[ks], I, 0, 0, 0);
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        hi[ks] = volt_operand(2, a, g, ks);
                        lo[ks] = volt_operand(3, a, g, ks);
                    }
#pragma unroll
                    for (int term = 0; term < NOISY_TERMS; ++term)
#pragma unroll
                        for (int ks = 0; ks < KS; ++ks)
                            Q = __builtin_amdgcn_mfma_f32_32x32x16_f16(Fq[term][ks], hi[ks], Q, 0,
                                                                       0, 0);
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks)
                        Q = __builtin_amdgcn_mfma_f32_32x32x16_f16(Fq[0][ks], lo[ks], Q, 0, 0, 0);
                } else {
                    v8h digits[KS];
                    // The digit sum over the read's rows (the two lanes of a vector hold
                    // rows 0-7 and 8-15 of each 16-row block).
                    u32 count = 0u;
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        const uint2 code = qcur[OUTN ? ks : 0];
                        digits[ks] = digits_f16(code, plan.in_shift[a], plan.in_mask4[a]);
                        const u32 sh = u32(plan.in_shift[a]);
                        count = __builtin_amdgcn_sad_u8((code.x >> sh) & plan.in_mask4[a], 0u, count);
                        count = __builtin_amdgcn_sad_u8((code.y >> sh) & plan.in_mask4[a], 0u, count);
                    }
                    count += u32(__shfl_xor(int(count), 32));
                    rowsum = float(count);
#pragma unroll
                    for (int term = 0; term < NOISY_TERMS; ++term)
#pragma unroll
                        for (int ks = 0; ks < KS; ++ks)
                            I = __builtin_amdgcn_mfma_f32_32x32x16_f16(Fg[term][ks], digits[ks], I,
                                                                       0, 0, 0);
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        const v8h squared = digits[ks] * digits[ks];
#pragma unroll
                        for (int term = 0; term < NOISY_TERMS; ++term)
                            Q = __builtin_amdgcn_mfma_f32_32x32x16_f16(Fq[term][ks], squared, Q, 0,
                                                                       0, 0);
                    }
                }
                // Sign-extended here so the compiler sees a 24-bit operand (v_mad_i32_i24).
                const u32 f24 = u32(int(plan.f24[a][w] << 8) >> 8);
                const float shift = plan.kl[w] * rowsum;
                const u64 base = u64((((n_out * G + g) * p_tiles + tile) * A + a) * W + w) * u64(C) +
                                 u64(cc0 + lhalf * 4);
                const NormalRun normals(base, args.read_seed, 60u);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float mean = (I[r] + shift) * plan.out_mean;
                    const float sd = __builtin_amdgcn_sqrtf(fmaxf(Q[r] * var_scale, 0.0f));
                    const float z = normals.at(u32((r >> 2) * 8 + (r & 3)), args.read_seed, 60u);
                    const float current = I[r] + (mean + sd * z);
                    float y = (NONLINEAR ? scurve(current, alpha) : current) + MAGIC;
                    y = __builtin_amdgcn_fmed3f(y, MAGIC, top);
                    const int low = int(__float_as_uint(y) << 8) >> 8;
                    Ti[r] += u32(low) * f24;
                    // One output at a time: interleaving the normals of all 16 outputs
                    // would spill registers.
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        };
        if (OUTN) {
            for (int w = 0; w < W; ++w) {
                load_terms(Fa, g, 2 * w);
                load_terms(Fb, g, 2 * w + 1);
                output_reads(Fa, Fb, w);
            }
        } else if (SLICE) {
            for (int w = 0; w < W; ++w)
                for (int a = 0; a < A; ++a) {
                    load_terms(Fa, g, w * A + a);
                    slice_reads(Fa, w, a, a + 1);
                }
        } else if (KS == 2) {
            for (int w = 0; w < W; ++w) {
                load_terms(Fa, g, w);
                slice_reads(Fa, w, 0, A);
            }
        } else {
            // Fa holds (g, 0) on entry; on exit it holds (g + 1, 0) when that read exists.
            int w = 0;
            for (; w + 1 < W; w += 2) {
                load_terms(Fb, g, w + 1);
                slice_reads(Fa, w, 0, A);
                if (w + 2 < W) load_terms(Fa, g, w + 2);
                else if (g + 1 < g1) load_terms(Fa, g + 1, 0);
                slice_reads(Fb, w + 1, 0, A);
            }
            if (w < W) {
                if (g + 1 < g1) load_terms(Fb, g + 1, 0);
                slice_reads(Fa, w, 0, A);
#pragma unroll
                for (int term = 0; term < NOISY_TERMS; ++term)
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) Fa[term][ks] = Fb[term][ks];
            }
        }
        float T[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) T[r] = float(int(Ti[r]));

        if (args.totals) {
            if (n_out < args.n) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const i64 c = col_tile + (r >> 2) * 8 + lhalf * 4 + (r & 3);
                    if (c < args.ncols) args.out[(n_out * G + g) * args.ldo + c] = T[r];
                }
            }
            continue;
        }

        // Scale restore (float(T) * xs) * ws and torch's cascade over reads.
        const float xs = n_out < args.n ? args.xscale[n_out * G + g] : 0.0f;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            const i64 c = col_tile + qd * 8 + lhalf * 4;
            v4fn ws = {0.0f, 0.0f, 0.0f, 0.0f};
            if (c + 3 < args.ncols) {
                ws = *reinterpret_cast<const v4fn *>(args.wscale + i64(g) * args.ldws + c);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (c + e < args.ncols) ws[e] = args.wscale[i64(g) * args.ldws + c + e];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float v = T[qd * 4 + e] * xs;
                v = v * ws[e];
                sum_set(0, qd * 4 + e, sum_get(0, qd * 4 + e) + v);
            }
        }
        const int count = g + 1;
        if ((count & 15) == 0) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                sum_set(1, r, sum_get(1, r) + sum_get(0, r));
                sum_set(0, r, 0.0f);
            }
            if ((count & 255) == 0) {
                // Level 2 of the cascade lives in `out` (more than 255 reads).
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const i64 c = col_tile + (r >> 2) * 8 + lhalf * 4 + (r & 3);
                    if (n_out < args.n && c < args.ncols) {
                        float *dst = args.out + n_out * args.ldo + c;
                        *dst = count == 256 ? sum_get(1, r) : *dst + sum_get(1, r);
                    }
                    sum_set(1, r, 0.0f);
                }
            }
        }
    }
    if (args.totals || n_out >= args.n) return;

    bool finite = true;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
        const i64 c = col_tile + qd * 8 + lhalf * 4;
        float *dst = args.out + n_out * args.ldo + c;
        v4fn v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float s = sum_get(0, qd * 4 + e) + sum_get(1, qd * 4 + e);
            if (g1 >= 256 && c + e < args.ncols) s = s + dst[e];
            v[e] = s;
            finite = finite && (c + e >= args.ncols || fabsf(s) <= FLT_MAX);
        }
        if (c + 3 < args.ncols) {
            *reinterpret_cast<v4fn *>(dst) = v;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (c + e < args.ncols) dst[e] = v[e];
        }
    }
    if (!finite && args.status) atomicOr(args.status, u32(MF_STATUS_OUTPUT));
}

// Split reads of small batches (at most 32 vectors): one workgroup per (32-column block,
// read) with one wave per weight slice, so a read's 25 pairs (config 3) run on five waves
// at once instead of one after another.  Each wave loads its weight slice's terms once (a
// block reads every term of its read once) and converts its pairs with every input slice,
// whose digits it builds from the read's codes (fa*fw*(0x400000 + code) modulo 2^32, as
// noisy_read); the waves add their words in LDS (integer sums: any order gives the same
// totals) and the block writes the read's slice totals [n, G, ldo], or with args.restored
// their scale restore (float(T) * xs) * ws rounded as the fused epilogue rounds it;
// k_restore_sum_f32 or k_gru_step sums them over the reads in torch's order.  Plain and
// S-curve reads (terms event-independent or shared read noise).
template <int KS, int NA, bool NONLINEAR>
__global__ __launch_bounds__(512) void k_noisy_pairs(const NoisyPlan plan, const NoisyArgs args) {
    const float MAGIC = 12582912.0f;   // 1.5 * 2^23
    constexpr int P = 16 * KS;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // this wave's weight slice
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int W = plan.n_w, A = plan.n_in;
    const i64 cb = blockIdx.x;                       // chunk-relative 32-column block
    const i64 v0 = i64(blockIdx.y) * 32;
    const int g = int(args.g_begin + blockIdx.z);
    const i64 G = args.G, kp = args.kp;
    const i64 vrows = (args.n - v0) < 32 ? (args.n - v0) : 32;
    const __amdgpu_buffer_rsrc_t qbuf = noisy_buffer(args.q + v0 * kp, vrows * kp);
    const int q_off = lrow * int(kp) + lhalf * 8 + g * P;
    // Terms of (weight slice w, column block cb, read g): [w][CB][G][term][KS][64 lanes].
    const uint4 *frag = args.gs + (cb * G + g) * NOISY_TERMS * KS * 64 + lane +
                        w * (args.CB * G * NOISY_TERMS * KS * 64);
    v8h F[NOISY_TERMS][KS];
#pragma unroll
    for (int term = 0; term < NOISY_TERMS; ++term)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            F[term][ks] = __builtin_bit_cast(v8h, frag[(term * KS + ks) * 64]);
    uint2 codes[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
        codes[ks] = make_uint2(__builtin_amdgcn_raw_buffer_load_b32(qbuf, q_off + ks * 16, 0, 0),
                               __builtin_amdgcn_raw_buffer_load_b32(qbuf, q_off + ks * 16 + 4, 0, 0));
    // LDS: first the digits of every input slice (wave w builds slices w, w + W, ..), then
    // the waves' total words.
    __shared__ u32 shared_words[8 * 16 * 64];
    uint4 *sdigits = reinterpret_cast<uint4 *>(shared_words);   // [a][ks][64 lanes]
    for (int a = w; a < A; a += W)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            sdigits[(a * KS + ks) * 64 + lane] = __builtin_bit_cast(
                uint4, digits_f16(codes[ks], plan.in_shift[a], plan.in_mask4[a]));
    __syncthreads();
    // The epilogue's scales (outputs r = w, w + W, ..: the first four) are loaded now, so
    // their latency overlaps the pairs.
    const i64 n_out = v0 + lrow;
    const i64 col_tile = args.c_begin + cb * 32;
    auto column = [&](int r) { return col_tile + (r >> 2) * 8 + lhalf * 4 + (r & 3); };
    const float xs = args.restored && n_out < args.n ? args.xscale[n_out * G + g] : 0.0f;
    float ws_first[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = w + j * W;
        if (args.restored && r < 16 && column(r) < args.ncols)
            ws_first[j] = args.wscale[i64(g) * args.ldws + column(r)];
    }
    u32 Ti[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) Ti[r] = 0u;
    const float top = plan.top_magic[w], alpha = plan.alpha[w];
    // The MFMA order of noisy_read (terms outer, row blocks inner), so the totals are its
    // totals bit for bit.  Unrolled over the input slices (at most NA), so that a slice's
    // MFMAs can issue while the previous slice's currents are converted.
#pragma unroll
    for (int a = 0; a < NA; ++a) {
        if (a >= A) break;
        v8h digits[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            digits[ks] = __builtin_bit_cast(v8h, sdigits[(a * KS + ks) * 64 + lane]);
        v16f I = {};
#pragma unroll
        for (int term = 0; term < NOISY_TERMS; ++term)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                I = __builtin_amdgcn_mfma_f32_32x32x16_f16(F[term][ks], digits[ks], I, 0, 0, 0);
        const u32 f24 = u32(int(plan.f24[a][w] << 8) >> 8);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float y = (NONLINEAR ? scurve(I[r], alpha) : I[r]) + MAGIC;
            y = __builtin_amdgcn_fmed3f(y, MAGIC, top);
            const int low = int(__float_as_uint(y) << 8) >> 8;
            Ti[r] += u32(low) * f24;
        }
    }
    // Sum the slices' words: wave w writes its plane, then wave w adds outputs r = w, w + W..
    // (in the digits' LDS, once every wave has read them).
    u32 (*planes)[16][64] = reinterpret_cast<u32 (*)[16][64]>(shared_words);
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) planes[w][r][lane] = Ti[r];
    __syncthreads();
    for (int j = 0, r = w; r < 16; ++j, r += W) {
        u32 total = plan.bias;
        for (int k = 0; k < W; ++k) total += planes[k][r][lane];
        const i64 c = column(r);
        if (n_out < args.n && c < args.ncols) {
            float v = float(int(total));
            if (args.restored) {
                v = v * xs;
                // (selects, not an index: a dynamic index would put ws_first in scratch)
                const float ws = j == 0 ? ws_first[0] : j == 1 ? ws_first[1] : j == 2 ? ws_first[2]
                                 : j == 3 ? ws_first[3] : args.wscale[i64(g) * args.ldws + c];
                v = v * ws;
            }
            args.out[(n_out * G + g) * args.ldo + c] = v;
        }
    }
}

#define MF_PAIRS_INST(KS, NA)                                                                  \
    template __global__ void k_noisy_pairs<KS, NA, false>(const NoisyPlan, const NoisyArgs);  \
    template __global__ void k_noisy_pairs<KS, NA, true>(const NoisyPlan, const NoisyArgs);
MF_PAIRS_INST(2, 5)
MF_PAIRS_INST(2, 8)
MF_PAIRS_INST(4, 5)
#undef MF_PAIRS_INST

// The read kernel.  The output-mode variant (16 in-kernel normals per pair) runs three waves
// per SIMD at 32-row reads (a few spilled registers cost less than a wave fewer) and one at
// 64-row reads, which hold two slices' terms.
template <int KS, int NA, bool NONLINEAR, bool VNOISE, bool SLICE, bool OUTN>
__global__ __launch_bounds__(256, OUTN ? (KS == 2 && !VNOISE ? 3 : KS == 2 ? 2 : 1) : (KS == 2 && NA <= 5 && !VNOISE ? 4 : 2)) void k_noisy(
    const NoisyPlan plan,
                                                             const NoisyArgs args) {
    noisy_read<KS, NA, NONLINEAR, VNOISE, SLICE, OUTN>(plan, args);
}

__global__ void k_restore_sum_f32(const float *totals, i64 n, i64 G, i64 g_run, i64 ldt,
                                  i64 ncols, const float *xscale, const float *wscale, i64 ldws,
                                  float *out, i64 ldo, int lp, int restored, u32 *status) {
    // Reads arrive in batches of RESTORE_BATCH: a batch's loads are all issued before
    // its values enter the cascade, so a thread waits on memory once per batch rather
    // than once per read.  The arithmetic and the summation order are unchanged.
    constexpr int RESTORE_BATCH = 8;
    bool finite = true;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < n * ncols;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 v = i / ncols, c = i - v * ncols;
        const float *tv = totals + v * G * ldt + c;
        const float *xv = xscale + v * G;
        const float *wv = wscale + c;
        Cascade<float> cascade;
        cascade.reset();
        for (i64 g0 = 0; g0 < g_run; g0 += RESTORE_BATCH) {
            float t[RESTORE_BATCH], xs[RESTORE_BATCH], ws[RESTORE_BATCH];
#pragma unroll
            for (int j = 0; j < RESTORE_BATCH; ++j) {
                const i64 g = g0 + j < g_run ? g0 + j : g_run - 1;   // past the end: unused
                t[j] = tv[g * ldt];
                if (!restored) {
                    xs[j] = xv[g];
                    ws[j] = wv[g * ldws];
                }
            }
#pragma unroll
            for (int j = 0; j < RESTORE_BATCH; ++j) {
                if (g0 + j < g_run) {
                    float x = t[j];
                    if (!restored) {
                        x = x * xs[j];
                        x = x * ws[j];
                    }
                    cascade.push(x, lp);
                }
            }
        }
        const float s = cascade.finish();
        out[v * ldo + c] = s;
        finite = finite && fabsf(s) <= FLT_MAX;
    }
    if (!finite && status) atomicOr(status, u32(MF_STATUS_OUTPUT));
}

#define MF_NOISY_INST1(KS, NA, NL, VN, SL, ON) \
    template __global__ void k_noisy<KS, NA, NL, VN, SL, ON>(const NoisyPlan, const NoisyArgs);
#define MF_NOISY_INST(KS, NA)                                                                    \
    MF_NOISY_INST1(KS, NA, false, false, false, false) MF_NOISY_INST1(KS, NA, true, false, false, false) \
    MF_NOISY_INST1(KS, NA, false, true, false, false) MF_NOISY_INST1(KS, NA, true, true, false, false)   \
    MF_NOISY_INST1(KS, NA, false, false, true, false) MF_NOISY_INST1(KS, NA, true, false, true, false)   \
    MF_NOISY_INST1(KS, NA, false, true, true, false) MF_NOISY_INST1(KS, NA, true, true, true, false)     \
    MF_NOISY_INST1(KS, NA, false, false, false, true) MF_NOISY_INST1(KS, NA, true, false, false, true)   \
    MF_NOISY_INST1(KS, NA, false, true, false, true) MF_NOISY_INST1(KS, NA, true, true, false, true)
MF_NOISY_INST(2, 5)
MF_NOISY_INST(2, 8)
MF_NOISY_INST(4, 5)
#undef MF_NOISY_INST
#undef MF_NOISY_INST1

}  // namespace mf
