// Ideal-device sliced array read on gfx950 int8 MFMA, fused with the scale
// restore and torch's read-order summation.  Only `out` is written to HBM.
//
// With every device effect off the ADC count of slice pair (a, w) is the closed
// form code = min(S_aw, max_w), S_aw = sum_r da[n,r] * dw[r,c] (memfast/
// reference.py:63-117 with ideal conductances; exact because FP32 current
// errors stay far below half a count, checked on the host).  Per read:
//   * T = sum_aw fa*fw*min(S_aw, max_w) starts as the linear part
//     sum_aw fa*fw*S_aw, which is the plain int8 x int8 MFMA of the codes;
//   * pairs that can exceed max_w are tested on precomputed digit sums per
//     wave block (S <= Mw*max_n sum_r da, or S <= Ma*max_c sum_r dw); most
//     are proven clamp-free and need nothing more;
//   * each remaining pair gets its own MFMA on natural operand forms (masked
//     bytes whose int8 value is factor*digit), Y = fa*fw*S, a wave-wide
//     max (min) test against fa*fw*max_w, and -- only if some output exceeds
//     it -- the correction min(Y, lim) - Y per output.
// T is restored as (float(T) * xs[n,g]) * ws[g,c] and summed over reads in
// torch's CPU cascade order (level step 16; level 2 kept in `out`).
//
// Orientation: the MFMA A operand is the weight codes (tile rows = output
// columns c), the B operand the input codes (tile columns = vectors n), so the
// per-weight-slice masks are built once per wave and shared by TN vector tiles.
// Block = 4 waves: 2 (columns) x 2 (vectors); wave tile 32 columns x 32*TN
// vectors; LDS holds codes [64 x 32*KS] and [64*TN x 32*KS] per read, double
// buffered.  Roofline: int8 MFMA, with the VALU epilogue as co-bound.
#include <cfloat>
#include <type_traits>

#include "mf_kernels.h"

namespace mf {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32 sext_bytes(u32 x, int bits) {
    const u32 sign = (x >> (bits - 1)) & 0x01010101u;
    const u32 ext = (0xFFu << bits) & 0xFFu;
    return x | (sign * ext);
}

__device__ __forceinline__ v4i sext4(v4i x, int bits) {
    return v4i{int(sext_bytes(u32(x.x), bits)), int(sext_bytes(u32(x.y), bits)),
               int(sext_bytes(u32(x.z), bits)), int(sext_bytes(u32(x.w), bits))};
}

__device__ __forceinline__ v4i and4(v4i x, u32 m) {
    const int mi = int(m);
    return v4i{x.x & mi, x.y & mi, x.z & mi, x.w & mi};
}

__device__ __forceinline__ v16i mfma(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// Per-read digit sums, maximized over blocks of `block` (32 or 64) rows, then
// tested against the slot thresholds: out[rb][g] = mask of proven slots.
// Workgroup = 64 reads (one per lane, so a wave loads 64 consecutive P-byte
// runs of a row) x 16 waves that split the block's rows; LDS combines the
// partial maxima.  Digit sums use SWAR: (word >> shift) & mask per byte, then
// v_sad_u8 adds the four bytes.  Requires P in {32, 64} and reads that start
// at g * P (R a multiple of P).
template <int P>
__global__ __launch_bounds__(64 * DIGIT_WAVES) void k_digit_bits(
    const DigitJob a, const DigitJob b, i64 first_blocks, i64 kp, i64 G) {
    constexpr int CHUNKS = P / 16;
    __shared__ int partial[DIGIT_WAVES][8][64];
    const bool second = i64(blockIdx.y) >= first_blocks;
    const DigitJob &job = second ? b : a;
    const u8 *codes = job.codes;
    const i64 rows = job.rows;
    const int block = job.block;
    const SliceLayout &layout = job.layout;
    const SlotTests &tests = job.tests;
    uint64_t *out = job.out;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const i64 g = i64(blockIdx.x) * 64 + lane;
    const i64 rb = second ? i64(blockIdx.y) - first_blocks : i64(blockIdx.y);
    const int S = layout.count;
    const int per = block / DIGIT_WAVES;
    int best[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    u32 masks[8];
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) masks[sl] = sl < S ? u32(layout.mask[sl]) * 0x01010101u : 0u;
    // Every row's loads are issued before the first digit sum.
    constexpr int MAX_PER = 64 / DIGIT_WAVES;
    uint4 chunk[MAX_PER][CHUNKS];
    bool live[MAX_PER];
#pragma unroll
    for (int i = 0; i < MAX_PER; ++i) {
        const i64 row = rb * block + wave * per + i;
        live[i] = g < G && i < per && row < rows;
        const uint4 *src = reinterpret_cast<const uint4 *>(codes + row * kp + g * P);
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c)
            chunk[i][c] = live[i] ? src[c] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < MAX_PER; ++i) {
        if (!live[i]) continue;
#pragma unroll
        for (int sl = 0; sl < 8; ++sl) {
            if (sl >= S) break;
            const int sh = layout.shift[sl];
            const u32 mk = masks[sl];
            u32 sum = 0;
#pragma unroll
            for (int c = 0; c < CHUNKS; ++c) {
                sum = __builtin_amdgcn_sad_u8((chunk[i][c].x >> sh) & mk, 0u, sum);
                sum = __builtin_amdgcn_sad_u8((chunk[i][c].y >> sh) & mk, 0u, sum);
                sum = __builtin_amdgcn_sad_u8((chunk[i][c].z >> sh) & mk, 0u, sum);
                sum = __builtin_amdgcn_sad_u8((chunk[i][c].w >> sh) & mk, 0u, sum);
            }
            best[sl] = max(best[sl], int(sum));
        }
    }
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) partial[wave][sl][lane] = best[sl];
    __syncthreads();
    if (wave > 0 || g >= G || rb * block >= rows) return;
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {
        if (sl >= S) break;
        int m = best[sl];
        for (int w = 1; w < DIGIT_WAVES; ++w) m = max(m, partial[w][sl][lane]);
        partial[0][sl][lane] = m;
    }
    // Only this lane reads back its own words: no barrier needed.
    uint64_t bits = 0;
    uint64_t slots = tests.exists;
    while (slots) {
        const int slot = __builtin_ctzll(slots);
        slots &= slots - 1;
        if (partial[0][tests.slice[slot]][lane] <= tests.thr[slot]) bits |= uint64_t(1) << slot;
    }
    out[rb * G + g] = bits;
}

// Buffer resource over [base, base + bytes): loads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void *base, i64 bytes) {
    const int records = bytes > 0x7FFFFFFF ? 0x7FFFFFFF : int(bytes < 0 ? 0 : bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), short(0), records,
                                             0x00020000);
}

// T += min(Y, lim) - Y for a positive pair (max() for a negative one, lim < 0),
// skipped when no output of the 32x32 tile crosses lim (the usual case).  A positive
// pair has Y >= 0 and lim > 0, so min(Y, lim) - Y = -(Y -sat lim), an unsigned
// saturating subtract (one instruction).
template <bool POSITIVE>
__device__ __forceinline__ void correct_tile(v16i &T, const v16i &y, int lim) {
    int e = y[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) e = POSITIVE ? max(e, y[r]) : min(e, y[r]);
    if (__builtin_amdgcn_ballot_w64(POSITIVE ? e > lim : e < lim) == 0) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        if (POSITIVE)
            T[r] = int(u32(T[r]) - __builtin_elementwise_sub_sat(u32(y[r]), u32(lim)));
        else
            T[r] += max(lim - y[r], 0);
    }
}

template <int TN, int KS>
__global__ __launch_bounds__(256, TN == 1 && KS == 1 ? 5 : 2) void k_ideal(const IdealPlan plan,
                                                                           const IdealArgs args) {
    constexpr int BC = 64;                 // output columns per block
    constexpr int BV = 2 * TN * 32;        // vectors per block
    constexpr int KB = 32 * KS;            // code bytes per row and read (= P)
    constexpr int STRIDE = KB + 16;        // LDS row stride (conflict-free b128 reads)
    constexpr int CHUNKS = KB / 16;
    constexpr int W_LOADS = (BC * CHUNKS + 255) / 256;
    constexpr int X_LOADS = (BV * CHUNKS + 255) / 256;
    __shared__ __align__(16) u8 sW[2][BC * STRIDE];
    __shared__ __align__(16) u8 sX[2][BV * STRIDE];
    __shared__ __align__(16) float sWS[2][BC];
    __shared__ __align__(16) float sXS[2][BV];
    // Level 1 of the cascade, per wave and lane (it changes once per 16 reads;
    // keeping it out of registers leaves room for a fifth wave per SIMD).
    __shared__ float sAcc1[4][TN][16][64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wc = wave & 1, wv = wave >> 1;
    const i64 c0 = i64(blockIdx.x) * BC;
    const i64 v0 = i64(blockIdx.y) * BV;
    const int G = int(args.G);
    const i64 cblock = (c0 + wc * 32) / 32;          // weight digit-bits block (32 columns)
    const i64 vblock = (v0 + wv * TN * 32) / 64;     // input digit-bits block (64 vectors)
    const int lrow = lane & 31, lhalf = lane >> 5;
    const i64 kp = args.kp;

    // Block-local buffers: rows past n / ncols read as zero.
    const i64 wrows = (args.ncols - c0) < BC ? (args.ncols - c0) : BC;
    const i64 vrows = (args.n - v0) < BV ? (args.n - v0) : BV;
    const __amdgpu_buffer_rsrc_t wbuf = buffer_of(args.wt + c0 * kp, wrows * kp);
    const __amdgpu_buffer_rsrc_t xbuf = buffer_of(args.q + v0 * kp, vrows * kp);
    const __amdgpu_buffer_rsrc_t wsbuf =
        buffer_of(args.wscale + c0, (i64(G) * args.ldws - c0) * 4);
    const __amdgpu_buffer_rsrc_t xsbuf = buffer_of(args.xscale + v0 * G, vrows * G * 4);

    // Per-thread load slots (fixed across reads; the read adds g * P bytes).
    int w_off[W_LOADS], x_off[X_LOADS];
#pragma unroll
    for (int e = 0; e < W_LOADS; ++e) {
        const int c = tid + e * 256;
        w_off[e] = (c / CHUNKS) * int(kp) + (c % CHUNKS) * 16;
    }
#pragma unroll
    for (int e = 0; e < X_LOADS; ++e) {
        const int c = tid + e * 256;
        x_off[e] = (c / CHUNKS) * int(kp) + (c % CHUNKS) * 16;
    }
    // Wave 0 loads the column scales, the next BV / 64 waves the vector scales
    // (wave-uniform conditions, so the loads need no lane masks).
    static_assert(BC == 64 && BV % 64 == 0 && BC + BV <= 256, "scale loaders");
    const bool scale_w = wave == 0;
    const bool scale_x = wave >= 1 && wave <= BV / 64;
    const int scale_off = scale_w ? tid * 4 : (tid - BC) * G * 4;

    v4i rw[W_LOADS], rx[X_LOADS];
    float rscale = 0.0f;
    auto fetch = [&](int g) {
        const int kofs = g * KB;
#pragma unroll
        for (int e = 0; e < W_LOADS; ++e)
            rw[e] = __builtin_amdgcn_raw_buffer_load_b128(wbuf, w_off[e] + kofs, 0, 0);
#pragma unroll
        for (int e = 0; e < X_LOADS; ++e)
            rx[e] = __builtin_amdgcn_raw_buffer_load_b128(xbuf, x_off[e] + kofs, 0, 0);
        if (scale_w)
            rscale = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                wsbuf, scale_off + g * int(args.ldws) * 4, 0, 0));
        else if (scale_x)
            rscale = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                xsbuf, scale_off + g * 4, 0, 0));
    };
    // Tile rows are whole waves (multiples of 64 chunks), so the store conditions are
    // wave-uniform.
    auto stash = [&](int buf) {
#pragma unroll
        for (int e = 0; e < W_LOADS; ++e) {
            const int c = tid + e * 256;
            if (W_LOADS * 256 == BC * CHUNKS || wave + 4 * e < BC * CHUNKS / 64) {
                v4i v = rw[e];
                if (args.w_bits < 8) v = sext4(v, args.w_bits);
                *reinterpret_cast<v4i *>(&sW[buf][(c / CHUNKS) * STRIDE + (c % CHUNKS) * 16]) = v;
            }
        }
#pragma unroll
        for (int e = 0; e < X_LOADS; ++e) {
            const int c = tid + e * 256;
            if (X_LOADS * 256 == BV * CHUNKS || wave + 4 * e < BV * CHUNKS / 64) {
                v4i v = rx[e];
                if (args.a_bits < 8) v = sext4(v, args.a_bits);
                *reinterpret_cast<v4i *>(&sX[buf][(c / CHUNKS) * STRIDE + (c % CHUNKS) * 16]) = v;
            }
        }
        if (scale_w) sWS[buf][tid] = rscale;
        else if (scale_x) sXS[buf][tid - BC] = rscale;
    };

    float acc0[TN][16];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int r = 0; r < 16; ++r) { acc0[tn][r] = 0.0f; sAcc1[wave][tn][r][lane] = 0.0f; }

    fetch(0);
    stash(0);
    __syncthreads();

    const uint64_t *xbits = args.xbits + vblock * G;
    const uint64_t *wbits = args.wbits + cblock * G;
    const int G_run = int(args.G_run);   // reads past G_run hold only zero padding
    // One read; the LDS buffer index is a constant in each of the two copies.
    auto read = [&](const int g, auto buffer) {
        constexpr int cur = decltype(buffer)::value;
        if (g + 1 < G_run) fetch(g + 1);

        v4i Wr[KS], Xr[TN][KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            Wr[ks] = *reinterpret_cast<const v4i *>(
                &sW[cur][(wc * 32 + lrow) * STRIDE + ks * 32 + lhalf * 16]);
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
                Xr[tn][ks] = *reinterpret_cast<const v4i *>(
                    &sX[cur][(wv * TN * 32 + tn * 32 + lrow) * STRIDE + ks * 32 + lhalf * 16]);
        }

        // Linear part: sum over all pairs of fa*fw*S = the plain int8 product of
        // the (sign-extended) codes, one MFMA per 32 rows.
        v16i T[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            T[tn] = mfma(Wr[0], Xr[tn][0], v16i{});
#pragma unroll
            for (int ks = 1; ks < KS; ++ks) T[tn] = mfma(Wr[ks], Xr[tn][ks], T[tn]);
        }

        // Clamp candidates (pairs that can exceed max_w) not proven clamp-free
        // by the digit sums are recomputed alone, Y = fa*fw*S; only a tile where
        // some |Y| exceeds the limit lim = fa*fw*max_w pays the per-output
        // correction min(Y, lim) - Y (max() for negative pairs).  Slots are
        // numbered cw * 8 + ca, so one weight slice's failing slots share its
        // masked operand; the slot constants are scalar loads from the plan.
        uint64_t fail = plan.exists & ~(xbits[g] | wbits[g]);
        while (fail) {
            const int cw = __builtin_ctzll(fail) >> 3;
            u32 group = u32(fail >> (cw * 8)) & 0xFFu;
            fail &= ~(uint64_t(0xFF) << (cw * 8));
            const u32 wm = plan.cw_wnat[cw];
            const int wlim = plan.cw_limit[cw];
            v4i Wm[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) Wm[ks] = and4(Wr[ks], wm);
            // Positive pairs (fa * fw > 0) first, then negative ones.
            const u32 negative = plan.cw_negative_ca[cw];
            auto candidates = [&](u32 set, auto positive) {
                while (set) {
                    const int ca = __builtin_ctz(set);
                    set &= set - 1;
                    const u32 xm = plan.ca_xnat[ca];
                    const int lim = plan.ca_factor[ca] * wlim;
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn) {
                        v16i y = mfma(Wm[0], and4(Xr[tn][0], xm), v16i{});
#pragma unroll
                        for (int ks = 1; ks < KS; ++ks)
                            y = mfma(Wm[ks], and4(Xr[tn][ks], xm), y);
                        correct_tile<decltype(positive)::value>(T[tn], y, lim);
                    }
                }
            };
            candidates(group & ~negative, std::true_type{});
            candidates(group & negative, std::false_type{});
        }

        // Scale restore (float(T) * xs) * ws and cascade accumulation.
        v4f ws4[4];
#pragma unroll
        for (int qd = 0; qd < 4; ++qd)
            ws4[qd] = *reinterpret_cast<const v4f *>(&sWS[cur][wc * 32 + qd * 8 + lhalf * 4]);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            const float xs = sXS[cur][wv * TN * 32 + tn * 32 + lrow];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float v = float(T[tn][r]) * xs;
                v = v * ws4[r >> 2][r & 3];
                acc0[tn][r] = acc0[tn][r] + v;
            }
        }
        const int count = g + 1;
        if ((count & 15) == 0) {
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    sAcc1[wave][tn][r][lane] = sAcc1[wave][tn][r][lane] + acc0[tn][r];
                    acc0[tn][r] = 0.0f;
                }
            if ((count & 255) == 0) {
                // Level 2 of the cascade lives in `out` (more than 255 reads).
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
                    const i64 n = v0 + wv * TN * 32 + tn * 32 + lrow;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const i64 c = c0 + wc * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
                        const float a1 = sAcc1[wave][tn][r][lane];
                        if (n < args.n && c < args.ncols) {
                            float *dst = args.out + n * args.ldo + c;
                            *dst = count == 256 ? a1 : *dst + a1;
                        }
                        sAcc1[wave][tn][r][lane] = 0.0f;
                    }
                }
            }
        }

        if (g + 1 < G_run) stash(cur ^ 1);
        __syncthreads();
    };
    for (int g = 0; g < G_run; g += 2) {
        read(g, std::integral_constant<int, 0>{});
        if (g + 1 < G_run) read(g + 1, std::integral_constant<int, 1>{});
    }

    bool finite = true;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
        const i64 n = v0 + wv * TN * 32 + tn * 32 + lrow;
        if (n >= args.n) continue;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            const i64 c = c0 + wc * 32 + qd * 8 + lhalf * 4;
            float *dst = args.out + n * args.ldo + c;
            v4f v;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float s = acc0[tn][qd * 4 + e] + sAcc1[wave][tn][qd * 4 + e][lane];
                if (G_run >= 256 && c + e < args.ncols) s = s + dst[e];
                v[e] = s;
                finite = finite && (c + e >= args.ncols || fabsf(s) <= FLT_MAX);
            }
            if (c + 3 < args.ncols) {
                *reinterpret_cast<v4f *>(dst) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (c + e < args.ncols) dst[e] = v[e];
            }
        }
    }
    if (!finite && args.status) atomicOr(args.status, u32(MF_STATUS_OUTPUT));
    // The quantizers finished before this read began, so their status bits are final: the
    // first workgroup hands them to the caller, which then need not wait for the whole read.
    if (args.mailbox && blockIdx.x == 0 && blockIdx.y == 0 && tid == 0)
        publish_status(args.status, args.mailbox);
}

template __global__ void k_digit_bits<32>(const DigitJob, const DigitJob, i64, i64, i64);
template __global__ void k_digit_bits<64>(const DigitJob, const DigitJob, i64, i64, i64);

#define MF_IDEAL_INST(TN, KS) template __global__ void k_ideal<TN, KS>(const IdealPlan, const IdealArgs);
MF_IDEAL_INST(2, 1)
MF_IDEAL_INST(1, 1)
MF_IDEAL_INST(1, 2)

}  // namespace mf
