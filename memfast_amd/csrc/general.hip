// General sliced array read on gfx950: every non-wide configuration, every
// device effect.  Used for noisy devices and as the parity entry point.
//
// Model (memfast/reference.py:63-117, memfast/kernels.cu:71-202): for each
// read group g = i*Gr + j, input slice a and weight slice w,
//   I = sum_r V_a[n,r] * (G_w[r,c] - L)            (ascending-row FMA)
//   code = round(clamp(S(I * (Ma*Mw) * (1/unit)), 0, max_w))
//   T[n,g,c] = sum_a sum_w fa * fw * code           (int64)
// and the fused epilogue (memfast/simulator.py:582-585) accumulates
// (float(T) * xs[n,g]) * ws[g,c] over g in torch's CPU `sum` order.
//
// Block: 8 vectors x 32 columns, one thread per output.  Per 32-row chunk the
// block stages voltages (up to 8 input slices at a time) and conductances (a
// group of weight slices) in LDS.  Bound: VALU FMAs, K*A*W per output.
//
// WIDE (precisions above 8 bits or BFP, memfast/config.py `wide`): 32-bit
// codes, FP64 scales, and the epilogue of memfast/simulator.py:578-585:
// restore_scales (FP64 frexp/ldexp) summed over reads in torch's FP64 order.
#include <cfloat>
#include <type_traits>

#include "mf_kernels.h"

namespace mf {

constexpr int GV = 8;         // vectors per block
constexpr int GC = 32;        // columns per block
constexpr int GROWS = 32;     // rows per staged chunk
constexpr int GMAX_A = 8;     // input slices supported (activation_bits <= 8)

template <typename Phys>
__device__ __forceinline__ Phys load_g(const void *g, i64 idx) {
    return reinterpret_cast<const Phys *>(g)[idx];
}

template <typename Phys>
__device__ __forceinline__ Phys adc_count(const mf_config &cfg, Phys current, int a, int w);

template <>
__device__ __forceinline__ float adc_count<float>(const mf_config &cfg, float current, int a,
                                                  int w) {
    float z = current * float(i64(cfg.in_mask[a]) * cfg.w_mask[w]);
    z = z * cfg.f_inv_unit;
    if (cfg.has_nonlinear) z = z / (1.0f + fabsf(cfg.f_alpha_over_max[w] * z));
    const float top = float(cfg.adc_max[w]);
    z = z < 0.0f ? 0.0f : z;
    z = z > top ? top : z;
    return rintf(z);
}

template <>
__device__ __forceinline__ double adc_count<double>(const mf_config &cfg, double current, int a,
                                                    int w) {
    double z = current * double(i64(cfg.in_mask[a]) * cfg.w_mask[w]);
    z = z * cfg.d_inv_unit;
    if (cfg.has_nonlinear) z = z / (1.0 + fabs(cfg.d_alpha_over_max[w] * z));
    const double top = double(cfg.adc_max[w]);
    z = z < 0.0 ? 0.0 : z;
    z = z > top ? top : z;
    return rint(z);
}

// Column class for torch's sum over reads: the reference sums chunks of two
// tiles ([N, G, width*C] tensors); columns inside whole 4-row vector groups of
// a chunk use the cascade, the rest the interleaved cascade.
// FP64 sums interleave the columns beyond 16 * floor(width*C / 16).
template <bool WIDE>
__device__ __forceinline__ bool interleaved_column(i64 col, int C, i64 p) {
    const i64 t = col / C;
    const i64 first = (t / 2) * 2;
    const i64 chunk_width = (p - first) < 2 ? (p - first) : 2;
    const i64 wc = chunk_width * C;
    const i64 pos = col - first * C;
    const i64 span = WIDE ? 16 : (wc >= 8 ? 32 : 4);
    return pos >= (wc / span) * span;
}

template <typename Phys, int WG, bool OUTPUT_NOISE, bool WIDE>
__global__ __launch_bounds__(256) void k_general(const mf_config cfg, const GeneralArgs args,
                                                 int out_kind) {
    typedef typename std::conditional<WIDE, u32, u8>::type Code;
    typedef typename std::conditional<WIDE, double, float>::type Out;
    __shared__ Phys volt[GMAX_A][GV][GROWS];
    __shared__ Phys cond[WG][GROWS][GC + 1];
    const Code *q_codes = static_cast<const Code *>(args.q);
    const Code *packed = static_cast<const Code *>(args.packed);
    const Out *xscale = static_cast<const Out *>(args.xscale);
    const Out *wscale = static_cast<const Out *>(args.wscale);
    Out *out = static_cast<Out *>(args.out);

    const int R = cfg.rows, C = cfg.cols, P = cfg.read_rows, Gr = cfg.reads;
    const int A = cfg.n_in, W = cfg.n_w;
    const i64 m = args.m;
    const i64 G = m * Gr;
    const i64 ncols = args.width * C;
    const int tc = threadIdx.x % GC, tv = threadIdx.x / GC;
    const i64 col = i64(blockIdx.y) * GC + tc;
    const i64 vec0 = i64(blockIdx.x) * GV;
    const i64 vec = vec0 + tv;
    const bool live = col < ncols && vec < args.n;
    const i64 tt = live ? col / C : 0;            // tile relative to begin
    const int cc = int(col % C);
    const i64 kp = m * R;
    const u64 read_seed = event_seed(args.seed, args.event);
    const Phys low = low_of<Phys>(cfg);
    const Phys volt_level = sizeof(Phys) == 8 ? Phys(cfg.d_voltage) : Phys(cfg.f_voltage);

    Cascade<Out> cascade;
    Interleaved<Out> interleaved;
    cascade.reset();
    interleaved.reset();
    const bool use_interleaved = live && out_kind == OUT_FUSED &&
                                 interleaved_column<WIDE>(args.begin * C + col, C, args.p);

    for (i64 g = 0; g < G; ++g) {
        const i64 i = g / Gr;
        const int j = int(g % Gr);
        const int row0 = j * P;
        const int len = (R - row0) < P ? (R - row0) : P;
        i64 total = 0;
        // Input slices in chunks of GMAX_A (more than 8 only with wide codes).
        for (int a0 = 0; a0 < A; a0 += GMAX_A)
        for (int w0 = 0; w0 < W; w0 += WG) {
            Phys cur[GMAX_A][WG];
            Phys mean[OUTPUT_NOISE ? GMAX_A : 1][WG];
            Phys var[OUTPUT_NOISE ? GMAX_A : 1][WG];
#pragma unroll
            for (int a = 0; a < GMAX_A; ++a)
#pragma unroll
                for (int wl = 0; wl < WG; ++wl) {
                    cur[a][wl] = Phys(0);
                    if (OUTPUT_NOISE) { mean[a][wl] = Phys(0); var[a][wl] = Phys(0); }
                }
            for (int ch = 0; ch < len; ch += GROWS) {
                const int clen = (len - ch) < GROWS ? (len - ch) : GROWS;
                __syncthreads();
                // Stage voltages V_a[n, r] for input slices a0 .. a0 + GMAX_A - 1.
                const int a_count = (A - a0) < GMAX_A ? (A - a0) : GMAX_A;
                for (int e = threadIdx.x; e < a_count * GV * GROWS; e += blockDim.x) {
                    const int al = e / (GV * GROWS);
                    const int a = a0 + al;
                    const int v = (e / GROWS) % GV;
                    const int rr = e % GROWS;
                    const i64 nn = vec0 + v;
                    Phys value = Phys(0);
                    if (nn < args.n && rr < clen) {
                        const int r = row0 + ch + rr;
                        const int mask = cfg.in_mask[a];
                        const int digit =
                            int((u32(q_codes[nn * kp + i * R + r]) >> cfg.in_shift[a]) & u32(mask));
                        value = Phys(digit) / Phys(mask) * volt_level;
                        if (cfg.has_vnoise) {
                            const u64 address = u64(((nn * m + i) * A + a) * R + r);
                            const float z = normal(address, read_seed, 40u, cfg.f_two_pi);
                            value = value * Phys(1.0f + cfg.f_vnoise * z);
                        }
                    }
                    volt[al][v][rr] = value;
                }
                const int plane_lo = args.planes > 1 ? a0 : 0;
                const int plane_hi = args.planes > 1 ? a0 + a_count : 1;
                for (int plane = plane_lo; plane < plane_hi; ++plane) {
                    if (plane != plane_lo) __syncthreads();
                    // Stage conductances G_w[r, c] for this group of weight slices.
                    for (int e = threadIdx.x; e < WG * GROWS * GC; e += blockDim.x) {
                        const int wl = e / (GROWS * GC);
                        const int rr = (e / GC) % GROWS;
                        const int ccol = e % GC;
                        const int w = w0 + wl;
                        const i64 gcol = i64(blockIdx.y) * GC + ccol;
                        Phys value = low;
                        if (w < W && rr < clen && gcol < ncols) {
                            const int r = row0 + ch + rr;
                            const i64 t_rel = gcol / C;
                            const int c = int(gcol % C);
                            if (args.g) {
                                const i64 idx =
                                    ((((i64(plane) * m + i) * args.width + t_rel) * W + w) * R + r) *
                                        C + c;
                                value = load_g<Phys>(args.g, idx);
                            } else {
                                const i64 t = args.begin + t_rel;
                                const u32 code = packed[((i * args.p + t) * R + r) * C + c];
                                const int mask = cfg.w_mask[w];
                                const int digit = int((code >> cfg.w_shift[w]) & u32(mask));
                                value = nominal_level<Phys>(cfg, digit, mask) * drift_of<Phys>(cfg);
                            }
                        }
                        cond[wl][rr][ccol] = value;
                    }
                    __syncthreads();
                    // slice_pair planes: plane p holds input slice p's conductances.
                    const int a_lo = args.planes > 1 ? plane - a0 : 0;
                    const int a_hi = args.planes > 1 ? plane - a0 + 1 : a_count;
                    for (int rr = 0; rr < clen; ++rr) {
#pragma unroll
                        for (int wl = 0; wl < WG; ++wl) {
                            const Phys base = cond[wl][rr][tc];
                            const Phys eff = base - low;
#pragma unroll
                            for (int a = 0; a < GMAX_A; ++a) {
                                if (a < a_lo || a >= a_hi) continue;
                                const Phys v = volt[a][tv][rr];
                                cur[a][wl] = fma(v, eff, cur[a][wl]);
                                if (OUTPUT_NOISE) {
                                    mean[a][wl] = fma(v, base, mean[a][wl]);
                                    var[a][wl] = fma(v * v, base * base, var[a][wl]);
                                }
                            }
                        }
                    }
                }
            }
            // ADC and signed shift-add for this group of weight slices.
            if (live) {
#pragma unroll
                for (int al = 0; al < GMAX_A; ++al) {
                    const int a = a0 + al;
                    if (a >= A) continue;
#pragma unroll
                    for (int wl = 0; wl < WG; ++wl) {
                        const int w = w0 + wl;
                        if (w >= W) continue;
                        Phys current = cur[al][wl];
                        if (OUTPUT_NOISE) {
                            const i64 t = args.begin + tt;
                            const u64 address = u64(
                                ((((vec * m * Gr + g) * args.p + t) * A + a) * W + w) * C + cc);
                            const float z = normal(address, read_seed, 60u, cfg.f_two_pi);
                            const Phys mu = mean[al][wl] * Phys(cfg.f_out_mean);
                            const Phys sd = sqrt(var[al][wl] * Phys(cfg.f_out_var));
                            current = current + (mu + sd * Phys(z));
                        }
                        const Phys code = adc_count<Phys>(cfg, current, a, w);
                        const i64 icode = i64(code);
                        if (args.codes)
                            args.codes[(((vec * G + g) * A + a) * W + w) * ncols + col] =
                                int32_t(icode);
                        total += icode * (cfg.in_factor[a] * cfg.w_factor[w]);
                    }
                }
            }
        }
        if (!live) continue;
        if (out_kind == OUT_TOTALS) {
            out[((vec * G + g) * args.width + tt) * C + cc] = Out(total);
        } else {
            const i64 o = args.begin * C + col;
            Out value;
            if (WIDE) {
                value = Out(restore_f64(double(total), double(xscale[vec * G + g]),
                                        double(wscale[g * args.ldws + o])));
            } else {
                value = Out(total) * xscale[vec * G + g];
                value = value * wscale[g * args.ldws + o];
            }
            if (use_interleaved) interleaved.push(value, int(G), args.lp_interleaved);
            else cascade.push(value, args.lp_cascade);
        }
    }
    if (live && out_kind == OUT_FUSED) {
        const i64 o = args.begin * C + col;
        const Out value = use_interleaved ? interleaved.finish(int(G)) : cascade.finish();
        out[vec * args.ldo + o] = value;
        if (!(fabs(double(value)) <= (WIDE ? DBL_MAX : double(FLT_MAX))) && args.status)
            atomicOr(args.status, u32(MF_STATUS_OUTPUT));
    }
}

#define MF_GENERAL_INST(PHYS, WG, OUT, WIDE)                                                  \
    template __global__ void k_general<PHYS, WG, OUT, WIDE>(const mf_config, const GeneralArgs, \
                                                            int);
MF_GENERAL_INST(float, 8, false, false)
MF_GENERAL_INST(float, 2, true, false)
MF_GENERAL_INST(double, 4, false, false)
MF_GENERAL_INST(double, 2, true, false)
MF_GENERAL_INST(float, 8, false, true)
MF_GENERAL_INST(float, 2, true, true)
MF_GENERAL_INST(double, 4, false, true)
MF_GENERAL_INST(double, 2, true, true)

}  // namespace mf
