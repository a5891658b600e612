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

// FP64 MFMA read for precise currents (memfast/config.py:215-224: FP64 conductances and
// currents), every device effect but voltage variation and output-mode read noise.
// Block: 16 vectors x 16 columns, four waves; slice pair q = a*W + w goes to wave q % 4,
// which computes its current on v_mfma_f64_16x16x4_f64 over the read's rows, converts it
// (the reference's FP64 ADC) and adds fa*fw*code.  The waves' partial totals meet in LDS,
// and each thread restores and sums one output over the reads in torch's order, as
// k_general does (or, with OUT_TOTALS, writes the totals as k_general does).  The current
// is z = sum_r d_a[n,r] * x_w[r,c] with x = (G - L) * (V*Mw/unit), the reference's
// (sum_r (V*d/Ma)*(G - L)) * (Ma*Mw) / unit up to FP64 rounding; with ideal devices z is an
// integer to within a few ulps, so the counts are exact.
// STAGED (one plane of conductances, at most MFMA64_STAGED_MAX_W weight slices): per chunk of
// MFMA64_ROWS rows the block stages the chunk's codes and every weight slice's x in LDS, and
// each wave keeps up to MFMA64_PAIRS pairs' currents in registers across the chunks.
// Otherwise (slice_pair planes, more weight slices) each step loads its operands itself.
// Bound: FP64 MFMA, K*A*W FMAs per output.
constexpr int MFMA64_ROWS = 32;
constexpr int MFMA64_PAIRS = 8;

__device__ __forceinline__ double adc_count_f64(const mf_config &cfg, double z, int w) {
    if (cfg.has_nonlinear) z = z / (1.0 + fabs(cfg.d_alpha_over_max[w] * z));
    const double top = double(cfg.adc_max[w]);
    z = z < 0.0 ? 0.0 : z;
    z = z > top ? top : z;
    return rint(z);
}

template <bool WIDE, bool STAGED>
__global__ __launch_bounds__(256) void k_general_mfma64(const mf_config cfg,
                                                        const GeneralArgs args, int out_kind) {
    typedef typename std::conditional<WIDE, u32, u8>::type Code;
    typedef typename std::conditional<WIDE, double, float>::type Out;
    typedef double v4d __attribute__((ext_vector_type(4)));
    __shared__ i64 part[4][256];
    __shared__ double xs_l[STAGED ? MFMA64_STAGED_MAX_W : 1][MFMA64_ROWS][16];
    __shared__ u32 cs_l[16][MFMA64_ROWS + 1];
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
    const i64 kp = m * R;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 15, lk = lane >> 4;
    const i64 v0 = i64(blockIdx.x) * 16, c0 = i64(blockIdx.y) * 16;
    // MFMA operands: A (16 vectors x 4 rows): lane -> vector v0 + li, row lk of the step;
    // B (4 rows x 16 columns): lane -> column c0 + li, row lk.  The result's element e
    // (e = 0..3): lane -> column c0 + li, vector v0 + lk + 4*e (measured on gfx950).
    const i64 a_vec = v0 + li;
    const bool a_live = a_vec < args.n;
    const i64 b_col = c0 + li;
    const bool b_live = b_col < ncols;
    const i64 b_t = b_live ? b_col / C : 0;   // tile relative to begin
    const int b_c = int(b_col % C);
    // The output this thread restores and sums: vector v0 + tid / 16, column c0 + tid % 16.
    const i64 o_vec = v0 + (threadIdx.x >> 4), o_col = c0 + (threadIdx.x & 15);
    const bool o_live = o_vec < args.n && o_col < ncols;
    const double low = cfg.d_low;
    // Conductance at (plane, array i, row r, weight slice w) of this lane's B column.
    auto level_at = [&](int plane, i64 i, int r, int w, i64 t, int c) {
        if (args.g) {
            const i64 idx = ((((i64(plane) * m + i) * args.width + t) * W + w) * R + r) * C + c;
            return load_g<double>(args.g, idx);
        }
        const u32 code = packed[((i * args.p + args.begin + t) * R + r) * C + c];
        const int wmask = cfg.w_mask[w];
        return nominal_level<double>(cfg, int((code >> u32(cfg.w_shift[w])) & u32(wmask)), wmask) *
               drift_of<double>(cfg);
    };
    auto k1_of = [&](int w) { return cfg.d_voltage * double(cfg.w_mask[w]) * cfg.d_inv_unit; };

    Cascade<Out> cascade;
    Interleaved<Out> interleaved;
    cascade.reset();
    interleaved.reset();
    const bool use_interleaved = o_live && out_kind == OUT_FUSED &&
                                 interleaved_column<WIDE>(args.begin * C + o_col, C, args.p);
    const int pairs = A * W;
    for (i64 g = 0; g < G; ++g) {
        const i64 i = g / Gr;
        const int j = int(g % Gr);
        const int row0 = j * P;
        const int len = (R - row0) < P ? (R - row0) : P;
        i64 t[4] = {0, 0, 0, 0};
        if (STAGED) {
            for (int base = 0; base < pairs; base += 4 * MFMA64_PAIRS) {
                v4d cur[MFMA64_PAIRS];
#pragma unroll
                for (int k = 0; k < MFMA64_PAIRS; ++k) cur[k] = v4d{0.0, 0.0, 0.0, 0.0};
                for (int ch = 0; ch < len; ch += MFMA64_ROWS) {
                    const int clen = (len - ch) < MFMA64_ROWS ? (len - ch) : MFMA64_ROWS;
                    __syncthreads();   // every wave is done with the previous chunk
                    for (int e = threadIdx.x; e < 16 * MFMA64_ROWS; e += 256) {
                        const int v = e / MFMA64_ROWS, r = e % MFMA64_ROWS;
                        const i64 vec = v0 + v;
                        cs_l[v][r] = vec < args.n && r < clen
                                         ? u32(q_codes[vec * kp + i * R + row0 + ch + r])
                                         : 0u;
                    }
                    for (int e = threadIdx.x; e < W * MFMA64_ROWS * 16; e += 256) {
                        const int w = e / (MFMA64_ROWS * 16), r = (e / 16) % MFMA64_ROWS;
                        const int c = e % 16;
                        const i64 col = c0 + c;
                        double x = 0.0;
                        if (col < ncols && r < clen)
                            x = (level_at(0, i, row0 + ch + r, w, col / C, int(col % C)) - low) *
                                k1_of(w);
                        xs_l[w][r][c] = x;
                    }
                    __syncthreads();
                    // Steps outside, pairs inside: consecutive MFMAs feed different
                    // accumulators, so none waits for the one before.
#pragma unroll
                    for (int st = 0; st < MFMA64_ROWS / 4; ++st) {
                        const int r = 4 * st + lk;   // rows past clen were staged as zero
                        const u32 code = cs_l[li][r];
#pragma unroll
                        for (int k = 0; k < MFMA64_PAIRS; ++k) {
                            const int pq = base + wave + 4 * k;
                            if (pq < pairs) {
                                const int a = pq / W, w = pq - a * W;
                                const double d =
                                    double((code >> u32(cfg.in_shift[a])) & u32(cfg.in_mask[a]));
                                cur[k] = __builtin_amdgcn_mfma_f64_16x16x4f64(d, xs_l[w][r][li],
                                                                              cur[k], 0, 0, 0);
                            }
                        }
                    }
                }
#pragma unroll
                for (int k = 0; k < MFMA64_PAIRS; ++k) {
                    const int pq = base + wave + 4 * k;
                    if (pq >= pairs) break;
                    const int a = pq / W, w = pq - a * W;
                    const i64 f = cfg.in_factor[a] * cfg.w_factor[w];
#pragma unroll
                    for (int e = 0; e < 4; ++e) t[e] += i64(adc_count_f64(cfg, cur[k][e], w)) * f;
                }
            }
        } else {
            for (int pq = wave; pq < pairs; pq += 4) {
                const int a = pq / W, w = pq - a * W;
                const int plane = args.planes > 1 ? a : 0;
                const double k1 = k1_of(w);
                const u32 ashift = u32(cfg.in_shift[a]), amask = u32(cfg.in_mask[a]);
                const Code *qrow = q_codes + a_vec * kp + i * R + row0 + lk;
                v4d cur = {0.0, 0.0, 0.0, 0.0};
                for (int r4 = 0; r4 < len; r4 += 4) {
                    const bool row_ok = r4 + lk < len;
                    double d = 0.0;
                    if (a_live && row_ok) d = double((u32(qrow[r4]) >> ashift) & amask);
                    double x = 0.0;
                    if (b_live && row_ok) x = (level_at(plane, i, row0 + r4 + lk, w, b_t, b_c) - low) * k1;
                    cur = __builtin_amdgcn_mfma_f64_16x16x4f64(d, x, cur, 0, 0, 0);
                }
                const i64 f = cfg.in_factor[a] * cfg.w_factor[w];
#pragma unroll
                for (int e = 0; e < 4; ++e) t[e] += i64(adc_count_f64(cfg, cur[e], w)) * f;
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) part[wave][(lk + 4 * e) * 16 + li] = t[e];
        __syncthreads();
        const i64 total = part[0][threadIdx.x] + part[1][threadIdx.x] + part[2][threadIdx.x] +
                          part[3][threadIdx.x];
        __syncthreads();
        if (o_live && out_kind == OUT_TOTALS) {
            out[((o_vec * G + g) * args.width + o_col / C) * C + o_col % C] = Out(total);
        } else if (o_live) {
            const i64 o = args.begin * C + o_col;
            Out value;
            if (WIDE) {
                value = Out(restore_f64(double(total), double(xscale[o_vec * G + g]),
                                        double(wscale[g * args.ldws + o])));
            } else {
                value = Out(total) * xscale[o_vec * G + g];
                value = value * wscale[g * args.ldws + o];
            }
            if (use_interleaved) interleaved.push(value, int(G), args.lp_interleaved);
            else cascade.push(value, args.lp_cascade);
        }
    }
    if (o_live && out_kind == OUT_FUSED) {
        const i64 o = args.begin * C + o_col;
        const Out value = use_interleaved ? interleaved.finish(int(G)) : cascade.finish();
        out[o_vec * args.ldo + o] = value;
        if (!(fabs(double(value)) <= (WIDE ? DBL_MAX : double(FLT_MAX))) && args.status)
            atomicOr(args.status, u32(MF_STATUS_OUTPUT));
    }
}
#define MF_MFMA64_INST(WIDE, STAGED)                                                            \
    template __global__ void k_general_mfma64<WIDE, STAGED>(const mf_config, const GeneralArgs, \
                                                            int);
MF_MFMA64_INST(false, false)
MF_MFMA64_INST(false, true)
MF_MFMA64_INST(true, false)
MF_MFMA64_INST(true, true)
#undef MF_MFMA64_INST

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
