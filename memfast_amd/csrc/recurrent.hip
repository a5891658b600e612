// GRU gate equations over analog projections (memfast/nn/recurrent.py), fused
// into one elementwise pass:
//   r = sigmoid(ir + hr), z = sigmoid(iz + hz), n = tanh(in + r * hn),
//   h = (1 - z) * n + z * hx,
// each operation rounded to FP32 in the order PyTorch's separate elementwise
// ops use (sigmoid(v) = 1 / (1 + exp(-v)); no contraction: the library builds
// with -ffp-contract=off).  inputs/hidden are [n, 3H] (gate chunks r, z, n).
// With `bias` the hidden projection's bias is added first (hidden + bias, one
// FP32 add per element, as the separate bias kernel does) and a non-finite sum
// sets `flag` in *status.
#include <cfloat>
#include <cmath>

#include "mf_kernels.h"

namespace mf {

__device__ __forceinline__ float gate_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

__global__ __launch_bounds__(256) void k_gru_gates(const float *inputs, i64 ldi, const float *hidden,
                                                   i64 ldh, const float *hx, i64 ldx, float *out,
                                                   i64 ldo, i64 n, i64 width, const float *bias,
                                                   u32 *status, u32 flag) {
    const i64 total = n * width;
    bool finite = true;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 v = i / width, c = i - v * width;
        const float *in = inputs + v * ldi, *hd = hidden + v * ldh;
        float hr = hd[c], hz = hd[width + c], hn = hd[2 * width + c];
        if (bias) {
            hr = hr + bias[c];
            hz = hz + bias[width + c];
            hn = hn + bias[2 * width + c];
            finite = finite && fabsf(hr) <= FLT_MAX && fabsf(hz) <= FLT_MAX &&
                     fabsf(hn) <= FLT_MAX;
        }
        const float r = gate_sigmoid(in[c] + hr);
        const float z = gate_sigmoid(in[width + c] + hz);
        const float rn = r * hn;
        const float cand = tanhf(in[2 * width + c] + rn);
        const float keep = (1.0f - z) * cand;
        const float carry = z * hx[v * ldx + c];
        out[v * ldo + c] = keep + carry;
    }
    if (!finite && status) atomicOr(status, flag);
}

// The hidden projection values of NC columns cc[] of row b: the split read's values summed
// over its reads in torch's cascade order, BATCH reads' loads at a time (RESTORED: the
// values are already (float(T) * xs) * ws; else they are integer totals restored here).
template <bool RESTORED, int BATCH, int NC>
__device__ __forceinline__ void restore_columns(const GruStepArgs &a, i64 b, const i64 (&cc)[NC],
                                                float (&v)[NC]) {
    Cascade<float> cascade[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) cascade[k].reset();
    const float *tv = a.totals + b * a.G * a.ldt;
    const float *xv = a.xscale_in + b * a.G;
    for (i64 g0 = 0; g0 < a.g_run; g0 += BATCH) {
        float tt[NC][BATCH], ws[NC][BATCH], xs[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
            const i64 g = g0 + j < a.g_run ? g0 + j : a.g_run - 1;   // past the end: unused
            if (!RESTORED) xs[j] = xv[g];
#pragma unroll
            for (int k = 0; k < NC; ++k) {
                tt[k][j] = tv[g * a.ldt + cc[k]];
                if (!RESTORED) ws[k][j] = a.wscale[g * a.ldws + cc[k]];
            }
        }
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
            if (g0 + j < a.g_run) {
#pragma unroll
                for (int k = 0; k < NC; ++k) {
                    float x = tt[k][j];
                    if (!RESTORED) {
                        x = x * xs[j];
                        x = x * ws[k][j];
                    }
                    cascade[k].push(x, a.lp);
                }
            }
        }
    }
#pragma unroll
    for (int k = 0; k < NC; ++k) v[k] = cascade[k].finish();
}

// k_restore_sum_f32, k_gru_gates and k_row_groups_wave of one step in one launch, one
// workgroup per batch row, bit for bit their results.  A thread owns hidden units c (c =
// thread, + blockDim, ...) and their three projection columns c, H + c, 2H + c:
// 1. each hidden projection value is (float(T) * xs) * ws (or the read's already restored
//    values) summed over the reads in torch's cascade order (Cascade<float>; loads issued a
//    batch of reads at a time), or read from the fused read's output, plus the bias;
// 2. the gates as k_gru_gates (bias first; FP32 in PyTorch's order), the new state kept in
//    LDS (H floats, dynamic shared memory; each thread reads back only its own units);
// 3. the new state's row is one quantization group: its peak (fmaxf, NaN ignored) gives
//    the scale, every read of the row gets it, codes past H are zero.
// Flags: a non-finite hidden value (restore) or biased sum sets MF_STATUS_OUTPUT; a
// non-finite new state sets MF_STATUS_INPUT when it is quantized.
__global__ __launch_bounds__(1024) void k_gru_step(const GruStepArgs a) {
    extern __shared__ float state[];   // [H]
    __shared__ float wave_peak[16];
    const i64 b = blockIdx.x;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, threads = blockDim.x;
    const i64 H = a.width;
    const float *in = a.inputs + b * a.ldi;
    bool out_finite = true, state_finite = true;
    float peak = 0.0f;
    for (i64 c = t; c < H; c += threads) {
        const i64 cc[3] = {c, H + c, 2 * H + c};
        // Gate operands and biases first, so their latency overlaps the restore.
        float gate_in[3], bias[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            gate_in[k] = in[cc[k]];
            if (a.bias) bias[k] = a.bias[cc[k]];
        }
        const float hx = a.hx[b * a.ldx + c];
        float v[3];
        if (!a.totals) {
#pragma unroll
            for (int k = 0; k < 3; ++k) v[k] = a.hidden[b * a.ldh + cc[k]];
        } else if (a.restored) {
            restore_columns<true, 16, 3>(a, b, cc, v);
        } else {
            restore_columns<false, 8, 3>(a, b, cc, v);
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            if (a.totals) out_finite = out_finite && fabsf(v[k]) <= FLT_MAX;
            if (a.bias) {
                v[k] = v[k] + bias[k];
                out_finite = out_finite && fabsf(v[k]) <= FLT_MAX;
            }
        }
        const float r = gate_sigmoid(gate_in[0] + v[0]);
        const float z = gate_sigmoid(gate_in[1] + v[1]);
        const float rn = r * v[2];
        const float cand = tanhf(gate_in[2] + rn);
        const float keep = (1.0f - z) * cand;
        const float carry = z * hx;
        const float h = keep + carry;
        a.out[b * a.ldo + c] = h;
        state[c] = h;
        const float mag = fabsf(h);
        state_finite = state_finite && mag <= FLT_MAX;
        peak = fmaxf(peak, mag);
    }
    if (!out_finite && a.status) atomicOr(a.status, u32(MF_STATUS_OUTPUT));
    if (!a.quantize) return;
    for (int off = 1; off < 64; off <<= 1) peak = fmaxf(peak, __shfl_xor(peak, off, 64));
    if (lane == 0) wave_peak[wave] = peak;
    // Also orders this row's restore reads of xscale_in before the writes of xscale_out below.
    __syncthreads();
    peak = 0.0f;
    for (int w = 0; w < (threads + 63) / 64; ++w) peak = fmaxf(peak, wave_peak[w]);
    const float s = group_scale(peak, a.upper);
    if (t == 0) a.scale[b] = s;
    for (i64 g = t; g < a.G; g += threads) a.xscale_out[b * a.G + g] = s;
    u8 *dst = a.q + b * a.kp;
    for (i64 c = t; c < a.kp; c += threads)
        dst[c] = c < H ? quantize_code(state[c], s, -a.upper, a.upper, a.mask) : u8(0);
    if (!state_finite && a.status) atomicOr(a.status, u32(MF_STATUS_INPUT));
}

}  // namespace mf
