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

}  // namespace mf
