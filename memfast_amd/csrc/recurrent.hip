// GRU gate equations over analog projections (memfast/nn/recurrent.py), fused
// into one elementwise pass:
//   r = sigmoid(ir + hr), z = sigmoid(iz + hz), n = tanh(in + r * hn),
//   h = (1 - z) * n + z * hx,
// each operation rounded to FP32 in the order PyTorch's separate elementwise
// ops use (sigmoid(v) = 1 / (1 + exp(-v)); no contraction: the library builds
// with -ffp-contract=off).  inputs/hidden are [n, 3H] (gate chunks r, z, n).
#include <cmath>

#include "mf_kernels.h"

namespace mf {

__device__ __forceinline__ float gate_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

__global__ __launch_bounds__(256) void k_gru_gates(const float *inputs, i64 ldi, const float *hidden,
                                                   i64 ldh, const float *hx, i64 ldx, float *out,
                                                   i64 ldo, i64 n, i64 width) {
    const i64 total = n * width;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 v = i / width, c = i - v * width;
        const float *in = inputs + v * ldi, *hd = hidden + v * ldh;
        const float r = gate_sigmoid(in[c] + hd[c]);
        const float z = gate_sigmoid(in[width + c] + hd[width + c]);
        const float rn = r * hd[2 * width + c];
        const float cand = tanhf(in[2 * width + c] + rn);
        const float keep = (1.0f - z) * cand;
        const float carry = z * hx[v * ldx + c];
        out[v * ldo + c] = keep + carry;
    }
}

}  // namespace mf
