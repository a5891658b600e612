// Overflow-safe FP64 scale restore and read sum of slice totals: the path the
// reference takes for wide precisions and when the FP32 restore overflows
// (memfast/simulator.py:57-66 restore_scales, :578-585 and :614-615).
//
// restore_scales computes frexp mantissas and exponents of T, xs and ws,
// multiplies the mantissas ((vm*xm)*wm, two FP64 roundings) and applies the
// exponent sum with torch.ldexp, which multiplies by 2^e held in a double.
// The read sum follows torch's CPU `sum(1)` over [N, G, width*C] FP64: the
// level-16 cascade per column, with the last columns of each chunk (beyond
// 16 * floor(width*C / 16)) summed as four interleaved streams.
#include "mf_kernels.h"

namespace mf {

// One thread per (vector, column of the chunk): totals [n, G, width*C] (FP32,
// integer valued), xscale [n, G], wscale [G, ldws] at columns col0 + col;
// writes out[vec * ldo + col0 + col].
__global__ void k_stable_sum(const float *totals, i64 n, i64 G, i64 wc, const float *xscale,
                             const float *wscale, i64 ldws, i64 col0, double *out, i64 ldo,
                             int lp_cascade, int lp_interleaved) {
    const i64 total = n * wc;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 vec = i / wc, col = i - vec * wc;
        const bool interleave = col >= (wc / 16) * 16;
        Cascade<double> cascade;
        Interleaved<double> interleaved;
        cascade.reset();
        interleaved.reset();
        for (i64 g = 0; g < G; ++g) {
            const double v = restore_f64(double(totals[(vec * G + g) * wc + col]),
                                         double(xscale[vec * G + g]),
                                         double(wscale[g * ldws + col0 + col]));
            if (interleave) interleaved.push(v, int(G), lp_interleaved);
            else cascade.push(v, lp_cascade);
        }
        out[vec * ldo + col0 + col] = interleave ? interleaved.finish(int(G)) : cascade.finish();
    }
}

}  // namespace mf
