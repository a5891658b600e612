// Programmed and read conductances of packed weight cells on gfx950.
//
// One thread per (plane, array, tile, weight slice, row, column) cell, as
// memfast/reference.py:10-51 (restored) and the read-noise factor of the
// slice_pair mode (memfast/reference.py:86-93).  The arithmetic order of the
// CPU reference is kept (nominal level, x write noise, x drift, stuck-at
// override, x shared read noise) with FP32 constants rounded as torch rounds
// Python scalars.  Output layout g[plane][m][width][W][R][C] (HBM-bound pass,
// 4 or 8 bytes written per cell, RNG-bound when noise is on).
#include "mf_kernels.h"

namespace mf {

template <typename Phys, typename Code>
__global__ __launch_bounds__(256) void k_restore(const mf_config cfg, const Code *packed, i64 m,
                                                 i64 p, i64 begin, i64 width, u32 seed,
                                                 u64 event, int planes, Phys *g) {
    const int R = cfg.rows, C = cfg.cols, W = cfg.n_w;
    const i64 per_plane = m * width * W * R * C;
    const i64 total = per_plane * planes;
    const u64 read_seed = event_seed(seed, event);
    for (i64 idx = i64(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += i64(gridDim.x) * blockDim.x) {
        i64 rest = idx;
        const int c = int(rest % C); rest /= C;
        const int r = int(rest % R); rest /= R;
        const int w = int(rest % W); rest /= W;
        const i64 tt = rest % width; rest /= width;
        const i64 i = rest % m;
        const int plane = int(rest / m);
        const i64 t = begin + tt;
        const u64 cell = u64((((i * p + t) * W + w) * R + r) * C + c);
        const u32 code = packed[((i * p + t) * R + r) * C + c];
        Phys raw = cell_conductance<Phys>(cfg, code, w, cell, seed, read_seed);
        if (planes > 1) {
            // slice_pair: an independent read field per activation slice.
            const u64 address = cell * u64(cfg.n_in) + u64(plane);
            raw = raw * Phys(noise_factor<Phys>(cfg, cfg.f_read, address, read_seed, 20u));
        }
        g[idx] = raw;
    }
}

template __global__ void k_restore<float, u8>(const mf_config, const u8 *, i64, i64, i64, i64,
                                              u32, u64, int, float *);
template __global__ void k_restore<double, u8>(const mf_config, const u8 *, i64, i64, i64, i64,
                                               u32, u64, int, double *);
template __global__ void k_restore<float, u32>(const mf_config, const u32 *, i64, i64, i64, i64,
                                               u32, u64, int, float *);
template __global__ void k_restore<double, u32>(const mf_config, const u32 *, i64, i64, i64, i64,
                                                u32, u64, int, double *);

}  // namespace mf
