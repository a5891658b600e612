// Physical conductance levels and noise factors shared by the gfx950 kernels.
//
// Arithmetic order and FP32 rounding of constants follow the CPU reference
// memfast/reference.py:10-51 (restored) so that ideal and noisy levels match it.
#pragma once

#include "mf_device.h"

namespace mf {

template <typename Phys>
__device__ __forceinline__ Phys nominal_level(const mf_config &cfg, int digit, int mask);

template <>
__device__ __forceinline__ float nominal_level<float>(const mf_config &cfg, int digit, int mask) {
    if (mask == 1) return digit ? cfg.f_high : cfg.f_low;
    return cfg.f_low + cfg.f_span * (float(digit) / float(mask));
}

template <>
__device__ __forceinline__ double nominal_level<double>(const mf_config &cfg, int digit,
                                                        int mask) {
    if (mask == 1) return digit ? cfg.d_high : cfg.d_low;
    return cfg.d_low + cfg.d_span * (double(digit) / double(mask));
}

template <typename Phys>
__device__ __forceinline__ Phys drift_of(const mf_config &cfg);
template <>
__device__ __forceinline__ float drift_of<float>(const mf_config &cfg) { return cfg.f_drift; }
template <>
__device__ __forceinline__ double drift_of<double>(const mf_config &cfg) { return cfg.d_drift; }

template <typename Phys>
__device__ __forceinline__ Phys low_of(const mf_config &cfg);
template <>
__device__ __forceinline__ float low_of<float>(const mf_config &cfg) { return cfg.f_low; }
template <>
__device__ __forceinline__ double low_of<double>(const mf_config &cfg) { return cfg.d_low; }

template <typename Phys>
__device__ __forceinline__ Phys high_of(const mf_config &cfg);
template <>
__device__ __forceinline__ float high_of<float>(const mf_config &cfg) { return cfg.f_high; }
template <>
__device__ __forceinline__ double high_of<double>(const mf_config &cfg) { return cfg.d_high; }

// exp(sigma * n) for a noise sample n at `address`.  FP64 currents resolve conductance
// differences far below one FP32 ulp of g (high - low down to 1e-4 of high), and one ulp of an
// FP32 factor near 1 is 2^-23 of g, so they sample with OCML's logf/cosf/sqrtf/expf, which stay
// within an ulp or two of torch CPU's; FP32 currents use the hardware approximations
// (normal_fast, exp_small).
template <typename Phys>
__device__ __forceinline__ float noise_factor(const mf_config &cfg, float sigma, u64 address,
                                              u64 seed, u32 stream) {
    if constexpr (sizeof(Phys) == sizeof(double))
        return expf(sigma * normal(address, seed, stream, cfg.f_two_pi));
    else
        return exp_small(sigma * normal_fast(address, seed, stream));
}

// Programmed + (shared) read conductance of one cell.
template <typename Phys>
__device__ __forceinline__ Phys cell_conductance(const mf_config &cfg, u32 code, int w, u64 cell,
                                                 u32 seed, u64 read_seed) {
    const int mask = cfg.w_mask[w];
    const int digit = int((code >> cfg.w_shift[w]) & u32(mask));
    Phys raw = nominal_level<Phys>(cfg, digit, mask);
    if (cfg.has_write) raw = raw * Phys(noise_factor<Phys>(cfg, cfg.f_write, cell, seed, 10u));
    raw = raw * drift_of<Phys>(cfg);
    if (cfg.has_saf) {
        const float u = uniform(cell, seed, 30u);
        if (u < cfg.f_saf_low) raw = low_of<Phys>(cfg);
        else if (u < cfg.f_saf_band) raw = high_of<Phys>(cfg);
    }
    if (cfg.read_mode == MF_READ_SHARED && cfg.has_read)
        raw = raw * Phys(noise_factor<Phys>(cfg, cfg.f_read, cell, read_seed, 20u));
    return raw;
}

}  // namespace mf
