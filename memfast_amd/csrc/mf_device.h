// Device-side helpers shared by the gfx950 kernels of the sliced analog engine.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/memfast_hip.h"

namespace mf {

typedef uint8_t u8;
typedef uint32_t u32;
typedef uint64_t u64;
typedef int64_t i64;

// ---------------------------------------------------------------------------
// Counter-based RNG keyed by physical address (memfast/random.py:8-33,
// memfast/kernels.cu:22-41).  The integer part is exact; normal() uses OCML's
// logf/cosf/sqrtf and normal_fast() the hardware instructions (neither is bit-identical
// to torch CPU's).
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ u32 mix(u32 x) {
    x = (x ^ (x >> 16)) * 0x7feb352du;
    x = (x ^ (x >> 15)) * 0x846ca68bu;
    return x ^ (x >> 16);
}

// uniform() in two parts: uniform_fold() depends on the address's high word, the seed
// and the stream only, so addresses that share a high word share it.
__device__ __forceinline__ u32 uniform_fold(u32 hi, u64 seed, u32 stream) {
    const u32 key = mix(u32(seed) ^ (stream * 0x9e3779b9u));
    u32 fold = mix(hi ^ mix(u32(seed >> 32)));
    if (hi != 0u) fold ^= mix(hi ^ key);
    return fold ^ key;
}

__device__ __forceinline__ float uniform_finish(u32 lo, u32 fold) {
    const u32 h = mix(lo ^ fold);
    // ((h >> 8) + 0.5) / 2^24 is exact in FP32.
    return (float(h >> 8) + 0.5f) * (1.0f / 16777216.0f);
}

__device__ __forceinline__ float uniform(u64 address, u64 seed, u32 stream) {
    return uniform_finish(u32(address), uniform_fold(u32(address >> 32), seed, stream));
}

__device__ __forceinline__ float normal(u64 address, u64 seed, u32 stream, float two_pi) {
    const float u = uniform(address, seed, stream);
    const float v = uniform(address, seed, stream + 1u);
    // torch: sqrt(-2 * log(u)) * cos((2*pi) * v), all FP32.
    return sqrtf(-2.0f * logf(u)) * cosf(two_pi * v);
}

// normal() on the hardware transcendentals: log2 (v_log_f32), cos(2*pi*v) with v in
// revolutions (v_cos_f32) and sqrt (v_sqrt_f32), one instruction each.  Over every uniform
// value (k + 0.5) / 2^24, sqrt(-2 ln u) stays within 4.8e-7 and cos(2*pi*v) within 1.3e-7
// of the exact values (OCML's sqrtf(-2 logf(u)): 5.9e-7).
__device__ __forceinline__ float box_muller(float u, float v) {
    // -2 ln u = -2 ln(2) log2(u).
    return __builtin_amdgcn_sqrtf(-1.38629436f * __builtin_amdgcn_logf(u)) *
           __builtin_amdgcn_cosf(v);
}

__device__ __forceinline__ float normal_fast(u64 address, u64 seed, u32 stream) {
    return box_muller(uniform(address, seed, stream), uniform(address, seed, stream + 1u));
}

// exp(x) for the noise exponents as exp2(x * log2(e)) on v_exp_f32: within 1 ulp of
// exp(x) for |x| <= 0.5 and 4 ulp for |x| <= 4 (measured over 2^24 points).
__device__ __forceinline__ float exp_small(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504f);
}

// The S-curve of memfast/reference.py:57-59 in FP32 with the reference's roundings:
// t = RN(alpha * z) (alpha = fp32(nonlinearity / max)), d = RN(1 + |t|), then RN(z / d).
// The quotient is v_rcp_f32's estimate r of 1/d (within 1 ulp) refined by one residual
// step: q0 = RN(z * r) is within an ulp of z / d, so e = z - q0 * d is exact in one FMA and
// RN(q0 + e * r) is the correctly rounded quotient (Markstein).  A CPU check over 2e8
// arguments with r = RN(1/d) and with r one ulp either side found every rounded integer
// equal to rint(RN(z / d)).
__device__ __forceinline__ float scurve(float z, float alpha) {
    const float t = z * alpha;
    const float d = 1.0f + fabsf(t);
    const float r = __builtin_amdgcn_rcpf(d);
    const float q0 = z * r;
    const float e = fmaf(-q0, d, z);
    return fmaf(e, r, q0);
}

// Tile (x, y) of workgroup L (its linear id) in a grid of nx (fast) by ny tiles, arranged so
// that the workgroups one XCD runs take one contiguous run of tiles in x-fastest order. The
// dispatcher deals workgroup L to XCD L % 8 (MI355X: 8 XCDs, one L2 each), so with the plain
// order neighbouring tiles, which share the operand indexed by y, land on eight different L2s;
// here the tiles in flight on an XCD share it.  A bijection of [0, nx*ny): the last
// (nx*ny) % 8 workgroups keep their own index.
__device__ __forceinline__ void xcd_tile(u32 L, u32 nx, u32 ny, u32 &x, u32 &y) {
    const u32 per = (nx * ny) / 8;
    const u32 P = L < per * 8 ? (L % 8) * per + L / 8 : L;
    x = P % nx;
    y = P / nx;
}

// Copy a status word to a caller's pinned host word, marked MF_STATUS_PUBLISHED.  Called by
// one lane of a kernel that started after the kernels setting those bits had finished: the
// device-scope load sees their atomics, and the system-scope store writes through to host
// memory.  Call it after the kernel's last load of read-only inputs: the compiler counts this
// store as a possible write to them, and loads after it become vector loads.
__device__ __forceinline__ void publish_status(u32 *status, u32 *mailbox) {
    const u32 flags = status ? __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                             : 0u;
    __hip_atomic_store(mailbox, flags | MF_STATUS_PUBLISHED, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}

// INT code of x in a group of scale s (memfast/quantization.py:41: round half to even,
// clamp, two's complement masked to the code width), FP32 division as torch's.
__device__ __forceinline__ u8 quantize_code(float x, float s, float lower, float upper,
                                            u32 mask) {
    float c = rintf(x / s);
    c = c < lower ? lower : c;
    c = c > upper ? upper : c;
    return u8(u32(int(c)) & mask);
}

// scale of one group from its peak |x| (quantization.py:25-31 for INT codes).
__device__ __forceinline__ float group_scale(float peak, float upper) {
    float s = (peak > 0.0f ? peak : 1.0f) / upper;
    const float tiny = __uint_as_float(1u);
    return s < tiny ? tiny : s;
}

__host__ __device__ __forceinline__ u64 event_seed(u32 seed, u64 event) {
    return u64(seed ^ mix(u32(event))) | (u64(mix(u32(event >> 32))) << 32);
}

// ---------------------------------------------------------------------------
// Overflow-safe FP64 scale restore of memfast/simulator.py:57-66
// (restore_scales): frexp mantissas multiplied as (vm*xm)*wm, the exponent sum
// applied with torch.ldexp, which multiplies by 2^e held in a double.
// ---------------------------------------------------------------------------
// x * 2^e with 2^e formed as a double (0 below 2^-1074, inf above 2^1023).
__device__ __forceinline__ double times_pow2(double x, int e) {
    double scale;
    if (e > 1023) scale = __longlong_as_double(0x7FF0000000000000LL);
    else if (e >= -1022) scale = __longlong_as_double(i64(e + 1023) << 52);
    else if (e >= -1074) scale = __longlong_as_double(1LL << (e + 1074));
    else scale = 0.0;
    return x * scale;
}

__device__ __forceinline__ double restore_f64(double value, double xs, double ws) {
    int ve, xe, we;
    const double vm = frexp(value, &ve);
    const double xm = frexp(xs, &xe);
    const double wm = frexp(ws, &we);
    const double mantissa = (vm * xm) * wm;
    if (mantissa == 0.0) return 0.0;
    const int exponent = ve + xe + we;
    const int first = exponent < -1022 ? -1022 : (exponent > 1023 ? 1023 : exponent);
    return times_pow2(times_pow2(mantissa, first), exponent - first);
}

// ---------------------------------------------------------------------------
// torch CPU reduction order of `sum` over the read dimension
// (aten/src/ATen/native/cpu/SumKernel.cpp as shipped in torch 2.x):
// a 4-level cascade whose level step is 2^lp; each full block of 2^lp values is
// summed sequentially from zero and pushed up the levels, the tail stays in
// level 0, and the levels are finally folded low-first.  Columns outside the
// 4-row-vector chunks use four interleaved cascades (rows k, k+4, ...), then
// the leftover rows are added to the first one and the four are folded.
// ---------------------------------------------------------------------------
template <typename T>
struct Cascade {
    T acc[4];
    int count;
    __device__ __forceinline__ void reset() {
        acc[0] = acc[1] = acc[2] = acc[3] = T(0);
        count = 0;
    }
    __device__ __forceinline__ void push(T x, int lp) {
        acc[0] = acc[0] + x;
        ++count;
        const int step_mask = (1 << lp) - 1;
        if ((count & step_mask) == 0) {
#pragma unroll
            for (int j = 1; j < 4; ++j) {
                acc[j] = acc[j] + acc[j - 1];
                acc[j - 1] = T(0);
                if ((count & (step_mask << (j * lp))) != 0) break;
            }
        }
    }
    __device__ __forceinline__ T finish() const {
        T r = acc[0];
        r = r + acc[1];
        r = r + acc[2];
        r = r + acc[3];
        return r;
    }
};

// Interleaved (ILP 4) variant: values arrive in read order g = 0..total-1.
template <typename T>
struct Interleaved {
    Cascade<T> stream[4];
    T first;   // finalized stream 0 plus leftover rows
    int seen;
    __device__ __forceinline__ void reset() {
#pragma unroll
        for (int k = 0; k < 4; ++k) stream[k].reset();
        first = T(0);
        seen = 0;
    }
    // total: number of values; lp: level power of each stream (size total/4).
    __device__ __forceinline__ void push(T x, int total, int lp) {
        const int full = (total / 4) * 4;
        if (seen < full) {
            const int k = seen & 3;
            // Stream k receives its q-th value; dispatch without dynamic indexing.
            if (k == 0) stream[0].push(x, lp);
            else if (k == 1) stream[1].push(x, lp);
            else if (k == 2) stream[2].push(x, lp);
            else stream[3].push(x, lp);
            if (seen + 1 == full) first = stream[0].finish();
        } else {
            if (full == 0 && seen == 0) first = T(0);
            first = first + x;
        }
        ++seen;
    }
    __device__ __forceinline__ T finish(int total) const {
        const int full = (total / 4) * 4;
        T r = first;
        if (full) {
            r = r + stream[1].finish();
            r = r + stream[2].finish();
            r = r + stream[3].finish();
        }
        return r;
    }
};

}  // namespace mf
