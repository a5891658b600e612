// Grouped INT quantization, slicing layout and per-read scale gathering on gfx950.
//
// Semantics follow memfast/quantization.py for INT codes of at most 8 bits
// (FP32 arithmetic): grouped_quantize (:9-44), read_starts (:76-79),
// pack_weight (:94-112) and input_tiles (:115-137).  Division is IEEE
// correctly rounded FP32 (as torch CPU's true division) and rounding is
// round-half-even (rintf), so codes and scales are bit-identical to the CPU
// reference.  All kernels are HBM-bound elementwise passes.
#include <cfloat>

#include "mf_kernels.h"

namespace mf {

// out[v, c] += bias[c] (one FP32 add, as torch's broadcast add), flagging a
// non-finite sum in the status word.
__global__ void k_bias_add(float *out, i64 n, i64 o, i64 ldo, const float *bias, u32 *status,
                           u32 flag) {
    bool finite = true;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < n * o;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 v = i / o, c = i - v * o;
        const float s = out[v * ldo + c] + bias[c];
        out[v * ldo + c] = s;
        finite = finite && fabsf(s) <= FLT_MAX;
    }
    if (!finite && status) atomicOr(status, flag);
}

// out[v, c] = float(in[v * ld + c]) for c < cols (round to nearest even, as torch's cast
// of an FP64 tensor to FP32), flagging a non-finite result in the status word.
__global__ void k_narrow_f64(const double *in, i64 n, i64 cols, i64 ld, float *out, u32 *status,
                             u32 flag) {
    bool finite = true;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < n * cols;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 v = i / cols, c = i - v * cols;
        const float f = float(in[v * ld + c]);
        out[i] = f;
        finite = finite && fabsf(f) <= FLT_MAX;
    }
    if (!finite && status) atomicOr(status, flag);
}

__global__ void k_fill_u32(u32 *p, i64 count, u32 value) {
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += i64(gridDim.x) * blockDim.x)
        p[i] = value;
}

// Per-group max |x| via an integer atomicMax on the FP32 bit pattern (|x| >= 0
// orders like its bits).  Each thread first folds a run of up to 8 elements
// of one row that lie in the same group, to cut atomic traffic.  A non-finite
// element ORs `flag` into *status (when status is non-null).
__global__ void k_group_max(const float *x, i64 rows, i64 cols, i64 ld, i64 gr, i64 gc,
                            i64 ncg, u32 *work, u32 *status, u32 flag) {
    const i64 runs_per_row = (cols + 7) / 8;
    const i64 total = rows * runs_per_row;
    bool finite = true;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 r = i / runs_per_row;
        const i64 c0 = (i % runs_per_row) * 8;
        const float *row = x + r * ld;
        u32 best = 0;
        i64 group = -1;
        for (int e = 0; e < 8; ++e) {
            const i64 c = c0 + e;
            if (c >= cols) break;
            const i64 g = c / gc;
            if (g != group) {
                if (group >= 0) atomicMax(&work[(r / gr) * ncg + group], best);
                group = g;
                best = 0;
            }
            const float v = fabsf(row[c]);
            finite = finite && v <= FLT_MAX;
            const u32 bits = __float_as_uint(v);
            best = bits > best ? bits : best;
        }
        if (group >= 0) atomicMax(&work[(r / gr) * ncg + group], best);
    }
    if (!finite && status) atomicOr(status, flag);
}

// scale = (max > 0 ? max : 1) / upper, clamped below by the smallest subnormal.
__global__ void k_group_scale(const u32 *work, i64 groups, float upper, float *scale) {
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < groups;
         i += i64(gridDim.x) * blockDim.x) {
        const float peak = __uint_as_float(work[i]);
        float s = (peak > 0.0f ? peak : 1.0f) / upper;
        const float tiny = __uint_as_float(1u);
        s = s < tiny ? tiny : s;
        scale[i] = s;
    }
}

// quantize_code() for many values of one group at the cost of one division.  The
// quotient is taken as q = x * y with y = RN(1/s): then |q - x/s| <= |x/s| * 2^-23 and the
// reference's RN(x/s) is within |x/s| * 2^-24 of x/s, so for |x/s| <= 256 the two lie
// within 2^-14.4 of each other and round to the same integer unless q is within that of
// a half-integer.  Such values (|q - rint(q)| >= 0.5 - 2^-12), NaN, and every value of a
// group whose 1/s overflows (s subnormal) take the IEEE division.  Beyond |x/s| = 256 both
// quotients clamp to the same code, as long as |lower|, upper <= 128 (codes of at most
// 8 bits).
struct GroupCodes {
    float s, y;
    bool fast;
    __device__ __forceinline__ explicit GroupCodes(float scale)
        : s(scale), y(1.0f / scale), fast(y <= FLT_MAX) {}
    __device__ __forceinline__ u8 operator()(float x, float lower, float upper, u32 mask) const {
        const float q = x * y;
        float c = rintf(q);
        if (!fast || !(fabsf(q - c) < 0.5f - 0x1p-12f)) c = rintf(x / s);
        c = c < lower ? lower : c;
        c = c > upper ? upper : c;
        return u8(u32(int(c)) & mask);
    }
};

// Fused grouped quantization of row-local groups (gr == 1, the activation
// layout): one thread per (row, group of gc columns) computes the group's peak,
// its scale (stored in the grid scale [n, ncg]) and the codes of q [n, kp]; the
// thread of a row's last group also writes the zero padding [k, kp).  The
// second pass over the group re-reads it from cache.  VEC: 16-byte loads and
// 4-byte code stores (gc, k, kp and ld multiples of 4, x 16-byte aligned).
template <bool VEC>
__global__ void k_row_groups(const float *x, i64 n, i64 k, i64 ld, i64 gc, i64 ncg, i64 kp,
                             float lower, float upper, u32 mask, u8 *q, float *scale,
                             u32 *status, u32 flag) {
    const i64 total = n * ncg;
    bool finite = true;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 row = i / ncg, j = i - row * ncg;
        const i64 c0 = j * gc, c1 = (c0 + gc) < k ? (c0 + gc) : k;
        const float *src = x + row * ld;
        u8 *dst = q + row * kp;
        float peak = 0.0f;
        if (VEC) {
            for (i64 c = c0; c < c1; c += 4) {
                const float4 v = *reinterpret_cast<const float4 *>(src + c);
                const float a0 = fabsf(v.x), a1 = fabsf(v.y), a2 = fabsf(v.z), a3 = fabsf(v.w);
                finite = finite && a0 <= FLT_MAX && a1 <= FLT_MAX && a2 <= FLT_MAX && a3 <= FLT_MAX;
                peak = fmaxf(peak, fmaxf(fmaxf(a0, a1), fmaxf(a2, a3)));
            }
        } else {
            for (i64 c = c0; c < c1; ++c) {
                const float a = fabsf(src[c]);
                finite = finite && a <= FLT_MAX;
                peak = fmaxf(peak, a);
            }
        }
        const float s = group_scale(peak, upper);
        scale[i] = s;
        if (VEC) {
            for (i64 c = c0; c < c1; c += 4) {
                const float4 v = *reinterpret_cast<const float4 *>(src + c);
                const u32 word = u32(quantize_code(v.x, s, lower, upper, mask)) |
                                 u32(quantize_code(v.y, s, lower, upper, mask)) << 8 |
                                 u32(quantize_code(v.z, s, lower, upper, mask)) << 16 |
                                 u32(quantize_code(v.w, s, lower, upper, mask)) << 24;
                *reinterpret_cast<u32 *>(dst + c) = word;
            }
            if (j == ncg - 1)
                for (i64 c = k; c < kp; c += 4) *reinterpret_cast<u32 *>(dst + c) = 0u;
        } else {
            for (i64 c = c0; c < c1; ++c) dst[c] = quantize_code(src[c], s, lower, upper, mask);
            if (j == ncg - 1)
                for (i64 c = k; c < kp; ++c) dst[c] = 0;
        }
    }
    if (!finite && status) atomicOr(status, flag);
}
template __global__ void k_row_groups<true>(const float *, i64, i64, i64, i64, i64, i64, float,
                                            float, u32, u8 *, float *, u32 *, u32);
template __global__ void k_row_groups<false>(const float *, i64, i64, i64, i64, i64, i64, float,
                                             float, u32, u8 *, float *, u32 *, u32);

// Cooperative row groups of gc = 4*L floats (L a power of two <= 64): L lanes
// share a group, each holding one float4, so a wave reads 1 KiB contiguous per
// load and writes 256 contiguous code bytes.  The group peak is a shuffle
// reduction over the L lanes.  Requires the VEC conditions of k_row_groups.
__global__ void k_row_groups_lanes(const float *x, i64 n, i64 k, i64 ld, int L, i64 ncg, i64 kp,
                                   float lower, float upper, u32 mask, u8 *q, float *scale,
                                   u32 *status, u32 flag) {
    const i64 t = i64(blockIdx.x) * blockDim.x + threadIdx.x;
    const i64 total = n * ncg * L;
    if (t >= total) return;   // whole groups: L divides 64 and total
    const i64 grp = t / L;
    const int member = int(t - grp * L);
    const i64 row = grp / ncg, j = grp - row * ncg;
    const i64 col = j * 4 * L + member * 4;
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (col < k) v = *reinterpret_cast<const float4 *>(x + row * ld + col);
    const float a0 = fabsf(v.x), a1 = fabsf(v.y), a2 = fabsf(v.z), a3 = fabsf(v.w);
    const bool finite = a0 <= FLT_MAX && a1 <= FLT_MAX && a2 <= FLT_MAX && a3 <= FLT_MAX;
    float peak = fmaxf(fmaxf(a0, a1), fmaxf(a2, a3));
    for (int off = 1; off < L; off <<= 1) peak = fmaxf(peak, __shfl_xor(peak, off, 64));
    const float s = group_scale(peak, upper);
    if (member == 0) scale[grp] = s;
    u8 *dst = q + row * kp;
    if (col < k) {
        const u32 word = u32(quantize_code(v.x, s, lower, upper, mask)) |
                         u32(quantize_code(v.y, s, lower, upper, mask)) << 8 |
                         u32(quantize_code(v.z, s, lower, upper, mask)) << 16 |
                         u32(quantize_code(v.w, s, lower, upper, mask)) << 24;
        *reinterpret_cast<u32 *>(dst + col) = word;
    }
    if (j == ncg - 1)
        for (i64 c = k + member * 4; c < kp; c += 4 * L) *reinterpret_cast<u32 *>(dst + c) = 0u;
    if (!finite && status) atomicOr(status, flag);
}

// Wave-wide row groups of gc = 256*V floats: one wave per group, V float4 per
// lane kept in registers (one pass), peak reduced across the wave.  With `reads`
// (not NULL) the wave also writes the per-read scale table xscale [n, G] for the
// reads whose first physical row (clamped to k-1, as k_input_scales takes it)
// lies in its group, so no separate gather pass is needed.
template <int V>
__global__ void k_row_groups_wave(const float *x, i64 n, i64 k, i64 ld, i64 ncg, i64 kp,
                                  float lower, float upper, u32 mask, u8 *q, float *scale,
                                  u32 *status, u32 flag, const ReadTable reads) {
    const i64 t = i64(blockIdx.x) * blockDim.x + threadIdx.x;
    const i64 grp = t >> 6;
    const int lane = int(t & 63);
    if (grp >= n * ncg) return;   // whole waves
    const i64 row = grp / ncg, j = grp - row * ncg;
    const i64 c0 = j * 256 * V;
    const float *src = x + row * ld;
    float4 v[V];
    float peak = 0.0f;
    bool finite = true;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const i64 col = c0 + (i * 64 + lane) * 4;
        v[i] = col < k ? *reinterpret_cast<const float4 *>(src + col)
                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float a0 = fabsf(v[i].x), a1 = fabsf(v[i].y), a2 = fabsf(v[i].z), a3 = fabsf(v[i].w);
        finite = finite && a0 <= FLT_MAX && a1 <= FLT_MAX && a2 <= FLT_MAX && a3 <= FLT_MAX;
        peak = fmaxf(peak, fmaxf(fmaxf(a0, a1), fmaxf(a2, a3)));
    }
    for (int off = 1; off < 64; off <<= 1) peak = fmaxf(peak, __shfl_xor(peak, off, 64));
    const float s = group_scale(peak, upper);
    if (lane == 0) scale[grp] = s;
    if (reads.xscale) {
        for (i64 rd = lane; rd < reads.G; rd += 64) {
            i64 first = (rd / reads.Gr) * reads.R + (rd % reads.Gr) * reads.P;
            first = first < k ? first : k - 1;
            if (first / (256 * V) == j) reads.xscale[row * reads.G + rd] = s;
        }
    }
    u8 *dst = q + row * kp;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const i64 col = c0 + (i * 64 + lane) * 4;
        if (col < k) {
            const u32 word = u32(quantize_code(v[i].x, s, lower, upper, mask)) |
                             u32(quantize_code(v[i].y, s, lower, upper, mask)) << 8 |
                             u32(quantize_code(v[i].z, s, lower, upper, mask)) << 16 |
                             u32(quantize_code(v[i].w, s, lower, upper, mask)) << 24;
            *reinterpret_cast<u32 *>(dst + col) = word;
        }
    }
    if (j == ncg - 1)
        for (i64 c = k + lane * 4; c < kp; c += 256) *reinterpret_cast<u32 *>(dst + c) = 0u;
    if (!finite && status) atomicOr(status, flag);
}
template __global__ void k_row_groups_wave<2>(const float *, i64, i64, i64, i64, i64, float, float,
                                              u32, u8 *, float *, u32 *, u32, const ReadTable);
template __global__ void k_row_groups_wave<4>(const float *, i64, i64, i64, i64, i64, float, float,
                                              u32, u8 *, float *, u32 *, u32, const ReadTable);
template __global__ void k_row_groups_wave<8>(const float *, i64, i64, i64, i64, i64, float, float,
                                              u32, u8 *, float *, u32 *, u32, const ReadTable);
template __global__ void k_row_groups_wave<16>(const float *, i64, i64, i64, i64, i64, float,
                                               float, u32, u8 *, float *, u32 *, u32,
                                               const ReadTable);

// Column groups of GR rows held in registers: thread = (physical column, one
// row group), so every lane issues its GR coalesced loads at once.  Writes the
// scale grid, packed [m, p, R, C] (bytes, coalesced across lanes) and the
// thread's GR contiguous bytes of packed_t (4-byte stores when WORD: kp % 4 == 0).
template <int GR, bool WORD>
__global__ void k_col_groups_reg(const float *b, i64 k, i64 o, i64 ld, int R, int C, i64 m,
                                 i64 p, float lower, float upper, u32 mask, u8 *packed,
                                 u8 *packed_t, float *scale, u32 *status, u32 flag) {
    const i64 kp = m * R, op = p * C;
    const i64 col = i64(blockIdx.x) * blockDim.x + threadIdx.x;
    if (col >= op) return;
    const i64 r0 = i64(blockIdx.y) * GR;
    const bool live = col < o;
    float v[GR];
#pragma unroll
    for (int i = 0; i < GR; ++i) {
        const i64 row = r0 + i;
        v[i] = (live && row < k) ? b[row * ld + col] : 0.0f;
    }
    float peak = 0.0f;
    bool finite = true;
#pragma unroll
    for (int i = 0; i < GR; ++i) {
        const float a = fabsf(v[i]);
        finite = finite && a <= FLT_MAX;
        peak = fmaxf(peak, a);
    }
    const float s = group_scale(peak, upper);
    if (live && r0 < k) scale[i64(blockIdx.y) * o + col] = s;
    const i64 t = col / C, c = col - t * C;
    i64 tile = r0 / R, r = r0 - tile * R;
    u8 *column_t = packed_t ? packed_t + col * kp : nullptr;
    u32 word = 0;
#pragma unroll
    for (int i = 0; i < GR; ++i) {
        const i64 row = r0 + i;
        if (row >= kp) break;
        const u8 code = (live && row < k) ? quantize_code(v[i], s, lower, upper, mask) : u8(0);
        packed[((tile * p + t) * R + r) * C + c] = code;
        if (++r == R) { r = 0; ++tile; }
        if (column_t) {
            if (WORD) {
                word |= u32(code) << (8 * (i & 3));
                if ((i & 3) == 3) {
                    *reinterpret_cast<u32 *>(column_t + row - 3) = word;
                    word = 0;
                }
            } else {
                column_t[row] = code;
            }
        }
    }
    if (!finite && status) atomicOr(status, flag);
}
// The proven-slot mask of one side from its slices' digit-sum maxima (the test
// k_digit_bits applies): slot s passes when maxima[tests.slice[s]] <= tests.thr[s].
__device__ __forceinline__ uint64_t proven_slots(const SlotTests &tests, const int *maxima) {
    uint64_t bits = 0, slots = tests.exists;
    while (slots) {
        const int slot = __builtin_ctzll(slots);
        slots &= slots - 1;
        if (maxima[tests.slice[slot]] <= tests.thr[slot]) bits |= uint64_t(1) << slot;
    }
    return bits;
}

// Column groups through an LDS tile: workgroup = 64 physical columns (lanes)
// x 4 row groups of GR rows (waves), i.e. a [4*GR x 64] code tile.  Each lane
// holds its group's GR values in registers (coalesced 256-byte row loads),
// writes its codes into the tile, and the workgroup then stores the tile as
// 64-byte row segments of packed [m, p, R, C] and 4*GR-byte column runs of
// packed_t [p*C, m*R], 16 bytes per store.  Requires C % 64 == 0, R % (4*GR)
// == 0 (row segments stay inside one array tile) and kp % 16 == 0.
// GIVEN: the group scales [ceil(k/gr), o] are already in `scale` (any gr, from
// a separate group-maximum pass); each row takes its group's scale.
// With `digits` (GR == 32 == rows per read), each wave also reduces its read's
// digit sums over the 32-column blocks of the tile into their proven-slot masks.
template <int GR, bool GIVEN>
__device__ __forceinline__ void col_tile(const float *b, i64 k, i64 o, i64 ld, int R, int C, i64 m,
                                         i64 p, float lower, float upper, u32 mask, u8 *packed,
                                         u8 *packed_t, float *scale, i64 gr, u32 *status, u32 flag,
                                         i64 bx, i64 by, const TileDigits *digits) {
    constexpr int ROWS = 4 * GR;
    __shared__ __align__(16) u8 tile_rc[ROWS][64 + 16];   // row-major codes
    __shared__ __align__(16) u8 tile_cr[64][ROWS + 16];   // column-major codes
    const i64 kp = m * R;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const i64 c0 = bx * 64, r_block = by * ROWS;
    const i64 col = c0 + lane;
    const i64 r0 = r_block + wave * GR;
    const bool live = col < o;
    float v[GR];
#pragma unroll
    for (int i = 0; i < GR; ++i) {
        const i64 row = r0 + i;
        v[i] = (live && row < k) ? b[row * ld + col] : 0.0f;
    }
    bool finite = true, large = false;
    if (GIVEN) {
        i64 g = r0 / gr, boundary = (g + 1) * gr;
        float sc = (live && r0 < k) ? scale[g * o + col] : 1.0f;
#pragma unroll
        for (int i = 0; i < GR; ++i) {
            const i64 row = r0 + i;
            if (live && row < k && row >= boundary) {
                g = row / gr;
                boundary = (g + 1) * gr;
                sc = scale[g * o + col];
            }
            const u8 code = (live && row < k) ? quantize_code(v[i], sc, lower, upper, mask) : u8(0);
            tile_rc[wave * GR + i][lane] = code;
            tile_cr[lane][wave * GR + i] = code;
        }
    } else {
        float peak = 0.0f;
#pragma unroll
        for (int i = 0; i < GR; ++i) {
            const float a = fabsf(v[i]);
            finite = finite && a <= FLT_MAX;
            peak = fmaxf(peak, a);
        }
        const float sc = group_scale(peak, upper);
        if (live && r0 < k) scale[(r0 / GR) * o + col] = sc;
        large = digits && live && r0 < k && sc > digits->scale_bound;
        const GroupCodes codes(sc);
#pragma unroll
        for (int i = 0; i < GR; ++i) {
            const u8 code = (live && r0 + i < k) ? codes(v[i], lower, upper, mask) : u8(0);
            tile_rc[wave * GR + i][lane] = code;
            tile_cr[lane][wave * GR + i] = code;
        }
    }
    __syncthreads();
    // packed: ROWS rows x 64 bytes = 4 x 16-byte chunks per row.
    const i64 t = c0 / C, cc0 = c0 - t * C;
    for (int e = threadIdx.x; e < ROWS * 4; e += 256) {
        const int rr = e >> 2, chunk = e & 3;
        const i64 row = r_block + rr;
        if (row >= kp) continue;
        const i64 i = row / R, r = row - i * R;
        *reinterpret_cast<uint4 *>(packed + ((i * p + t) * R + r) * C + cc0 + chunk * 16) =
            *reinterpret_cast<const uint4 *>(&tile_rc[rr][chunk * 16]);
    }
    // packed_t: 64 columns x ROWS bytes = ROWS/16 chunks per column.
    if (packed_t) {
        for (int e = threadIdx.x; e < 64 * (ROWS / 16); e += 256) {
            const int cl = e / (ROWS / 16), chunk = e % (ROWS / 16);
            const i64 row = r_block + chunk * 16;
            if (row >= kp) continue;
            *reinterpret_cast<uint4 *>(packed_t + (c0 + cl) * kp + row) =
                *reinterpret_cast<const uint4 *>(&tile_cr[cl][chunk * 16]);
        }
    }
    if (GR == 32 && digits && r0 < kp) {
        // This wave's rows are one read (g = r0 / 32) of all 64 columns.
        __shared__ int col_max[4][2][8];
        const uint4 *mine = reinterpret_cast<const uint4 *>(&tile_cr[lane][wave * GR]);
        const uint4 lo = mine[0], hi = mine[1];
        const SliceLayout &layout = digits->layout;
#pragma unroll
        for (int sl = 0; sl < 8; ++sl) {
            if (sl >= layout.count) break;
            const int sh = layout.shift[sl];
            const u32 mk = u32(layout.mask[sl]) * 0x01010101u;
            u32 sum = __builtin_amdgcn_sad_u8((lo.x >> sh) & mk, 0u, 0u);
            sum = __builtin_amdgcn_sad_u8((lo.y >> sh) & mk, 0u, sum);
            sum = __builtin_amdgcn_sad_u8((lo.z >> sh) & mk, 0u, sum);
            sum = __builtin_amdgcn_sad_u8((lo.w >> sh) & mk, 0u, sum);
            sum = __builtin_amdgcn_sad_u8((hi.x >> sh) & mk, 0u, sum);
            sum = __builtin_amdgcn_sad_u8((hi.y >> sh) & mk, 0u, sum);
            sum = __builtin_amdgcn_sad_u8((hi.z >> sh) & mk, 0u, sum);
            sum = __builtin_amdgcn_sad_u8((hi.w >> sh) & mk, 0u, sum);
            int best = int(sum);
#pragma unroll
            for (int off = 1; off < 32; off <<= 1) best = max(best, __shfl_xor(best, off, 64));
            if ((lane & 31) == 0) col_max[wave][lane >> 5][sl] = best;
        }
        // Lanes 0 and 32 read back only the words they wrote.
        if ((lane & 31) == 0)
            digits->bits[((c0 + lane) / 32) * digits->G + r0 / GR] =
                proven_slots(digits->tests, col_max[wave][lane >> 5]);
    }
    if (!finite && status) atomicOr(status, flag);
    if (large && status) atomicOr(status, u32(MF_STATUS_RANGE));
}

template <int GR, bool GIVEN>
__global__ __launch_bounds__(256) void k_col_groups_tile(
    const float *b, i64 k, i64 o, i64 ld, int R, int C, i64 m, i64 p, float lower, float upper,
    u32 mask, u8 *packed, u8 *packed_t, float *scale, i64 gr, u32 *status, u32 flag) {
    col_tile<GR, GIVEN>(b, k, o, ld, R, C, m, p, lower, upper, mask, packed, packed_t, scale, gr,
                        status, flag, blockIdx.x, blockIdx.y, nullptr);
}
#define MF_COL_TILE_INST(GR, GIVEN)                                                             \
    template __global__ void k_col_groups_tile<GR, GIVEN>(const float *, i64, i64, i64, int, int, \
                                                          i64, i64, float, float, u32, u8 *, u8 *,  \
                                                          float *, i64, u32 *, u32);
MF_COL_TILE_INST(16, false)
MF_COL_TILE_INST(32, false)
MF_COL_TILE_INST(32, true)
#undef MF_COL_TILE_INST

// Input row groups of one read (P = 32 values of one vector) for the ideal read, with
// its digit-sum pre-pass: one workgroup quantizes reads 4j .. 4j+3 of 64 vectors (one
// (vector, read) group per lane, whole 128-byte lines of q) into q and the per-read
// scale table xscale [n, G], and reduces each read's digit sums over the 64 vectors into
// the proven-slot mask of that vector block (what k_digit_bits computes from q).
// Requires k == m*R, G % 4 == 0, ldx % 4 == 0 and 16-byte aligned x and q.
__device__ __forceinline__ void input_read_block(const ReadGroupArgs &a, i64 block) {
    __shared__ int wave_max[4][4][8];
    __shared__ int block_max[4][8];
    const i64 G = a.G, quads = G / 4;
    const i64 vb = block / quads, g0 = (block - vb * quads) * 4;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int rd = t & 3;
    const i64 row = vb * 64 + (t >> 2), g = g0 + rd;
    const bool live = row < a.n;
    float4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (live) {
        const float4 *src = reinterpret_cast<const float4 *>(a.x + row * a.ldx + g * 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = src[i];
    }
    bool finite = true;
    float peak = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float e0 = fabsf(v[i].x), e1 = fabsf(v[i].y), e2 = fabsf(v[i].z), e3 = fabsf(v[i].w);
        finite = finite && e0 <= FLT_MAX && e1 <= FLT_MAX && e2 <= FLT_MAX && e3 <= FLT_MAX;
        peak = fmaxf(fmaxf(peak, fmaxf(e0, e1)), fmaxf(e2, e3));
    }
    const float s = group_scale(peak, a.xupper);
    const float lo = -a.xupper, hi = a.xupper;
    const u32 mk = a.xmask;
    const GroupCodes codes(s);
    u32 w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        w[i] = u32(codes(v[i].x, lo, hi, mk)) | u32(codes(v[i].y, lo, hi, mk)) << 8 |
               u32(codes(v[i].z, lo, hi, mk)) << 16 | u32(codes(v[i].w, lo, hi, mk)) << 24;
    if (live) {
        a.xscale[row * G + g] = s;
        uint4 *dst = reinterpret_cast<uint4 *>(a.q + row * a.k + g * 32);
        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
    // Digit sums of this lane's (vector, read), maximized over the wave's 16 vectors of
    // the same read and then over the workgroup's 4 waves.  Rows past n hold zero codes.
    const SliceLayout &layout = a.xdigits.layout;
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {
        if (sl >= layout.count) break;
        const int sh = layout.shift[sl];
        const u32 dm = u32(layout.mask[sl]) * 0x01010101u;
        u32 sum = 0u;
#pragma unroll
        for (int i = 0; i < 8; ++i) sum = __builtin_amdgcn_sad_u8((w[i] >> sh) & dm, 0u, sum);
        int best = int(sum);
#pragma unroll
        for (int off = 4; off < 64; off <<= 1) best = max(best, __shfl_xor(best, off, 64));
        if (lane < 4) wave_max[wave][lane][sl] = best;
    }
    __syncthreads();
    if (t < 4) {
        for (int sl = 0; sl < layout.count && sl < 8; ++sl)
            block_max[t][sl] = max(max(wave_max[0][t][sl], wave_max[1][t][sl]),
                                   max(wave_max[2][t][sl], wave_max[3][t][sl]));
        a.xdigits.bits[vb * G + g0 + t] = proven_slots(a.xdigits.tests, block_max[t]);
    }
    if (!finite && a.status) atomicOr(a.status, u32(MF_STATUS_INPUT));
    if (live && s > a.xdigits.scale_bound && a.status) atomicOr(a.status, u32(MF_STATUS_RANGE));
}

// Both operands of the ideal read in read-sized groups, with its digit-sum pre-pass, in
// one launch: workgroups [0, wblocks) program B through the LDS code tile (32-row column
// groups), the rest quantize A (one read of 64 vectors each).
__global__ __launch_bounds__(256) void k_read_groups(const ReadGroupArgs a) {
    const i64 block = blockIdx.x;
    if (block < a.wblocks) {
        const i64 bx = block % a.wgrid_x, by = block / a.wgrid_x;
        col_tile<32, false>(a.b, a.k, a.o, a.ldb, a.R, a.C, a.m, a.p, a.wlower, a.wupper,
                            a.wmask, a.packed, a.packed_t, a.wscale, 32, a.status,
                            u32(MF_STATUS_WEIGHT), bx, by, &a.wdigits);
    } else {
        input_read_block(a, block - a.wblocks);
    }
}

#define MF_COL_REG_INST(GR, WORD)                                                               \
    template __global__ void k_col_groups_reg<GR, WORD>(const float *, i64, i64, i64, int, int, \
                                                        i64, i64, float, float, u32, u8 *, u8 *,  \
                                                        float *, u32 *, u32);
MF_COL_REG_INST(8, true)
MF_COL_REG_INST(8, false)
MF_COL_REG_INST(16, true)
MF_COL_REG_INST(16, false)
MF_COL_REG_INST(32, true)
MF_COL_REG_INST(32, false)
MF_COL_REG_INST(64, true)
MF_COL_REG_INST(64, false)

// Fused grouped quantization of column-local groups (gc == 1, the weight
// layout of quantization.py:82-112): thread = one physical column `col` of the
// padded [kp, op] code matrix and one chunk of `span` rows (a multiple of gr,
// so groups never straddle chunks).  Lanes take consecutive columns, so the
// FP32 reads, the packed [m, p, R, C] bytes and the scale grid [nrg, o] are
// coalesced; each thread writes its run of packed_t [op, kp] (column-major)
// itself, four rows per 4-byte store when WORD (kp and span multiples of 4).
template <bool WORD>
__global__ void k_col_groups(const float *b, i64 k, i64 o, i64 ld, i64 gr, i64 span, int R,
                             int C, i64 m, i64 p, float lower, float upper, u32 mask,
                             u8 *packed, u8 *packed_t, float *scale, u32 *status, u32 flag) {
    const i64 kp = m * R, op = p * C;
    const i64 col = i64(blockIdx.x) * blockDim.x + threadIdx.x;
    if (col >= op) return;
    const i64 r0 = i64(blockIdx.y) * span;
    const i64 r1 = (r0 + span) < kp ? (r0 + span) : kp;
    if (r0 >= r1) return;
    const i64 t = col / C, c = col - t * C;
    i64 tile = r0 / R, r = r0 - tile * R;   // packed coordinates of the current row
    u8 *column_t = packed_t ? packed_t + col * kp : nullptr;
    u32 word = 0;
    bool finite = true;
    auto put = [&](i64 row, u8 code) {
        packed[((tile * p + t) * R + r) * C + c] = code;
        if (++r == R) { r = 0; ++tile; }
        if (column_t) {
            if (WORD) {
                word |= u32(code) << (8 * (row & 3));
                if ((row & 3) == 3) {
                    *reinterpret_cast<u32 *>(column_t + row - 3) = word;
                    word = 0;
                }
            } else {
                column_t[row] = code;
            }
        }
    };
    i64 row = r0;
    if (col < o) {
        const i64 live = r1 < k ? r1 : k;
        while (row < live) {
            const i64 g_end = (row + gr) < live ? (row + gr) : live;
            float peak = 0.0f;
            for (i64 rr = row; rr < g_end; ++rr) {
                const float a = fabsf(b[rr * ld + col]);
                finite = finite && a <= FLT_MAX;
                peak = fmaxf(peak, a);
            }
            const float s = group_scale(peak, upper);
            scale[(row / gr) * o + col] = s;
            for (; row < g_end; ++row) put(row, quantize_code(b[row * ld + col], s, lower, upper, mask));
        }
    }
    for (; row < r1; ++row) put(row, 0);
    if (!finite && status) atomicOr(status, flag);
}
template __global__ void k_col_groups<true>(const float *, i64, i64, i64, i64, i64, int, int, i64,
                                            i64, float, float, u32, u8 *, u8 *, float *, u32 *,
                                            u32);
template __global__ void k_col_groups<false>(const float *, i64, i64, i64, i64, i64, int, int, i64,
                                             i64, float, float, u32, u8 *, u8 *, float *, u32 *,
                                             u32);

// Codes of column-local groups (gc == 1) from precomputed group scales
// [ceil(k/gr), o] (any gr): the layout of k_col_groups with rows in chunks of
// `span` (a multiple of 4) independent of the group size.
template <bool WORD>
__global__ void k_col_codes(const float *b, i64 k, i64 o, i64 ld, i64 gr, i64 span, int R, int C,
                            i64 m, i64 p, const float *scale, float lower, float upper, u32 mask,
                            u8 *packed, u8 *packed_t) {
    const i64 kp = m * R, op = p * C;
    const i64 col = i64(blockIdx.x) * blockDim.x + threadIdx.x;
    if (col >= op) return;
    const i64 r0 = i64(blockIdx.y) * span;
    const i64 r1 = (r0 + span) < kp ? (r0 + span) : kp;
    if (r0 >= r1) return;
    const i64 t = col / C, c = col - t * C;
    i64 tile = r0 / R, r = r0 - tile * R;   // packed coordinates of the current row
    u8 *column_t = packed_t ? packed_t + col * kp : nullptr;
    u32 word = 0;
    auto put = [&](i64 row, u8 code) {
        packed[((tile * p + t) * R + r) * C + c] = code;
        if (++r == R) { r = 0; ++tile; }
        if (column_t) {
            if (WORD) {
                word |= u32(code) << (8 * (row & 3));
                if ((row & 3) == 3) {
                    *reinterpret_cast<u32 *>(column_t + row - 3) = word;
                    word = 0;
                }
            } else {
                column_t[row] = code;
            }
        }
    };
    const bool live_col = col < o;
    const i64 live = live_col ? (r1 < k ? r1 : k) : r0;   // rows with data: [r0, live)
    i64 g = r0 / gr, boundary = (g + 1) * gr;
    float s = live_col && r0 < live ? scale[g * o + col] : 1.0f;
    // Four rows per step: independent loads in flight.
    for (i64 row = r0; row < r1; row += 4) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = row + u < live ? b[(row + u) * ld + col] : 0.0f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const i64 rr = row + u;
            if (rr >= r1) break;
            if (rr < live && rr >= boundary) {
                g = rr / gr;
                boundary = (g + 1) * gr;
                s = scale[g * o + col];
            }
            put(rr, rr < live ? quantize_code(v[u], s, lower, upper, mask) : u8(0));
        }
    }
}
template __global__ void k_col_codes<true>(const float *, i64, i64, i64, i64, i64, int, int, i64,
                                           i64, const float *, float, float, u32, u8 *, u8 *);
template __global__ void k_col_codes<false>(const float *, i64, i64, i64, i64, i64, int, int, i64,
                                            i64, const float *, float, float, u32, u8 *, u8 *);

// q [n, kp] with kp = m*R; columns >= k are zero padding.
__global__ void k_input_codes(const float *x, i64 n, i64 k, i64 ld, i64 kp, const float *scale,
                              i64 gr, i64 gc, i64 ncg, int fixed, float lower, float upper,
                              u32 mask, u8 *q) {
    const i64 total = n * kp;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 row = i / kp, col = i % kp;
        u8 code = 0;
        if (col < k) {
            const float s = fixed ? scale[col] : scale[(row / gr) * ncg + col / gc];
            code = quantize_code(x[row * ld + col], s, lower, upper, mask);
        }
        q[i] = code;
    }
}

// Four consecutive columns per thread: one 16-byte load and one 4-byte store.
// Needs k % 4 == 0, kp % 4 == 0, ld % 4 == 0, a 16-byte aligned x and a 4-byte
// aligned q.  I is the index type: u32 when n*kp/4 plus one grid stride, kp, gr
// and gc all stay below 2^31, else i64.  The column group advances incrementally
// over the four columns instead of a division per column.
template <typename I>
__global__ __launch_bounds__(256) void k_input_codes4(const float *x, i64 n, i64 k, i64 ld, i64 kp,
                                                      const float *scale, i64 gr, i64 gc, i64 ncg,
                                                      int fixed, float lower, float upper, u32 mask,
                                                      u8 *q) {
    const I kq = I(kp / 4), total = I(n) * kq;
    const I group_rows = I(gr), group_cols = I(gc);
    for (I e = I(blockIdx.x) * I(blockDim.x) + I(threadIdx.x); e < total;
         e += I(gridDim.x) * I(blockDim.x)) {
        const I row = e / kq, col = (e - row * kq) * 4;
        u32 word = 0;
        if (i64(col) < k) {
            const float4 v = *reinterpret_cast<const float4 *>(x + i64(row) * ld + i64(col));
            float sc[4];
            if (fixed) {
#pragma unroll
                for (int j = 0; j < 4; ++j) sc[j] = scale[i64(col) + j];
            } else {
                const float *srow = scale + i64(row / group_rows) * ncg;
                I g = col / group_cols, rem = col - g * group_cols;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    sc[j] = srow[g];
                    if (++rem == group_cols) {
                        ++g;
                        rem = 0;
                    }
                }
            }
            word = u32(quantize_code(v.x, sc[0], lower, upper, mask)) |
                   u32(quantize_code(v.y, sc[1], lower, upper, mask)) << 8 |
                   u32(quantize_code(v.z, sc[2], lower, upper, mask)) << 16 |
                   u32(quantize_code(v.w, sc[3], lower, upper, mask)) << 24;
        }
        *reinterpret_cast<u32 *>(q + i64(row) * kp + i64(col)) = word;
    }
}
template __global__ void k_input_codes4<u32>(const float *, i64, i64, i64, i64, const float *, i64,
                                             i64, i64, int, float, float, u32, u8 *);
template __global__ void k_input_codes4<i64>(const float *, i64, i64, i64, i64, const float *, i64,
                                             i64, i64, int, float, float, u32, u8 *);

// ---- implicit im2col: input tiles of a convolution's patch matrix ----------
// Patch row r = b * L + oh * wo + ow (L = ho * wo), column k = (c * kh + i) * kw + j
// (F.unfold's order) holds x[b, c0 + c, oh*sh - ph + i*dh, ow*sw - pw + j*dw], or 0
// outside the image.  Lanes own consecutive patch rows, so for one k a wave reads
// neighbouring pixels of one image row (coalesced); k is uniform across the wave and
// its (c, i, j) decomposition advances incrementally in scalar registers.
struct ConvLane {
    i64 pixel;    // offset of x[b, c0, ih0, iw0] (may point outside the image)
    int ih0, iw0;
};

__device__ __forceinline__ ConvLane conv_lane(const mf_conv_geometry &g, u32 row) {
    const u32 wo = u32(g.out_width), L = u32(g.out_height) * wo;
    const u32 b = row / L, l = row - b * L;
    const u32 oh = l / wo, ow = l - oh * wo;
    ConvLane lane;
    lane.ih0 = int(oh) * g.sh - g.ph;
    lane.iw0 = int(ow) * g.sw - g.pw;
    lane.pixel = (i64(b) * g.channels + g.c0) * g.height * g.width + i64(lane.ih0) * g.width +
                 lane.iw0;
    return lane;
}

// Position (c, i, j) of column k in the patch and its offset from the patch origin.
struct ConvTap {
    int c, i, j;
    i64 delta;   // c*H*W + i*dh*W + j*dw
    int di, dj;  // i*dh, j*dw

    __device__ __forceinline__ void start(const mf_conv_geometry &g, int k) {
        const int kk = g.kh * g.kw;
        c = k / kk;
        const int rem = k - c * kk;
        i = rem / g.kw;
        j = rem - i * g.kw;
        di = i * g.dh;
        dj = j * g.dw;
        delta = i64(c) * g.height * g.width + i64(di) * g.width + dj;
    }
    __device__ __forceinline__ void next(const mf_conv_geometry &g) {
        if (++j < g.kw) {
            dj += g.dw;
            delta += g.dw;
            return;
        }
        j = 0;
        delta -= i64(dj);
        dj = 0;
        if (++i < g.kh) {
            di += g.dh;
            delta += i64(g.dh) * g.width;
            return;
        }
        i = 0;
        delta += i64(g.height - di) * g.width;
        di = 0;
        ++c;
    }
};

__device__ __forceinline__ float conv_load(const float *x, const mf_conv_geometry &g,
                                           const ConvLane &lane, bool live, const ConvTap &t) {
    const u32 ih = u32(lane.ih0 + t.di), iw = u32(lane.iw0 + t.dj);
    return live && ih < u32(g.height) && iw < u32(g.width) ? x[lane.pixel + t.delta] : 0.0f;
}

// Codes q [rows, kp] (zero past K) for a tile of 64 rows x CONV_CHUNK columns per
// block, with a fixed per-column scale (gc == 0) or per-(gr rows, gc columns) group
// scales [ceil(rows/gr), ncg].  Each wave quantizes CONV_CHUNK/4 columns of the 64
// rows into LDS; the block then writes whole row segments.
constexpr int CONV_CHUNK = CONV_CHUNK_COLS;
constexpr int CONV_PITCH = CONV_CHUNK / 4 + 1;   // dwords per LDS row (odd: no conflicts)

__global__ __launch_bounds__(256) void k_conv_codes(const float *x, const mf_conv_geometry g,
                                                    i64 K, i64 kp, const float *scale, i64 gr,
                                                    i64 gc, i64 ncg, float lower, float upper,
                                                    u32 mask, u8 *q, int vec, u32 *status,
                                                    u32 flag) {
    __shared__ u32 tile[64 * CONV_PITCH];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const i64 rows = g.n * g.out_height * g.out_width;
    const i64 r0 = i64(blockIdx.x) * 64;
    const i64 kc = i64(blockIdx.y) * CONV_CHUNK;
    const bool live = r0 + lane < rows;
    const ConvLane me = conv_lane(g, u32(live ? r0 + lane : r0));
    const int k0 = int(kc) + wave * (CONV_CHUNK / 4);
    bool finite = true;
    constexpr int CPW = CONV_CHUNK / 4;   // columns per wave
    if (k0 < K) {
        // Gather every value (and scale) first, so the loads are all in flight
        // before the first one is needed.
        float v[CPW], sc[CPW];
        ConvTap tap;
        tap.start(g, k0);
        const i64 rg = gc ? ((live ? r0 + lane : r0) / gr) * ncg : 0;
        i64 cg = gc ? k0 / gc : 0, cr = gc ? k0 - cg * gc : 0;
#pragma unroll
        for (int t = 0; t < CPW; ++t) {
            v[t] = 0.0f;
            sc[t] = 1.0f;
            if (k0 + t < K) {
                v[t] = conv_load(x, g, me, live, tap);
                sc[t] = gc ? scale[rg + cg] : scale[k0 + t];
                tap.next(g);
                if (gc && ++cr == gc) {
                    cr = 0;
                    ++cg;
                }
            }
        }
#pragma unroll
        for (int e = 0; e < CPW / 4; ++e) {
            u32 word = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int t = e * 4 + b;
                if (k0 + t < K) {
                    finite = finite && fabsf(v[t]) <= FLT_MAX;
                    word |= u32(quantize_code(v[t], sc[t], lower, upper, mask)) << (8 * b);
                }
            }
            tile[lane * CONV_PITCH + wave * (CPW / 4) + e] = word;
        }
    } else {
#pragma unroll
        for (int e = 0; e < CPW / 4; ++e) tile[lane * CONV_PITCH + wave * (CPW / 4) + e] = 0;
    }
    if (!finite && status) atomicOr(status, flag);
    __syncthreads();
    // Row `row` of the tile: 4 threads x CONV_CHUNK/4 bytes.
    const int row = threadIdx.x >> 2, part = threadIdx.x & 3;
    constexpr int WORDS = CONV_CHUNK / 16;
    if (r0 + row >= rows) return;
    const i64 col = kc + part * (CONV_CHUNK / 4);
    if (col >= kp) return;
    u32 w[WORDS];
#pragma unroll
    for (int e = 0; e < WORDS; ++e) w[e] = tile[row * CONV_PITCH + part * WORDS + e];
    u8 *dst = q + (r0 + row) * kp + col;
    if (vec) {   // kp and q 16-byte aligned: whole 16-byte pieces below kp
#pragma unroll
        for (int e = 0; e < WORDS; e += 4)
            if (col + 4 * e < kp)
                *reinterpret_cast<uint4 *>(dst + 4 * e) =
                    make_uint4(w[e], w[e + 1], w[e + 2], w[e + 3]);
    } else {
        const int count = int(kp - col < CONV_CHUNK / 4 ? kp - col : CONV_CHUNK / 4);
        for (int t = 0; t < count; ++t) dst[t] = u8(w[t >> 2] >> (8 * (t & 3)));
    }
}

// Group maxima |x| of the patch matrix for groups of gr rows and gc columns into
// work [ceil(rows/gr), ncg] (cleared; float bits).  A wave owns 64 rows and walks all
// K columns, flushing each lane's running maximum at column-group boundaries.
__global__ __launch_bounds__(256) void k_conv_group_max(const float *x, const mf_conv_geometry g,
                                                        i64 K, i64 gr, i64 gc, i64 ncg, u32 *work,
                                                        u32 *status, u32 flag) {
    const int lane = threadIdx.x & 63;
    const i64 rows = g.n * g.out_height * g.out_width;
    const i64 r0 = (i64(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 64;
    if (r0 >= rows) return;
    const bool live = r0 + lane < rows;
    const ConvLane me = conv_lane(g, u32(live ? r0 + lane : r0));
    u32 *target = work + ((live ? r0 + lane : r0) / gr) * ncg;
    ConvTap tap;
    tap.start(g, 0);
    bool finite = true;
    float peak = 0.0f;
    i64 cr = 0;
#pragma unroll 1
    for (i64 k = 0; k < K; ++k) {
        const float v = fabsf(conv_load(x, g, me, live, tap));
        finite = finite && v <= FLT_MAX;
        peak = v > peak || v != v ? v : peak;
        tap.next(g);
        if (++cr == gc || k + 1 == K) {
            if (live && __float_as_uint(peak)) atomicMax(target, __float_as_uint(peak));
            ++target;
            cr = 0;
            peak = 0.0f;
        }
    }
    if (!finite && status) atomicOr(status, flag);
}

// xscale [n, m*Gr]: scale of the read's first physical row, replicate-padded.
__global__ void k_input_scales(i64 n, i64 k, i64 groups, int R, int P, int Gr,
                               const float *scale, i64 gr, i64 gc, i64 ncg, int fixed,
                               float *xscale) {
    const i64 total = n * groups;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 row = i / groups, g = i % groups;
        i64 col = (g / Gr) * R + (g % Gr) * P;
        col = col < k ? col : k - 1;
        xscale[i] = fixed ? scale[col] : scale[(row / gr) * ncg + col / gc];
    }
}

// packed [m, p, R, C] and packed_t [p*C, m*R] from logical [k, o] weights.
__global__ void k_weight_codes(const float *b, i64 k, i64 o, i64 ld, int R, int C, i64 m,
                               i64 p, const float *scale, i64 gr, i64 gc, i64 ncg,
                               float lower, float upper, u32 mask, u8 *packed, u8 *packed_t) {
    const i64 kp = m * R, op = p * C;
    const i64 total = kp * op;
    for (i64 idx = i64(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += i64(gridDim.x) * blockDim.x) {
        const i64 row = idx / op, col = idx % op;
        u8 code = 0;
        if (row < k && col < o) {
            const float s = scale[(row / gr) * ncg + col / gc];
            code = quantize_code(b[row * ld + col], s, lower, upper, mask);
        }
        const i64 i = row / R, r = row % R, t = col / C, c = col % C;
        packed[((i * p + t) * R + r) * C + c] = code;
        if (packed_t) packed_t[col * kp + row] = code;
    }
}

// wscale [m*Gr, p*C]: replicate-padded scale at each read's first row.
__global__ void k_weight_scales(i64 k, i64 o, i64 groups, i64 op, int R, int P, int Gr,
                                const float *scale, i64 gr, i64 gc, i64 ncg, float *wscale) {
    const i64 total = groups * op;
    for (i64 idx = i64(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += i64(gridDim.x) * blockDim.x) {
        const i64 g = idx / op, col = idx % op;
        i64 row = (g / Gr) * R + (g % Gr) * P;
        row = row < k ? row : k - 1;
        const i64 cc = col < o ? col : o - 1;
        wscale[idx] = scale[(row / gr) * ncg + cc / gc];
    }
}

__global__ void k_transpose_packed(const u8 *packed, int R, int C, i64 m, i64 p, u8 *packed_t) {
    const i64 kp = m * R, op = p * C;
    const i64 total = kp * op;
    for (i64 idx = i64(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += i64(gridDim.x) * blockDim.x) {
        const i64 col = idx / kp, row = idx % kp;  // coalesced writes along rows
        const i64 i = row / R, r = row % R, t = col / C, c = col % C;
        packed_t[idx] = packed[((i * p + t) * R + r) * C + c];
    }
}

}  // namespace mf

// ---------------------------------------------------------------------------
// Wide configurations (precision above 8 bits or BFP): FP64 arithmetic and
// 32-bit codes, as memfast/quantization.py:9-44 computes in FP64 there.
// ---------------------------------------------------------------------------
namespace mf {

// Group max |x| of FP64 values (S = float: FP32 values, widened exactly) via atomicMax on
// the bit pattern.
template <typename S>
__global__ void k_group_max_f64(const S *x, i64 rows, i64 cols, i64 ld, i64 gr, i64 gc,
                                i64 ncg, u64 *work, u32 *status, u32 flag) {
    const i64 total = rows * cols;
    bool finite = true;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 r = i / cols, c = i - r * cols;
        const double v = fabs(double(x[r * ld + c]));
        finite = finite && v <= DBL_MAX;
        const u64 bits = u64(__double_as_longlong(v));
        if (bits) atomicMax(reinterpret_cast<unsigned long long *>(&work[(r / gr) * ncg + c / gc]),
                            static_cast<unsigned long long>(bits));
    }
    if (!finite && status) atomicOr(status, flag);
}

// |x| as its bit pattern (which orders like the value for |x| >= 0) and the
// largest finite magnitude, for FP32 (u32 bits) and FP64 (u64 bits).
template <typename T> struct AbsBits;
template <> struct AbsBits<float> {
    typedef u32 U;
    static __device__ __forceinline__ U of(float v) { return __float_as_uint(v); }
    static constexpr float LARGEST = FLT_MAX;
};
template <> struct AbsBits<double> {
    typedef unsigned long long U;
    static __device__ __forceinline__ U of(double v) { return U(__double_as_longlong(v)); }
    static constexpr double LARGEST = DBL_MAX;
};

// Groups of gr rows x gc columns, reduced along the rows first: block = 64
// column lanes x 4 row lanes over a chunk of `chunk` rows; each column lane
// covers V adjacent columns (V > 1: one 16-byte load per row, needs cols % V
// == 0, ld % V == 0 and a 16-byte aligned x), so a wave reads 64*V*sizeof(T)
// contiguous bytes per row.  Each thread keeps running maxima while its rows
// stay in one row group; LDS folds the four row lanes; then the block's 64*V
// column maxima go to their column groups: a block maximum and one atomicMax
// when all its columns lie in one group, else a shuffle maximum over aligned
// segments of `seg` columns (the largest power of two dividing gc, at most 64:
// such a segment never crosses a group boundary) and one atomicMax per
// segment.  work [ceil(rows/gr), ncg].  S: the stored type (FP32 values widened exactly to
// T = double for the wide quantizers' FP32 operands).
template <typename T> struct __align__(16) Vec16 { T e[16 / sizeof(T)]; };
template <typename T, typename U, int V, typename S>
__global__ __launch_bounds__(256) void k_col_group_max(const S *x, i64 rows, i64 cols, i64 ld,
                                                       i64 gr, i64 gc, i64 ncg, i64 chunk,
                                                       U *work, u32 *status, u32 flag) {
    static_assert(V == 1 || V * sizeof(S) == 16, "V columns per lane fill one 16-byte load");
    constexpr int BC = 64 * V;   // columns per block
    __shared__ U part[4][BC];
    __shared__ U wave_max[4];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const i64 c0 = i64(blockIdx.x) * BC;
    const i64 c = c0 + i64(tx) * V;
    const i64 r0 = i64(blockIdx.y) * chunk;
    const i64 r1 = (r0 + chunk) < rows ? (r0 + chunk) : rows;
    const i64 c_last = (c0 + BC - 1) < (cols - 1) ? (c0 + BC - 1) : (cols - 1);
    const bool one_group = c0 / gc == c_last / gc;
    const i64 low_bit = gc & -gc;
    const int seg = low_bit < 64 ? int(low_bit) : 64;
    bool finite = true;
    // Row groups that intersect this chunk, handled one at a time (uniform loop).
    for (i64 g = r0 / gr; g * gr < r1; ++g) {
        const i64 lo = (g * gr) > r0 ? (g * gr) : r0;
        const i64 hi = ((g + 1) * gr) < r1 ? ((g + 1) * gr) : r1;
        U best[V];
#pragma unroll
        for (int j = 0; j < V; ++j) best[j] = 0;
        if (c < cols) {
            i64 r = lo + ty;
            // Four rows per step: independent loads in flight.
            for (; r + 12 < hi; r += 16) {
                Vec16<S> v[4];
                S w[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (V > 1) v[u] = *reinterpret_cast<const Vec16<S> *>(x + (r + 4 * u) * ld + c);
                    else w[u] = x[(r + 4 * u) * ld + c];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
#pragma unroll
                    for (int j = 0; j < V; ++j) {
                        const T a = fabs(T(V > 1 ? v[u].e[j] : w[u]));
                        finite = finite && a <= AbsBits<T>::LARGEST;
                        const U bits = U(AbsBits<T>::of(a));
                        best[j] = bits > best[j] ? bits : best[j];
                    }
                }
            }
            for (; r < hi; r += 4) {
                Vec16<S> v;
                S w = 0;
                if (V > 1) v = *reinterpret_cast<const Vec16<S> *>(x + r * ld + c);
                else w = x[r * ld + c];
#pragma unroll
                for (int j = 0; j < V; ++j) {
                    const T a = fabs(T(V > 1 ? v.e[j] : w));
                    finite = finite && a <= AbsBits<T>::LARGEST;
                    const U bits = U(AbsBits<T>::of(a));
                    best[j] = bits > best[j] ? bits : best[j];
                }
            }
        }
#pragma unroll
        for (int j = 0; j < V; ++j) part[ty][tx * V + j] = best[j];
        __syncthreads();
        // Thread t folds column c0 + t of the block (threads >= BC hold 0).
        const int t = threadIdx.x;
        U m = 0;
        if (t < BC) {
            m = part[0][t];
            m = part[1][t] > m ? part[1][t] : m;
            m = part[2][t] > m ? part[2][t] : m;
            m = part[3][t] > m ? part[3][t] : m;
        }
        if (one_group) {
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) {
                const U other = U(__shfl_xor(m, d, 64));
                m = other > m ? other : m;
            }
            if (tx == 0) wave_max[ty] = m;
            __syncthreads();
            if (t == 0) {
                U b = wave_max[0];
                b = wave_max[1] > b ? wave_max[1] : b;
                b = wave_max[2] > b ? wave_max[2] : b;
                b = wave_max[3] > b ? wave_max[3] : b;
                if (b) atomicMax(&work[g * ncg + c0 / gc], b);
            }
        } else {
            for (int d = seg >> 1; d >= 1; d >>= 1) {
                const U other = U(__shfl_xor(m, d, 64));
                m = other > m ? other : m;
            }
            const i64 col = c0 + t;
            if (t < BC && (t & (seg - 1)) == 0 && col < cols && m)
                atomicMax(&work[g * ncg + col / gc], m);
        }
        __syncthreads();
    }
    if (!finite && status) atomicOr(status, flag);
}

// Row groups (gr == 1, gc >= 64): one wave per row and chunk of ROW_CHUNK
// columns (coalesced); per group in the chunk a lane maximum, a wave maximum by
// shuffles, and one atomicMax per (row, group, chunk).  work [rows, ncg].
constexpr int ROW_CHUNK = ROW_CHUNK_COLS;
template <typename T, typename U, typename S>
__global__ __launch_bounds__(256) void k_row_group_max(const S *x, i64 rows, i64 cols, i64 ld,
                                                       i64 gc, i64 ncg, U *work, u32 *status,
                                                       u32 flag) {
    const int lane = threadIdx.x & 63;
    const i64 row = i64(blockIdx.y) * 4 + (threadIdx.x >> 6);
    const i64 c0 = i64(blockIdx.x) * ROW_CHUNK;
    if (row >= rows) return;
    const i64 c1 = (c0 + ROW_CHUNK) < cols ? (c0 + ROW_CHUNK) : cols;
    const S *src = x + row * ld;
    bool finite = true;
    for (i64 g = c0 / gc; g * gc < c1; ++g) {
        const i64 lo = (g * gc) > c0 ? (g * gc) : c0;
        const i64 hi = ((g + 1) * gc) < c1 ? ((g + 1) * gc) : c1;
        U best = 0;
        for (i64 c = lo + lane; c < hi; c += 64) {
            const T v = fabs(T(src[c]));
            finite = finite && v <= AbsBits<T>::LARGEST;
            const U bits = U(AbsBits<T>::of(v));
            best = bits > best ? bits : best;
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            const U other = U(__shfl_xor(best, d, 64));
            best = other > best ? other : best;
        }
        if (lane == 0 && best) atomicMax(&work[row * ncg + g], best);
    }
    if (!finite && status) atomicOr(status, flag);
}

typedef unsigned long long ull;
template __global__ void k_col_group_max<float, u32, 1, float>(const float *, i64, i64, i64, i64,
                                                               i64, i64, i64, u32 *, u32 *, u32);
template __global__ void k_col_group_max<float, u32, 4, float>(const float *, i64, i64, i64, i64,
                                                               i64, i64, i64, u32 *, u32 *, u32);
template __global__ void k_col_group_max<double, ull, 1, double>(const double *, i64, i64, i64, i64,
                                                                 i64, i64, i64, ull *, u32 *, u32);
template __global__ void k_col_group_max<double, ull, 2, double>(const double *, i64, i64, i64, i64,
                                                                 i64, i64, i64, ull *, u32 *, u32);
template __global__ void k_col_group_max<double, ull, 1, float>(const float *, i64, i64, i64, i64,
                                                                i64, i64, i64, ull *, u32 *, u32);
template __global__ void k_col_group_max<double, ull, 4, float>(const float *, i64, i64, i64, i64,
                                                                i64, i64, i64, ull *, u32 *, u32);
template __global__ void k_row_group_max<float, u32, float>(const float *, i64, i64, i64, i64, i64,
                                                            u32 *, u32 *, u32);
template __global__ void k_row_group_max<double, ull, double>(const double *, i64, i64, i64, i64,
                                                              i64, ull *, u32 *, u32);
template __global__ void k_row_group_max<double, ull, float>(const float *, i64, i64, i64, i64,
                                                             i64, ull *, u32 *, u32);
template __global__ void k_group_max_f64<double>(const double *, i64, i64, i64, i64, i64, i64,
                                                 u64 *, u32 *, u32);
template __global__ void k_group_max_f64<float>(const float *, i64, i64, i64, i64, i64, i64, u64 *,
                                                u32 *, u32);

// floor() of the correctly rounded log2(x) for normal x > 0: ilogb(x), or one
// more when log2(x) lies within half a unit in the last place below the next
// integer (so that it rounds up to it).
__device__ __forceinline__ int floor_log2_rounded(double x) {
    const int e = ilogb(x);
    const double top = ldexp(1.0, e + 1);
    const double distance = ((top - x) / top) * 1.4426950408889634;   // ~ (e+1) - log2(x)
    const double target = double(e + 1);
    const double gap = target - nextafter(target, -INFINITY);
    return distance < 0.5 * gap ? e + 1 : e;
}

// INT: scale = (max > 0 ? max : 1) / upper, at least the smallest FP64
// subnormal.  BFP (bw_e > 0): e = clamp(floor(log2(max(max, DBL_MIN))),
// 1 - L, L) with L = 2^(bw_e-1) - 1, scale = 2^(e + 2 - bits).
// `narrow`: an INT operand of at most 8 bits in a wide configuration, which the reference
// quantizes in FP32 (memfast/quantization.py:9-31 picks the dtype per operand): the FP32
// scale of the FP32 peak, stored exactly as a double.
// A scale above `bound` sets MF_STATUS_RANGE in *status (may be null).
__global__ void k_group_scale_f64(const u64 *work, i64 groups, int bits, int bw_e, double upper,
                                  int narrow, double *scale, double bound, u32 *status) {
    bool large = false;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < groups;
         i += i64(gridDim.x) * blockDim.x) {
        const double peak = __longlong_as_double(static_cast<long long>(work[i]));
        double s;
        if (narrow && !bw_e) {
            s = double(group_scale(float(peak), float(upper)));
        } else if (bw_e) {
            const int limit = (1 << (bw_e - 1)) - 1;
            int e = floor_log2_rounded(peak > DBL_MIN ? peak : DBL_MIN);
            e = e < 1 - limit ? 1 - limit : (e > limit ? limit : e);
            s = ldexp(1.0, e + 2 - bits);
        } else {
            s = (peak > 0.0 ? peak : 1.0) / upper;
            const double tiny = __longlong_as_double(1LL);
            s = s < tiny ? tiny : s;
        }
        scale[i] = s;
        large = large || s > bound;
    }
    if (large && status) atomicOr(status, u32(MF_STATUS_RANGE));
}

// `narrow`: the FP32 code of the FP32 value and scale (see k_group_scale_f64).
__device__ __forceinline__ u32 quantize_code_f64(double x, double s, double lower, double upper,
                                                 u64 mask, int narrow) {
    if (narrow) return quantize_code(float(x), float(s), float(lower), float(upper), u32(mask));
    double c = rint(x / s);
    c = c < lower ? lower : c;
    c = c > upper ? upper : c;
    return u32(u64(i64(c)) & mask);
}

// q [n, kp] u32 codes; `scale` is the group grid, or a [k] row when fixed.
template <typename S>
__global__ void k_input_codes_f64(const S *x, i64 n, i64 k, i64 ld, i64 kp,
                                  const double *scale, i64 gr, i64 gc, i64 ncg, int fixed,
                                  double lower, double upper, u64 mask, int narrow, u32 *q) {
    const i64 total = n * kp;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 row = i / kp, col = i - row * kp;
        u32 code = 0;
        if (col < k) {
            const double s = fixed ? scale[col] : scale[(row / gr) * ncg + col / gc];
            code = quantize_code_f64(double(x[row * ld + col]), s, lower, upper, mask, narrow);
        }
        q[i] = code;
    }
}

// packed [m, p, R, C] as int64 (the checkpoint layout) and u32 (kernel copy).
template <typename S>
__global__ void k_weight_codes_f64(const S *b, i64 k, i64 o, i64 ld, int R, int C, i64 m,
                                   i64 p, const double *scale, i64 gr, i64 gc, i64 ncg,
                                   double lower, double upper, u64 mask, int narrow, i64 *packed,
                                   u32 *packed32) {
    const i64 kp = m * R, op = p * C;
    const i64 total = kp * op;
    for (i64 idx = i64(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += i64(gridDim.x) * blockDim.x) {
        // idx enumerates the packed layout, so both outputs are written in order.
        const i64 c = idx % C;
        const i64 r = (idx / C) % R;
        const i64 t = (idx / (i64(C) * R)) % p;
        const i64 i = idx / (i64(C) * R * p);
        const i64 row = i * R + r, col = t * C + c;
        u32 code = 0;
        if (row < k && col < o)
            code = quantize_code_f64(double(b[row * ld + col]), scale[(row / gr) * ncg + col / gc], lower,
                                     upper, mask, narrow);
        packed[idx] = i64(code);
        packed32[idx] = code;
    }
}

#define MF_CODES_F64_INST(S)                                                                   \
    template __global__ void k_input_codes_f64<S>(const S *, i64, i64, i64, i64, const double *,  \
                                                  i64, i64, i64, int, double, double, u64, int,  \
                                                  u32 *);                                        \
    template __global__ void k_weight_codes_f64<S>(const S *, i64, i64, i64, int, int, i64, i64, \
                                                   const double *, i64, i64, i64, double, double, \
                                                   u64, int, i64 *, u32 *);
MF_CODES_F64_INST(double)
MF_CODES_F64_INST(float)
#undef MF_CODES_F64_INST

// Per-read scales gathered at each read's first row, replicate-padded
// (memfast/quantization.py:76-79, :104-111, :133-136), for FP64 scales.
__global__ void k_input_scales_f64(i64 n, i64 k, i64 groups, int R, int P, int Gr,
                                   const double *scale, i64 gr, i64 gc, i64 ncg, int fixed,
                                   double *xscale) {
    const i64 total = n * groups;
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += i64(gridDim.x) * blockDim.x) {
        const i64 row = i / groups, g = i % groups;
        i64 col = (g / Gr) * R + (g % Gr) * P;
        col = col < k ? col : k - 1;
        xscale[i] = fixed ? scale[col] : scale[(row / gr) * ncg + col / gc];
    }
}

__global__ void k_weight_scales_f64(i64 k, i64 o, i64 groups, i64 op, int R, int P, int Gr,
                                    const double *scale, i64 gr, i64 gc, i64 ncg, double *wscale) {
    const i64 total = groups * op;
    for (i64 idx = i64(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += i64(gridDim.x) * blockDim.x) {
        const i64 g = idx / op, col = idx % op;
        i64 row = (g / Gr) * R + (g % Gr) * P;
        row = row < k ? row : k - 1;
        const i64 cc = col < o ? col : o - 1;
        wscale[idx] = scale[(row / gr) * ncg + cc / gc];
    }
}

// ---- implicit im2col for wide configurations ------------------------------
// The patch matrix of k_conv_codes (same row and column order) gathered from an FP64
// NCHW image, one element per thread: wide configurations are the rarer case, and
// their codes are 32-bit words, so the LDS byte tiling of the narrow kernel does not
// apply.

// Value of patch element (row, col) of the geometry, 0 outside the image.
__device__ __forceinline__ double conv_value_f64(const double *x, const mf_conv_geometry &g,
                                                 i64 row, i64 col) {
    const i64 plane = g.out_height * g.out_width;
    const i64 b = row / plane, l = row - b * plane;
    const i64 oh = l / g.out_width, ow = l - oh * g.out_width;
    const i64 taps = i64(g.kh) * g.kw;
    const i64 c = col / taps, rem = col - c * taps;
    const i64 i = rem / g.kw, j = rem - i * g.kw;
    const i64 ih = oh * g.sh - g.ph + i * g.dh, iw = ow * g.sw - g.pw + j * g.dw;
    if (ih < 0 || ih >= g.height || iw < 0 || iw >= g.width) return 0.0;
    return x[((b * g.channels + g.c0 + c) * g.height + ih) * g.width + iw];
}

// Group maxima |v| of the patch matrix as FP64 bit patterns into work [ceil(rows/gr), ncg]
// (cleared); a non-finite gathered value sets `flag`.
__global__ void k_conv_group_max_f64(const double *x, const mf_conv_geometry g, i64 K, i64 gr,
                                     i64 gc, i64 ncg, u64 *work, u32 *status, u32 flag) {
    const i64 rows = g.n * g.out_height * g.out_width;
    bool finite = true;
    for (i64 e = i64(blockIdx.x) * blockDim.x + threadIdx.x; e < rows * K;
         e += i64(gridDim.x) * blockDim.x) {
        const i64 row = e / K, col = e - row * K;
        const double v = fabs(conv_value_f64(x, g, row, col));
        finite = finite && v <= DBL_MAX;
        const u64 bits = u64(__double_as_longlong(v));
        if (bits)
            atomicMax(reinterpret_cast<unsigned long long *>(&work[(row / gr) * ncg + col / gc]),
                      static_cast<unsigned long long>(bits));
    }
    if (!finite && status) atomicOr(status, flag);
}

// Codes q [rows, kp] (zero past K) with group scales [ceil(rows/gr), ncg], or with a
// fixed per-column scale [K] (`fixed`); a non-finite gathered value sets `flag`.
__global__ void k_conv_codes_f64(const double *x, const mf_conv_geometry g, i64 K, i64 kp,
                                 const double *scale, i64 gr, i64 gc, i64 ncg, int fixed,
                                 double lower, double upper, u64 mask, int narrow, u32 *q,
                                 u32 *status, u32 flag) {
    const i64 rows = g.n * g.out_height * g.out_width;
    bool finite = true;
    for (i64 e = i64(blockIdx.x) * blockDim.x + threadIdx.x; e < rows * kp;
         e += i64(gridDim.x) * blockDim.x) {
        const i64 row = e / kp, col = e - row * kp;
        u32 code = 0;
        if (col < K) {
            const double v = conv_value_f64(x, g, row, col);
            finite = finite && fabs(v) <= DBL_MAX;
            const double s = fixed ? scale[col] : scale[(row / gr) * ncg + col / gc];
            code = quantize_code_f64(v, s, lower, upper, mask, narrow);
        }
        q[e] = code;
    }
    if (!finite && status) atomicOr(status, flag);
}

}  // namespace mf
