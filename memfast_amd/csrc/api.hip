// extern "C" entry points of libmemfast_hip.so (declared in include/memfast_hip.h).
//
// Host side of the gfx950 engine: argument validation, kernel selection, the
// ideal-device MFMA plan, launches on the caller's stream and error strings.
// Nothing here allocates device memory; the caller owns every buffer.
#include <algorithm>
#include <atomic>
#include <cfloat>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <thread>
#include <utility>
#include <vector>

#include "mf_kernels.h"

#ifndef MF_SOURCE_HASH
#define MF_SOURCE_HASH "unknown"
#endif

namespace mf {

__global__ void k_rng(const u64 *address, i64 count, u64 seed, u32 stream, int kind, float two_pi,
                      float *out) {
    for (i64 i = i64(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += i64(gridDim.x) * blockDim.x)
        out[i] = kind ? normal(address[i], seed, stream, two_pi) : uniform(address[i], seed, stream);
}

// ---------------------------------------------------------------------------
thread_local char g_error[1024] = "";

// Read-kernel timing for benchmarks: event pairs recorded around the main read
// kernel of each mf_mm call while enabled.  The event lists are guarded by a mutex;
// a call that must not create events (mf_mm_static) turns timing off for its own
// thread only.
struct ProfileState {
    std::atomic<bool> enabled{false};
    std::mutex lock;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pending, spare;
};
ProfileState g_profile;
thread_local bool g_profile_off = false;

bool profiling() { return g_profile.enabled.load(std::memory_order_relaxed) && !g_profile_off; }

std::pair<hipEvent_t, hipEvent_t> profile_pair() {
    {
        std::lock_guard<std::mutex> guard(g_profile.lock);
        if (!g_profile.spare.empty()) {
            auto pair = g_profile.spare.back();
            g_profile.spare.pop_back();
            return pair;
        }
    }
    std::pair<hipEvent_t, hipEvent_t> pair{nullptr, nullptr};
    if (hipEventCreate(&pair.first) != hipSuccess || hipEventCreate(&pair.second) != hipSuccess)
        return {nullptr, nullptr};
    return pair;
}

void profile_push(std::pair<hipEvent_t, hipEvent_t> pair) {
    std::lock_guard<std::mutex> guard(g_profile.lock);
    g_profile.pending.push_back(pair);
}

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(MF_E_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
    return MF_OK;
}

unsigned grid_for(i64 total, int block = 256) {
    i64 blocks = (total + block - 1) / block;
    if (blocks < 1) blocks = 1;
    if (blocks > 65536 * 8) blocks = 65536 * 8;
    return unsigned(blocks);
}

int check_config(const mf_config *cfg) {
    if (!cfg) return fail(MF_E_INVALID, "config descriptor is NULL");
    if (cfg->abi_version != MF_ABI_VERSION)
        return fail(MF_E_INVALID, "config ABI version %d, library expects %d", cfg->abi_version,
                    MF_ABI_VERSION);
    if (cfg->rows < 1 || cfg->cols < 4 || cfg->cols % 4 || cfg->read_rows < 1 ||
        cfg->read_rows > cfg->rows || cfg->reads != (cfg->rows + cfg->read_rows - 1) / cfg->read_rows)
        return fail(MF_E_INVALID, "invalid array geometry");
    if (cfg->n_in < 1 || cfg->n_in > MF_MAX_SLICES || cfg->n_w < 1 || cfg->n_w > MF_MAX_SLICES)
        return fail(MF_E_INVALID, "invalid slice counts");
    if (cfg->activation_bits < 2 || cfg->activation_bits > 32 || cfg->weight_bits < 2 ||
        cfg->weight_bits > 32)
        return fail(MF_E_INVALID, "precisions must be 2..32 bits");
    const bool wide = cfg->activation_bits > 8 || cfg->weight_bits > 8 || cfg->bw_e != 0;
    if (bool(cfg->wide) != wide) return fail(MF_E_INVALID, "descriptor wide flag is inconsistent");
    return MF_OK;
}

// Narrow (u8 codes, FP32 scales) and wide (u32 codes, FP64 scales) entry points.
int check_narrow(const mf_config *cfg) {
    const int status = check_config(cfg);
    if (status) return status;
    if (cfg->wide) return fail(MF_E_INVALID, "wide configuration: use the *_wide entry point");
    return MF_OK;
}

int check_wide(const mf_config *cfg) {
    const int status = check_config(cfg);
    if (status) return status;
    if (!cfg->wide) return fail(MF_E_INVALID, "narrow configuration: use the u8 entry point");
    return MF_OK;
}

int ceil_log2_torch(i64 x) {
    // c10 utils::CeilLog2 as used by the CPU sum kernel.
    if (x <= 2) return 1;
    int bits = 0;
    u64 v = u64(x - 1);
    while (v) { ++bits; v >>= 1; }
    return bits;
}

int level_power(i64 size) {
    const int lp = ceil_log2_torch(size) / 4;
    return lp > 4 ? lp : 4;
}

bool needs_conductances(const mf_config *cfg) {
    return cfg->has_write || cfg->has_saf ||
           (cfg->has_read && cfg->read_mode != MF_READ_OUTPUT);
}

int restore_planes(const mf_config *cfg) {
    return (cfg->has_read && cfg->read_mode == MF_READ_SLICE_PAIR) ? cfg->n_in : 1;
}

// Whether every output column uses the plain cascade of torch's sum.
bool all_cascade_columns(int C, i64 p) {
    for (i64 first = 0; first < p; first += 2) {
        const i64 wc = ((p - first) < 2 ? (p - first) : 2) * C;
        const i64 span = wc >= 8 ? 32 : 4;
        if (wc % span) return false;
    }
    return true;
}

int byte_mask(int shift, int mask, bool sign_slice) {
    int m = (mask << shift) & 0xFF;
    if (sign_slice) m |= (0xFF << shift) & 0xFF;
    return m;
}

u32 replicate(int m) { return u32(m) * 0x01010101u; }

// Natural operand mask of one slice: masked two's complement bytes whose int8
// value is factor*digit (sign-extended bits included for codes narrower than 8).
struct SliceForm {
    u32 nat;
};

SliceForm slice_form(int shift, int mask, bool sign_slice, int bits) {
    SliceForm f{};
    f.nat = replicate(byte_mask(shift, mask, sign_slice && bits < 8));
    return f;
}

// Ideal-device MFMA eligibility and plan.  Returns false (with reason) when the
// general kernel must be used.
bool build_ideal_plan(const mf_config *cfg, i64 m, i64 p, IdealPlan *plan, SlotTests *xtests,
                      SlotTests *wtests, int *ks, const char **why) {
    if (cfg->wide) { *why = "wide codes"; return false; }
    if (cfg->has_write || cfg->has_read || cfg->has_vnoise || cfg->has_nonlinear || cfg->has_saf ||
        cfg->has_drift) {
        *why = "device effects enabled";
        return false;
    }
    if (!cfg->weight_signed) { *why = "unsigned weights"; return false; }
    if (cfg->n_in > IDEAL_MAX_CA || cfg->n_w > IDEAL_MAX_CW) { *why = "too many slices"; return false; }
    if (cfg->read_rows % 32 || cfg->rows % cfg->read_rows || cfg->read_rows > 64) {
        *why = "rows_per_read must be 32 or 64 and divide the array rows";
        return false;
    }
    const i64 G = m * cfg->reads;
    if (G >= 4096) { *why = "more than 4095 reads per output"; return false; }
    if (!all_cascade_columns(cfg->cols, p)) { *why = "interleaved summation columns"; return false; }
    const int P = cfg->read_rows;
    // Closed-form exactness: FP32 (or FP64) current error stays below 1/4 count.
    const double unit_err = cfg->precise ? std::ldexp(1.0, -53) : std::ldexp(1.0, -24);
    const double span = cfg->precise ? cfg->d_span : double(cfg->f_span);
    const double high = cfg->precise ? cfg->d_high : double(cfg->f_high);
    double bound_abs = 0.0;
    for (int a = 0; a < cfg->n_in; ++a)
        for (int w = 0; w < cfg->n_w; ++w) {
            const double ma = cfg->in_mask[a], mw = cfg->w_mask[w];
            double zcap = P * ma * mw;
            if (zcap > cfg->adc_max[w] + 1.0) zcap = cfg->adc_max[w] + 1.0;
            const double rel = (P + 16.0 + mw * high / span) * unit_err;
            if (zcap * rel > bound_abs) bound_abs = zcap * rel;
        }
    if (bound_abs >= 0.25) { *why = "FP32 currents may move ADC counts"; return false; }
    double fa_sum = 0.0, fw_sum = 0.0;
    for (int a = 0; a < cfg->n_in; ++a) fa_sum += std::fabs(double(cfg->in_factor[a]));
    for (int w = 0; w < cfg->n_w; ++w)
        fw_sum += std::fabs(double(cfg->w_factor[w])) * cfg->adc_max[w];
    if (fa_sum * fw_sum >= 2147483647.0) { *why = "slice totals exceed int32"; return false; }

    memset(plan, 0, sizeof(*plan));
    // A pair is clamp-free when even P rows of full digits stay within max_w.
    bool is_free[MF_MAX_SLICES][MF_MAX_SLICES];
    for (int w = 0; w < cfg->n_w; ++w)
        for (int a = 0; a < cfg->n_in; ++a)
            is_free[a][w] = i64(P) * cfg->in_mask[a] * cfg->w_mask[w] <= cfg->adc_max[w];
    SliceForm xf[MF_MAX_SLICES], wf[MF_MAX_SLICES];
    for (int a = 0; a < cfg->n_in; ++a)
        xf[a] = slice_form(cfg->in_shift[a], cfg->in_mask[a], a == cfg->n_in - 1,
                           cfg->activation_bits);
    for (int w = 0; w < cfg->n_w; ++w)
        wf[w] = slice_form(cfg->w_shift[w], cfg->w_mask[w], w == cfg->n_w - 1,
                           cfg->weight_bits);
    // Clamp-candidate grid: slot cw * 8 + ca (a weight slice's slots are adjacent).
    int ca_of[MF_MAX_SLICES], cw_of[MF_MAX_SLICES];
    for (int a = 0; a < cfg->n_in; ++a) {
        ca_of[a] = -1;
        for (int w = 0; w < cfg->n_w; ++w)
            if (!is_free[a][w]) { ca_of[a] = plan->n_ca++; break; }
        if (ca_of[a] >= 0) {
            plan->ca_xnat[ca_of[a]] = xf[a].nat;
            plan->ca_factor[ca_of[a]] = int(cfg->in_factor[a]);
        }
    }
    for (int w = 0; w < cfg->n_w; ++w) {
        cw_of[w] = -1;
        for (int a = 0; a < cfg->n_in; ++a)
            if (!is_free[a][w]) { cw_of[w] = plan->n_cw++; break; }
        if (cw_of[w] >= 0) {
            plan->cw_wnat[cw_of[w]] = wf[w].nat;
            plan->cw_limit[cw_of[w]] = int(cfg->w_factor[w] * cfg->adc_max[w]);
        }
    }
    memset(xtests, 0, sizeof(*xtests));
    memset(wtests, 0, sizeof(*wtests));
    for (int a = 0; a < cfg->n_in; ++a)
        for (int w = 0; w < cfg->n_w; ++w) {
            if (is_free[a][w]) continue;
            const int slot = cw_of[w] * 8 + ca_of[a];
            plan->exists |= uint64_t(1) << slot;
            if ((cfg->in_factor[a] < 0) != (cfg->w_factor[w] < 0))
                plan->cw_negative_ca[cw_of[w]] |= 1u << ca_of[a];
            // S <= Mw * sum_r da  and  S <= Ma * sum_r dw.
            xtests->exists |= uint64_t(1) << slot;
            xtests->slice[slot] = a;
            xtests->thr[slot] = cfg->adc_max[w] / cfg->w_mask[w];
            wtests->exists |= uint64_t(1) << slot;
            wtests->slice[slot] = w;
            wtests->thr[slot] = cfg->adc_max[w] / cfg->in_mask[a];
        }
    *ks = P / 32;
    return true;
}

i64 align256(i64 x) { return (x + 255) / 256 * 256; }

void ideal_workspace(const mf_config *cfg, i64 n, i64 m, i64 p, i64 *xbytes, i64 *wbytes) {
    const i64 G = m * cfg->reads;
    *xbytes = align256((n + 63) / 64 * G * 8);
    *wbytes = align256((p * cfg->cols + 31) / 32 * G * 8);
}

// Whether every conductance term k1[w] * (g - L) fits fp16 with margin.  The
// sampled normals are sqrt(-2 ln u) cos(2 pi v) with u >= 2^-25, so |z| < 5.9;
// programming and shared read noise multiply g by at most exp(5.9 sigma) each,
// drift by the drift factor, and stuck-at faults set L or H.
bool fp16_terms_fit(const mf_config *cfg) {
    const double zmax = 5.9;
    double high = cfg->f_high;
    if (cfg->has_write) high *= std::exp(zmax * double(cfg->f_write));
    if (cfg->has_read) high *= std::exp(zmax * double(cfg->f_read));
    if (cfg->has_drift && cfg->f_drift > 1.0f) high *= double(cfg->f_drift);
    const double low = cfg->f_low;
    const double span = std::max(high - low, low);   // |g - L| for g in [0, high]
    for (int w = 0; w < cfg->n_w; ++w) {
        const double k1 = double(float(cfg->d_voltage * double(cfg->w_mask[w]) * cfg->d_inv_unit));
        if (!(k1 * span < 16384.0)) return false;
    }
    return true;
}

// Noisy-device MFMA eligibility and plan (noisy_mfma.hip): FP32 currents,
// conductances that do not depend on the input slice (no slice_pair read
// noise), no voltage or output-mode read noise, reads of 32 or 64 rows that
// tile the array, plain cascade columns, FP32-exact totals.
// Planes of conductance terms of the noisy read: slice_pair read noise gives every
// input slice its own read of each cell.
int noisy_term_planes(const mf_config *cfg) {
    if (cfg->has_read && cfg->read_mode == MF_READ_SLICE_PAIR) return cfg->n_in;
    if (cfg->has_read && cfg->read_mode == MF_READ_OUTPUT) return 2;
    return 1;
}

bool build_noisy_plan(const mf_config *cfg, i64 m, i64 p, NoisyPlan *plan, int *ks,
                      const char **why) {
    if (cfg->wide) { *why = "wide codes"; return false; }
    if (cfg->precise) { *why = "FP64 currents"; return false; }
    const bool output_noise = cfg->has_read && cfg->read_mode == MF_READ_OUTPUT;
    if (output_noise) {
        // Squared digits must be exact in fp16 and the noise addresses of a wave's 32
        // columns must share one array tile.
        if (cfg->cols % 32) { *why = "output-mode read noise needs array columns in multiples of 32"; return false; }
        for (int a = 0; a < cfg->n_in; ++a)
            if (cfg->in_mask[a] > 15) { *why = "output-mode read noise with input digits above 15"; return false; }
    }
    if ((cfg->read_rows != 32 && cfg->read_rows != 64) || cfg->rows % cfg->read_rows) {
        *why = "rows_per_read must be 32 or 64 and divide the array rows";
        return false;
    }
    if (cfg->read_rows == 64 && cfg->n_in > 5) { *why = "more than 5 input slices at 64-row reads"; return false; }
    if (cfg->n_in > 8 || cfg->n_w > 8) { *why = "too many slices"; return false; }
    const i64 G = m * cfg->reads;
    if (G >= 4096) { *why = "more than 4095 reads per output"; return false; }
    if (!all_cascade_columns(cfg->cols, p)) { *why = "interleaved summation columns"; return false; }
    double fa_sum = 0.0, fw_sum = 0.0;
    for (int a = 0; a < cfg->n_in; ++a) fa_sum += std::fabs(double(cfg->in_factor[a]));
    for (int w = 0; w < cfg->n_w; ++w) fw_sum += std::fabs(double(cfg->w_factor[w])) * cfg->adc_max[w];
    if (fa_sum * fw_sum >= 16777216.0) { *why = "slice totals exceed FP32 integers"; return false; }
    if (!fp16_terms_fit(cfg)) { *why = "conductance terms beyond the fp16 range"; return false; }
    memset(plan, 0, sizeof(*plan));
    plan->n_in = cfg->n_in;
    plan->n_w = cfg->n_w;
    plan->planes = noisy_term_planes(cfg);
    plan->out_noise = output_noise ? 1 : 0;
    plan->out_mean = cfg->f_out_mean;
    plan->two_pi = cfg->f_two_pi;
    for (int w = 0; w < cfg->n_w; ++w) {
        plan->k1[w] = float(cfg->d_voltage * double(cfg->w_mask[w]) * cfg->d_inv_unit);
        plan->top[w] = float(cfg->adc_max[w]);
        plan->alpha[w] = cfg->has_nonlinear ? cfg->f_alpha_over_max[w] : 0.0f;
        plan->fw[w] = float(cfg->w_factor[w]);
        plan->kl[w] = plan->k1[w] * cfg->f_low;
        plan->qk[w] = float(cfg->d_voltage * cfg->d_inv_unit);
        const float mw = float(cfg->w_mask[w]);
        plan->out_var[w] = mw * mw * cfg->f_out_var;
    }
    i64 factor_sum = 0;
    for (int a = 0; a < cfg->n_in; ++a) {
        plan->fa[a] = float(cfg->in_factor[a]);
        plan->in_shift[a] = cfg->in_shift[a];
        plan->in_mask4[a] = u32(cfg->in_mask[a]) * 0x01010101u;
        for (int w = 0; w < cfg->n_w; ++w) factor_sum += cfg->in_factor[a] * cfg->w_factor[w];
    }
    plan->bias = u32(0) - u32(u64(factor_sum) * 0x400000u);
    for (int a = 0; a < cfg->n_in; ++a)
        for (int w = 0; w < cfg->n_w; ++w) {
            if (std::abs(double(cfg->in_factor[a]) * double(cfg->w_factor[w])) >= 8388608.0) {
                *why = "slice factor product beyond 24 bits";
                return false;
            }
            const int f = int(plan->fa[a] * plan->fw[w]);
            plan->f24[a][w] = u32(int(u32(f) << 8) >> 8);
        }
    for (int w = 0; w < cfg->n_w; ++w) plan->top_magic[w] = 12582912.0f + plan->top[w];
    *ks = cfg->read_rows / 16;
    return true;
}

// Bytes of conductance terms per 32-column block: NOISY_TERMS fp16 terms per cell,
// weight slice and term plane.
i64 noisy_block_bytes(const mf_config *cfg, i64 m) {
    return i64(cfg->n_w) * noisy_term_planes(cfg) * 32 * m * cfg->rows * NOISY_TERMS * 2;
}

bool noisy_extent_ok(i64 n, i64 m, const mf_config *cfg) {
    const i64 kp = m * cfg->rows;
    return 64 * kp <= 0x7FFFFFFF && (n + 63) / 64 <= 0x7FFFFFFF;
}

// Blocks of the noisy read (64 columns x 64 vectors each) below which the
// reads are split across blocks (grid z): each block writes integer slice
// totals for its reads and k_restore_sum_f32 restores and sums them.
constexpr i64 NOISY_SPLIT_BELOW = 512;

i64 noisy_terms_bytes(const mf_config *cfg, i64 m, i64 p) {
    return (p * cfg->cols + 63) / 64 * 2 * noisy_block_bytes(cfg, m);
}

// Read chunks of a split read (1: not split).  `requested` (the variant's
// split field) overrides the automatic choice: 1 never splits, s >= 2 splits
// into s chunks (at most one per read).
i64 noisy_split(const mf_config *cfg, i64 n, i64 m, i64 p, int requested = 0) {
    const i64 G = m * cfg->reads;
    i64 z;
    if (requested > 0) {
        z = requested;
    } else {
        const i64 blocks = (p * cfg->cols + 63) / 64 * ((n + 63) / 64);
        if (G < 2 || blocks >= NOISY_SPLIT_BELOW) return 1;
        z = (NOISY_SPLIT_BELOW + blocks - 1) / blocks;
    }
    if (z > G) z = G;
    if (z < 2) return 1;
    const i64 step = (G + z - 1) / z;
    return (G + step - 1) / step;
}

i64 noisy_scratch_bytes(const mf_config *cfg, i64 n, i64 m, i64 p, int requested = 0) {
    if (noisy_split(cfg, n, m, p, requested) < 2) return 0;
    return align256(n * m * cfg->reads * p * cfg->cols * 4);
}

// Operand terms per input value with voltage variation: x hi and lo, and with output-mode
// read noise RN(x * x) hi and lo.
int voltage_terms(const mf_config *cfg) {
    return cfg->has_read && cfg->read_mode == MF_READ_OUTPUT ? 4 : 2;
}

// Voltage-variation input operands (k_voltage_terms): hi and lo fp16 per input
// slice, vector (in blocks of 32) and physical row.  They sit at the end of the
// workspace, so the conductance terms keep their place (and stay reusable) whatever
// the vector count.
i64 noisy_voltage_bytes(const mf_config *cfg, i64 n, i64 m) {
    const i64 vectors = (n + 31) / 32 * 32;
    return cfg->has_vnoise ? align256(voltage_terms(cfg) * i64(cfg->n_in) * vectors * m *
                                      cfg->rows * 2)
                           : 0;
}

// Whether a split noisy read runs k_noisy_pairs (one wave per weight slice, 32 vectors):
// batches of at most 32 vectors, where the four-wave tile (64 vectors, the slices one
// after another) would leave half its waves idle; plain and S-curve reads (no voltage,
// slice_pair or output-mode noise).
bool noisy_small_tile(const mf_config *cfg, i64 n) {
    const bool per_read_noise = cfg->has_vnoise ||
                                (cfg->has_read && cfg->read_mode != MF_READ_SHARED);
    return n <= 32 && !per_read_noise;
}

// Fields of the `variant` word (include/memfast_hip.h).
int variant_tile(int32_t v) { return v & 0xFF; }
int variant_split(int32_t v) { return (v >> MF_MM_SPLIT_SHIFT) & 0xF; }
int variant_tier(int32_t v) { return (v >> MF_MM_TIER_SHIFT) & 0xF; }
bool variant_valid(int32_t v) {
    const int32_t known = 0xFF | MF_MM_REUSE_TERMS | (0xF << MF_MM_SPLIT_SHIFT) |
                          (0xF << MF_MM_TIER_SHIFT);
    return (v & ~known) == 0 && variant_tile(v) <= 2 && variant_tier(v) <= 3;
}

// Conductance terms depend on the read event only through shared read noise.
bool terms_event_independent(const mf_config *cfg) { return !cfg->has_read; }

// Split conductances and run k_noisy over column chunks that fit `bytes` of
// workspace (at least 64 columns).  g: optional injected conductances.
// reuse: the workspace already holds this program's event-independent terms
// for every column (a previous call with the same codes, seed and config).
// ocols, g_run: output columns computed and reads executed (the logical matrix;
// columns past ocols are left unwritten, reads past g_run hold only padding).
int launch_noisy(const mf_config *cfg, const NoisyPlan &plan, int ks, const u8 *q,
                 const float *xscale, i64 n, i64 m, const u8 *packed_t, const float *wscale, i64 p,
                 const float *g, u32 seed, u64 event, float *out, i64 ldo, void *workspace,
                 i64 bytes, int totals, u32 *status, hipStream_t s, bool reuse = false,
                 i64 ocols = -1, i64 g_run = -1, int split_request = 0,
                 const float **split_totals = nullptr, bool *split_restored = nullptr) {
    const i64 kp = m * cfg->rows, ncols = p * cfg->cols, G = m * cfg->reads;
    if (ocols < 0) ocols = ncols;
    if (g_run < 0) g_run = G;
    const i64 vbytes = noisy_voltage_bytes(cfg, n, m);
    if (bytes < vbytes) return fail(MF_E_RESOURCE, "workspace below the voltage operands");
    const uint4 *volt = nullptr;
    if (vbytes) {
        // Aligned down to 256 bytes at the end of the workspace.
        const i64 at = ((bytes - vbytes) / 256) * 256;
        uint4 *operands = reinterpret_cast<uint4 *>(static_cast<char *>(workspace) + at);
        hipLaunchKernelGGL(k_voltage_terms<u8>,
                           dim3(grid_for(i64(cfg->n_in) * ((n + 31) / 32 * 32) * (kp / 8))),
                           dim3(256), 0, s, *cfg, q, n, m, seed, event,
                           int(voltage_terms(cfg) == 4), operands);
        volt = operands;
        bytes = at;
    }
    const i64 per_block = noisy_block_bytes(cfg, m);
    // Split read (fused output only, when the whole program's terms fit).
    const i64 split = totals ? 1 : noisy_split(cfg, n, m, p, split_request);
    const i64 full = noisy_terms_bytes(cfg, m, p);
    const i64 scratch = noisy_scratch_bytes(cfg, n, m, p, split_request);
    const bool use_split = split > 1 && bytes >= full + scratch;
    if (split > 1 && split_request > 1 && !use_split)
        return fail(MF_E_RESOURCE,
                    "workspace of %lld bytes below the %lld a %lld-way read split needs",
                    static_cast<long long>(bytes), static_cast<long long>(full + scratch),
                    static_cast<long long>(split));
    const i64 max_cb = use_split ? full / per_block : (bytes / per_block) / 2 * 2;
    if (max_cb < 2) return fail(MF_E_RESOURCE, "workspace below one 64-column chunk");
    reuse = reuse && g == nullptr && terms_event_independent(cfg) && max_cb * 32 >= ocols;
    uint4 *gs = static_cast<uint4 *>(workspace);
    float *partial = use_split ? reinterpret_cast<float *>(static_cast<char *>(workspace) + full)
                               : nullptr;
    for (i64 c_begin = 0; c_begin < ocols; c_begin += max_cb * 32) {
        const i64 cols = (ocols - c_begin) < max_cb * 32 ? (ocols - c_begin) : max_cb * 32;
        const i64 CB = (cols + 63) / 64 * 2;
        const i64 threads = i64(cfg->n_w) * CB * G * ks * 64;
        if (reuse) {
            // terms already in place
        } else if (ks == 2) {
            hipLaunchKernelGGL(k_split_conductances<2>, dim3(grid_for(threads)), dim3(256), 0, s, *cfg,
                               packed_t, g, m, p, ncols, seed, event, c_begin, CB, plan, gs);
        } else {
            hipLaunchKernelGGL(k_split_conductances<4>, dim3(grid_for(threads)), dim3(256), 0, s, *cfg,
                               packed_t, g, m, p, ncols, seed, event, c_begin, CB, plan, gs);
        }
        NoisyArgs args{};
        args.q = q;
        args.gs = gs;
        args.xscale = xscale;
        args.wscale = wscale;
        args.out = out;
        args.status = status;
        args.n = n;
        args.kp = kp;
        args.G = G;
        args.ldo = ldo;
        args.ldws = ncols;
        args.ncols = ocols;
        args.c_begin = c_begin;
        args.CB = CB;
        args.totals = totals;
        args.g_begin = 0;
        args.g_end = g_run;
        args.g_step = g_run;
        args.volt = volt;
        args.read_seed = event_seed(seed, event);
        args.C = cfg->cols;
        unsigned gz = 1;
        if (use_split) {
            args.totals = 1;
            args.out = partial;
            args.ldo = ncols;
            args.g_step = (g_run + split - 1) / split;
            gz = unsigned((g_run + args.g_step - 1) / args.g_step);
        }
        const bool nl = cfg->has_nonlinear != 0;
        const bool slice = plan.planes > 1 && !plan.out_noise;
        // A split read of at most 32 vectors runs k_noisy_pairs: one read per workgroup,
        // one wave per weight slice.
        const bool pairs = use_split && noisy_small_tile(cfg, n);
        const dim3 grid = pairs ? dim3{unsigned(CB), unsigned((n + 31) / 32), unsigned(g_run)}
                                : dim3{unsigned((n + 63) / 64), unsigned(CB / 2), gz};
        const dim3 block{pairs ? unsigned(64 * cfg->n_w) : 256u};
        if (pairs) {
            args.g_step = 1;
            args.restored = 1;   // the values (float(T) * xs) * ws; consumers only sum them
        }
        // Benchmark timing brackets the read kernel alone (not the conductance split).
        std::pair<hipEvent_t, hipEvent_t> timing{nullptr, nullptr};
        if (profiling() && (timing = profile_pair()).first) hipEventRecord(timing.first, s);
#define MF_NOISY_LAUNCH1(KS, NA, NL, VN, SL, ON) \
    hipLaunchKernelGGL((k_noisy<KS, NA, NL, VN, SL, ON>), grid, block, 0, s, plan, args)
#define MF_NOISY_LAUNCH2(KS, NA, VN, SL, ON)                    \
    {                                                          \
        if (nl) MF_NOISY_LAUNCH1(KS, NA, true, VN, SL, ON);    \
        else MF_NOISY_LAUNCH1(KS, NA, false, VN, SL, ON);      \
    }
#define MF_NOISY_LAUNCH(KS, NA)                                                                \
    {                                                                                         \
        if (pairs && nl)                                                                      \
            hipLaunchKernelGGL((k_noisy_pairs<KS, NA, true>), grid, block, 0, s, plan, args);  \
        else if (pairs)                                                                       \
            hipLaunchKernelGGL((k_noisy_pairs<KS, NA, false>), grid, block, 0, s, plan, args); \
        else if (plan.out_noise && volt) MF_NOISY_LAUNCH2(KS, NA, true, false, true)          \
        else if (plan.out_noise) MF_NOISY_LAUNCH2(KS, NA, false, false, true)                 \
        else if (volt && slice) MF_NOISY_LAUNCH2(KS, NA, true, true, false)                   \
        else if (volt) MF_NOISY_LAUNCH2(KS, NA, true, false, false)                           \
        else if (slice) MF_NOISY_LAUNCH2(KS, NA, false, true, false)                          \
        else MF_NOISY_LAUNCH2(KS, NA, false, false, false)                                    \
    }
        if (ks == 4) MF_NOISY_LAUNCH(4, 5)
        else if (cfg->n_in <= 5) MF_NOISY_LAUNCH(2, 5)
        else MF_NOISY_LAUNCH(2, 8)
#undef MF_NOISY_LAUNCH
#undef MF_NOISY_LAUNCH2
#undef MF_NOISY_LAUNCH1
        if (timing.first) {
            hipEventRecord(timing.second, s);
            profile_push(timing);
        }
    }
    // With split_totals the caller restores and sums a split read's totals [n, G, ncols]
    // itself (null when the read wrote `out`).
    const bool restored = use_split && noisy_small_tile(cfg, n);   // k_noisy_pairs restored
    if (split_totals) *split_totals = use_split ? partial : nullptr;
    if (split_restored) *split_restored = restored;
    if (use_split && !split_totals)
        hipLaunchKernelGGL(k_restore_sum_f32, dim3(grid_for(n * ocols)), dim3(256), 0, s, partial, n,
                           G, g_run, ncols, ocols, xscale, wscale, ncols, out, ldo, level_power(G),
                           int(restored), status);
    return check_launch("noisy MFMA read");
}

// Whether every output column of a wide read uses the plain cascade of torch's
// FP64 sum (columns beyond 16 * floor(width*C / 16) of a two-tile chunk are
// interleaved).
bool all_cascade_columns_wide(int C, i64 p) {
    for (i64 first = 0; first < p; first += 2) {
        const i64 wc = ((p - first) < 2 ? (p - first) : 2) * C;
        if (wc % 16) return false;
    }
    return true;
}

// Planes of conductance terms per weight slice of the wide read: one per input slice with
// slice_pair read noise (an independent read factor per cell and input slice), else one.
int wide_term_planes(const mf_config *cfg) {
    return cfg->has_read && cfg->read_mode == MF_READ_SLICE_PAIR ? cfg->n_in : 1;
}

// Wide noisy-device MFMA eligibility and plan (noisy_wide.hip): the narrow
// kernel's device model, input codes of at most 16 bits with digits up to 255,
// fewer than 256 reads, exact int32 totals.
bool build_noisy_wide_plan(const mf_config *cfg, i64 m, i64 p, NoisyWidePlan *plan, int *ks,
                           const char **why) {
    if (!cfg->wide) { *why = "narrow codes"; return false; }
    if (cfg->precise) { *why = "FP64 currents"; return false; }
    if (cfg->has_read && cfg->read_mode == MF_READ_OUTPUT) { *why = "output-mode read noise"; return false; }
    if ((cfg->read_rows != 32 && cfg->read_rows != 64) || cfg->rows % cfg->read_rows) {
        *why = "rows_per_read must be 32 or 64 and divide the array rows";
        return false;
    }
    if (cfg->activation_bits > 16) { *why = "input codes wider than 16 bits"; return false; }
    if (!fp16_terms_fit(cfg)) { *why = "conductance terms beyond the fp16 range"; return false; }
    if (cfg->n_in > WIDE_MFMA_MAX_A || cfg->n_w > WIDE_MFMA_MAX_W ||
        cfg->n_w * NOISY_TERMS * (cfg->read_rows / 16) > WIDE_FRAGS_LARGE) {
        *why = "too many slices";
        return false;
    }
    const i64 G = m * cfg->reads;
    if (G >= 256) { *why = "256 or more reads per output"; return false; }
    if (!all_cascade_columns_wide(cfg->cols, p)) { *why = "interleaved summation columns"; return false; }
    double fa_sum = 0.0, fw_sum = 0.0;
    for (int a = 0; a < cfg->n_in; ++a) {
        if (cfg->in_mask[a] > 255) { *why = "input digits above 255"; return false; }
        fa_sum += std::fabs(double(cfg->in_factor[a]));
    }
    for (int w = 0; w < cfg->n_w; ++w) fw_sum += std::fabs(double(cfg->w_factor[w])) * cfg->adc_max[w];
    if (fa_sum * fw_sum >= 2147483647.0) { *why = "slice totals exceed int32"; return false; }
    for (int a = 0; a < cfg->n_in; ++a)
        for (int w = 0; w < cfg->n_w; ++w)
            if (std::fabs(double(cfg->in_factor[a]) * double(cfg->w_factor[w])) >= 8388608.0) {
                *why = "slice factor products beyond 24 bits";
                return false;
            }
    memset(plan, 0, sizeof(*plan));
    plan->n_in = cfg->n_in;
    plan->n_w = cfg->n_w;
    plan->planes = wide_term_planes(cfg);
    i64 factor_sum = 0;
    for (int w = 0; w < cfg->n_w; ++w) {
        plan->k1[w] = float(cfg->d_voltage * double(cfg->w_mask[w]) * cfg->d_inv_unit);
        plan->top[w] = float(cfg->adc_max[w]);
        plan->alpha[w] = cfg->has_nonlinear ? cfg->f_alpha_over_max[w] : 0.0f;
        plan->fw[w] = int(cfg->w_factor[w]);
    }
    for (int a = 0; a < cfg->n_in; ++a) {
        plan->fa[a] = int(cfg->in_factor[a]);
        plan->in_shift[a] = cfg->in_shift[a];
        plan->in_mask2[a] = u32(cfg->in_mask[a]) * 0x00010001u;
        for (int w = 0; w < cfg->n_w; ++w) factor_sum += cfg->in_factor[a] * cfg->w_factor[w];
    }
    plan->bias = u32(0) - u32(u64(factor_sum) * 0x400000u);
    *ks = cfg->read_rows / 16;
    return true;
}

// Workspace of the wide MFMA read: 16-bit input codes, then the conductance
// terms of up to every 32-column block (NOISY_TERMS fp16 terms per cell and slice).
i64 wide_codes_bytes(i64 n, i64 m, const mf_config *cfg) { return align256(n * m * cfg->rows * 2); }
// Voltage-variation input operands of the wide read (k_voltage_terms<u32>): hi and lo
// fp16 per input slice, vector (in blocks of 32) and physical row.
i64 wide_voltage_bytes(i64 n, i64 m, const mf_config *cfg) {
    const i64 vectors = (n + 31) / 32 * 32;
    return cfg->has_vnoise ? align256(2 * i64(cfg->n_in) * vectors * m * cfg->rows * 2) : 0;
}
// Workspace of the wide read before its conductance terms: the 16-bit codes, then the
// voltage operands.
i64 wide_prefix_bytes(i64 n, i64 m, const mf_config *cfg) {
    return wide_codes_bytes(n, m, cfg) + wide_voltage_bytes(n, m, cfg);
}
i64 wide_block_bytes(const mf_config *cfg, i64 m) {
    return i64(cfg->n_w) * wide_term_planes(cfg) * 32 * m * cfg->rows * NOISY_TERMS * 2;
}

bool wide_extent_ok(i64 n, i64 m, const mf_config *cfg) {
    const i64 kp = m * cfg->rows;
    return 64 * kp <= 0x7FFFFFFF && (n + 127) / 128 <= 65535;
}

// Repack codes to 16 bits, split conductances and run k_noisy_wide over column
// chunks that fit the workspace.  g: optional injected conductances.
int launch_noisy_wide(const mf_config *cfg, const NoisyWidePlan &plan, int ks,
                      const u32 *q, const double *xscale, i64 n, i64 m, const u32 *packed,
                      const double *wscale, i64 p, const float *g, u32 seed, u64 event,
                      double *out, i64 ldo, void *workspace, i64 bytes, int totals, u32 *status,
                      hipStream_t s, int tier_request = 0) {
    const i64 kp = m * cfg->rows, ncols = p * cfg->cols, G = m * cfg->reads;
    const i64 codes_bytes = wide_codes_bytes(n, m, cfg);
    const i64 prefix = wide_prefix_bytes(n, m, cfg);
    const i64 per_block = wide_block_bytes(cfg, m);
    const i64 max_cb = (bytes - prefix) / per_block;
    if (max_cb < 2) return fail(MF_E_RESOURCE, "workspace below one 64-column chunk");
    const int frags = cfg->n_w * NOISY_TERMS * ks;
    if (frags > WIDE_FRAGS_LARGE) return fail(MF_E_RESOURCE, "too many weight slices for LDS");
    // Automatic: the smallest capacity that holds a read.
    int tier = frags > WIDE_FRAGS_SMALL ? 2 : frags > WIDE_FRAGS_TINY ? 1 : 0;
    if (tier_request > 0) {
        // A tuned schedule's LDS capacity: 24, 36 or 72 fragments per read.
        const int capacity[3] = {WIDE_FRAGS_TINY, WIDE_FRAGS_SMALL, WIDE_FRAGS_LARGE};
        if (frags > capacity[tier_request - 1])
            return fail(MF_E_RESOURCE, "LDS tier of %d fragments below a read's %d",
                        capacity[tier_request - 1], frags);
        tier = tier_request - 1;
    }
    uint16_t *q16 = static_cast<uint16_t *>(workspace);
    uint4 *volt = cfg->has_vnoise
                      ? reinterpret_cast<uint4 *>(static_cast<char *>(workspace) + codes_bytes)
                      : nullptr;
    uint4 *gs = reinterpret_cast<uint4 *>(static_cast<char *>(workspace) + prefix);
    hipLaunchKernelGGL(k_codes16, dim3(grid_for(n * kp)), dim3(256), 0, s, q, n * kp, q16);
    if (volt)
        hipLaunchKernelGGL(k_voltage_terms<u32>,
                           dim3(grid_for(i64(cfg->n_in) * ((n + 31) / 32 * 32) * (kp / 8))),
                           dim3(256), 0, s, *cfg, q, n, m, seed, event, 0, volt);
    for (i64 c_begin = 0; c_begin < ncols; c_begin += max_cb * 32) {
        const i64 cols = (ncols - c_begin) < max_cb * 32 ? (ncols - c_begin) : max_cb * 32;
        const i64 CB = (cols + 31) / 32;
        const i64 threads = CB * G * cfg->n_w * ks * 64;
        if (ks == 2)
            hipLaunchKernelGGL(k_split_wide<2>, dim3(grid_for(threads)), dim3(256), 0, s, *cfg,
                               packed, g, m, p, ncols, seed, event, c_begin, CB, plan, gs);
        else
            hipLaunchKernelGGL(k_split_wide<4>, dim3(grid_for(threads)), dim3(256), 0, s, *cfg,
                               packed, g, m, p, ncols, seed, event, c_begin, CB, plan, gs);
        NoisyWideArgs args{};
        args.q16 = q16;
        args.gs = gs;
        args.xscale = xscale;
        args.wscale = wscale;
        args.out = out;
        args.status = status;
        args.n = n;
        args.kp = kp;
        args.G = G;
        args.ldo = ldo;
        args.ldws = ncols;
        args.ncols = ncols;
        args.c_begin = c_begin;
        args.totals = totals;
        args.volt = volt;
        const dim3 grid{unsigned(CB), unsigned((n + 127) / 128), 1u};
        const bool nl = cfg->has_nonlinear != 0;
        // slice_pair read noise: a plane of terms per (weight, input) slice pair, staged in
        // LDS one input slice at a time (the kernel's SLICE form).
        const bool sl = plan.planes > 1;
#define MF_WIDE_LAUNCH2(KS, FR, SL)                                                              \
    if (volt && nl)                                                                              \
        hipLaunchKernelGGL((k_noisy_wide<KS, true, FR, true, SL>), grid, dim3(256), 0, s, plan,     \
                           args);                                                                \
    else if (volt)                                                                               \
        hipLaunchKernelGGL((k_noisy_wide<KS, false, FR, true, SL>), grid, dim3(256), 0, s, plan,    \
                           args);                                                                \
    else if (nl)                                                                                 \
        hipLaunchKernelGGL((k_noisy_wide<KS, true, FR, false, SL>), grid, dim3(256), 0, s, plan,    \
                           args);                                                                \
    else                                                                                         \
        hipLaunchKernelGGL((k_noisy_wide<KS, false, FR, false, SL>), grid, dim3(256), 0, s, plan,   \
                           args);
#define MF_WIDE_LAUNCH(KS, FR)                                                                   \
    if (sl) { MF_WIDE_LAUNCH2(KS, FR, true) } else { MF_WIDE_LAUNCH2(KS, FR, false) }
        if (ks == 4) {
            if (tier == 2) { MF_WIDE_LAUNCH(4, WIDE_FRAGS_LARGE) }
            else if (tier == 1) { MF_WIDE_LAUNCH(4, WIDE_FRAGS_SMALL) }
            else { MF_WIDE_LAUNCH(4, WIDE_FRAGS_TINY) }
        } else {
            if (tier == 2) { MF_WIDE_LAUNCH(2, WIDE_FRAGS_LARGE) }
            else if (tier == 1) { MF_WIDE_LAUNCH(2, WIDE_FRAGS_SMALL) }
            else { MF_WIDE_LAUNCH(2, WIDE_FRAGS_TINY) }
        }
#undef MF_WIDE_LAUNCH
#undef MF_WIDE_LAUNCH2
    }
    return check_launch("wide noisy MFMA read");
}

SliceLayout layout_of(const int32_t *shift, const int32_t *mask, int count) {
    SliceLayout l{};
    l.count = count;
    for (int i = 0; i < count; ++i) { l.shift[i] = shift[i]; l.mask[i] = mask[i]; }
    return l;
}

template <typename Phys>
int launch_general(const mf_config *cfg, const GeneralArgs &args, int out_kind, hipStream_t s) {
    const i64 ncols = args.width * cfg->cols;
    const i64 col_blocks = (ncols + 31) / 32;
    const i64 vec_blocks = (args.n + 7) / 8;
    if (col_blocks > 65535) return fail(MF_E_RESOURCE, "too many output columns for one launch");
    if (vec_blocks > 2147483647) return fail(MF_E_RESOURCE, "too many input vectors");
    const dim3 grid{unsigned(vec_blocks), unsigned(col_blocks), 1u};
    const bool output_noise = cfg->has_read && cfg->read_mode == MF_READ_OUTPUT;
#define MF_GENERAL_LAUNCH(WIDE)                                                                  \
    if (sizeof(Phys) == 4) {                                                                     \
        if (output_noise)                                                                        \
            hipLaunchKernelGGL((k_general<float, 2, true, WIDE>), grid, dim3(256), 0, s, *cfg,     \
                               args, out_kind);                                                  \
        else                                                                                     \
            hipLaunchKernelGGL((k_general<float, 8, false, WIDE>), grid, dim3(256), 0, s, *cfg,    \
                               args, out_kind);                                                  \
    } else {                                                                                     \
        if (output_noise)                                                                        \
            hipLaunchKernelGGL((k_general<double, 2, true, WIDE>), grid, dim3(256), 0, s, *cfg,    \
                               args, out_kind);                                                  \
        else                                                                                     \
            hipLaunchKernelGGL((k_general<double, 4, false, WIDE>), grid, dim3(256), 0, s, *cfg,   \
                               args, out_kind);                                                  \
    }
    if (cfg->wide) {
        MF_GENERAL_LAUNCH(true)
    } else {
        MF_GENERAL_LAUNCH(false)
    }
#undef MF_GENERAL_LAUNCH
    return check_launch("general read");
}

// Precise currents run on FP64 MFMA (k_general_mfma64) unless voltage variation or
// output-mode read noise needs the general kernel.
static bool precise_mfma_ok(const mf_config *cfg) {
    return cfg->precise && !cfg->has_vnoise &&
           !(cfg->has_read && cfg->read_mode == MF_READ_OUTPUT);
}

static int launch_general_mfma64(const mf_config *cfg, const GeneralArgs &args, int out_kind,
                                 hipStream_t s) {
    const i64 ncols = args.width * cfg->cols;
    const i64 col_blocks = (ncols + 15) / 16;
    const i64 vec_blocks = (args.n + 15) / 16;
    if (col_blocks > 65535) return fail(MF_E_RESOURCE, "too many output columns for one launch");
    if (vec_blocks > 2147483647) return fail(MF_E_RESOURCE, "too many input vectors");
    const dim3 grid{unsigned(vec_blocks), unsigned(col_blocks), 1u};
    const bool staged = args.planes == 1 && cfg->n_w <= MFMA64_STAGED_MAX_W;
#define MF_MFMA64_LAUNCH(WIDE, STAGED)                                                           \
    hipLaunchKernelGGL((k_general_mfma64<WIDE, STAGED>), grid, dim3(256), 0, s, *cfg, args,     \
                       out_kind)
    if (cfg->wide) {
        if (staged) MF_MFMA64_LAUNCH(true, true);
        else MF_MFMA64_LAUNCH(true, false);
    } else {
        if (staged) MF_MFMA64_LAUNCH(false, true);
        else MF_MFMA64_LAUNCH(false, false);
    }
#undef MF_MFMA64_LAUNCH
    return check_launch("precise MFMA read");
}

// The general read (fused or to totals): FP32 currents on k_general, precise ones on FP64
// MFMA where that applies and no per-pair codes are asked for, else k_general in FP64.
static int launch_general_read(const mf_config *cfg, const GeneralArgs &args, int out_kind,
                               hipStream_t s) {
    if (!cfg->precise) return launch_general<float>(cfg, args, out_kind, s);
    return precise_mfma_ok(cfg) && !args.codes ? launch_general_mfma64(cfg, args, out_kind, s)
                                               : launch_general<double>(cfg, args, out_kind, s);
}

// Group maxima |x| into work[row group][col group] (cleared): column groups and
// wide row groups by chunked reductions with few atomics, others elementwise.
static void launch_input_codes(const float *x, i64 n, i64 k, i64 ld, i64 kp, const float *scale,
                               i64 gr, i64 gc, i64 ncg, int fixed, float lower, float upper,
                               u32 mask, u8 *q, hipStream_t s) {
    const bool vec = k % 4 == 0 && kp % 4 == 0 && ld % 4 == 0 &&
                     reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(q) % 4 == 0;
    if (vec) {
        const i64 quads = n * (kp / 4);
        const unsigned grid = grid_for(quads);
        const i64 limit = i64(1) << 31;
        if (quads + i64(grid) * 256 < limit && kp < limit && gr < limit && gc < limit)
            hipLaunchKernelGGL(k_input_codes4<u32>, dim3(grid), dim3(256), 0, s, x, n, k, ld, kp,
                               scale, gr, gc, ncg, fixed, lower, upper, mask, q);
        else
            hipLaunchKernelGGL(k_input_codes4<i64>, dim3(grid), dim3(256), 0, s, x, n, k, ld, kp,
                               scale, gr, gc, ncg, fixed, lower, upper, mask, q);
    } else {
        hipLaunchKernelGGL(k_input_codes, dim3(grid_for(n * kp)), dim3(256), 0, s, x, n, k, ld, kp,
                           scale, gr, gc, ncg, fixed, lower, upper, mask, q);
    }
}

static void launch_group_max_f32(const float *x, i64 rows, i64 cols, i64 ld, i64 gr, i64 gc,
                                 i64 ncg, u32 *work, u32 *status, u32 flag, hipStream_t s) {
    const i64 chunks = (rows + COL_CHUNK_ROWS - 1) / COL_CHUNK_ROWS;
    const i64 row_chunks = (cols + ROW_CHUNK_COLS - 1) / ROW_CHUNK_COLS;
    const bool vec_ok = cols % 4 == 0 && ld % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (gr == 1 && gc >= 64 && (rows + 3) / 4 <= 65535 && row_chunks <= 2147483647) {
        hipLaunchKernelGGL((k_row_group_max<float, u32>),
                           dim3(unsigned(row_chunks), unsigned((rows + 3) / 4)), dim3(256), 0, s, x,
                           rows, cols, ld, gc, ncg, work, status, flag);
    } else if ((gr > 1 || gc == 1) && vec_ok && (cols + 63) / 64 <= 2147483647 &&
               (rows + COL_CHUNK_ROWS_VEC - 1) / COL_CHUNK_ROWS_VEC <= 65535) {
        hipLaunchKernelGGL((k_col_group_max<float, u32, 4>),
                           dim3(unsigned((cols + 255) / 256),
                                unsigned((rows + COL_CHUNK_ROWS_VEC - 1) / COL_CHUNK_ROWS_VEC)),
                           dim3(256), 0, s, x, rows, cols, ld, gr, gc, ncg, i64(COL_CHUNK_ROWS_VEC),
                           work, status, flag);
    } else if ((gr > 1 || gc == 1) && (cols + 63) / 64 <= 2147483647 && chunks <= 65535) {
        hipLaunchKernelGGL((k_col_group_max<float, u32, 1>),
                           dim3(unsigned((cols + 63) / 64), unsigned(chunks)), dim3(256), 0, s, x,
                           rows, cols, ld, gr, gc, ncg, i64(COL_CHUNK_ROWS), work, status, flag);
    } else {
        hipLaunchKernelGGL(k_group_max, dim3(grid_for(rows * ((cols + 7) / 8))), dim3(256), 0, s, x,
                           rows, cols, ld, gr, gc, ncg, work, status, flag);
    }
}

}  // namespace mf

using namespace mf;

// Shape checks shared by the implicit im2col entry points.
static int check_conv_geometry(const mf_conv_geometry &g) {
    if (g.n < 1 || g.channels < 1 || g.height < 1 || g.width < 1 || g.c0 < 0 ||
        g.group_channels < 1 || g.c0 + g.group_channels > g.channels || g.kh < 1 || g.kw < 1 ||
        g.sh < 1 || g.sw < 1 || g.ph < 0 || g.pw < 0 || g.dh < 1 || g.dw < 1)
        return fail(MF_E_INVALID, "invalid convolution geometry");
    if (g.height > 0x3FFFFFFF || g.width > 0x3FFFFFFF || g.ph > 0x3FFFFFFF || g.pw > 0x3FFFFFFF ||
        i64(g.dh) * (g.kh - 1) > 0x3FFFFFFF || i64(g.dw) * (g.kw - 1) > 0x3FFFFFFF)
        return fail(MF_E_UNSUPPORTED, "convolution extent too large");
    const i64 ho = (g.height + 2 * i64(g.ph) - i64(g.dh) * (g.kh - 1) - 1) / g.sh + 1;
    const i64 wo = (g.width + 2 * i64(g.pw) - i64(g.dw) * (g.kw - 1) - 1) / g.sw + 1;
    if (g.height + 2 * i64(g.ph) <= i64(g.dh) * (g.kh - 1) ||
        g.width + 2 * i64(g.pw) <= i64(g.dw) * (g.kw - 1) || g.out_height != ho ||
        g.out_width != wo)
        return fail(MF_E_INVALID, "convolution output size does not match the geometry");
    return MF_OK;
}

// One lane: the status word as the kernels queued before it left it, to the mailbox.
__global__ void k_publish_status(u32 *status, u32 *mailbox) { publish_status(status, mailbox); }

extern "C" {

int32_t mf_abi_version(void) { return MF_ABI_VERSION; }

const char *mf_last_error(void) { return g_error; }

const char *mf_source_hash(void) { return MF_SOURCE_HASH; }

int mf_device_identity(int device, mf_identity *out) {
    if (!out) return fail(MF_E_INVALID, "identity output is NULL");
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return fail(MF_E_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    memset(out, 0, sizeof(*out));
    snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
    snprintf(out->name, sizeof(out->name), "%s", prop.name);
    out->compute_units = prop.multiProcessorCount;
    out->memory_bytes = int64_t(prop.totalGlobalMem);
    int version = 0;
    if (hipDriverGetVersion(&version) == hipSuccess) out->driver_version = version;
    if (hipRuntimeGetVersion(&version) == hipSuccess) out->runtime_version = version;
    return MF_OK;
}

int mf_input_tiles(const mf_config *cfg, const float *x, int64_t n, int64_t k, int64_t ld,
                   const float *scale, uint8_t *q, float *xscale, void *stream) {
    int status = check_narrow(cfg);
    if (status) return status;
    if (!x || !scale || !q || !xscale || n < 1 || k < 1 || ld < k)
        return fail(MF_E_INVALID, "invalid input-tile arguments");
    const int R = cfg->rows, P = cfg->read_rows, Gr = cfg->reads;
    const i64 m = (k + R - 1) / R;
    const i64 kp = m * R;
    const int bits = cfg->activation_bits;
    const float upper = float((1 << (bits - 1)) - 1);
    const u32 mask = (1u << bits) - 1u;
    hipStream_t s = static_cast<hipStream_t>(stream);
    launch_input_codes(x, n, k, ld, kp, scale, 1, 1, k, 1, -upper, upper, mask, q, s);
    hipLaunchKernelGGL(k_input_scales, dim3(grid_for(n * m * Gr)), dim3(256), 0, s, n, k, m * Gr,
                       R, P, Gr, scale, i64(1), i64(1), k, 1, xscale);
    return check_launch("input tiles");
}

int mf_conv_input_tiles(const mf_config *cfg, const float *x, const mf_conv_geometry *geom,
                        const float *fixed_scale, int64_t gr, int64_t gc, uint32_t *work,
                        float *scale, uint8_t *q, float *xscale, uint32_t *status, void *stream) {
    int st = check_narrow(cfg);
    if (st) return st;
    if (!x || !geom || !q || !xscale) return fail(MF_E_INVALID, "invalid conv input-tile arguments");
    const mf_conv_geometry g = *geom;
    st = check_conv_geometry(g);
    if (st) return st;
    const i64 rows = g.n * g.out_height * g.out_width;
    const i64 K = g.group_channels * g.kh * g.kw;
    const int R = cfg->rows, P = cfg->read_rows, Gr = cfg->reads;
    const i64 m = (K + R - 1) / R, kp = m * R;
    const int bits = cfg->activation_bits;
    const float upper = float((1 << (bits - 1)) - 1);
    const u32 mask = (1u << bits) - 1u;
    if (rows > 0x7FFFFFFF || K > 0x7FFFFFFF || (kp + CONV_CHUNK_COLS - 1) / CONV_CHUNK_COLS > 65535)
        return fail(MF_E_UNSUPPORTED, "too many patches or patch columns");
    const dim3 grid((unsigned)((rows + 63) / 64), (unsigned)((kp + CONV_CHUNK_COLS - 1) / CONV_CHUNK_COLS));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int vec = kp % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0;
    if (fixed_scale) {
        hipLaunchKernelGGL(k_conv_codes, grid, dim3(256), 0, s, x, g, K, kp, fixed_scale, i64(1),
                           i64(0), i64(1), -upper, upper, mask, q, vec, status,
                           u32(MF_STATUS_INPUT));
        hipLaunchKernelGGL(k_input_scales, dim3(grid_for(rows * m * Gr)), dim3(256), 0, s, rows, K,
                           m * Gr, R, P, Gr, fixed_scale, i64(1), i64(1), K, 1, xscale);
        return check_launch("conv input tiles");
    }
    if (!work || !scale || gr < 1 || gc < 1)
        return fail(MF_E_INVALID, "dynamic conv input tiles need work, scale and group sizes");
    gr = gr < rows ? gr : rows;
    gc = gc < K ? gc : K;
    const i64 nrg = (rows + gr - 1) / gr, ncg = (K + gc - 1) / gc;
    hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(nrg * ncg)), dim3(256), 0, s, work, nrg * ncg, 0u);
    hipLaunchKernelGGL(k_conv_group_max, dim3(unsigned((rows + 255) / 256)), dim3(256), 0, s, x, g,
                       K, gr, gc, ncg, work, status, u32(MF_STATUS_INPUT));
    hipLaunchKernelGGL(k_group_scale, dim3(grid_for(nrg * ncg)), dim3(256), 0, s, work, nrg * ncg,
                       upper, scale);
    hipLaunchKernelGGL(k_conv_codes, grid, dim3(256), 0, s, x, g, K, kp, scale, gr, gc, ncg, -upper,
                       upper, mask, q, vec, status, u32(MF_STATUS_INPUT));
    hipLaunchKernelGGL(k_input_scales, dim3(grid_for(rows * m * Gr)), dim3(256), 0, s, rows, K,
                       m * Gr, R, P, Gr, scale, gr, gc, ncg, 0, xscale);
    return check_launch("conv input tiles");
}

int mf_conv_input_tiles_wide(const mf_config *cfg, const double *x, const mf_conv_geometry *geom,
                             const double *fixed_scale, int64_t gr, int64_t gc, uint64_t *work,
                             double *scale, uint32_t *q, double *xscale, uint32_t *status,
                             void *stream) {
    int st = check_wide(cfg);
    if (st) return st;
    if (!x || !geom || !q || !xscale) return fail(MF_E_INVALID, "invalid conv input-tile arguments");
    const mf_conv_geometry g = *geom;
    st = check_conv_geometry(g);
    if (st) return st;
    const i64 rows = g.n * g.out_height * g.out_width;
    const i64 K = g.group_channels * g.kh * g.kw;
    const int R = cfg->rows, P = cfg->read_rows, Gr = cfg->reads;
    const i64 m = (K + R - 1) / R, kp = m * R;
    const int bits = cfg->activation_bits;
    const double upper = double((i64(1) << (bits - 1)) - 1);
    const double lower = cfg->bw_e ? -double(i64(1) << (bits - 1)) : -upper;
    const u64 mask = bits == 64 ? ~u64(0) : (u64(1) << bits) - 1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (fixed_scale) {
        hipLaunchKernelGGL(k_conv_codes_f64, dim3(grid_for(rows * kp)), dim3(256), 0, s, x, g, K,
                           kp, fixed_scale, i64(1), i64(1), K, 1, lower, upper, mask, 0, q,
                           status, u32(MF_STATUS_INPUT));
        hipLaunchKernelGGL(k_input_scales_f64, dim3(grid_for(rows * m * Gr)), dim3(256), 0, s,
                           rows, K, m * Gr, R, P, Gr, fixed_scale, i64(1), i64(1), K, 1, xscale);
        return check_launch("wide conv input tiles");
    }
    if (!work || !scale || gr < 1 || gc < 1)
        return fail(MF_E_INVALID, "dynamic conv input tiles need work, scale and group sizes");
    gr = gr < rows ? gr : rows;
    gc = gc < K ? gc : K;
    const i64 nrg = (rows + gr - 1) / gr, ncg = (K + gc - 1) / gc;
    hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(2 * nrg * ncg)), dim3(256), 0, s,
                       reinterpret_cast<u32 *>(work), 2 * nrg * ncg, 0u);
    hipLaunchKernelGGL(k_conv_group_max_f64, dim3(grid_for(rows * K)), dim3(256), 0, s, x, g, K,
                       gr, gc, ncg, work, status, u32(MF_STATUS_INPUT));
    const int narrow = bits <= 8 && !cfg->bw_e;   // FP32 quantization, as the reference's
    hipLaunchKernelGGL(k_group_scale_f64, dim3(grid_for(nrg * ncg)), dim3(256), 0, s, work,
                       nrg * ncg, bits, cfg->bw_e, upper, narrow, scale, HUGE_VAL,
                       static_cast<u32 *>(nullptr));
    hipLaunchKernelGGL(k_conv_codes_f64, dim3(grid_for(rows * kp)), dim3(256), 0, s, x, g, K, kp,
                       scale, gr, gc, ncg, 0, lower, upper, mask, narrow, q, status,
                       u32(MF_STATUS_INPUT));
    hipLaunchKernelGGL(k_input_scales_f64, dim3(grid_for(rows * m * Gr)), dim3(256), 0, s, rows,
                       K, m * Gr, R, P, Gr, scale, gr, gc, ncg, 0, xscale);
    return check_launch("wide conv input tiles");
}

static i64 lcm4(i64 gr) { return gr % 4 == 0 ? gr : (gr % 2 == 0 ? 2 * gr : 4 * gr); }

int mf_quantize_inputs(const mf_config *cfg, const float *x, int64_t n, int64_t k, int64_t ld,
                       int64_t gr, int64_t gc, uint32_t *work, float *scale, uint8_t *q,
                       float *xscale, uint32_t *status, void *stream) {
    int status_code = check_narrow(cfg);
    if (status_code) return status_code;
    if (!x || !scale || !q || !xscale || n < 1 || k < 1 || ld < k || gr < 1 || gc < 1)
        return fail(MF_E_INVALID, "invalid input quantization arguments");
    const int R = cfg->rows, P = cfg->read_rows, Gr = cfg->reads;
    const i64 m = (k + R - 1) / R, kp = m * R;
    gr = gr < n ? gr : n;
    gc = gc < k ? gc : k;
    const i64 nrg = (n + gr - 1) / gr, ncg = (k + gc - 1) / gc;
    // scale == xscale: groups of exactly one read and no padded reads make the
    // group grid the per-read scale table itself, and the gather is skipped.
    const bool direct = scale == xscale;
    if (direct && !(gr == 1 && gc == P && kp == k))
        return fail(MF_E_INVALID, "scale may alias xscale only for groups of one read "
                                  "(gr == 1, gc == read rows, k == m*R)");
    const int bits = cfg->activation_bits;
    const float upper = float((1 << (bits - 1)) - 1);
    const u32 mask = (1u << bits) - 1u;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool vec = gc % 4 == 0 && k % 4 == 0 && kp % 4 == 0 && ld % 4 == 0 &&
                     reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(q) % 4 == 0;
    const i64 quads = gc / 4;
    const bool pow2 = quads > 0 && (quads & (quads - 1)) == 0;
    if (gr == 1 && vec && pow2 && quads <= 64) {
        const int L = int(quads);
        hipLaunchKernelGGL(k_row_groups_lanes, dim3(unsigned((n * ncg * L + 255) / 256)), dim3(256),
                           0, s, x, n, k, ld, L, ncg, kp, -upper, upper, mask, q, scale, status,
                           u32(MF_STATUS_INPUT));
    } else if (gr == 1 && vec && pow2 && quads <= 1024) {
        const dim3 grid{unsigned((n * ncg * 64 + 255) / 256)};
        const int V = int(quads / 64);
        // The waves fill the per-read scale table themselves.
        const ReadTable reads{direct ? nullptr : xscale, m * Gr, R, P, Gr};
        if (V == 2)
            hipLaunchKernelGGL(k_row_groups_wave<2>, grid, dim3(256), 0, s, x, n, k, ld, ncg, kp,
                               -upper, upper, mask, q, scale, status, u32(MF_STATUS_INPUT), reads);
        else if (V == 4)
            hipLaunchKernelGGL(k_row_groups_wave<4>, grid, dim3(256), 0, s, x, n, k, ld, ncg, kp,
                               -upper, upper, mask, q, scale, status, u32(MF_STATUS_INPUT), reads);
        else if (V == 8)
            hipLaunchKernelGGL(k_row_groups_wave<8>, grid, dim3(256), 0, s, x, n, k, ld, ncg, kp,
                               -upper, upper, mask, q, scale, status, u32(MF_STATUS_INPUT), reads);
        else
            hipLaunchKernelGGL(k_row_groups_wave<16>, grid, dim3(256), 0, s, x, n, k, ld, ncg, kp,
                               -upper, upper, mask, q, scale, status, u32(MF_STATUS_INPUT), reads);
        return check_launch("input quantization");
    } else if (gr == 1 && gc <= 1024) {
        if (vec)
            hipLaunchKernelGGL(k_row_groups<true>, dim3(grid_for(n * ncg)), dim3(256), 0, s, x, n, k,
                               ld, gc, ncg, kp, -upper, upper, mask, q, scale, status, u32(MF_STATUS_INPUT));
        else
            hipLaunchKernelGGL(k_row_groups<false>, dim3(grid_for(n * ncg)), dim3(256), 0, s, x, n,
                               k, ld, gc, ncg, kp, -upper, upper, mask, q, scale, status,
                               u32(MF_STATUS_INPUT));
    } else {
        if (!work) return fail(MF_E_INVALID, "grouped input quantization needs a work buffer");
        hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(nrg * ncg)), dim3(256), 0, s, work, nrg * ncg, 0u);
        launch_group_max_f32(x, n, k, ld, gr, gc, ncg, work, status, u32(MF_STATUS_INPUT), s);
        hipLaunchKernelGGL(k_group_scale, dim3(grid_for(nrg * ncg)), dim3(256), 0, s, work,
                           nrg * ncg, upper, scale);
        launch_input_codes(x, n, k, ld, kp, scale, gr, gc, ncg, 0, -upper, upper, mask, q, s);
    }
    if (!direct)
        hipLaunchKernelGGL(k_input_scales, dim3(grid_for(n * m * Gr)), dim3(256), 0, s, n, k,
                           m * Gr, R, P, Gr, scale, gr, gc, ncg, 0, xscale);
    return check_launch("input quantization");
}

int mf_quantize_weights(const mf_config *cfg, const float *b, int64_t k, int64_t o, int64_t ld,
                        int64_t gr, int64_t gc, uint32_t *work, float *scale, uint8_t *packed,
                        uint8_t *packed_t, float *wscale, uint32_t *status, void *stream) {
    int status_code = check_narrow(cfg);
    if (status_code) return status_code;
    if (!b || !scale || !packed || !wscale || k < 1 || o < 1 || ld < o || gr < 1 || gc < 1)
        return fail(MF_E_INVALID, "invalid weight quantization arguments");
    const int R = cfg->rows, C = cfg->cols, P = cfg->read_rows, Gr = cfg->reads;
    const i64 m = (k + R - 1) / R, p = (o + C - 1) / C, kp = m * R, op = p * C;
    gr = gr < k ? gr : k;
    gc = gc < o ? gc : o;
    const i64 nrg = (k + gr - 1) / gr, ncg = (o + gc - 1) / gc;
    // scale == wscale: column groups of exactly one read, no padded reads or
    // columns: the group grid is the per-read scale table, no gather runs.
    const bool direct = scale == wscale;
    if (direct && !(gc == 1 && gr == P && kp == k && op == o))
        return fail(MF_E_INVALID, "scale may alias wscale only for groups of one read "
                                  "(gc == 1, gr == read rows, k == m*R, o == p*C)");
    const int bits = cfg->weight_bits;
    const float upper = float((1 << (bits - (cfg->weight_signed ? 1 : 0))) - 1);
    const float lower = cfg->weight_signed ? -upper : 0.0f;
    const u32 mask = (1u << bits) - 1u;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const i64 unit = lcm4(gr);
    const i64 span = unit >= 128 ? unit : unit * (128 / unit);
    const bool reg_group = gr == 8 || gr == 16 || gr == 32 || gr == 64;
    const bool tiled = (gr == 16 || gr == 32) && cfg->cols % 64 == 0 && R % (4 * gr) == 0 &&
                       kp % 16 == 0;
    if (gc == 1 && tiled && kp / (4 * gr) <= 65535) {
        const dim3 grid{unsigned(op / 64), unsigned(kp / (4 * gr)), 1u};
        if (gr == 16)
            hipLaunchKernelGGL((k_col_groups_tile<16, false>), grid, dim3(256), 0, s, b, k, o, ld, R,
                               C, m, p, lower, upper, mask, packed, packed_t, scale, gr, status,
                               u32(MF_STATUS_WEIGHT));
        else
            hipLaunchKernelGGL((k_col_groups_tile<32, false>), grid, dim3(256), 0, s, b, k, o, ld, R,
                               C, m, p, lower, upper, mask, packed, packed_t, scale, gr, status,
                               u32(MF_STATUS_WEIGHT));
    } else if (gc == 1 && reg_group && (kp + gr - 1) / gr <= 65535) {
        const dim3 grid{unsigned((op + 255) / 256), unsigned((kp + gr - 1) / gr), 1u};
        const bool word = kp % 4 == 0;
#define MF_COL_REG_LAUNCH(GR)                                                                    \
    if (gr == GR) {                                                                              \
        if (word)                                                                                \
            hipLaunchKernelGGL((k_col_groups_reg<GR, true>), grid, dim3(256), 0, s, b, k, o, ld, R, \
                               C, m, p, lower, upper, mask, packed, packed_t, scale, status,      \
                               u32(MF_STATUS_WEIGHT));                                           \
        else                                                                                     \
            hipLaunchKernelGGL((k_col_groups_reg<GR, false>), grid, dim3(256), 0, s, b, k, o, ld, \
                               R, C, m, p, lower, upper, mask, packed, packed_t, scale, status,   \
                               u32(MF_STATUS_WEIGHT));                                           \
    }
        MF_COL_REG_LAUNCH(8)
        MF_COL_REG_LAUNCH(16)
        MF_COL_REG_LAUNCH(32)
        MF_COL_REG_LAUNCH(64)
#undef MF_COL_REG_LAUNCH
    } else if (gc == 1 && gr <= 256 && (kp + span - 1) / span <= 65535) {
        const dim3 grid{unsigned((op + 255) / 256), unsigned((kp + span - 1) / span), 1u};
        if (kp % 4 == 0)
            hipLaunchKernelGGL(k_col_groups<true>, grid, dim3(256), 0, s, b, k, o, ld, gr, span, R, C,
                               m, p, lower, upper, mask, packed, packed_t, scale, status,
                               u32(MF_STATUS_WEIGHT));
        else
            hipLaunchKernelGGL(k_col_groups<false>, grid, dim3(256), 0, s, b, k, o, ld, gr, span, R,
                               C, m, p, lower, upper, mask, packed, packed_t, scale, status,
                               u32(MF_STATUS_WEIGHT));
    } else if (gc == 1 && (kp + 255) / 256 <= 65535) {
        // Tall column groups: maxima reduced along the rows, then codes in 256-row chunks.
        if (!work) return fail(MF_E_INVALID, "grouped weight quantization needs a work buffer");
        hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(nrg * ncg)), dim3(256), 0, s, work, nrg * ncg, 0u);
        launch_group_max_f32(b, k, o, ld, gr, gc, ncg, work, status, u32(MF_STATUS_WEIGHT), s);
        hipLaunchKernelGGL(k_group_scale, dim3(grid_for(nrg * ncg)), dim3(256), 0, s, work,
                           nrg * ncg, upper, scale);
        if (cfg->cols % 64 == 0 && R % 128 == 0 && kp % 16 == 0 && kp / 128 <= 65535) {
            // The LDS tile of 32-row groups, each row taking its group's scale.
            const dim3 grid{unsigned(op / 64), unsigned(kp / 128), 1u};
            hipLaunchKernelGGL((k_col_groups_tile<32, true>), grid, dim3(256), 0, s, b, k, o, ld, R,
                               C, m, p, lower, upper, mask, packed, packed_t, scale, gr, status,
                               u32(MF_STATUS_WEIGHT));
        } else {
            const dim3 grid{unsigned((op + 255) / 256), unsigned((kp + 255) / 256), 1u};
            if (kp % 4 == 0)
                hipLaunchKernelGGL(k_col_codes<true>, grid, dim3(256), 0, s, b, k, o, ld, gr,
                                   i64(256), R, C, m, p, scale, lower, upper, mask, packed,
                                   packed_t);
            else
                hipLaunchKernelGGL(k_col_codes<false>, grid, dim3(256), 0, s, b, k, o, ld, gr,
                                   i64(256), R, C, m, p, scale, lower, upper, mask, packed,
                                   packed_t);
        }
    } else {
        if (!work) return fail(MF_E_INVALID, "grouped weight quantization needs a work buffer");
        hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(nrg * ncg)), dim3(256), 0, s, work, nrg * ncg, 0u);
        launch_group_max_f32(b, k, o, ld, gr, gc, ncg, work, status, u32(MF_STATUS_WEIGHT), s);
        hipLaunchKernelGGL(k_group_scale, dim3(grid_for(nrg * ncg)), dim3(256), 0, s, work,
                           nrg * ncg, upper, scale);
        hipLaunchKernelGGL(k_weight_codes, dim3(grid_for(kp * op)), dim3(256), 0, s, b, k, o, ld, R,
                           C, m, p, scale, gr, gc, ncg, lower, upper, mask, packed, packed_t);
    }
    if (!direct)
        hipLaunchKernelGGL(k_weight_scales, dim3(grid_for(m * Gr * op)), dim3(256), 0, s, k, o,
                           m * Gr, op, R, P, Gr, scale, gr, gc, ncg, wscale);
    return check_launch("weight quantization");
}

int mf_transpose_packed(const mf_config *cfg, const uint8_t *packed, int64_t m, int64_t p,
                        uint8_t *packed_t, void *stream) {
    int status = check_narrow(cfg);
    if (status) return status;
    if (!packed || !packed_t || m < 1 || p < 1) return fail(MF_E_INVALID, "invalid transpose arguments");
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(k_transpose_packed, dim3(grid_for(m * cfg->rows * p * cfg->cols)), dim3(256),
                       0, s, packed, cfg->rows, cfg->cols, m, p, packed_t);
    return check_launch("transpose packed");
}

int mf_restore(const mf_config *cfg, const uint8_t *packed, int64_t m, int64_t p, int64_t begin,
               int64_t end, uint32_t seed, uint64_t event, void *g, void *stream) {
    int status = check_narrow(cfg);
    if (status) return status;
    if (!packed || !g || m < 1 || p < 1 || begin < 0 || end <= begin || end > p)
        return fail(MF_E_INVALID, "invalid restore arguments");
    const int planes = restore_planes(cfg);
    const i64 total = i64(planes) * m * (end - begin) * cfg->n_w * cfg->rows * cfg->cols;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (cfg->precise)
        hipLaunchKernelGGL((k_restore<double, u8>), dim3(grid_for(total)), dim3(256), 0, s, *cfg, packed, m,
                           p, begin, end - begin, seed, event, planes, static_cast<double *>(g));
    else
        hipLaunchKernelGGL((k_restore<float, u8>), dim3(grid_for(total)), dim3(256), 0, s, *cfg, packed, m,
                           p, begin, end - begin, seed, event, planes, static_cast<float *>(g));
    return check_launch("restore");
}

int mf_partial(const mf_config *cfg, const uint8_t *q, int64_t n, int64_t m, const uint8_t *packed,
               int64_t p, int64_t begin, int64_t end, const void *g, uint32_t seed,
               uint64_t event, float *totals, int32_t *codes, void *stream) {
    int status = check_narrow(cfg);
    if (status) return status;
    if (!q || !packed || !totals || n < 1 || m < 1 || p < 1 || begin < 0 || end <= begin || end > p)
        return fail(MF_E_INVALID, "invalid partial arguments");
    if (cfg->n_in > 8 || cfg->n_w > 8) return fail(MF_E_UNSUPPORTED, "more than 8 slices");
    if (!g && needs_conductances(cfg))
        return fail(MF_E_INVALID, "device noise needs restored conductances (g)");
    GeneralArgs args{};
    args.q = q;
    args.packed = packed;
    args.g = g;
    args.out = totals;
    args.codes = codes;
    args.n = n;
    args.m = m;
    args.p = p;
    args.begin = begin;
    args.width = end - begin;
    args.seed = seed;
    args.event = event;
    args.planes = g ? restore_planes(cfg) : 1;
    const i64 G = m * cfg->reads;
    args.lp_cascade = level_power(G);
    args.lp_interleaved = level_power(G / 4);
    hipStream_t s = static_cast<hipStream_t>(stream);
    return launch_general_read(cfg, args, OUT_TOTALS, s);
}

// Extents the MFMA kernel addresses with 32-bit buffer offsets (a block's code
// slab of up to 128 rows and the whole per-read weight-scale table) and its grid.
static bool ideal_extent_ok(const mf_config *cfg, i64 n, i64 m, i64 p) {
    const i64 kp = m * cfg->rows, ncols = p * cfg->cols, G = m * cfg->reads;
    const i64 limit = 0x7FFFFFFF;
    return 128 * kp <= limit && G * ncols * 4 <= limit && 128 * G * 4 <= limit &&
           (n + 63) / 64 + (ncols + 31) / 32 <= 65535;
}

static bool wide_plan_ok(const mf_config *cfg, i64 n, i64 m, i64 p) {
    NoisyWidePlan plan;
    int ks = 0;
    const char *why = "";
    return wide_extent_ok(n, m, cfg) && build_noisy_wide_plan(cfg, m, p, &plan, &ks, &why);
}

int mf_mm_kernel(const mf_config *cfg, int64_t n, int64_t m, int64_t p, int32_t has_packed_t,
                 int32_t *kernel_id) {
    int status = check_config(cfg);
    if (status) return status;
    if (!kernel_id) return fail(MF_E_INVALID, "kernel_id is NULL");
    IdealPlan plan;
    SlotTests xt, wt;
    int ks = 0;
    const char *why = "";
    NoisyPlan noisy;
    if (has_packed_t && ideal_extent_ok(cfg, n, m, p) &&
        build_ideal_plan(cfg, m, p, &plan, &xt, &wt, &ks, &why))
        *kernel_id = 1;
    else if (has_packed_t && noisy_extent_ok(n, m, cfg) &&
             build_noisy_plan(cfg, m, p, &noisy, &ks, &why))
        *kernel_id = 2;
    else if (wide_plan_ok(cfg, n, m, p))
        *kernel_id = 3;
    else
        *kernel_id = 0;
    return MF_OK;
}

int mf_mm_workspace(const mf_config *cfg, int64_t n, int64_t m, int64_t p, int32_t variant,
                    int64_t *bytes) {
    int status = check_config(cfg);
    if (status) return status;
    if (!bytes || n < 1 || m < 1 || p < 1) return fail(MF_E_INVALID, "invalid workspace query");
    if (!variant_valid(variant)) return fail(MF_E_INVALID, "unknown kernel variant 0x%x", variant);
    IdealPlan plan;
    SlotTests xt, wt;
    NoisyPlan noisy;
    int ks = 0;
    const char *why = "";
    if (build_ideal_plan(cfg, m, p, &plan, &xt, &wt, &ks, &why)) {
        i64 xb, wb;
        ideal_workspace(cfg, n, m, p, &xb, &wb);
        *bytes = xb + wb;
    } else if (build_noisy_plan(cfg, m, p, &noisy, &ks, &why)) {
        *bytes = noisy_terms_bytes(cfg, m, p) +
                 noisy_scratch_bytes(cfg, n, m, p, variant_split(variant)) +
                 noisy_voltage_bytes(cfg, n, m);
    } else if (wide_plan_ok(cfg, n, m, p)) {
        // At least the two 32-column blocks the wide read's chunking needs, even for
        // outputs narrower than 64 columns.
        const i64 blocks = std::max<i64>(2, (p * cfg->cols + 31) / 32);
        *bytes = wide_prefix_bytes(n, m, cfg) + blocks * wide_block_bytes(cfg, m);
    } else {
        *bytes = 0;
    }
    return MF_OK;
}

// The ideal read proper once both sides' proven-slot masks are in xbits / wbits.
// The largest group scale for which no FP32 step of the ideal read's restore can overflow:
// each read's total obeys |T| <= Tmax = sum over slice pairs of |fa*fw| * P * mask_a * mask_w,
// so with every scale <= s, |(T*xs)*ws| <= Tmax*s^2*(1+2^-24)^2 and a sum of G such terms in
// any order stays below G*Tmax*s^2*1.07 (G < 2^20).  s = sqrt(FLT_MAX / (2*G*Tmax)), rounded
// down to FP32.
static float finite_output_scale_bound(const mf_config *cfg, i64 G) {
    double tmax = 0.0;
    for (int a = 0; a < cfg->n_in; ++a)
        for (int w = 0; w < cfg->n_w; ++w)
            tmax += std::fabs(double(cfg->in_factor[a]) * double(cfg->w_factor[w])) *
                    double(cfg->read_rows) * double(cfg->in_mask[a]) * double(cfg->w_mask[w]);
    const double bound = std::sqrt(double(FLT_MAX) / (2.0 * double(G) * std::max(tmax, 1.0)));
    float f = float(bound);
    if (double(f) > bound) f = std::nextafter(f, 0.0f);
    return f;
}

static int launch_ideal(const mf_config *cfg, const IdealPlan &plan, int ks, const u8 *q,
                        const float *xscale, const u8 *packed_t, const float *wscale,
                        const uint64_t *xbits, const uint64_t *wbits, i64 n, i64 m, i64 p,
                        i64 out_cols, i64 g_run, float *out, i64 ldo, int32_t variant,
                        u32 *status, hipStream_t s, u32 *mailbox = nullptr) {
    const i64 kp = m * cfg->rows, ncols = p * cfg->cols, G = m * cfg->reads;
    IdealArgs args{};
    args.q = q;
    args.wt = packed_t;
    args.xscale = xscale;
    args.wscale = wscale;
    args.xbits = xbits;
    args.wbits = wbits;
    args.out = out;
    args.status = status;
    args.mailbox = mailbox;
    args.n = n;
    args.kp = kp;
    args.G = G;
    args.G_run = g_run;
    args.ldo = ldo;
    args.ldws = ncols;
    args.ncols = out_cols;
    args.Gr = cfg->reads;
    args.R = cfg->rows;
    args.P = cfg->read_rows;
    args.a_bits = cfg->activation_bits;
    args.w_bits = cfg->weight_bits;
    // Tile variants: 0 default (32 vectors per wave), 1 = 64 vectors per wave,
    // 2 = 32 vectors per wave.
    const int tn = (ks == 1 && variant_tile(variant) == 1) ? 2 : 1;
    const i64 gy = (n + 64 * tn - 1) / (64 * tn), gx = (out_cols + 63) / 64;
    if (gy > 65535 || gx > 2147483647) return fail(MF_E_RESOURCE, "grid too large");
    const dim3 grid{unsigned(gx), unsigned(gy), 1u};
    std::pair<hipEvent_t, hipEvent_t> timing{nullptr, nullptr};
    if (profiling() && (timing = profile_pair()).first) hipEventRecord(timing.first, s);
    if (ks == 1 && tn == 2) hipLaunchKernelGGL((k_ideal<2, 1>), grid, dim3(256), 0, s, plan, args);
    else if (ks == 1) hipLaunchKernelGGL((k_ideal<1, 1>), grid, dim3(256), 0, s, plan, args);
    else hipLaunchKernelGGL((k_ideal<1, 2>), grid, dim3(256), 0, s, plan, args);
    if (timing.first) {
        hipEventRecord(timing.second, s);
        profile_push(timing);
    }
    return check_launch("ideal MFMA read");
}

// Reads that hold at least one of the first k_rows rows (reads tile the
// arrays: R a multiple of P, as the MFMA kernels require).
static i64 reads_with_rows(const mf_config *cfg, i64 m, i64 k_rows) {
    const i64 G = m * cfg->reads;
    if (cfg->rows % cfg->read_rows) return G;
    const i64 used = (k_rows + cfg->read_rows - 1) / cfg->read_rows;
    return used < G ? used : G;
}

// mf_mm; with `split_totals` a noisy MFMA read split across blocks leaves its totals to the
// caller (*split_totals, [n, G, p*C]) instead of restoring them into `out` (null otherwise);
// *split_restored says whether they are already restored ((float(T) * xs) * ws).
static int mm_read(const mf_config *cfg, const uint8_t *q, const float *xscale, int64_t n,
                   int64_t m, const uint8_t *packed, const uint8_t *packed_t, const float *wscale,
                   int64_t p, int64_t out_cols, int64_t k_rows, const void *g, uint32_t seed,
                   uint64_t event, float *out, int64_t ldo, void *workspace,
                   int64_t workspace_bytes, int32_t variant, uint32_t *status, void *stream,
                   const float **split_totals, bool *split_restored = nullptr) {
    if (split_totals) *split_totals = nullptr;
    const int valid = check_narrow(cfg);
    if (valid) return valid;
    if (!q || !xscale || !packed || !wscale || !out || n < 1 || m < 1 || p < 1 ||
        ldo < p * cfg->cols)
        return fail(MF_E_INVALID, "invalid mm arguments");
    if (out_cols < 1 || out_cols > p * cfg->cols || k_rows < 1 || k_rows > m * cfg->rows)
        return fail(MF_E_INVALID, "out_cols must be in [1, p*C] and k_rows in [1, m*R]");
    const i64 g_run = reads_with_rows(cfg, m, k_rows);
    if (cfg->n_in > 8 || cfg->n_w > 8) return fail(MF_E_UNSUPPORTED, "more than 8 slices");
    if (!variant_valid(variant)) return fail(MF_E_INVALID, "unknown kernel variant 0x%x", variant);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const i64 G = m * cfg->reads;
    IdealPlan plan;
    int ks = 0;
    const char *why = "";
    const bool aligned = (reinterpret_cast<uintptr_t>(q) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(packed_t) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(out) % 16 == 0) && ldo % 4 == 0;
    i64 xbytes = 0, wbytes = 0;
    ideal_workspace(cfg, n, m, p, &xbytes, &wbytes);
    const bool room = workspace && workspace_bytes >= xbytes + wbytes;
    SlotTests xtests, wtests;
    if (!g && packed_t && aligned && room && ideal_extent_ok(cfg, n, m, p) &&
        build_ideal_plan(cfg, m, p, &plan, &xtests, &wtests, &ks, &why)) {
        uint64_t *xbits = static_cast<uint64_t *>(workspace);
        uint64_t *wbits = reinterpret_cast<uint64_t *>(static_cast<char *>(workspace) + xbytes);
        const i64 kp = m * cfg->rows, ncols = p * cfg->cols;
        const SliceLayout xl = layout_of(cfg->in_shift, cfg->in_mask, cfg->n_in);
        const SliceLayout wl = layout_of(cfg->w_shift, cfg->w_mask, cfg->n_w);
        const unsigned gblocks = unsigned((G + 63) / 64);
        const DigitJob xjob{q, n, 64, xl, xtests, xbits};
        const DigitJob wjob{packed_t, ncols, 32, wl, wtests, wbits};
        const i64 xblocks = (n + 63) / 64;
        const dim3 dgrid(gblocks, unsigned(xblocks + (ncols + 31) / 32));
        if (cfg->read_rows == 64)
            hipLaunchKernelGGL(k_digit_bits<64>, dgrid, dim3(64 * DIGIT_WAVES), 0, s, xjob, wjob,
                               xblocks, kp, G);
        else
            hipLaunchKernelGGL(k_digit_bits<32>, dgrid, dim3(64 * DIGIT_WAVES), 0, s, xjob, wjob,
                               xblocks, kp, G);
        return launch_ideal(cfg, plan, ks, q, xscale, packed_t, wscale, xbits, wbits, n, m, p,
                            out_cols, g_run, out, ldo, variant, status, s);
    }
    NoisyPlan noisy;
    if (!g && packed_t && aligned && workspace && ideal_extent_ok(cfg, n, m, p) &&
        noisy_extent_ok(n, m, cfg) && build_noisy_plan(cfg, m, p, &noisy, &ks, &why) &&
        workspace_bytes >= noisy_voltage_bytes(cfg, n, m) + 2 * noisy_block_bytes(cfg, m)) {
        return launch_noisy(cfg, noisy, ks, q, xscale, n, m, packed_t, wscale, p, nullptr, seed,
                            event, out, ldo, workspace, workspace_bytes, 0, status, s,
                            (variant & MF_MM_REUSE_TERMS) != 0, out_cols, g_run,
                            variant_split(variant), split_totals, split_restored);
    }
    if (!g && needs_conductances(cfg))
        return fail(MF_E_INVALID, "device noise needs restored conductances (g)");
    GeneralArgs args{};
    args.q = q;
    args.packed = packed;
    args.g = g;
    args.xscale = xscale;
    args.wscale = wscale;
    args.out = out;
    args.status = status;
    args.n = n;
    args.m = m;
    args.p = p;
    args.begin = 0;
    args.width = p;
    args.ldo = ldo;
    args.ldws = p * cfg->cols;
    args.seed = seed;
    args.event = event;
    args.planes = g ? restore_planes(cfg) : 1;
    args.lp_cascade = level_power(G);
    args.lp_interleaved = level_power(G / 4);
    std::pair<hipEvent_t, hipEvent_t> timing{nullptr, nullptr};
    if (profiling() && (timing = profile_pair()).first) hipEventRecord(timing.first, s);
    const int launched = launch_general_read(cfg, args, OUT_FUSED, s);
    if (timing.first) {
        hipEventRecord(timing.second, s);
        profile_push(timing);
    }
    return launched;
}

int mf_mm(const mf_config *cfg, const uint8_t *q, const float *xscale, int64_t n, int64_t m,
          const uint8_t *packed, const uint8_t *packed_t, const float *wscale, int64_t p,
          int64_t out_cols, int64_t k_rows, const void *g, uint32_t seed, uint64_t event,
          float *out, int64_t ldo, void *workspace, int64_t workspace_bytes, int32_t variant,
          uint32_t *status, void *stream) {
    return mm_read(cfg, q, xscale, n, m, packed, packed_t, wscale, p, out_cols, k_rows, g, seed,
                   event, out, ldo, workspace, workspace_bytes, variant, status, stream, nullptr);
}

int mf_mm_from_float(const mf_config *cfg, const float *x, int64_t n, int64_t k, int64_t ldx,
                     const float *b, int64_t o, int64_t ldb, int64_t x_gr, int64_t x_gc,
                     int64_t w_gr, int64_t w_gc, uint8_t *q, float *xscale, uint8_t *packed,
                     uint8_t *packed_t, float *wscale, float *out, int64_t ldo, void *workspace,
                     int64_t workspace_bytes, int32_t variant, uint32_t *status,
                     uint32_t *mailbox, void *stream) {
    const int valid = check_narrow(cfg);
    if (valid) return valid;
    if (!x || !b || !q || !xscale || !packed || !packed_t || !wscale || !out || n < 1 || k < 1 ||
        o < 1 || ldx < k || ldb < o || ldo < o)
        return fail(MF_E_INVALID, "invalid mm_from_float arguments");
    if (!variant_valid(variant)) return fail(MF_E_INVALID, "unknown kernel variant 0x%x", variant);
    const int R = cfg->rows, C = cfg->cols, P = cfg->read_rows;
    const i64 m = (k + R - 1) / R, p = (o + C - 1) / C, G = m * cfg->reads;
    // Groups of one read on both sides, whole arrays, and the tile and vector layouts the
    // fused quantizer assumes; anything else takes mf_quantize_inputs/_weights + mf_mm.
    const bool shapes = P == 32 && R % 128 == 0 && C % 64 == 0 && k == m * R && o == p * C &&
                        G % 4 == 0 &&
                        (x_gr < n ? x_gr : n) == 1 && x_gc == P && w_gr == P && w_gc == 1;
    const bool aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldx % 4 == 0 &&
                         reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(packed_t) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(packed) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(out) % 16 == 0 && ldo % 4 == 0;
    i64 xbytes = 0, wbytes = 0;
    ideal_workspace(cfg, n, m, p, &xbytes, &wbytes);
    const bool room = workspace && workspace_bytes >= xbytes + wbytes;
    IdealPlan plan;
    SlotTests xtests, wtests;
    int ks = 0;
    const char *why = "";
    const i64 wgrid_x = o / 64, wblocks = wgrid_x * (m * R / 128), xblocks = (n + 63) / 64 * (G / 4);
    if (!shapes || !aligned || !room || !ideal_extent_ok(cfg, n, m, p) ||
        wblocks + xblocks > 0x7FFFFFFF || !build_ideal_plan(cfg, m, p, &plan, &xtests, &wtests, &ks, &why))
        return fail(MF_E_UNSUPPORTED, "mm_from_float not applicable");
    u32 *device_mailbox = nullptr;
    if (mailbox) {
        __atomic_store_n(mailbox, 0u, __ATOMIC_RELAXED);
        const hipError_t e =
            hipHostGetDevicePointer(reinterpret_cast<void **>(&device_mailbox), mailbox, 0);
        if (e != hipSuccess)
            return fail(MF_E_INVALID, "mailbox is not pinned host memory: %s", hipGetErrorString(e));
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint64_t *xbits = static_cast<uint64_t *>(workspace);
    uint64_t *wbits = reinterpret_cast<uint64_t *>(static_cast<char *>(workspace) + xbytes);
    const float bound = finite_output_scale_bound(cfg, G);
    ReadGroupArgs a{};
    a.b = b;
    a.k = k;
    a.o = o;
    a.ldb = ldb;
    a.R = R;
    a.C = C;
    a.m = m;
    a.p = p;
    const int wbits_n = cfg->weight_bits;
    a.wupper = float((1 << (wbits_n - (cfg->weight_signed ? 1 : 0))) - 1);
    a.wlower = cfg->weight_signed ? -a.wupper : 0.0f;
    a.wmask = (1u << wbits_n) - 1u;
    a.packed = packed;
    a.packed_t = packed_t;
    a.wscale = wscale;
    a.wgrid_x = wgrid_x;
    a.wblocks = wblocks;
    a.x = x;
    a.n = n;
    a.ldx = ldx;
    a.xupper = float((1 << (cfg->activation_bits - 1)) - 1);
    a.xmask = (1u << cfg->activation_bits) - 1u;
    a.q = q;
    a.xscale = xscale;
    a.G = G;
    a.wdigits = TileDigits{layout_of(cfg->w_shift, cfg->w_mask, cfg->n_w), wtests, wbits, G, bound};
    a.xdigits = TileDigits{layout_of(cfg->in_shift, cfg->in_mask, cfg->n_in), xtests, xbits, G,
                           bound};
    a.status = status;
    hipLaunchKernelGGL(k_read_groups, dim3(unsigned(wblocks + xblocks)), dim3(256), 0, s, a);
    const int launched = check_launch("read-group quantization");
    if (launched) return launched;
    return launch_ideal(cfg, plan, ks, q, xscale, packed_t, wscale, xbits, wbits, n, m, p, o, G,
                        out, ldo, variant, status, s, device_mailbox);
}

int mf_status_publish(const uint32_t *status, uint32_t *mailbox, void *stream) {
    if (!status || !mailbox) return fail(MF_E_INVALID, "invalid status_publish arguments");
    __atomic_store_n(mailbox, 0u, __ATOMIC_RELAXED);
    u32 *device_mailbox = nullptr;
    const hipError_t e =
        hipHostGetDevicePointer(reinterpret_cast<void **>(&device_mailbox), mailbox, 0);
    if (e != hipSuccess)
        return fail(MF_E_INVALID, "mailbox is not pinned host memory: %s", hipGetErrorString(e));
    hipLaunchKernelGGL(k_publish_status, dim3(1), dim3(1), 0, static_cast<hipStream_t>(stream),
                       const_cast<u32 *>(status), device_mailbox);
    return check_launch("status publish");
}

int mf_status_wait(const uint32_t *mailbox, int64_t timeout_us, uint32_t *flags,
                   int32_t *published) {
    if (!mailbox || !flags || !published || timeout_us < 0)
        return fail(MF_E_INVALID, "invalid status_wait arguments");
    using clock = std::chrono::steady_clock;
    const auto start = clock::now();
    for (int64_t i = 0;; ++i) {
        const uint32_t word = __atomic_load_n(mailbox, __ATOMIC_ACQUIRE);
        if (word & MF_STATUS_PUBLISHED) {
            *flags = word & ~MF_STATUS_PUBLISHED;
            *published = 1;
            return MF_OK;
        }
        if (i % 64 == 0) {
            const int64_t waited =
                std::chrono::duration_cast<std::chrono::microseconds>(clock::now() - start).count();
            if (waited >= timeout_us) {
                *flags = 0;
                *published = 0;
                return MF_OK;
            }
            // Spin for the first 2 ms (a read's quantizers take tens of microseconds), then
            // poll in short sleeps behind longer queued work.
            if (waited >= 2000) std::this_thread::sleep_for(std::chrono::microseconds(20));
        }
#if defined(__x86_64__)
        __builtin_ia32_pause();
#endif
    }
}

}  // extern "C"

// Scratch of mf_mm_static: device memory the library holds on each GPU it runs
// on (the code object's zero-initialised data, mapped when the module loads on
// that device) until the process ends.  Host code never passes this name to a
// kernel: on the host it is only a stand-in for the per-device address that
// hipGetSymbolAddress returns, which static_scratch() records once per device.
static __device__ __align__(256) unsigned char scratch[MF_STATIC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first call).
int static_scratch(void **out) {
    int device = -1;
    const hipError_t got = hipGetDevice(&device);
    if (got != hipSuccess) return fail(MF_E_HIP, "hipGetDevice: %s", hipGetErrorString(got));
    if (device < 0 || device >= kMaxDevices)
        return fail(MF_E_UNSUPPORTED, "device %d beyond the %d the static scratch serves", device,
                    kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_lock);
    if (!g_scratch_ptr[device]) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(MF_E_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", device,
                        hipGetErrorString(e));
        g_scratch_ptr[device] = ptr;
    }
    *out = g_scratch_ptr[device];
    return MF_OK;
}
}  // namespace

extern "C" {

int mf_mm_static(const mf_config *cfg, const uint8_t *q, const float *xscale, int64_t n,
                 int64_t m, const uint8_t *packed, const uint8_t *packed_t, const float *wscale,
                 int64_t p, int64_t out_cols, int64_t k_rows, const void *g, uint32_t seed,
                 uint64_t event, float *out, int64_t ldo, int32_t variant, uint32_t *status,
                 void *stream) {
    const int valid = check_narrow(cfg);
    if (valid) return valid;
    if (n < 1 || m < 1 || p < 1) return fail(MF_E_INVALID, "invalid mm arguments");
    // The least scratch each read kernel can run in: the ideal kernel's digit masks,
    // or one 64-column chunk of noisy conductance terms (mf_mm runs wider noisy
    // reads chunk by chunk within the scratch it is given).
    i64 need = 0;
    const char *what = "";
    IdealPlan plan;
    SlotTests xt, wt;
    NoisyPlan noisy;
    int ks = 0;
    const char *why = "";
    if (!g && packed_t && build_ideal_plan(cfg, m, p, &plan, &xt, &wt, &ks, &why)) {
        i64 xb = 0, wb = 0;
        ideal_workspace(cfg, n, m, p, &xb, &wb);
        need = xb + wb;
        what = "digit masks of the ideal-device read";
    } else if (!g && packed_t && build_noisy_plan(cfg, m, p, &noisy, &ks, &why)) {
        need = noisy_voltage_bytes(cfg, n, m) + 2 * noisy_block_bytes(cfg, m);
        what = cfg->has_vnoise ? "voltage-noise operands and one 64-column chunk of noisy "
                                 "conductance terms"
                               : "one 64-column chunk of noisy conductance terms";
    }
    if (need > MF_STATIC_SCRATCH_BYTES)
        return fail(MF_E_RESOURCE,
                    "mf_mm_static needs %lld bytes of scratch for the %s; its static scratch "
                    "holds %lld (MF_STATIC_SCRATCH_BYTES)",
                    static_cast<long long>(need), what,
                    static_cast<long long>(MF_STATIC_SCRATCH_BYTES));
    void *ptr = nullptr;
    const int found = static_scratch(&ptr);
    if (found) return found;
    // The scratch is shared by every call on this GPU, so it never holds this
    // program's conductance terms from an earlier call: sample them again.
    // Benchmark timing (hipEventCreate) stays off for this thread's call.
    variant &= ~MF_MM_REUSE_TERMS;
    const bool was_off = g_profile_off;
    g_profile_off = true;
    const int launched = mf_mm(cfg, q, xscale, n, m, packed, packed_t, wscale, p, out_cols,
                               k_rows, g, seed, event, out, ldo, ptr, MF_STATIC_SCRATCH_BYTES,
                               variant, status, stream);
    g_profile_off = was_off;
    return launched;
}

int mf_mm_totals(const mf_config *cfg, const uint8_t *q, int64_t n, int64_t m,
                 const uint8_t *packed_t, int64_t p, const float *g, uint32_t seed, uint64_t event,
                 float *totals, void *workspace, int64_t workspace_bytes, void *stream) {
    const int valid = check_narrow(cfg);
    if (valid) return valid;
    if (!q || !packed_t || !totals || !workspace || n < 1 || m < 1 || p < 1)
        return fail(MF_E_INVALID, "invalid totals arguments");
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(packed_t)) % 16)
        return fail(MF_E_INVALID, "codes must be 16-byte aligned");
    NoisyPlan noisy;
    int ks = 0;
    const char *why = "";
    if (!ideal_extent_ok(cfg, n, m, p) || !noisy_extent_ok(n, m, cfg) ||
        !build_noisy_plan(cfg, m, p, &noisy, &ks, &why))
        return fail(MF_E_UNSUPPORTED, "noisy MFMA read not applicable: %s", why);
    const i64 ncols = p * cfg->cols;
    return launch_noisy(cfg, noisy, ks, q, nullptr, n, m, packed_t, nullptr, p, g, seed, event,
                        totals, ncols, workspace, workspace_bytes, 1, nullptr,
                        static_cast<hipStream_t>(stream));
}

int mf_bias_add(float *out, int64_t n, int64_t o, int64_t ldo, const float *bias,
                uint32_t *status, void *stream) {
    if (!out || !bias || n < 1 || o < 1 || ldo < o) return fail(MF_E_INVALID, "invalid bias arguments");
    hipLaunchKernelGGL(k_bias_add, dim3(grid_for(n * o)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), out, n, o, ldo, bias, status,
                       u32(MF_STATUS_OUTPUT));
    return check_launch("bias add");
}

int mf_narrow_output(const double *in, int64_t n, int64_t cols, int64_t ld, float *out,
                     uint32_t *status, void *stream) {
    if (!in || !out || n < 1 || cols < 1 || ld < cols)
        return fail(MF_E_INVALID, "invalid output cast arguments");
    hipLaunchKernelGGL(k_narrow_f64, dim3(grid_for(n * cols)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), in, n, cols, ld, out, status,
                       u32(MF_STATUS_OUTPUT));
    return check_launch("output cast");
}

int mf_gru_gates(const float *inputs, int64_t ldi, const float *hidden, int64_t ldh,
                 const float *hx, int64_t ldx, float *out, int64_t ldo, int64_t n, int64_t width,
                 void *stream) {
    if (!inputs || !hidden || !hx || !out || n < 1 || width < 1 || ldi < 3 * width ||
        ldh < 3 * width || ldx < width || ldo < width)
        return fail(MF_E_INVALID, "invalid GRU gate arguments");
    hipLaunchKernelGGL(k_gru_gates, dim3(grid_for(n * width)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), inputs, ldi, hidden, ldh, hx, ldx, out, ldo,
                       n, width, nullptr, nullptr, 0u);
    return check_launch("GRU gates");
}

int mf_gru_sequence(const mf_config *cfg, int64_t steps, int32_t reverse, int64_t batch,
                    int64_t width, const float *projected, int64_t proj_step, int64_t proj_row,
                    const float *h0, int64_t ld_h0, int64_t gr, int64_t gc, uint32_t *work,
                    float *scale, uint8_t *q, float *xscale, const uint8_t *packed,
                    const uint8_t *packed_t, const float *wscale, int64_t m, int64_t p,
                    const float *bias, uint32_t seed, uint64_t event0, float *hidden,
                    int64_t ld_hidden, void *workspace, int64_t workspace_bytes, int32_t variant,
                    float *out, int64_t out_step, int64_t out_row, uint32_t *status,
                    void *stream) {
    const int valid = check_narrow(cfg);
    if (valid) return valid;
    if (!projected || !h0 || !q || !xscale || !scale || !packed || !wscale || !hidden || !out ||
        !status || steps < 1 || batch < 1 || width < 1 || m < 1 || p < 1)
        return fail(MF_E_INVALID, "invalid GRU sequence arguments");
    if (proj_row < 3 * width || proj_step < batch * proj_row || ld_h0 < width ||
        out_row < width || out_step < batch * out_row || ld_hidden < p * cfg->cols ||
        3 * width > p * cfg->cols || width > m * cfg->rows ||
        (width + cfg->rows - 1) / cfg->rows != m)
        return fail(MF_E_INVALID, "GRU sequence shapes do not match the hidden program");
    if (event0 > uint64_t(INT64_MAX) - uint64_t(steps))
        return fail(MF_E_INVALID, "read events of the sequence exceed the signed 64-bit range");
    hipStream_t s = static_cast<hipStream_t>(stream);
    // With one input group per state row, each step after its read is one k_gru_step: the
    // split read's restore and sum, the gates, and the next read's input codes.  Otherwise
    // the step quantizes, reads (restoring its own totals) and runs k_gru_gates.
    const i64 G = m * cfg->reads, ncols = p * cfg->cols;
    const bool fused = (gr < batch ? gr : batch) == 1 && (gc < width ? gc : width) == width &&
                       (scale != xscale || G == 1) && width <= 5120;   // 3H floats of LDS, under 64 KiB
    for (i64 i = 0; i < steps; ++i) {
        const i64 t = reverse ? steps - 1 - i : i;
        const float *hx = i == 0 ? h0 : out + (reverse ? t + 1 : t - 1) * out_step;
        const i64 ldx = i == 0 ? ld_h0 : out_row;
        int rc = MF_OK;
        if (i == 0 || !fused) {
            rc = mf_quantize_inputs(cfg, hx, batch, width, ldx, gr, gc, work, scale, q, xscale,
                                    status, stream);
            if (rc) return rc;
        }
        // The first read writes the program's event-independent conductance terms
        // into the workspace (unless the caller's variant says they are there);
        // later reads of the same program reuse them.
        const int32_t v = i == 0 ? variant : (variant | MF_MM_REUSE_TERMS);
        const float *totals = nullptr;
        bool restored = false;
        rc = mm_read(cfg, q, xscale, batch, m, packed, packed_t, wscale, p, 3 * width, width,
                     nullptr, seed, event0 + uint64_t(i), hidden, ld_hidden, workspace,
                     workspace_bytes, v, status, stream, fused ? &totals : nullptr,
                     fused ? &restored : nullptr);
        if (rc) return rc;
        if (fused) {
            GruStepArgs a{};
            a.inputs = projected + t * proj_step;
            a.ldi = proj_row;
            a.hidden = hidden;
            a.ldh = ld_hidden;
            a.totals = totals;
            a.restored = restored;
            a.G = G;
            a.g_run = reads_with_rows(cfg, m, width);
            a.ldt = ncols;
            a.lp = level_power(G);
            a.xscale_in = xscale;
            a.wscale = wscale;
            a.ldws = ncols;
            a.bias = bias;
            a.hx = hx;
            a.ldx = ldx;
            a.out = out + t * out_step;
            a.ldo = out_row;
            a.width = width;
            a.quantize = i + 1 < steps;
            a.kp = m * cfg->rows;
            a.upper = float((1 << (cfg->activation_bits - 1)) - 1);
            a.mask = (1u << cfg->activation_bits) - 1u;
            a.q = q;
            a.scale = scale;
            a.xscale_out = xscale;
            a.status = status;
            // One thread per hidden unit (up to 1024; more units loop).
            const unsigned threads = unsigned(width >= 1024 ? 1024 : (width + 63) / 64 * 64);
            hipLaunchKernelGGL(k_gru_step, dim3(unsigned(batch)), dim3(threads), width * 4, s, a);
        } else {
            hipLaunchKernelGGL(k_gru_gates, dim3(grid_for(batch * width)), dim3(256), 0, s,
                               projected + t * proj_step, proj_row, hidden, ld_hidden, hx, ldx,
                               out + t * out_step, out_row, batch, width, bias, status,
                               u32(MF_STATUS_OUTPUT));
        }
        rc = check_launch("GRU sequence gates");
        if (rc) return rc;
    }
    return MF_OK;
}

int mf_stable_sum(const mf_config *cfg, const float *totals, int64_t n, int64_t G, int64_t width,
                  const float *xscale, const float *wscale, int64_t ldws, int64_t col0, double *out,
                  int64_t ldo, void *stream) {
    const int valid = check_narrow(cfg);
    if (valid) return valid;
    const i64 wc = width * cfg->cols;
    if (!totals || !xscale || !wscale || !out || n < 1 || G < 1 || width < 1 || col0 < 0 ||
        ldws < col0 + wc || ldo < col0 + wc || G > 0x7FFFFFFF)
        return fail(MF_E_INVALID, "invalid stable-sum arguments");
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(k_stable_sum, dim3(grid_for(n * wc)), dim3(256), 0, s, totals, n, G, wc,
                       xscale, wscale, ldws, col0, out, ldo, level_power(G), level_power(G / 4));
    return check_launch("stable sum");
}

}  // extern "C"

// Group maxima |x| of an FP64 matrix (S = float: FP32 values, widened exactly) into
// work[row group][col group] (cleared).
template <typename S>
static void launch_group_max_f64(const S *x, i64 rows, i64 cols, i64 ld, i64 gr, i64 gc,
                                 i64 ncg, u64 *work, u32 *status, u32 flag, hipStream_t s) {
    constexpr int V = 16 / sizeof(S);   // columns per lane of the vector path
    const i64 chunks = (rows + COL_CHUNK_ROWS - 1) / COL_CHUNK_ROWS;
    const i64 row_chunks = (cols + ROW_CHUNK_COLS - 1) / ROW_CHUNK_COLS;
    unsigned long long *w = reinterpret_cast<unsigned long long *>(work);
    const bool vec_ok = cols % V == 0 && ld % V == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (gr == 1 && gc >= 64 && (rows + 3) / 4 <= 65535 && row_chunks <= 2147483647) {
        hipLaunchKernelGGL((k_row_group_max<double, unsigned long long, S>),
                           dim3(unsigned(row_chunks), unsigned((rows + 3) / 4)), dim3(256), 0, s, x,
                           rows, cols, ld, gc, ncg, w, status, flag);
    } else if ((gr > 1 || gc == 1) && vec_ok && (cols + 64 * V - 1) / (64 * V) <= 2147483647 &&
               (rows + COL_CHUNK_ROWS_VEC - 1) / COL_CHUNK_ROWS_VEC <= 65535) {
        hipLaunchKernelGGL((k_col_group_max<double, unsigned long long, V, S>),
                           dim3(unsigned((cols + 64 * V - 1) / (64 * V)),
                                unsigned((rows + COL_CHUNK_ROWS_VEC - 1) / COL_CHUNK_ROWS_VEC)),
                           dim3(256), 0, s, x, rows, cols, ld, gr, gc, ncg, i64(COL_CHUNK_ROWS_VEC),
                           w, status, flag);
    } else if ((gr > 1 || gc == 1) && (cols + 63) / 64 <= 2147483647 && chunks <= 65535) {
        hipLaunchKernelGGL((k_col_group_max<double, unsigned long long, 1, S>),
                           dim3(unsigned((cols + 63) / 64), unsigned(chunks)), dim3(256), 0, s, x,
                           rows, cols, ld, gr, gc, ncg, i64(COL_CHUNK_ROWS), w, status, flag);
    } else {
        hipLaunchKernelGGL(k_group_max_f64<S>, dim3(grid_for(rows * cols)), dim3(256), 0, s, x,
                           rows, cols, ld, gr, gc, ncg, work, status, flag);
    }
}

// Largest group scale of a wide operand below which no read of G reads can leave an output
// beyond FLT_MAX / 2 once cast to FP32: every read's slice total obeys
// |T| <= sum|fa| * sum|fw| * adc_max (the ADC clamps each count), so with input and weight
// scales below s the FP64 sum of G restores is at most G * Tmax * s^2 (times 1 + 2^-50 for
// its roundings).  Scales above it flag MF_STATUS_RANGE (the caller then reads the status
// word after the read instead of returning on the quantizers' bits).
static double wide_scale_bound(const mf_config *cfg, i64 G) {
    double fa = 0.0, fw = 0.0;
    for (int a = 0; a < cfg->n_in; ++a) fa += std::fabs(double(cfg->in_factor[a]));
    for (int w = 0; w < cfg->n_w; ++w)
        fw += std::fabs(double(cfg->w_factor[w])) * double(cfg->adc_max[w]);
    return std::sqrt(double(FLT_MAX) / (2.0 * double(G) * std::max(fa * fw, 1.0)));
}

// ---- wide configurations (u32 codes, FP64 scales and outputs) -------------
// The wide quantizers over FP64 operands, or FP32 ones (S = float) widened exactly as they
// are read, which gives the codes and scales of the FP64 copy without making it.
template <typename S>
static int quantize_inputs_wide(const mf_config *cfg, const S *x, int64_t n, int64_t k,
                                int64_t ld, int64_t gr, int64_t gc, uint64_t *work, double *scale,
                                uint32_t *q, double *xscale, uint32_t *status, void *stream) {
    const int valid = check_wide(cfg);
    if (valid) return valid;
    if (!x || !work || !scale || !q || !xscale || n < 1 || k < 1 || ld < k || gr < 1 || gc < 1)
        return fail(MF_E_INVALID, "invalid input quantization arguments");
    const int R = cfg->rows, P = cfg->read_rows, Gr = cfg->reads;
    const i64 m = (k + R - 1) / R, kp = m * R;
    gr = gr < n ? gr : n;
    gc = gc < k ? gc : k;
    const i64 nrg = (n + gr - 1) / gr, ncg = (k + gc - 1) / gc;
    const int bits = cfg->activation_bits;
    const double upper = double((i64(1) << (bits - 1)) - 1);
    const double lower = cfg->bw_e ? -double(i64(1) << (bits - 1)) : -upper;
    const u64 mask = bits == 64 ? ~u64(0) : (u64(1) << bits) - 1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(2 * nrg * ncg)), dim3(256), 0, s,
                       reinterpret_cast<u32 *>(work), 2 * nrg * ncg, 0u);
    launch_group_max_f64(x, n, k, ld, gr, gc, ncg, work, status, u32(MF_STATUS_INPUT), s);
    const int narrow = bits <= 8 && !cfg->bw_e;   // FP32 quantization, as the reference's
    hipLaunchKernelGGL(k_group_scale_f64, dim3(grid_for(nrg * ncg)), dim3(256), 0, s, work,
                       nrg * ncg, bits, cfg->bw_e, upper, narrow, scale,
                       wide_scale_bound(cfg, ((k) + R - 1) / R * Gr), status);
    hipLaunchKernelGGL(k_input_codes_f64<S>, dim3(grid_for(n * kp)), dim3(256), 0, s, x, n, k, ld,
                       kp, scale, gr, gc, ncg, 0, lower, upper, mask, narrow, q);
    hipLaunchKernelGGL(k_input_scales_f64, dim3(grid_for(n * m * Gr)), dim3(256), 0, s, n, k,
                       m * Gr, R, P, Gr, scale, gr, gc, ncg, 0, xscale);
    return check_launch("wide input quantization");
}

template <typename S>
static int quantize_weights_wide(const mf_config *cfg, const S *b, int64_t k, int64_t o,
                                 int64_t ld, int64_t gr, int64_t gc, uint64_t *work, double *scale,
                                 int64_t *packed, uint32_t *packed32, double *wscale,
                                 uint32_t *status, void *stream) {
    const int valid = check_wide(cfg);
    if (valid) return valid;
    if (!b || !work || !scale || !packed || !packed32 || !wscale || k < 1 || o < 1 || ld < o ||
        gr < 1 || gc < 1)
        return fail(MF_E_INVALID, "invalid weight quantization arguments");
    const int R = cfg->rows, C = cfg->cols, P = cfg->read_rows, Gr = cfg->reads;
    const i64 m = (k + R - 1) / R, p = (o + C - 1) / C, kp = m * R, op = p * C;
    gr = gr < k ? gr : k;
    gc = gc < o ? gc : o;
    const i64 nrg = (k + gr - 1) / gr, ncg = (o + gc - 1) / gc;
    const int bits = cfg->weight_bits;
    const bool is_signed = cfg->weight_signed != 0;
    const double upper = double((i64(1) << (bits - (is_signed ? 1 : 0))) - 1);
    const double lower = cfg->bw_e ? -double(i64(1) << (bits - 1)) : (is_signed ? -upper : 0.0);
    const u64 mask = (u64(1) << bits) - 1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(2 * nrg * ncg)), dim3(256), 0, s,
                       reinterpret_cast<u32 *>(work), 2 * nrg * ncg, 0u);
    launch_group_max_f64(b, k, o, ld, gr, gc, ncg, work, status, u32(MF_STATUS_WEIGHT), s);
    const int narrow = bits <= 8 && !cfg->bw_e;   // FP32 quantization, as the reference's
    hipLaunchKernelGGL(k_group_scale_f64, dim3(grid_for(nrg * ncg)), dim3(256), 0, s, work,
                       nrg * ncg, bits, cfg->bw_e, upper, narrow, scale,
                       wide_scale_bound(cfg, ((k) + R - 1) / R * Gr), status);
    hipLaunchKernelGGL(k_weight_codes_f64<S>, dim3(grid_for(kp * op)), dim3(256), 0, s, b, k, o,
                       ld, R, C, m, p, scale, gr, gc, ncg, lower, upper, mask, narrow, packed,
                       packed32);
    hipLaunchKernelGGL(k_weight_scales_f64, dim3(grid_for(m * Gr * op)), dim3(256), 0, s, k, o,
                       m * Gr, op, R, P, Gr, scale, gr, gc, ncg, wscale);
    return check_launch("wide weight quantization");
}

extern "C" {

int mf_quantize_inputs_wide(const mf_config *cfg, const double *x, int64_t n, int64_t k,
                            int64_t ld, int64_t gr, int64_t gc, uint64_t *work, double *scale,
                            uint32_t *q, double *xscale, uint32_t *status, void *stream) {
    return quantize_inputs_wide(cfg, x, n, k, ld, gr, gc, work, scale, q, xscale, status, stream);
}

int mf_quantize_inputs_wide_f32(const mf_config *cfg, const float *x, int64_t n, int64_t k,
                                int64_t ld, int64_t gr, int64_t gc, uint64_t *work, double *scale,
                                uint32_t *q, double *xscale, uint32_t *status, void *stream) {
    return quantize_inputs_wide(cfg, x, n, k, ld, gr, gc, work, scale, q, xscale, status, stream);
}

int mf_input_tiles_wide(const mf_config *cfg, const double *x, int64_t n, int64_t k, int64_t ld,
                        const double *scale, uint32_t *q, double *xscale, void *stream) {
    const int valid = check_wide(cfg);
    if (valid) return valid;
    if (!x || !scale || !q || !xscale || n < 1 || k < 1 || ld < k)
        return fail(MF_E_INVALID, "invalid input-tile arguments");
    const int R = cfg->rows, P = cfg->read_rows, Gr = cfg->reads;
    const i64 m = (k + R - 1) / R, kp = m * R;
    const int bits = cfg->activation_bits;
    const double upper = double((i64(1) << (bits - 1)) - 1);
    const double lower = cfg->bw_e ? -double(i64(1) << (bits - 1)) : -upper;
    const u64 mask = (u64(1) << bits) - 1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(k_input_codes_f64<double>, dim3(grid_for(n * kp)), dim3(256), 0, s, x, n, k, ld, kp,
                       scale, i64(1), i64(1), k, 1, lower, upper, mask, 0, q);
    hipLaunchKernelGGL(k_input_scales_f64, dim3(grid_for(n * m * Gr)), dim3(256), 0, s, n, k,
                       m * Gr, R, P, Gr, scale, i64(1), i64(1), k, 1, xscale);
    return check_launch("wide input tiles");
}

int mf_quantize_weights_wide(const mf_config *cfg, const double *b, int64_t k, int64_t o,
                             int64_t ld, int64_t gr, int64_t gc, uint64_t *work, double *scale,
                             int64_t *packed, uint32_t *packed32, double *wscale, uint32_t *status,
                             void *stream) {
    return quantize_weights_wide(cfg, b, k, o, ld, gr, gc, work, scale, packed, packed32, wscale,
                                 status, stream);
}

int mf_quantize_weights_wide_f32(const mf_config *cfg, const float *b, int64_t k, int64_t o,
                                 int64_t ld, int64_t gr, int64_t gc, uint64_t *work, double *scale,
                                 int64_t *packed, uint32_t *packed32, double *wscale,
                                 uint32_t *status, void *stream) {
    return quantize_weights_wide(cfg, b, k, o, ld, gr, gc, work, scale, packed, packed32, wscale,
                                 status, stream);
}

int mf_restore_wide(const mf_config *cfg, const uint32_t *packed, int64_t m, int64_t p,
                    int64_t begin, int64_t end, uint32_t seed, uint64_t event, void *g,
                    void *stream) {
    const int valid = check_wide(cfg);
    if (valid) return valid;
    if (!packed || !g || m < 1 || p < 1 || begin < 0 || end <= begin || end > p)
        return fail(MF_E_INVALID, "invalid restore arguments");
    const int planes = restore_planes(cfg);
    const i64 total = i64(planes) * m * (end - begin) * cfg->n_w * cfg->rows * cfg->cols;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (cfg->precise)
        hipLaunchKernelGGL((k_restore<double, u32>), dim3(grid_for(total)), dim3(256), 0, s, *cfg,
                           packed, m, p, begin, end - begin, seed, event, planes,
                           static_cast<double *>(g));
    else
        hipLaunchKernelGGL((k_restore<float, u32>), dim3(grid_for(total)), dim3(256), 0, s, *cfg,
                           packed, m, p, begin, end - begin, seed, event, planes,
                           static_cast<float *>(g));
    return check_launch("wide restore");
}

int mf_partial_wide(const mf_config *cfg, const uint32_t *q, int64_t n, int64_t m,
                    const uint32_t *packed, int64_t p, int64_t begin, int64_t end, const void *g,
                    uint32_t seed, uint64_t event, double *totals, int32_t *codes, void *stream) {
    const int valid = check_wide(cfg);
    if (valid) return valid;
    if (!q || !packed || !totals || n < 1 || m < 1 || p < 1 || begin < 0 || end <= begin || end > p)
        return fail(MF_E_INVALID, "invalid partial arguments");
    if (!g && needs_conductances(cfg))
        return fail(MF_E_INVALID, "device noise needs restored conductances (g)");
    GeneralArgs args{};
    args.q = q;
    args.packed = packed;
    args.g = g;
    args.out = totals;
    args.codes = codes;
    args.n = n;
    args.m = m;
    args.p = p;
    args.begin = begin;
    args.width = end - begin;
    args.seed = seed;
    args.event = event;
    args.planes = g ? restore_planes(cfg) : 1;
    const i64 G = m * cfg->reads;
    args.lp_cascade = level_power(G);
    args.lp_interleaved = level_power(G / 4);
    hipStream_t s = static_cast<hipStream_t>(stream);
    return launch_general_read(cfg, args, OUT_TOTALS, s);
}

int mf_mm_wide(const mf_config *cfg, const uint32_t *q, const double *xscale, int64_t n, int64_t m,
               const uint32_t *packed, const double *wscale, int64_t p, const void *g,
               uint32_t seed, uint64_t event, double *out, int64_t ldo, void *workspace,
               int64_t workspace_bytes, int32_t variant, uint32_t *status, void *stream) {
    const int valid = check_wide(cfg);
    if (valid) return valid;
    if (!variant_valid(variant)) return fail(MF_E_INVALID, "unknown kernel variant 0x%x", variant);
    if (!q || !xscale || !packed || !wscale || !out || n < 1 || m < 1 || p < 1 ||
        ldo < p * cfg->cols)
        return fail(MF_E_INVALID, "invalid mm arguments");
    NoisyWidePlan wplan;
    int ks = 0;
    const char *why = "";
    if (!g && workspace && (reinterpret_cast<uintptr_t>(workspace) % 256) == 0 &&
        wide_extent_ok(n, m, cfg) && build_noisy_wide_plan(cfg, m, p, &wplan, &ks, &why) &&
        workspace_bytes >= wide_prefix_bytes(n, m, cfg) + 2 * wide_block_bytes(cfg, m)) {
        hipStream_t s = static_cast<hipStream_t>(stream);
        std::pair<hipEvent_t, hipEvent_t> timing{nullptr, nullptr};
        if (profiling() && (timing = profile_pair()).first) hipEventRecord(timing.first, s);
        const int launched = launch_noisy_wide(cfg, wplan, ks, q, xscale, n, m, packed,
                                               wscale, p, nullptr, seed, event, out, ldo,
                                               workspace, workspace_bytes, 0, status, s,
                                               variant_tier(variant));
        if (timing.first) {
            hipEventRecord(timing.second, s);
            profile_push(timing);
        }
        return launched;
    }
    if (!g && needs_conductances(cfg))
        return fail(MF_E_INVALID, "device noise needs restored conductances (g)");
    GeneralArgs args{};
    args.q = q;
    args.packed = packed;
    args.g = g;
    args.xscale = xscale;
    args.wscale = wscale;
    args.out = out;
    args.status = status;
    args.n = n;
    args.m = m;
    args.p = p;
    args.begin = 0;
    args.width = p;
    args.ldo = ldo;
    args.ldws = p * cfg->cols;
    args.seed = seed;
    args.event = event;
    args.planes = g ? restore_planes(cfg) : 1;
    const i64 G = m * cfg->reads;
    args.lp_cascade = level_power(G);
    args.lp_interleaved = level_power(G / 4);
    hipStream_t s = static_cast<hipStream_t>(stream);
    std::pair<hipEvent_t, hipEvent_t> timing{nullptr, nullptr};
    if (profiling() && (timing = profile_pair()).first) hipEventRecord(timing.first, s);
    const int launched = launch_general_read(cfg, args, OUT_FUSED, s);
    if (timing.first) {
        hipEventRecord(timing.second, s);
        profile_push(timing);
    }
    return launched;
}

int mf_mm_totals_wide(const mf_config *cfg, const uint32_t *q, int64_t n, int64_t m,
                      const uint32_t *packed, int64_t p, const float *g, uint32_t seed,
                      uint64_t event, double *totals, void *workspace, int64_t workspace_bytes,
                      void *stream) {
    const int valid = check_wide(cfg);
    if (valid) return valid;
    if (!q || !packed || !totals || !workspace || n < 1 || m < 1 || p < 1)
        return fail(MF_E_INVALID, "invalid totals arguments");
    if (reinterpret_cast<uintptr_t>(workspace) % 256)
        return fail(MF_E_INVALID, "workspace must be 256-byte aligned");
    NoisyWidePlan plan;
    int ks = 0;
    const char *why = "";
    if (!wide_extent_ok(n, m, cfg) || !build_noisy_wide_plan(cfg, m, p, &plan, &ks, &why))
        return fail(MF_E_UNSUPPORTED, "wide MFMA read not applicable: %s", why);
    if (workspace_bytes < wide_prefix_bytes(n, m, cfg) + 2 * wide_block_bytes(cfg, m))
        return fail(MF_E_RESOURCE, "workspace below one 64-column chunk");
    const i64 ncols = p * cfg->cols;
    return launch_noisy_wide(cfg, plan, ks, q, nullptr, n, m, packed, nullptr, p, g, seed,
                             event, totals, ncols, workspace, workspace_bytes, 1, nullptr,
                             static_cast<hipStream_t>(stream));
}

int mf_profile_kernels(int32_t enable) {
    g_profile.enabled.store(enable != 0);
    return MF_OK;
}

int mf_profile_collect(int64_t *launches, double *milliseconds) {
    if (!launches || !milliseconds) return fail(MF_E_INVALID, "profile outputs are NULL");
    *launches = 0;
    *milliseconds = 0.0;
    int status = MF_OK;
    std::lock_guard<std::mutex> guard(g_profile.lock);
    for (auto &pair : g_profile.pending) {
        float ms = 0.0f;
        hipError_t e = hipEventSynchronize(pair.second);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, pair.first, pair.second);
        if (e != hipSuccess && status == MF_OK)
            status = fail(MF_E_HIP, "kernel timing failed: %s", hipGetErrorString(e));
        *milliseconds += ms;
        ++*launches;
        g_profile.spare.push_back(pair);
    }
    g_profile.pending.clear();
    return status;
}

int mf_resources_query(const mf_config *cfg, int32_t kernel_id, int64_t n, int32_t variant,
                       mf_resources *out) {
    int status = check_config(cfg);
    if (status) return status;
    if (!out) return fail(MF_E_INVALID, "resources output is NULL");
    if (!variant_valid(variant)) return fail(MF_E_INVALID, "unknown kernel variant 0x%x", variant);
    // The instance of the read kernel that mf_mm (mf_mm_wide) launches for this descriptor
    // and schedule (`variant`), chosen as launch_ideal, launch_noisy, launch_noisy_wide and
    // launch_general choose it.
    const bool nl = cfg->has_nonlinear != 0;
    const bool ks4 = cfg->read_rows == 64;
    const bool output_noise = cfg->has_read && cfg->read_mode == MF_READ_OUTPUT;
    const void *fn = nullptr;
    int threads = 256;
    if (kernel_id == 1) {
        // 32-row reads: 32 or (tile field 1) 64 vectors per wave; 64-row reads: KS 2.
        if (ks4) fn = reinterpret_cast<const void *>(&k_ideal<1, 2>);
        else if (variant_tile(variant) == 1) fn = reinterpret_cast<const void *>(&k_ideal<2, 1>);
        else fn = reinterpret_cast<const void *>(&k_ideal<1, 1>);
    } else if (kernel_id == 2) {
        // ks index 0: KS 2 with up to 5 slices, 1: KS 2 with 8, 2: KS 4.  The read split
        // does not change the instance.
#define MF_NOISY_FN(KS, NA, NL, VN, SL, ON) \
    reinterpret_cast<const void *>(&k_noisy<KS, NA, NL, VN, SL, ON>)
#define MF_NOISY_ROW(KS, NA)                                                                      \
    {{{MF_NOISY_FN(KS, NA, false, false, false, false), MF_NOISY_FN(KS, NA, true, false, false, false)}, \
      {MF_NOISY_FN(KS, NA, false, false, true, false), MF_NOISY_FN(KS, NA, true, false, true, false)}},  \
     {{MF_NOISY_FN(KS, NA, false, true, false, false), MF_NOISY_FN(KS, NA, true, true, false, false)},   \
      {MF_NOISY_FN(KS, NA, false, true, true, false), MF_NOISY_FN(KS, NA, true, true, true, false)}},    \
     {{MF_NOISY_FN(KS, NA, false, false, false, true), MF_NOISY_FN(KS, NA, true, false, false, true)},   \
      {MF_NOISY_FN(KS, NA, false, false, false, true), MF_NOISY_FN(KS, NA, true, false, false, true)}},  \
     {{MF_NOISY_FN(KS, NA, false, true, false, true), MF_NOISY_FN(KS, NA, true, true, false, true)},     \
      {MF_NOISY_FN(KS, NA, false, true, false, true), MF_NOISY_FN(KS, NA, true, true, false, true)}}}
        // [ks][plain, voltage, output, output and voltage noise][slice_pair][nonlinear]
        const void *table[3][4][2][2] = {MF_NOISY_ROW(2, 5), MF_NOISY_ROW(2, 8),
                                         MF_NOISY_ROW(4, 5)};
#undef MF_NOISY_ROW
#undef MF_NOISY_FN
        const int which = ks4 ? 2 : (cfg->n_in <= 5 ? 0 : 1);
        const int mode = output_noise ? (cfg->has_vnoise ? 3 : 2) : (cfg->has_vnoise ? 1 : 0);
        const bool slice = cfg->has_read && cfg->read_mode == MF_READ_SLICE_PAIR;
        fn = table[which][mode][slice ? 1 : 0][nl ? 1 : 0];
        if (n > 0 && noisy_small_tile(cfg, n) && variant_split(variant) != 1) {
            // A split read of at most 32 vectors (the automatic split applies below 512
            // four-wave blocks, 32768 output columns): k_noisy_pairs, one wave per weight
            // slice.
            const void *pairs[3][2] = {
                {reinterpret_cast<const void *>(&k_noisy_pairs<2, 5, false>),
                 reinterpret_cast<const void *>(&k_noisy_pairs<2, 5, true>)},
                {reinterpret_cast<const void *>(&k_noisy_pairs<2, 8, false>),
                 reinterpret_cast<const void *>(&k_noisy_pairs<2, 8, true>)},
                {reinterpret_cast<const void *>(&k_noisy_pairs<4, 5, false>),
                 reinterpret_cast<const void *>(&k_noisy_pairs<4, 5, true>)}};
            fn = pairs[which][nl ? 1 : 0];
            threads = 64 * cfg->n_w;
        }
    } else if (kernel_id == 3) {
        // The LDS tier: the schedule's (tier field 1-3), else launch_noisy_wide's automatic one.
        const int frags = cfg->n_w * NOISY_TERMS * (ks4 ? 4 : 2);
        int tier = frags > WIDE_FRAGS_SMALL ? 2 : frags > WIDE_FRAGS_TINY ? 1 : 0;
        if (variant_tier(variant) > 0) tier = variant_tier(variant) - 1;
        const bool vn = cfg->has_vnoise != 0;
        const bool sl = wide_term_planes(cfg) > 1;   // slice_pair: an LDS unit per input slice
#define MF_WIDE_FN2(KS, FR, SL)                                                                  \
    (vn ? (nl ? reinterpret_cast<const void *>(&k_noisy_wide<KS, true, FR, true, SL>)             \
              : reinterpret_cast<const void *>(&k_noisy_wide<KS, false, FR, true, SL>))           \
        : (nl ? reinterpret_cast<const void *>(&k_noisy_wide<KS, true, FR, false, SL>)            \
              : reinterpret_cast<const void *>(&k_noisy_wide<KS, false, FR, false, SL>)))
#define MF_WIDE_FN(KS, FR) (sl ? MF_WIDE_FN2(KS, FR, true) : MF_WIDE_FN2(KS, FR, false))
        if (ks4) fn = tier == 2 ? MF_WIDE_FN(4, WIDE_FRAGS_LARGE)
                      : tier == 1 ? MF_WIDE_FN(4, WIDE_FRAGS_SMALL) : MF_WIDE_FN(4, WIDE_FRAGS_TINY);
        else fn = tier == 2 ? MF_WIDE_FN(2, WIDE_FRAGS_LARGE)
                  : tier == 1 ? MF_WIDE_FN(2, WIDE_FRAGS_SMALL) : MF_WIDE_FN(2, WIDE_FRAGS_TINY);
#undef MF_WIDE_FN
#undef MF_WIDE_FN2
    } else if (kernel_id == 0) {
#define MF_GENERAL_FN(WIDE)                                                                      \
    (cfg->precise                                                                                \
         ? (precise_mfma_ok(cfg)                                                                 \
                ? (restore_planes(cfg) == 1 && cfg->n_w <= MFMA64_STAGED_MAX_W                   \
                       ? reinterpret_cast<const void *>(&k_general_mfma64<WIDE, true>)           \
                       : reinterpret_cast<const void *>(&k_general_mfma64<WIDE, false>))         \
            : output_noise ? reinterpret_cast<const void *>(&k_general<double, 2, true, WIDE>)    \
                         : reinterpret_cast<const void *>(&k_general<double, 4, false, WIDE>))    \
         : (output_noise ? reinterpret_cast<const void *>(&k_general<float, 2, true, WIDE>)       \
                         : reinterpret_cast<const void *>(&k_general<float, 8, false, WIDE>)))
        fn = cfg->wide ? MF_GENERAL_FN(true) : MF_GENERAL_FN(false);
#undef MF_GENERAL_FN
    } else {
        return fail(MF_E_INVALID, "unknown read kernel %d", kernel_id);
    }
    hipFuncAttributes attr;
    const hipError_t e = hipFuncGetAttributes(&attr, fn);
    if (e != hipSuccess) return fail(MF_E_HIP, "hipFuncGetAttributes: %s", hipGetErrorString(e));
    memset(out, 0, sizeof(*out));
    out->threads = threads;
    out->shared_bytes = int32_t(attr.sharedSizeBytes);
    out->registers = attr.numRegs;
    out->local_bytes = int32_t(attr.localSizeBytes);
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, threads, 0) == hipSuccess)
        out->max_blocks_per_cu = blocks;
    if (blocks == 0) return fail(MF_E_RESOURCE, "zero resident blocks");
    return MF_OK;
}

int mf_rng_uniform(const uint64_t *address, int64_t count, uint64_t seed, uint32_t stream,
                   float *out, void *stream_handle) {
    if (!address || !out || count < 0) return fail(MF_E_INVALID, "invalid rng arguments");
    if (count == 0) return MF_OK;
    hipLaunchKernelGGL(k_rng, dim3(grid_for(count)), dim3(256), 0,
                       static_cast<hipStream_t>(stream_handle), reinterpret_cast<const u64 *>(address),
                       count, u64(seed), stream, 0, 6.2831854820251465f, out);
    return check_launch("rng uniform");
}

int mf_rng_normal(const uint64_t *address, int64_t count, uint64_t seed, uint32_t stream,
                  float *out, void *stream_handle) {
    if (!address || !out || count < 0) return fail(MF_E_INVALID, "invalid rng arguments");
    if (count == 0) return MF_OK;
    hipLaunchKernelGGL(k_rng, dim3(grid_for(count)), dim3(256), 0,
                       static_cast<hipStream_t>(stream_handle), reinterpret_cast<const u64 *>(address),
                       count, u64(seed), stream, 1, 6.2831854820251465f, out);
    return check_launch("rng normal");
}

}  // extern "C"
