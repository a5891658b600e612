/*
 * Scalar C restatement of the ideal-device slice model and of the integer
 * part of the counter-based RNG (TEST INFRASTRUCTURE ONLY).
 *
 * It is an independent second restatement used to pin oracle/oracle.py:
 *   - ideal ADC counts: code = min(sum_r da*dw, max_w) for every input slice a,
 *     weight slice w and read group (memfast/reference.py:63-117 with every
 *     nonideality off; docs/user-guide.md:330-345),
 *   - T[n, i*Gr+j, t, c] = sum_a sum_w fa*fw*code  (memfast/reference.py:115),
 *   - the lowbias32-style hash, 24-bit uniform and event seed
 *     (memfast/random.py:8-27).
 * Loaded with ctypes from the CPU tests; never linked into the product.
 */
#include <stdint.h>

uint32_t brute_mix(uint32_t x) {
    x ^= x >> 16; x *= 0x7feb352du;
    x ^= x >> 15; x *= 0x846ca68bu;
    return x ^ (x >> 16);
}

/* Returns the 24-bit integer h>>8; the uniform is (h + 0.5) / 2^24. */
uint32_t brute_uniform_bits(uint64_t address, uint64_t seed, uint32_t stream) {
    uint32_t key = brute_mix((uint32_t)seed ^ (uint32_t)(stream * 0x9e3779b9u));
    uint32_t hi = (uint32_t)(address >> 32);
    uint32_t fold = brute_mix(hi ^ brute_mix((uint32_t)(seed >> 32)));
    if (hi != 0) fold ^= brute_mix(hi ^ key);
    return brute_mix((uint32_t)address ^ fold ^ key) >> 8;
}

uint64_t brute_event_seed(uint32_t seed, uint64_t event) {
    return (uint64_t)(seed ^ brute_mix((uint32_t)event)) |
           ((uint64_t)brute_mix((uint32_t)(event >> 32)) << 32);
}

/*
 * q:      [n][m][R]     codes (two's complement masked to the activation bits)
 * packed: [m][p][R][C]  codes (masked to the weight bits)
 * uint8 codes (brute_ideal_totals) or int64 codes of wide configurations
 * (brute_ideal_totals_wide); totals: int64 [n][m*Gr][p][C]
 */
static int64_t code_at(const void *codes, int wide, int64_t index) {
    return wide ? ((const int64_t *)codes)[index] : (int64_t)((const uint8_t *)codes)[index];
}

static void ideal_totals(const void *q, const void *packed, int wide, int n, int m, int p,
                         int R, int C, int P, int na, const int *ashift, const int64_t *amask,
                         const int64_t *afac, int nw, const int *wshift, const int64_t *wmask,
                         const int64_t *wfac, const int64_t *maxima, int64_t *totals) {
    int gr = (R + P - 1) / P;
    for (int v = 0; v < n; ++v)
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < gr; ++j) {
                int lo = j * P, hi = lo + P < R ? lo + P : R;
                for (int t = 0; t < p; ++t)
                    for (int c = 0; c < C; ++c) {
                        int64_t total = 0;
                        for (int a = 0; a < na; ++a)
                            for (int w = 0; w < nw; ++w) {
                                int64_t s = 0;
                                for (int r = lo; r < hi; ++r) {
                                    int64_t da = (code_at(q, wide, ((int64_t)v * m + i) * R + r)
                                                  >> ashift[a]) & amask[a];
                                    int64_t dw = (code_at(packed, wide,
                                                          (((int64_t)i * p + t) * R + r) * C + c)
                                                  >> wshift[w]) & wmask[w];
                                    s += da * dw;
                                }
                                if (s > maxima[w]) s = maxima[w];
                                total += afac[a] * wfac[w] * s;
                            }
                        totals[(((int64_t)v * m * gr + i * gr + j) * p + t) * C + c] = total;
                    }
            }
}

void brute_ideal_totals(const uint8_t *q, const uint8_t *packed, int n, int m, int p, int R,
                        int C, int P, int na, const int *ashift, const int64_t *amask,
                        const int64_t *afac, int nw, const int *wshift, const int64_t *wmask,
                        const int64_t *wfac, const int64_t *maxima, int64_t *totals) {
    ideal_totals(q, packed, 0, n, m, p, R, C, P, na, ashift, amask, afac, nw, wshift, wmask,
                 wfac, maxima, totals);
}

void brute_ideal_totals_wide(const int64_t *q, const int64_t *packed, int n, int m, int p,
                             int R, int C, int P, int na, const int *ashift,
                             const int64_t *amask, const int64_t *afac, int nw,
                             const int *wshift, const int64_t *wmask, const int64_t *wfac,
                             const int64_t *maxima, int64_t *totals) {
    ideal_totals(q, packed, 1, n, m, p, R, C, P, na, ashift, amask, afac, nw, wshift, wmask,
                 wfac, maxima, totals);
}
