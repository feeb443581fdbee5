// Host check of the reciprocal quantiser in bnn-train-infer_amd/csrc/bnn_quant.h (the
// one the gfx950 kernels compile) against the reference formulas
//   Q = clamp(roundf(F32(x / s)), -127, 127)      (soft-bnn-accelerator.c:197-208)
//   s = absmax == 0 ? 1 : F32(absmax / 127), FLT_TRUE_MIN if that is 0   (:187-195)
// Built with -O2 -fno-fast-math -ffp-contract=off (SSE binary32, IEEE division).
// quantize_rcp is checked with the reciprocal F32(1 / s) and with neighbours a few ulps
// away, standing for the device's estimate (bnn_quant.h bounds its error by 7 * 2^-24).
//   quant_sweep full <s_bits_hex>...   every finite x (2^32 - 2^24 - 2 patterns) per s, each
//                                      with one of F32(1 / s) and its two neighbours in turn
//   quant_sweep near <count> <seed>    `count` seeded scales s over all exponents, and for
//                                      every k in [-128, 128] the 129 floats nearest to
//                                      (k + 0.5) * s, each with F32(1 / s) and the floats up to
//                                      two ulps either side of it
//   quant_sweep scale                  quant_row_scale for every finite absmax >= 0
// Prints "checked N mismatches M" and the first mismatches; exit status 1 on any.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <thread>
#include <vector>

#include "bnn_quant.h"

static float from_bits(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}
static uint32_t to_bits(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    return b;
}

static int reference_q(float x, float s) {
    volatile float v = x / s;
    float r = roundf(v);
    if (r > 127.0f)
        r = 127.0f;
    else if (r < -127.0f)
        r = -127.0f;
    return (int)r;
}

#ifdef PLANTED_NO_DIVISION
// A planted mistake for the test of this checker: the reciprocal product alone.
static int planted_q(float x, float s, float rcp, bool exact) {
    const float y = exact ? x / s : x * rcp;
    return (int)fminf(fmaxf(roundf(y), -127.0f), 127.0f);
}
#define QUANTIZE planted_q
#else
#define QUANTIZE bnnhip::quantize_rcp
#endif

#ifdef PLANTED_NO_CORRECTION
// A planted mistake for the row-scale check: the product by F32(1 / 127) alone.
static float planted_scale(float a) {
    if (a == 0.0f)
        return 1.0f;
    const float s = a * 0x1.020408p-7f;
    return s == 0.0f ? 0x1p-149f : s;
}
#define ROW_SCALE planted_scale
#else
#define ROW_SCALE bnnhip::quant_row_scale
#endif

static float reference_scale(float a) {
    if (a == 0.0f)
        return 1.0f;
    volatile float s = a / 127.0f;
    return s == 0.0f ? 0x1p-149f : s;
}

// the float `ulps` steps from the positive finite r
static float step_ulps(float r, int ulps) {
    uint32_t b;
    memcpy(&b, &r, 4);
    b = (uint32_t)((int64_t)b + ulps);
    float f;
    memcpy(&f, &b, 4);
    return f;
}

static std::atomic<uint64_t> g_checked{0}, g_bad{0};
static std::atomic<int> g_reported{0};

static void check(float x, float s, float rcp, bool exact) {
    const int want = reference_q(x, s);
    const int got = QUANTIZE(x, s, rcp, exact);
    if (got != want) {
        g_bad++;
        if (g_reported++ < 10)
            printf("mismatch: s=%a x=%a got %d want %d\n", s, x, got, want);
    }
}

static void full(float s, unsigned threads) {
    const float r = 1.0f / s;
    const bool exact = bnnhip::quant_exact(s);
    // a subnormal s has an infinite or huge reciprocal, never used (exact)
    const float rcps[3] = {r, exact ? r : step_ulps(r, -1), exact ? r : step_ulps(r, 1)};
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < threads; ++t)
        pool.emplace_back([=] {
            uint64_t n = 0;
            for (uint64_t b = t; b <= 0xffffffffull; b += threads) {
                if (((uint32_t)b & 0x7f800000u) == 0x7f800000u)
                    continue;  // NaN / Inf: rejected before quantisation
                check(from_bits((uint32_t)b), s, rcps[b % 3u], exact);
                ++n;
            }
            g_checked += n;
        });
    for (auto& th : pool)
        th.join();
}

// splitmix64
static uint64_t next(uint64_t& st) {
    uint64_t z = (st += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static void near(unsigned count, uint64_t seed, unsigned threads) {
    std::vector<float> scales;
    uint64_t st = seed;
    // specials first, then s = F32(absmax / 127) for absmax of random sign-free bit patterns
    const float specials[] = {1.0f, 0x1p-126f, 0x1.000002p-126f, 0x1.fffffcp-127f, 0x1p-149f,
                              3.4028235e38f / 127.0f, 1.0f / 127.0f, 3.0f};
    for (float s : specials)
        scales.push_back(s);
    while (scales.size() < count) {
        const float amax = from_bits((uint32_t)(next(st) % 0x7f800000u));
        scales.push_back(bnnhip::quant_row_scale(amax));
    }
    std::atomic<unsigned> at{0};
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < threads; ++t)
        pool.emplace_back([&] {
            uint64_t n = 0;
            for (unsigned i; (i = at++) < scales.size();) {
                const float s = scales[i];
                const float r = 1.0f / s;
                const bool exact = bnnhip::quant_exact(s);
                for (int k = -128; k <= 128; ++k) {
                    const float c = (float)(((double)k + 0.5) * (double)s);
                    const uint32_t cb = to_bits(c);
                    for (int d = -64; d <= 64; ++d) {
                        // walk the float line through c (sign-magnitude bit patterns)
                        int64_t mag = (int64_t)(cb & 0x7fffffffu) * ((cb >> 31) ? -1 : 1) + d;
                        const uint32_t bits = mag < 0 ? (0x80000000u | (uint32_t)(-mag)) : (uint32_t)mag;
                        const float x = from_bits(bits);
                        if (!isfinite(x))
                            continue;
                        for (int u = -2; u <= 2; ++u)
                            check(x, s, exact ? r : step_ulps(r, u), exact);
                        n += 5;
                    }
                }
            }
            g_checked += n;
        });
    for (auto& th : pool)
        th.join();
}

int main(int argc, char** argv) {
    unsigned threads = std::thread::hardware_concurrency();
    if (const char* e = getenv("QUANT_SWEEP_THREADS"))
        threads = (unsigned)atoi(e);
    if (threads == 0)
        threads = 1;
    if (argc == 2 && strcmp(argv[1], "scale") == 0) {
        std::vector<std::thread> pool;
        for (unsigned t = 0; t < threads; ++t)
            pool.emplace_back([=] {
                uint64_t n = 0, bad = 0;
                for (uint64_t b = t; b < 0x7f800000ull; b += threads) {
                    const float a = from_bits((uint32_t)b);
                    const float want = reference_scale(a), got = ROW_SCALE(a);
                    if (to_bits(want) != to_bits(got)) {
                        ++bad;
                        if (g_reported++ < 10)
                            printf("mismatch: absmax=%a got %a want %a\n", a, got, want);
                    }
                    ++n;
                }
                g_checked += n;
                g_bad += bad;
            });
        for (auto& th : pool)
            th.join();
    } else if (argc >= 3 && strcmp(argv[1], "full") == 0) {
        for (int i = 2; i < argc; ++i)
            full(from_bits((uint32_t)strtoul(argv[i], nullptr, 16)), threads);
    } else if (argc == 4 && strcmp(argv[1], "near") == 0) {
        near((unsigned)atoi(argv[2]), strtoull(argv[3], nullptr, 10), threads);
    } else {
        fprintf(stderr, "usage: quant_sweep full <s_bits>... | near <count> <seed> | scale\n");
        return 2;
    }
    printf("checked %llu mismatches %llu\n", (unsigned long long)g_checked.load(), (unsigned long long)g_bad.load());
    return g_bad.load() ? 1 : 0;
}
