// Host check of the reciprocal quantiser in bnn-train-infer_amd/csrc/bnn_quant.h (the
// one the gfx950 kernels compile) against the reference formula
//   Q = clamp(roundf(F32(x / s)), -127, 127)      (soft-bnn-accelerator.c:197-208)
// Built with -O2 -fno-fast-math -ffp-contract=off (SSE binary32, IEEE division).
//   quant_sweep full <s_bits_hex>...   every finite x (2^32 - 2^24 - 2 patterns) per s
//   quant_sweep near <count> <seed>    `count` seeded scales s over all exponents, and for
//                                      every k in [-128, 128] the 129 floats nearest to
//                                      (k + 0.5) * s
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
    const float rcp = 1.0f / s;
    const bool exact = bnnhip::quant_exact(s);
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < threads; ++t)
        pool.emplace_back([=] {
            uint64_t n = 0;
            for (uint64_t b = t; b <= 0xffffffffull; b += threads) {
                if (((uint32_t)b & 0x7f800000u) == 0x7f800000u)
                    continue;  // NaN / Inf: rejected before quantisation
                check(from_bits((uint32_t)b), s, rcp, exact);
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
                const float rcp = 1.0f / s;
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
                        check(x, s, rcp, exact);
                        ++n;
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
    if (argc >= 3 && strcmp(argv[1], "full") == 0) {
        for (int i = 2; i < argc; ++i)
            full(from_bits((uint32_t)strtoul(argv[i], nullptr, 16)), threads);
    } else if (argc == 4 && strcmp(argv[1], "near") == 0) {
        near((unsigned)atoi(argv[2]), strtoull(argv[3], nullptr, 10), threads);
    } else {
        fprintf(stderr, "usage: quant_sweep full <s_bits>... | near <count> <seed>\n");
        return 2;
    }
    printf("checked %llu mismatches %llu\n", (unsigned long long)g_checked.load(), (unsigned long long)g_bad.load());
    return g_bad.load() ? 1 : 0;
}
