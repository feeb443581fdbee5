/* Test infrastructure: compares the device expf restatement (one shared source,
 * bnn-train-infer_amd/csrc/libc_expf.h) and the engine host step's four-lane form of it
 * (bnn-train-infer_amd/engine/host_expf.h, where the processor has AVX2 and FMA) with the
 * host C library's expf on every STRIDE-th float bit pattern (STRIDE 1 = all 2^32).  Prints
 * the mismatch count; NaN results compare equal to NaN.  Not part of the product. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../bnn-train-infer_amd/csrc/libc_expf.h"
#include "../bnn-train-infer_amd/engine/host_expf.h"

static int same(float want, float got) { return (isnan(want) && isnan(got)) || memcmp(&want, &got, 4) == 0; }

int main(int argc, char** argv) {
    const uint64_t stride = argc > 1 ? strtoull(argv[1], NULL, 10) : 1;
    static const uint64_t table[32] = BNNE_EXP2_TABLE;
    const int lanes = bnne_expf_lanes_usable();
    enum { kBatch = 4096 };
    static float xs[kBatch], ys[kBatch];
    uint32_t k = 0;
    uint64_t checked = 0, mismatches = 0, lane_mismatches = 0;
    for (uint64_t b = 0; b <= 0xffffffffull; b += stride ? stride : 1) {
        const uint32_t u = (uint32_t)b;
        float x, want, got;
        memcpy(&x, &u, 4);
        want = expf(x);
        got = bnne_expf_libc(x, table);
        checked++;
        if (!same(want, got)) {
            if (mismatches < 5)
                printf("x=%a libc=%a restated=%a\n", x, want, got);
            mismatches++;
        }
        xs[k++] = x;
        if (k == kBatch || b + (stride ? stride : 1) > 0xffffffffull) {
            if (lanes) {
                bnne_expf_lanes(xs, ys, k);
                for (uint32_t i = 0; i < k; ++i)
                    if (!same(expf(xs[i]), ys[i])) {
                        if (lane_mismatches < 5)
                            printf("x=%a libc=%a lanes=%a\n", xs[i], expf(xs[i]), ys[i]);
                        lane_mismatches++;
                    }
            }
            k = 0;
        }
    }
    printf("checked %llu (four-lane form %s) mismatches %llu\n", (unsigned long long)checked,
           lanes ? "checked too" : "not usable here", (unsigned long long)(mismatches + lane_mismatches));
    return mismatches + lane_mismatches != 0;
}
