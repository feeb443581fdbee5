/* Test infrastructure: compares the device expf restatement (one shared source,
 * bnn-train-infer_amd/csrc/libc_expf.h) with the host C library's expf on every
 * STRIDE-th float bit pattern (STRIDE 1 = all 2^32).  Prints the mismatch count;
 * NaN results compare equal to NaN.  Not part of the product. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../bnn-train-infer_amd/csrc/libc_expf.h"

int main(int argc, char** argv) {
    const uint64_t stride = argc > 1 ? strtoull(argv[1], NULL, 10) : 1;
    static const uint64_t table[32] = BNNE_EXP2_TABLE;
    uint64_t checked = 0, mismatches = 0;
    for (uint64_t b = 0; b <= 0xffffffffull; b += stride ? stride : 1) {
        const uint32_t u = (uint32_t)b;
        float x, want, got;
        memcpy(&x, &u, 4);
        want = expf(x);
        got = bnne_expf_libc(x, table);
        checked++;
        if (isnan(want) && isnan(got))
            continue;
        if (memcmp(&want, &got, 4) != 0) {
            if (mismatches < 5)
                printf("x=%a libc=%a restated=%a\n", x, want, got);
            mismatches++;
        }
    }
    printf("checked %llu mismatches %llu\n", (unsigned long long)checked, (unsigned long long)mismatches);
    return mismatches != 0;
}
