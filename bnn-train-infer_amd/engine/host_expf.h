/*
 * expf over arrays on the host, bit for bit the host C library's expf.
 *
 * On x86-64 processors with AVX2 and FMA, glibc 2.35's expf runs its FMA build of the
 * table-driven method that ../csrc/libc_expf.h restates (and that a test compares with
 * the C library on every float).  bnne_expf_lanes performs the restatement's operations
 * on four floats at a time in binary64 lanes (the same fused multiply-adds, the same
 * table, one rounding to float at the end); a group of four holding an |x| >= 88 or a
 * value that is not finite goes to the C library, as does the tail.  Callers use it only
 * where the processor has AVX2 and FMA (bnne_expf_lanes_usable) -- exactly where the C
 * library takes that build -- and the C library elsewhere.
 *
 * Plain C (shared by the engine and the test-side check against the C library).
 */
#ifndef BNNE_HOST_EXPF_H
#define BNNE_HOST_EXPF_H

#include <immintrin.h>
#include <math.h>
#include <stdint.h>

#include "../csrc/libc_expf.h"

static inline int bnne_expf_lanes_usable(void) {
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

__attribute__((target("avx2,fma"))) static inline void bnne_expf_lanes(const float* in, float* out, uint32_t n) {
    static const uint64_t table[32] = BNNE_EXP2_TABLE;
    const __m256d inv_ln2_n = _mm256_set1_pd(0x1.71547652b82fep+0 * 32), shift = _mm256_set1_pd(0x1.8p+52);
    const __m256d c0 = _mm256_set1_pd(0x1.c6af84b912394p-5 / 32 / 32 / 32);
    const __m256d c1 = _mm256_set1_pd(0x1.ebfce50fac4f3p-3 / 32 / 32);
    const __m256d c2 = _mm256_set1_pd(0x1.62e42ff0c52d6p-1 / 32), one = _mm256_set1_pd(1.0);
    uint32_t i = 0;
    for (; i + 4u <= n; i += 4u) {
        const __m128 x = _mm_loadu_ps(in + i);
        const __m128i abstop = _mm_and_si128(_mm_srli_epi32(_mm_castps_si128(x), 20), _mm_set1_epi32(0x7ff));
        if (_mm_movemask_epi8(_mm_cmpgt_epi32(abstop, _mm_set1_epi32(0x42a))) != 0) {
            for (uint32_t j = 0; j < 4u; ++j)
                out[i + j] = expf(in[i + j]);
            continue;
        }
        const __m256d xd = _mm256_cvtps_pd(x);
        __m256d kd = _mm256_fmadd_pd(inv_ln2_n, xd, shift);
        const __m256i ki = _mm256_castpd_si256(kd);
        kd = _mm256_sub_pd(kd, shift);
        const __m256d r = _mm256_fmsub_pd(inv_ln2_n, xd, kd);
        const __m256i t = _mm256_i64gather_epi64((const long long*)table, _mm256_and_si256(ki, _mm256_set1_epi64x(31)),
                                                 8);
        const __m256d s = _mm256_castsi256_pd(_mm256_add_epi64(t, _mm256_slli_epi64(ki, 47)));
        const __m256d z = _mm256_fmadd_pd(c0, r, c1);
        const __m256d r2 = _mm256_mul_pd(r, r);
        __m256d y = _mm256_fmadd_pd(c2, r, one);
        y = _mm256_fmadd_pd(z, r2, y);
        y = _mm256_mul_pd(y, s);
        _mm_storeu_ps(out + i, _mm256_cvtpd_ps(y));
    }
    for (; i < n; ++i)
        out[i] = expf(in[i]);
}

#endif
