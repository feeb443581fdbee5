// Per-row int8 quantisation of the F32 operations (reference
// bnn-accelerator/soft-bnn-accelerator.c:175-211), shared by the device kernels and
// the host-side checks: the same source is compiled by hipcc for gfx950 and by the
// host compiler.
#pragma once

#include <math.h>

#if defined(__HIPCC__)
#define BNN_QUANT_FN __host__ __device__ __forceinline__
#else
#define BNN_QUANT_FN static inline
#endif

namespace bnnhip {

// Row scale from the row's absmax (soft-bnn-accelerator.c:187-195): 1 for a zero row,
// else F32(absmax / 127), or the smallest subnormal when that quotient underflows.
BNN_QUANT_FN float quant_row_scale(float absmax) {
    if (absmax == 0.0f)
        return 1.0f;
    const float s = absmax / 127.0f;
    return s == 0.0f ? 0x1p-149f : s;
}

// Q = clamp(round-half-away(F32(x / s)), -127, 127)  (soft-bnn-accelerator.c:197-208),
// given rcp = F32(1 / s) and exact = (s is subnormal, where 1 / s may overflow).
// y = F32(x * F32(1 / s)) is within 1.6e-5 of x / s (|x / s| <= 128) and F32(x / s)
// within 3.9e-6, so both round to the same integer unless y lies within 2^-14 of a
// half-integer; those lanes (and all, when s is subnormal: `exact`) divide.  Beyond
// |x / s| = 128 both sides saturate at +-127.
BNN_QUANT_FN int quantize_rcp(float x, float s, float rcp, bool exact) {
    float y = x * rcp;
    float t = truncf(y), d = y - t;
    if (exact || fabsf(fabsf(d) - 0.5f) < 0x1p-14f) {
        y = x / s;
        t = truncf(y);
        d = y - t;
    }
    const float q = t + (fabsf(d) >= 0.5f ? copysignf(1.0f, y) : 0.0f);
    return (int)fminf(fmaxf(q, -127.0f), 127.0f);
}

BNN_QUANT_FN bool quant_exact(float s) { return s < 0x1p-126f; }

}  // namespace bnnhip
