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
// The quotient is Markstein's corrected product: q0 = F32(a * c) with c = F32(1 / 127),
// the residual a - 127 q0 (exact in one FMA), then F32(q0 + c * residual) in another.
// It equals the IEEE quotient for every finite a >= 0, subnormals included (all
// 2^31 - 2^23 patterns compared by tests/quant_sweep.cpp; the operations are IEEE
// binary32 ones on the host and the device alike), in three operations where a wave's
// IEEE division takes about ten.
BNN_QUANT_FN float quant_row_scale(float absmax) {
    if (absmax == 0.0f)
        return 1.0f;
    const float c = 0x1.020408p-7f;  // F32(1 / 127)
    const float q0 = absmax * c;
    const float s = fmaf(fmaf(-q0, 127.0f, absmax), c, q0);
    return s == 0.0f ? 0x1p-149f : s;
}

// Q = clamp(round-half-away(F32(x / s)), -127, 127)  (soft-bnn-accelerator.c:197-208),
// given rcp within relative error e <= 7 * 2^-24 of 1 / s (quant_rcp) and exact = (s
// is subnormal, where 1 / s may overflow).  For |x / s| <= 128, y = F32(x * rcp) lies
// within 128 e + 2^-18 of x / s and F32(x / s) within 2^-18, so the two are less than
// 2^-14 apart and round to the same integer unless y lies within 2^-14 of a
// half-integer; those lanes (and all, when s is subnormal: `exact`) divide.  Away from
// half-integers rounding half away from zero and half to even agree, so the other lanes
// take rint(y) (rounding to nearest even, the required mode), and |y - rint(y)| is the
// distance that decides.  Beyond |x / s| = 128 both sides saturate at +-127.
BNN_QUANT_FN int quantize_rcp(float x, float s, float rcp, bool exact) {
    const float y = x * rcp;
    float q = rintf(y);
    if (exact || fabsf(fabsf(y - q) - 0.5f) < 0x1p-14f) {
        const float z = x / s, t = truncf(z), d = z - t;
        q = t + (fabsf(d) >= 0.5f ? copysignf(1.0f, z) : 0.0f);
    }
    return (int)fminf(fmaxf(q, -127.0f), 127.0f);
}

BNN_QUANT_FN bool quant_exact(float s) { return s < 0x1p-126f; }

// The reciprocal quantize_rcp multiplies by, for a normal row scale s (every s below
// 2^122: absmax / 127 <= FLT_MAX / 127).  On the device: the hardware estimate r0 and
// one Newton step with the residual 1 - s r0 rounded once in an FMA, whose relative
// error is about d^2 + 2^-24 for an estimate within relative d -- at most 5.001 * 2^-24
// for any d <= 2^-11, inside quantize_rcp's 7 * 2^-24 (v_rcp_f32 itself measured within
// 0.77 * 2^-23 over every normal s below 2^122).  Three operations instead of an IEEE
// division.  The host divides.  A subnormal s takes quantize_rcp's division path and
// never uses the value.
BNN_QUANT_FN float quant_rcp(float s) {
#if defined(__HIP_DEVICE_COMPILE__)
    const float r0 = __builtin_amdgcn_rcpf(s);
    return fmaf(fmaf(-s, r0, 1.0f), r0, r0);
#else
    return 1.0f / s;
#endif
}

}  // namespace bnnhip
