// f32 arithmetic of the JIT kernels (src/jit/lower.rs) on gfx950: the
// polynomial exp, SiLU and a correctly rounded square root.  No fused
// multiply-add except where one is written out on purpose.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

namespace slm {

// emit_exp_f32x4 (lower.rs:22-65), one lane: clamp to [-87.3, 88.3],
// n = nearest(x * log2 e) (ties to even), Cody-Waite reduction with the two
// ln 2 constants, degree-5 Horner polynomial, times 2^n built from the
// exponent bits.  (fmaxf/fminf return the non-NaN operand where Cranelift's
// fmax/fmin propagate NaN; the paths here never feed them NaN from finite
// inputs.)
__device__ __forceinline__ float jit_exp(float x) {
#pragma clang fp contract(off)
    float xc = fmaxf(x, -87.3f);
    xc = fminf(xc, 88.3f);
    const float fx = xc * 1.44269504088896340736f;
    const float n = rintf(fx);
    const float n_hi = n * 0.69314575f;
    const float n_lo = n * 1.4286068e-6f;
    const float r_hi = xc - n_hi;
    const float r = r_hi - n_lo;
    float p = r * (1.0f / 120.0f);
    p = p + (1.0f / 24.0f);
    p = r * p;
    p = p + (1.0f / 6.0f);
    p = r * p;
    p = p + 0.5f;
    p = r * p;
    p = p + 1.0f;
    p = r * p;
    const float poly = p + 1.0f;
    const int ni = (int)n;  // |n| <= 128 after the clamp
    return poly * __int_as_float((ni + 127) << 23);
}

// Correctly rounded f32 square root (what Cranelift's `sqrt` is, x86
// sqrtps).  v_sqrt_f32 is within 1 ulp; the exact residuals x - s'*s of its
// neighbours s' = s -/+ 1 ulp (one fused multiply-add each, exact) tell
// whether the rounded root is s or a neighbour.  Tiny inputs are scaled by
// 2^32 first (root scaled by 2^16) so the residuals stay representable.
__device__ __forceinline__ float sqrt_rn(float x) {
    const bool tiny = x < 0x1.0p-96f;
    const float xs = tiny ? x * 0x1.0p+32f : x;
    float s = __builtin_amdgcn_sqrtf(xs);
    const float s_dn = __int_as_float(__float_as_int(s) - 1);
    const float s_up = __int_as_float(__float_as_int(s) + 1);
    const float r_dn = __builtin_fmaf(-s_dn, s, xs);
    const float r_up = __builtin_fmaf(-s_up, s, xs);
    s = r_dn <= 0.0f ? s_dn : s;
    s = r_up > 0.0f ? s_up : s;
    s = tiny ? s * 0x1.0p-16f : s;
    // zero, infinity and NaN pass through unchanged
    return (xs == 0.0f || xs == __builtin_inff() || xs != xs) ? __builtin_amdgcn_sqrtf(xs) : s;
}

// SiLU lowering (lower.rs:85-91): v / (1 + exp(-v)).
__device__ __forceinline__ float jit_silu(float v) {
#pragma clang fp contract(off)
    const float e = jit_exp(-v);
    const float den = 1.0f + e;
    return __fdiv_rn(v, den);
}

}  // namespace slm
