// Register math of the Paraplex pointwise chain (phase map, softplus,
// PvPowLU gate), shared by the Paraplex kernels and the fused decode FFN
// epilogue.  fp32.
#pragma once

#include "loom_common.h"

namespace loom {

// I_base = sin(pi/2 * beta / sqrt(1 + beta^2)) = sin(2*pi * beta/(4 sqrt(1+beta^2)))
__device__ __forceinline__ float phase_of(float beta) {
    return fsin_turns(0.25f * beta * frsq(1.0f + beta * beta));
}

// G(A) = max(A,1e-12)^(m/(sqrt(A)+1)) * sigmoid(A), with one reciprocal for
// both divisions: r = 1/((sqrt A + 1)(1 + e^-A)).
__device__ __forceinline__ float powlu_gate(float amp, float m) {
    const float safe = fmaxf(amp, 1.0e-12f);
    const float d1 = fsqrt(safe) + 1.0f;
    const float d2 = 1.0f + fexp(-amp);
    const float r = frcp(d1 * d2);
    const float expo = m * d2 * r;      // m / (sqrt(A) + 1)
    const float sig = d1 * r;           // 1 / (1 + e^-A)
    return __builtin_amdgcn_exp2f(expo * flog2(safe)) * sig;
}

// A = softplus(x) and G(A) for the fused chain, from one exponential
// E = e^min(x, 20):
//   A = log(1 + E), with the rounding of u = 1 + E put back
//       (log(u) + (E - (u - 1)) is log1p(E) to a few ulp for every E);
//       x > 20 -> A = x (torch's softplus threshold): log1p(E) > x for
//       every x <= 20 and E is capped at e^20, so A = max(x, log1p(E));
//   e^-A = 1/(1 + e^x), so sigmoid(A) = (1 + E)/(2 + E) = u/(1 + u)
//       (for x > 20 this is 1 - 5e-10, i.e. 1 in fp32, as torch gives);
//   G = A^(m/(sqrt A + 1)) * sigmoid(A), with one reciprocal for both
//       quotients: r = 1/((sqrt A + 1)(1 + u)).
// No branch and no select on the sign of x.
// EXACT = false drops the log1p rounding term: then A = log(u) exactly as
// rounded, off by at most 2^-24 absolute from log1p(E) (relative error below
// 2^-24 / E, under half a bf16 ulp for every E > 2^-16, and for smaller E both
// A and G are below the bf16 resolution of the output (A + r) * G).
template <bool EXACT = true>
__device__ __forceinline__ void softplus_gate(float x, float m, float& amp, float& gate) {
    const float e = x * kLog2e;
    const float E = __builtin_amdgcn_exp2f(fminf(e, 20.0f * kLog2e));
    const float u = 1.0f + E;
    const float a0 = EXACT ? fmaf(flog2(u), kLn2, E - (u - 1.0f)) : flog2(u) * kLn2;
    amp = __builtin_amdgcn_fmed3f(x, a0, 3.0e38f);   // max(x, a0) without a NaN-quieting pass
    const float safe = __builtin_amdgcn_fmed3f(amp, 1.0e-12f, 3.0e38f);
    const float d1 = fsqrt(safe) + 1.0f;
    const float r = frcp(fmaf(d1, u, d1));   // 1 / ((sqrt A + 1)(1 + u))
    const float expo = fmaf(m, u, m) * r;     // m (1 + u) r = m / (sqrt(A) + 1)
    const float sig = u * d1 * r;             // sigmoid(A)
    gate = __builtin_amdgcn_exp2f(expo * flog2(safe)) * sig;
}

}  // namespace loom
