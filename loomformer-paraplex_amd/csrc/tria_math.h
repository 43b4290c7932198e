// Register math of the Tria 3x3 carriers, shared by the Tria kernels and the
// fused decode FFN epilogue.  Row-major 3x3 matrices, fp32.
#pragma once

#include "loom_common.h"

namespace loom {

// Local carrier T(r,i,o) = (I + K(a,b,c)) @ R_axis,
// (a,b,c) = alpha * tanh(x / sqrt(mean(x^2) + eps)), x = (ri, ro, io).
// The axis is a compile-time parameter: the kernels are instantiated per axis.
template <int AXIS>
__device__ __forceinline__ void carrier9(float r, float i, float o, float alpha, float mt[9]) {
    const float x0 = r * i, x1 = r * o, x2 = i * o;
    const float inv = 1.0f / sqrtf((x0 * x0 + x1 * x1 + x2 * x2) * (1.0f / 3.0f) + 1e-6f);
    const float a = alpha * tanhf(x0 * inv);
    const float b = alpha * tanhf(x1 * inv);
    const float c = alpha * tanhf(x2 * inv);
    if constexpr (AXIS == 0) {          // about z
        mt[0] = -c;   mt[1] = -1.0f; mt[2] = b;
        mt[3] = 1.0f; mt[4] = -c;    mt[5] = -a;
        mt[6] = a;    mt[7] = b;     mt[8] = 1.0f;
    } else if constexpr (AXIS == 1) {   // about x
        mt[0] = 1.0f; mt[1] = b;     mt[2] = c;
        mt[3] = c;    mt[4] = -a;    mt[5] = -1.0f;
        mt[6] = -b;   mt[7] = 1.0f;  mt[8] = -a;
    } else {                  // about y
        mt[0] = -b;   mt[1] = -c;    mt[2] = 1.0f;
        mt[3] = a;    mt[4] = 1.0f;  mt[5] = c;
        mt[6] = -1.0f; mt[7] = a;    mt[8] = -b;
    }
}

// carrier9 with the hardware transcendentals, for the streaming chains where
// the libm forms dominate the instruction count:
//   1/sqrt -> v_rsq_f32, and tanh(y) = 1 - 2/(1 + 2^(2 y log2 e)) with v_exp_f32
//   and v_rcp_f32 (1 ulp each).  The tanh argument is x/rms(x), |y| <= sqrt(3),
//   so the exponential stays in range and the absolute error of alpha*tanh is
//   a few ulp of alpha.
template <int AXIS>
__device__ __forceinline__ void carrier9_fast(float r, float i, float o, float alpha,
                                              float mt[9]) {
    const float x0 = r * i, x1 = r * o, x2 = i * o;
    const float inv = __builtin_amdgcn_rsqf(
        fmaf(fmaf(x0, x0, fmaf(x1, x1, x2 * x2)), 1.0f / 3.0f, 1e-6f));
    const float k = 2.0f * 1.4426950408889634f * inv;   // 2 log2(e) / rms
    const float m2a = -2.0f * alpha;
    const float a = fmaf(m2a, __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x0 * k)), alpha);
    const float b = fmaf(m2a, __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x1 * k)), alpha);
    const float c = fmaf(m2a, __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x2 * k)), alpha);
    if constexpr (AXIS == 0) {
        mt[0] = -c;   mt[1] = -1.0f; mt[2] = b;
        mt[3] = 1.0f; mt[4] = -c;    mt[5] = -a;
        mt[6] = a;    mt[7] = b;     mt[8] = 1.0f;
    } else if constexpr (AXIS == 1) {
        mt[0] = 1.0f; mt[1] = b;     mt[2] = c;
        mt[3] = c;    mt[4] = -a;    mt[5] = -1.0f;
        mt[6] = -b;   mt[7] = 1.0f;  mt[8] = -a;
    } else {
        mt[0] = -b;   mt[1] = -c;    mt[2] = 1.0f;
        mt[3] = a;    mt[4] = 1.0f;  mt[5] = c;
        mt[6] = -1.0f; mt[7] = a;    mt[8] = -b;
    }
}

// 1 / sqrt(mean_9(v^2) + 1e-6) with v_rsq_f32
__device__ __forceinline__ float rms9_inv_fast(const float v[9]) {
    float s = v[0] * v[0];
#pragma unroll
    for (int k = 1; k < 9; ++k) s = fmaf(v[k], v[k], s);
    return __builtin_amdgcn_rsqf(fmaf(s, 1.0f / 9.0f, 1e-6f));
}

// out = A @ B for row-major 3x3
__device__ __forceinline__ void mm3(const float A[9], const float B[9], float out[9]) {
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int c = 0; c < 3; ++c)
            out[3 * r + c] = fmaf(A[3 * r + 2], B[6 + c], fmaf(A[3 * r + 1], B[3 + c], A[3 * r] * B[c]));
}

// rms over 9 entries with eps inside the root; returns the rms
__device__ __forceinline__ float rms9(const float v[9]) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 9; ++k) s = fmaf(v[k], v[k], s);
    return sqrtf(s * (1.0f / 9.0f) + 1e-6f);
}

// M <- M (I - beta/2 (G/s - I)), G = M^T M, s = max(mean(diag G), eps)
// (PolARM, tria.py:128-139), in place.
__device__ __forceinline__ void polarm9(float M[9], float beta, float eps) {
    float G[9];
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int c = 0; c < 3; ++c)
            G[3 * r + c] = fmaf(M[6 + r], M[6 + c], fmaf(M[3 + r], M[3 + c], M[r] * M[c]));
    const float s = fmaxf((G[0] + G[4] + G[8]) * (1.0f / 3.0f), eps);
    float C[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        const float id = (k == 0 || k == 4 || k == 8) ? 1.0f : 0.0f;
        C[k] = id - 0.5f * beta * (G[k] / s - id);
    }
    float R[9];
    mm3(M, C, R);
#pragma unroll
    for (int k = 0; k < 9; ++k) M[k] = R[k];
}

// v <- v / rms9(v)
__device__ __forceinline__ void normalize9(float v[9]) {
    const float inv = 1.0f / rms9(v);
#pragma unroll
    for (int k = 0; k < 9; ++k) v[k] *= inv;
}

}  // namespace loom
