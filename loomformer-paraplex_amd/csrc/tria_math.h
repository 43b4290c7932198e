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

}  // namespace loom
