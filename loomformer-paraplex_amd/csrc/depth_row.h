// One depth-attention row (bt, qh) on 16 lanes, shared by the depth
// attention kernel and the decode attention launch that folds the read in.
//
// Layout: element (bt, s, qh, d) of K/V lives at bt*stride_bt + s*stride_s +
// qh*HD + d.  Lane j of the row's 16 owns the EPL = HD/16 contiguous elements
// [j*EPL, (j+1)*EPL).  Scores for 8 depth slots are formed before any value is
// read (8 independent K loads in flight per lane), then folded into an fp32
// online softmax in log2 units.  The K/V rows are read
// once, with nontemporal loads.
//
// With RMS (DepthAttn under depth_attn_qkv_rms, loomformer.py:3397-3407) the
// query, key and value rows are read as fixed-RMS vectors, as fixed_rms
// (loomformer.py:840-844) forms them: the scale t / sqrt(mean(x^2) + 1e-6) with
// target qt, kt or vt is computed in fp32 from the stored row, rounded to the
// storage type, and each element x * scale rounded to the storage type again
// (both roundings vanish in fp32).  The stored history stays as projected.
#pragma once

#include "loom_common.h"

namespace loom {

constexpr int kDepthChunk = 8;

// target / sqrt(mean(x^2) + 1e-6) of a 16-lane row whose lanes hold EPL elements each
template <int EPL>
__device__ __forceinline__ float rms_scale(const float (&x)[EPL], float target) {
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < EPL; ++k) ss = fmaf(x[k], x[k], ss);
    ss = group_sum<16>(ss);
    return target * frsq(fmaf(ss, 1.0f / (float)(EPL * 16), 1e-6f));
}

// x <- x * scale in place, each term rounded to T as fixed_rms's bf16/fp16
// product is (scale itself rounded to T first)
template <typename T, int EPL>
__device__ __forceinline__ void fixed_rms_row(float (&x)[EPL], float target) {
    const float s = round_to<T>(rms_scale<EPL>(x, target));
#pragma unroll
    for (int k = 0; k < EPL; ++k) x[k] = round_to<T>(x[k] * s);
}

struct DepthRms {
    float qt, kt, vt;
};

// The read of row (bt, qh) = (row / QH, row % QH) on lane j of its 16:
// acc = unnormalised sum of p*v over the S slots, m / l the running max and
// sum (log2 units), qv the scaled query.  NT: the K/V rows are read once
// (nontemporal loads); otherwise they stay cached for other readers.
template <typename T, int EPL, int C, bool RMS, bool NT>
__device__ __forceinline__ void depth_row_core(const T* __restrict__ q, const T* __restrict__ hk,
                                               const T* __restrict__ hv, int64_t sbt, int64_t ss,
                                               int row, int j, int S, int QH, float scale,
                                               DepthRms rms, float (&qv)[EPL], float (&acc)[EPL],
                                               float& m, float& l) {
    constexpr int HD = EPL * 16;
    const int qh = row % QH;
    const int bt = row / QH;
    const int d0 = j * EPL;

    RowIO<T, EPL>::load(q + qh * HD + d0, qv);
    if constexpr (RMS) fixed_rms_row<T, EPL>(qv, rms.qt);
    const float qs = scale * kLog2e;                        // scores in log2 units
#pragma unroll
    for (int k = 0; k < EPL; ++k) qv[k] *= qs;

    const T* kp = hk + (int64_t)bt * sbt + qh * HD + d0;
    const T* vp = hv + (int64_t)bt * sbt + qh * HD + d0;
    m = -INFINITY;
    l = 0.0f;
#pragma unroll
    for (int k = 0; k < EPL; ++k) acc[k] = 0.0f;

    // the K and V rows of C depth slots are requested together (2C loads in
    // flight per lane), then scored and folded into the online softmax
    for (int s0 = 0; s0 < S; s0 += C) {
        RawRow<T, EPL> kr[C], vr[C];
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int sc_ = s0 + c < S ? s0 + c : S - 1;   // in range; masked below
            if constexpr (NT) {
                kr[c].load_nt(kp + (int64_t)sc_ * ss);
                vr[c].load_nt(vp + (int64_t)sc_ * ss);
            } else {
                kr[c].load(kp + (int64_t)sc_ * ss);
                vr[c].load(vp + (int64_t)sc_ * ss);
            }
        }
        float sc[C];
#pragma unroll
        for (int c = 0; c < C; ++c) {
            float kv[EPL];
            kr[c].to_float(kv);
            if constexpr (RMS) fixed_rms_row<T, EPL>(kv, rms.kt);
            float dot = 0.0f;
#pragma unroll
            for (int k = 0; k < EPL; ++k) dot = fmaf(qv[k], kv[k], dot);
            sc[c] = dot;
        }
        float cmax = -INFINITY;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            sc[c] = group_sum<16>(sc[c]);
            if (s0 + c < S) cmax = fmaxf(cmax, sc[c]);
        }
        const float m_new = fmaxf(m, cmax);
        const float corr = __builtin_amdgcn_exp2f(m - m_new);  // 0 on the first chunk
        l *= corr;
#pragma unroll
        for (int k = 0; k < EPL; ++k) acc[k] *= corr;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            float vv[EPL];
            vr[c].to_float(vv);
            if constexpr (RMS) fixed_rms_row<T, EPL>(vv, rms.vt);
            const float p = s0 + c < S ? __builtin_amdgcn_exp2f(sc[c] - m_new) : 0.0f;
            l += p;
#pragma unroll
            for (int k = 0; k < EPL; ++k) acc[k] = fmaf(p, vv[k], acc[k]);
        }
        m = m_new;
    }
}

template <typename T, int EPL, int C = kDepthChunk, bool RMS = false>
__device__ __forceinline__ void depth_row(const T* __restrict__ q, const T* __restrict__ hk,
                                          const T* __restrict__ hv, int64_t sbt, int64_t ss,
                                          T* __restrict__ d_out, T* __restrict__ w_out,
                                          float* __restrict__ lse_out, int row, int j, int S,
                                          int QH, float scale, DepthRms rms = DepthRms{}) {
    constexpr int HD = EPL * 16;
    const int qh = row % QH;
    const int bt = row / QH;
    const int d0 = j * EPL;
    const T* kp = hk + (int64_t)bt * sbt + qh * HD + d0;
    float qv[EPL], acc[EPL], m, l;
    depth_row_core<T, EPL, C, RMS, true>(q, hk, hv, sbt, ss, row, j, S, QH, scale, rms, qv, acc, m, l);
    const float inv_l = 1.0f / l;
#pragma unroll
    for (int k = 0; k < EPL; ++k) acc[k] *= inv_l;
    RowIO<T, EPL>::store(d_out + (int64_t)row * HD + d0, acc);
    if (lse_out != nullptr && j == 0) lse_out[row] = (m + flog2(l)) * kLn2;
    if (w_out != nullptr) {
        // weights: recompute each score (one more K read) and normalise
        for (int s = 0; s < S; ++s) {
            float kv[EPL];
            RowIO<T, EPL>::load(kp + (int64_t)s * ss, kv);
            if constexpr (RMS) fixed_rms_row<T, EPL>(kv, rms.kt);
            float dot = 0.0f;
#pragma unroll
            for (int k = 0; k < EPL; ++k) dot = fmaf(qv[k], kv[k], dot);
            dot = group_sum<16>(dot);
            if (j == 0) st(w_out + (int64_t)row * S + s, __builtin_amdgcn_exp2f(dot - m) * inv_l);
        }
    }
}

}  // namespace loom
