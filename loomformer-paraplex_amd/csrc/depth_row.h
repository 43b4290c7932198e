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
// query, key and value rows are read as fixed-RMS vectors: x * t / sqrt(mean(x^2)
// + 1e-6) with targets qt, kt, vt.  The key scale multiplies the group-summed
// score and the value scale the softmax weight of its row, so the stored
// history stays as projected.
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
    float qs = scale * kLog2e;                              // scores in log2 units
    if constexpr (RMS) qs *= rms_scale<EPL>(qv, rms.qt);
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
            float dot = 0.0f;
#pragma unroll
            for (int k = 0; k < EPL; ++k) dot = fmaf(qv[k], kv[k], dot);
            sc[c] = dot;
            if constexpr (RMS) sc[c] = group_sum<16>(sc[c]) * rms_scale<EPL>(kv, rms.kt);
        }
        float cmax = -INFINITY;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            if constexpr (!RMS) sc[c] = group_sum<16>(sc[c]);
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
            const float p = s0 + c < S ? __builtin_amdgcn_exp2f(sc[c] - m_new) : 0.0f;
            l += p;
            const float pv = RMS ? p * rms_scale<EPL>(vv, rms.vt) : p;
#pragma unroll
            for (int k = 0; k < EPL; ++k) acc[k] = fmaf(pv, vv[k], acc[k]);
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
            float dot = 0.0f;
#pragma unroll
            for (int k = 0; k < EPL; ++k) dot = fmaf(qv[k], kv[k], dot);
            dot = group_sum<16>(dot);
            if constexpr (RMS) dot *= rms_scale<EPL>(kv, rms.kt);
            if (j == 0) st(w_out + (int64_t)row * S + s, __builtin_amdgcn_exp2f(dot - m) * inv_l);
        }
    }
}

}  // namespace loom
