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

// Two reads over the same S history slots (one load of each K/V row): query
// q1's read normalised into d_out, and query q2's read as the normalised fp32
// row pd_out and its log-sum-exp lse_out (natural units, lane j == 0) -- the
// part of a later read over slots 0..S that the S slots here contribute.  The
// online softmax of q1 follows depth_row_core step for step.
template <typename T, int EPL, int C = kDepthChunk>
__device__ __forceinline__ void depth_row_pair(const T* __restrict__ q1, const T* __restrict__ q2,
                                               const T* __restrict__ hk, const T* __restrict__ hv,
                                               int64_t sbt, int64_t ss, T* __restrict__ d_out,
                                               float* __restrict__ pd_out,
                                               float* __restrict__ lse_out, int row, int j, int S,
                                               int QH, float scale) {
    constexpr int HD = EPL * 16;
    const int qh = row % QH;
    const int bt = row / QH;
    const int d0 = j * EPL;
    float qa[EPL], qb[EPL];
    RowIO<T, EPL>::load(q1 + qh * HD + d0, qa);
    RowIO<T, EPL>::load(q2 + qh * HD + d0, qb);
    const float qs = scale * kLog2e;                        // scores in log2 units
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
        qa[k] *= qs;
        qb[k] *= qs;
    }
    const T* kp = hk + (int64_t)bt * sbt + qh * HD + d0;
    const T* vp = hv + (int64_t)bt * sbt + qh * HD + d0;
    float ma = -INFINITY, la = 0.0f, mb = -INFINITY, lb = 0.0f, aa[EPL], ab[EPL];
#pragma unroll
    for (int k = 0; k < EPL; ++k) aa[k] = ab[k] = 0.0f;
    for (int s0 = 0; s0 < S; s0 += C) {
        RawRow<T, EPL> kr[C], vr[C];
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int sc_ = s0 + c < S ? s0 + c : S - 1;   // in range; masked below
            kr[c].load_nt(kp + (int64_t)sc_ * ss);
            vr[c].load_nt(vp + (int64_t)sc_ * ss);
        }
        float sa[C], sb[C];
#pragma unroll
        for (int c = 0; c < C; ++c) {
            float kv[EPL];
            kr[c].to_float(kv);
            float da = 0.0f, db = 0.0f;
#pragma unroll
            for (int k = 0; k < EPL; ++k) {
                da = fmaf(qa[k], kv[k], da);
                db = fmaf(qb[k], kv[k], db);
            }
            sa[c] = da;
            sb[c] = db;
        }
        float xa = -INFINITY, xb = -INFINITY;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            sa[c] = group_sum<16>(sa[c]);
            sb[c] = group_sum<16>(sb[c]);
            if (s0 + c < S) {
                xa = fmaxf(xa, sa[c]);
                xb = fmaxf(xb, sb[c]);
            }
        }
        const float na = fmaxf(ma, xa), nb = fmaxf(mb, xb);
        const float ca = __builtin_amdgcn_exp2f(ma - na), cb = __builtin_amdgcn_exp2f(mb - nb);
        la *= ca;
        lb *= cb;
#pragma unroll
        for (int k = 0; k < EPL; ++k) {
            aa[k] *= ca;
            ab[k] *= cb;
        }
#pragma unroll
        for (int c = 0; c < C; ++c) {
            float vv[EPL];
            vr[c].to_float(vv);
            const float pa = s0 + c < S ? __builtin_amdgcn_exp2f(sa[c] - na) : 0.0f;
            const float pb = s0 + c < S ? __builtin_amdgcn_exp2f(sb[c] - nb) : 0.0f;
            la += pa;
            lb += pb;
#pragma unroll
            for (int k = 0; k < EPL; ++k) {
                aa[k] = fmaf(pa, vv[k], aa[k]);
                ab[k] = fmaf(pb, vv[k], ab[k]);
            }
        }
        ma = na;
        mb = nb;
    }
    const float ia = 1.0f / la, ib = 1.0f / lb;
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
        aa[k] *= ia;
        ab[k] *= ib;
    }
    RowIO<T, EPL>::store(d_out + (int64_t)row * HD + d0, aa);
    RowIO<float, EPL>::store(pd_out + (int64_t)row * HD + d0, ab);
    if (j == 0) lse_out[row] = (mb + flog2(lb)) * kLn2;
}

// The read of one head row over slots 0..S-1 from the read over slots 0..S-2
// (pd: normalised fp32 row of this lane's EPL elements, lse: its log-sum-exp
// in natural units) and slot S-1's key kn and value vn: one softmax over the
// two parts.  qv: the query row's lane elements; scale = 1/sqrt(HD).
template <int EPL>
__device__ __forceinline__ void depth_fold_last(const float (&qv)[EPL], const float (&kn)[EPL],
                                                const float (&vn)[EPL], const float (&pd)[EPL],
                                                float lse, float scale, float (&out)[EPL]) {
    float dot = 0.0f;
#pragma unroll
    for (int k = 0; k < EPL; ++k) dot = fmaf(qv[k], kn[k], dot);
    const float s = group_sum<16>(dot) * scale;
    const float m = fmaxf(lse, s);
    const float w1 = fexp(lse - m), w2 = fexp(s - m);
    const float inv = 1.0f / (w1 + w2);
#pragma unroll
    for (int k = 0; k < EPL; ++k) out[k] = (pd[k] * w1 + vn[k] * w2) * inv;
}

}  // namespace loom
