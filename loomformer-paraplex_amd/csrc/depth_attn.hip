// Depth attention for gfx950: softmax over the depth axis of S history keys
// with one learned query per q-head.
//
// Layout: element (bt, s, qh, d) of K/V lives at bt*stride_bt + s*stride_s +
// qh*HD + d, so a [B,T,S,QH,HD] stack and a strided decode view
// hist[:, :, :S] of a [B,T,S_max,QH,HD] buffer are both read in place.
//
// Mapping: one (bt, qh) row per aligned group of 16 lanes (depth_row.h); a
// wavefront therefore covers 4 heads = 4*HD contiguous elements of one (bt, s)
// slice.
#include <cmath>
#include <type_traits>

#include "loom_common.h"
#include "depth_row.h"

namespace loom {

template <typename T, int EPL, int C, bool RMS>
__global__ void __launch_bounds__(256)
depth_attn_kernel(const T* __restrict__ q, const T* __restrict__ hk, const T* __restrict__ hv,
                  int64_t sbt, int64_t ss, T* __restrict__ d_out, T* __restrict__ w_out,
                  float* __restrict__ lse_out, int rows, int S, int QH, float scale, DepthRms rms) {
    const int row = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 4);
    if (row >= rows) return;  // all 16 lanes of a group leave together
    depth_row<T, EPL, C, RMS>(q, hk, hv, sbt, ss, d_out, w_out, lse_out, row, threadIdx.x & 15, S,
                              QH, scale, rms);
}

// target / sqrt(mean(x^2) + 1e-6) of the HD-element row at p, or 1 when target == 0
template <typename T>
__device__ __forceinline__ float row_rms_scale(const T* p, int HD, float target) {
    if (target == 0.0f) return 1.0f;
    float ss = 0.0f;
    for (int d = 0; d < HD; ++d) {
        const float x = ld(p + d);
        ss = fmaf(x, x, ss);
    }
    return target * frsq(ss / (float)HD + 1e-6f);
}

// Any HD: one thread per (bt, qh) row, online softmax, scalar loads.  With
// nonzero targets in rms the q, k, v rows are read as fixed-RMS vectors.
template <typename T>
__global__ void __launch_bounds__(256)
depth_attn_generic_kernel(const T* __restrict__ q, const T* __restrict__ hk,
                          const T* __restrict__ hv, int64_t sbt, int64_t ss,
                          T* __restrict__ d_out, T* __restrict__ w_out, float* __restrict__ lse_out,
                          int64_t rows, int S, int QH, int HD, float scale, DepthRms rms) {
    const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const int qh = (int)(row % QH);
    const int64_t bt = row / QH;
    const T* kp = hk + bt * sbt + qh * HD;
    const T* vp = hv + bt * sbt + qh * HD;
    // fixed-RMS rows as fixed_rms forms them: scale and scaled elements rounded
    // to T (with target 0 the scale is 1 and the rows are read as stored)
    const float qsc = round_to<T>(row_rms_scale(q + qh * HD, HD, rms.qt));
    auto score = [&](int s) {
        const float ksc = round_to<T>(row_rms_scale(kp + s * ss, HD, rms.kt));
        float dot = 0.0f;
        for (int d = 0; d < HD; ++d)
            dot = fmaf(round_to<T>(ld(q + qh * HD + d) * qsc), round_to<T>(ld(kp + s * ss + d) * ksc), dot);
        return dot * scale;
    };
    float m = -INFINITY, l = 0.0f;
    for (int s = 0; s < S; ++s) m = fmaxf(m, score(s));
    for (int s = 0; s < S; ++s) {
        const float p = fexp(score(s) - m);
        l += p;
        if (w_out != nullptr) st(w_out + row * S + s, p);
    }
    const float inv_l = 1.0f / l;
    for (int d = 0; d < HD; ++d) {
        float a = 0.0f;
        for (int s = 0; s < S; ++s)
            a = fmaf(fexp(score(s) - m),
                     round_to<T>(ld(vp + s * ss + d) * round_to<T>(row_rms_scale(vp + s * ss, HD, rms.vt))), a);
        st(d_out + row * HD + d, a * inv_l);
    }
    if (w_out != nullptr)
        for (int s = 0; s < S; ++s) st(w_out + row * S + s, ld(w_out + row * S + s) * inv_l);
    if (lse_out != nullptr) lse_out[row] = m + logf(l);
}

template <typename T>
static int dispatch_depth(const void* q, const void* hk, const void* hv, int64_t sbt, int64_t ss,
                          void* d_out, void* w_out, float* lse_out, int64_t BT, int64_t S,
                          int64_t QH, int64_t HD, hipStream_t stream, DepthRms rms = DepthRms{}) {
    const bool with_rms = rms.qt != 0.0f || rms.kt != 0.0f || rms.vt != 0.0f;
    const int64_t rows = BT * QH;
    const float scale = 1.0f / sqrtf((float)HD);
    // a small launch (a decode step's rows) takes one wave per block so it
    // spreads over as many CUs as it has waves
    const int threads = rows * 16 >= 256 * 256 ? 256 : 64;
    // the vector path moves pairs of elements (4 B for 16-bit types, 8 B for
    // fp32) and indexes rows with 32-bit integers
    const bool aligned = sbt % 2 == 0 && ss % 2 == 0 &&
                         (((uintptr_t)hk | (uintptr_t)hv | (uintptr_t)q | (uintptr_t)d_out) % 8 == 0) &&
                         rows * 16 < ((int64_t)1 << 31) && BT * sbt < ((int64_t)1 << 62);
    const int epl = (HD % 16 == 0) ? (int)(HD / 16) : 0;
#define LOOM_DA_LAUNCH(E, C, R)                                                                  \
        hipLaunchKernelGGL((depth_attn_kernel<T, E, C, R>), dim3((unsigned)ceil_div(rows * 16, threads)), \
                           dim3(threads), 0, stream, (const T*)q, (const T*)hk, (const T*)hv, sbt, \
                           ss, (T*)d_out, (T*)w_out, lse_out, (int)rows, (int)S, (int)QH, scale, rms);
#define LOOM_DA_CASE(E)                                                                          \
    case E:                                                                                      \
        if (with_rms) {                                                                          \
            LOOM_DA_LAUNCH(E, kDepthChunk, true)                                                 \
        } else {                                                                                 \
            LOOM_DA_LAUNCH(E, kDepthChunk, false)                                                \
        }                                                                                        \
        return launch_status("loom_depth_attn_forward");
    if (aligned) {
        switch (epl) {
            LOOM_DA_CASE(2)
            LOOM_DA_CASE(4)
            LOOM_DA_CASE(6)
            LOOM_DA_CASE(8)
            default: break;
        }
    }
#undef LOOM_DA_CASE
#undef LOOM_DA_LAUNCH
    hipLaunchKernelGGL((depth_attn_generic_kernel<T>), dim3((unsigned)ceil_div(rows, threads)),
                       dim3(threads), 0, stream, (const T*)q, (const T*)hk, (const T*)hv, sbt, ss,
                       (T*)d_out, (T*)w_out, lse_out, rows, (int)S, (int)QH, (int)HD, scale, rms);
    return launch_status("loom_depth_attn_forward");
}

// Two depth queries over the same S slots in one pass (depth_row_pair):
// q1's read into d_out, q2's as normalised fp32 rows and log-sum-exp.
template <typename T, int EPL>
__global__ void __launch_bounds__(256)
depth_attn_pair_kernel(const T* __restrict__ q1, const T* __restrict__ q2,
                       const T* __restrict__ hk, const T* __restrict__ hv, int64_t sbt, int64_t ss,
                       T* __restrict__ d_out, float* __restrict__ pd_out,
                       float* __restrict__ lse_out, int rows, int S, int QH, float scale) {
    const int row = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 4);
    if (row >= rows) return;  // all 16 lanes of a group leave together
    // two slots per step: 8 (the default) keeps 89 VGPRs, 5 waves per SIMD, and
    // loads 8 slots at S = 1..7 (the chunked prefill's reads have S = 1..19;
    // at 4096 tokens x 8 heads, S = 1 / 9 / 19: 14.4 / 29.4 / 48.2 us with 8,
    // 8.7 / 24.6 / 46.9 us with 2)
    depth_row_pair<T, EPL, 2>(q1, q2, hk, hv, sbt, ss, d_out, pd_out, lse_out, row,
                           threadIdx.x & 15, S, QH, scale);
}

// The read over slots 0..S-1 from the read over slots 0..S-2 (normalised fp32
// rows and log-sum-exp) and slot S-1: one slot row of K and V per (bt, qh).
template <typename T, int EPL>
__global__ void __launch_bounds__(256)
depth_attn_fold_kernel(const T* __restrict__ q, const T* __restrict__ hk,
                       const T* __restrict__ hv, int64_t sbt, int64_t ss, int S,
                       const float* __restrict__ pd, const float* __restrict__ plse,
                       T* __restrict__ d_out, int rows, int QH, float scale) {
    constexpr int HD = EPL * 16;
    const int row = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 4);
    if (row >= rows) return;
    const int j = threadIdx.x & 15, qh = row % QH, bt = row / QH, d0 = j * EPL;
    const int64_t off = (int64_t)bt * sbt + (int64_t)(S - 1) * ss + qh * HD + d0;
    float qv[EPL], kn[EPL], vn[EPL], part[EPL], out[EPL];
    RowIO<T, EPL>::load(q + qh * HD + d0, qv);
    RowIO<T, EPL>::load(hk + off, kn);
    RowIO<T, EPL>::load(hv + off, vn);
    RowIO<float, EPL>::load(pd + (int64_t)row * HD + d0, part);
    depth_fold_last<EPL>(qv, kn, vn, part, plse[row], scale, out);
    RowIO<T, EPL>::store(d_out + (int64_t)row * HD + d0, out);
}

template <typename T>
static int dispatch_pair_fold(bool pair, const void* q1, const void* q2, const void* hk,
                              const void* hv, int64_t sbt, int64_t ss, int64_t S, void* d_out,
                              float* pd, float* plse, int64_t BT, int64_t QH, int64_t HD,
                              hipStream_t stream) {
    const int64_t rows = BT * QH;
    const float scale = 1.0f / sqrtf((float)HD);
    const int threads = rows * 16 >= 256 * 256 ? 256 : 64;
    const dim3 grid((unsigned)ceil_div(rows * 16, threads));
#define LOOM_PF_CASE(E)                                                                          \
    case E:                                                                                      \
        if (pair)                                                                                \
            hipLaunchKernelGGL((depth_attn_pair_kernel<T, E>), grid, dim3(threads), 0, stream,   \
                               (const T*)q1, (const T*)q2, (const T*)hk, (const T*)hv, sbt, ss,  \
                               (T*)d_out, pd, plse, (int)rows, (int)S, (int)QH, scale);          \
        else                                                                                     \
            hipLaunchKernelGGL((depth_attn_fold_kernel<T, E>), grid, dim3(threads), 0, stream,   \
                               (const T*)q1, (const T*)hk, (const T*)hv, sbt, ss, (int)S, pd,    \
                               plse, (T*)d_out, (int)rows, (int)QH, scale);                      \
        return launch_status(pair ? "loom_depth_attn_pair" : "loom_depth_attn_fold");
    switch (HD / 16) {
        LOOM_PF_CASE(2)
        LOOM_PF_CASE(4)
        LOOM_PF_CASE(6)
        LOOM_PF_CASE(8)
    }
#undef LOOM_PF_CASE
    set_error("depth_attn_pair/fold: head_dim %lld not supported", (long long)HD);
    return LOOM_ERR_INVALID;
}

}  // namespace loom

using namespace loom;

// shape and layout checks shared by loom_depth_attn_pair and loom_depth_attn_fold
static int pair_fold_entry(bool pair, int dtype, const void* q1, const void* q2, const void* hk,
                           const void* hv, int64_t sbt, int64_t ss, int64_t S, void* d_out,
                           float* pd, float* plse, int64_t BT, int64_t QH, int64_t HD,
                           void* stream) {
    const char* what = pair ? "depth_attn_pair" : "depth_attn_fold";
    LOOM_CHECK(q1 && (!pair || q2) && hk && hv && d_out && pd && plse, "%s: null tensor argument", what);
    LOOM_CHECK(BT >= 0 && S >= (pair ? 1 : 2) && QH >= 1, "%s: bad shape BT=%lld S=%lld", what,
               (long long)BT, (long long)S);
    LOOM_CHECK((HD == 32 || HD == 64 || HD == 96 || HD == 128),
               "%s: head_dim must be 32, 64, 96 or 128, got %lld", what, (long long)HD);
    LOOM_CHECK(ss >= QH * HD && sbt >= S * ss,
               "%s: strides (bt=%lld, s=%lld) overlap the [S,QH,HD] block", what, (long long)sbt,
               (long long)ss);
    LOOM_CHECK(sbt % 2 == 0 && ss % 2 == 0 &&
                   ((((uintptr_t)hk | (uintptr_t)hv | (uintptr_t)q1 | (uintptr_t)q2 |
                      (uintptr_t)d_out | (uintptr_t)pd) % 8) == 0) &&
                   BT * QH * 16 < ((int64_t)1 << 31),
               "%s: rows need 8-byte alignment and even strides", what);
    if (BT == 0) return LOOM_OK;
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case LOOM_F32:
            return dispatch_pair_fold<float>(pair, q1, q2, hk, hv, sbt, ss, S, d_out, pd, plse, BT, QH, HD, st);
        case LOOM_BF16:
            return dispatch_pair_fold<bf16_t>(pair, q1, q2, hk, hv, sbt, ss, S, d_out, pd, plse, BT, QH, HD, st);
        case LOOM_F16:
            return dispatch_pair_fold<f16_t>(pair, q1, q2, hk, hv, sbt, ss, S, d_out, pd, plse, BT, QH, HD, st);
    }
    set_error("%s: unsupported dtype %d", what, dtype);
    return LOOM_ERR_INVALID;
}

extern "C" int loom_depth_attn_pair(int dtype, const void* q1, const void* q2, const void* hist_k,
                                    const void* hist_v, int64_t stride_bt, int64_t stride_s,
                                    void* d_out, float* part_d, float* part_lse, int64_t BT,
                                    int64_t S, int64_t QH, int64_t HD, void* stream) {
    clear_error();
    return pair_fold_entry(true, dtype, q1, q2, hist_k, hist_v, stride_bt, stride_s, S, d_out,
                           part_d, part_lse, BT, QH, HD, stream);
}

extern "C" int loom_depth_attn_fold(int dtype, const void* q, const void* hist_k,
                                    const void* hist_v, int64_t stride_bt, int64_t stride_s,
                                    int64_t S, const float* part_d, const float* part_lse,
                                    void* d_out, int64_t BT, int64_t QH, int64_t HD, void* stream) {
    clear_error();
    return pair_fold_entry(false, dtype, q, q, hist_k, hist_v, stride_bt, stride_s, S, d_out,
                           (float*)part_d, (float*)part_lse, BT, QH, HD, stream);
}

static int depth_entry(int dtype, const void* q, const void* hist_k, const void* hist_v,
                       int64_t stride_bt, int64_t stride_s, void* d_out, void* w_out,
                       float* lse_out, int64_t BT, int64_t S, int64_t QH, int64_t HD,
                       void* stream, DepthRms rms) {
    LOOM_CHECK(q && hist_k && hist_v && d_out, "depth_attn: null tensor argument");
    LOOM_CHECK(BT >= 0 && S >= 1 && QH >= 1 && HD >= 1, "depth_attn: bad shape BT=%lld S=%lld",
               (long long)BT, (long long)S);
    LOOM_CHECK(stride_s >= QH * HD && stride_bt >= S * stride_s,
               "depth_attn: strides (bt=%lld, s=%lld) overlap the [S,QH,HD] block",
               (long long)stride_bt, (long long)stride_s);
    if (BT == 0) return LOOM_OK;
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case LOOM_F32:
            return dispatch_depth<float>(q, hist_k, hist_v, stride_bt, stride_s, d_out, w_out,
                                         lse_out, BT, S, QH, HD, st, rms);
        case LOOM_BF16:
            return dispatch_depth<bf16_t>(q, hist_k, hist_v, stride_bt, stride_s, d_out, w_out,
                                          lse_out, BT, S, QH, HD, st, rms);
        case LOOM_F16:
            return dispatch_depth<f16_t>(q, hist_k, hist_v, stride_bt, stride_s, d_out, w_out,
                                         lse_out, BT, S, QH, HD, st, rms);
    }
    set_error("depth_attn: unsupported dtype %d", dtype);
    return LOOM_ERR_INVALID;
}

extern "C" int loom_depth_attn_forward(int dtype, const void* q, const void* hist_k,
                                       const void* hist_v, int64_t stride_bt, int64_t stride_s,
                                       void* d_out, void* w_out, float* lse_out, int64_t BT,
                                       int64_t S, int64_t QH, int64_t HD, void* stream) {
    clear_error();
    return depth_entry(dtype, q, hist_k, hist_v, stride_bt, stride_s, d_out, w_out, lse_out, BT, S,
                       QH, HD, stream, DepthRms{});
}

extern "C" int loom_depth_attn_forward_rms(int dtype, const void* q, const void* hist_k,
                                           const void* hist_v, int64_t stride_bt,
                                           int64_t stride_s, void* d_out, void* w_out,
                                           float* lse_out, int64_t BT, int64_t S, int64_t QH,
                                           int64_t HD, float q_target, float k_target,
                                           float v_target, void* stream) {
    clear_error();
    LOOM_CHECK(q_target > 0.0f && k_target > 0.0f && v_target > 0.0f,
               "depth_attn_rms: targets must be positive (q %g, k %g, v %g)", (double)q_target,
               (double)k_target, (double)v_target);
    return depth_entry(dtype, q, hist_k, hist_v, stride_bt, stride_s, d_out, w_out, lse_out, BT, S,
                       QH, HD, stream, DepthRms{q_target, k_target, v_target});
}
