// Decode-step kernels for gfx950: RoPE + KV-cache append, GQA decode
// attention with the dual readout (A.V and A.K_roped), fused residual add +
// LayerNorm, and the decode-time temporal Tria update (+ PolARM on fires).
#include <cmath>

#include "loom_common.h"

namespace loom {

// ------------------------------------------------------------------ RoPE + append
// qkv row b = [q (QH*HD) | k (KVH*HD) | v (KVH*HD)].  q_out[b] = rope(q);
// cache_k[b, pos] = rope(k); cache_v[b, pos] = v.  cos/sin: fp32 [*, HD] tables
// already scaled by the YaRN attention factor.
template <typename T>
__global__ void __launch_bounds__(256)
rope_append_kernel(const T* __restrict__ qkv, T* __restrict__ q_out, T* __restrict__ kc,
                   T* __restrict__ vc, const float* __restrict__ cosv, const float* __restrict__ sinv,
                   int64_t B, int64_t pos, int QH, int KVH, int HD, int64_t cstride_b,
                   int64_t cstride_t) {
    const int heads = QH + 2 * KVH;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= B * heads * HD) return;
    const int d = (int)(id % HD);
    const int hs = (int)((id / HD) % heads);
    const int64_t b = id / ((int64_t)HD * heads);
    const T* row = qkv + b * (int64_t)heads * HD;
    const int half = HD / 2;
    const float* cr = cosv + pos * HD;
    const float* sr = sinv + pos * HD;
    if (hs < QH + KVH) {
        const T* x = row + hs * HD;
        const float rot = d < half ? -ld(x + d + half) : ld(x + d - half);
        const float v = ld(x + d) * cr[d] + rot * sr[d];
        if (hs < QH)
            st(q_out + (b * QH + hs) * HD + d, v);
        else
            st(kc + b * cstride_b + pos * cstride_t + (hs - QH) * HD + d, v);
    } else {
        const int kvh = hs - QH - KVH;
        st(vc + b * cstride_b + pos * cstride_t + kvh * HD + d, ld(row + hs * HD + d));
    }
}

// ------------------------------------------------------------------ GQA attention
// Split over the sequence (flash-decoding): block (chunk, kvh, b) handles
// kAttnChunk positions for the G query heads that share kv head kvh and writes
// an unnormalised partial (m, l, sum p*v, sum p*k) per head; the combine
// kernel merges the chunks.  Lanes are grouped 16 per cache row, EPL = HD/16
// contiguous elements per lane.
constexpr int kAttnChunk = 256;
constexpr int kAttnMaxG = 8;

template <typename T, int EPL, int G, int LPR>
__global__ void __launch_bounds__(256)
gqa_partial_kernel(const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc,
                   int64_t cstride_b, int64_t cstride_t, float* __restrict__ ws, int64_t len,
                   int QH, int KVH, float scale) {
    constexpr int HD = EPL * LPR;
    constexpr int RG = 256 / LPR;          // rows handled concurrently by the block
    constexpr int RPW = 64 / LPR;          // row groups per wave
    __shared__ float sc[G][kAttnChunk];
    __shared__ float red[4][2 * G * HD];
    __shared__ float stat[G][2];
    const int chunk = blockIdx.x, kvh = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int nchunks = gridDim.x;
    const int tid = threadIdx.x, j = tid % LPR, grp = tid / LPR;
    const int64_t t0 = (int64_t)chunk * kAttnChunk;
    const int64_t t1 = t0 + kAttnChunk < len ? t0 + kAttnChunk : len;
    const int d0 = j * EPL;

    float qv[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) qv[g][e] = ld(q + (b * QH + kvh * G + g) * HD + d0 + e) * scale;

    const T* kbase = kc + b * cstride_b + kvh * HD + d0;
    const T* vbase = vc + b * cstride_b + kvh * HD + d0;
    // scores
    for (int64_t t = t0 + grp; t < t0 + kAttnChunk; t += RG) {
        float dot[G];
#pragma unroll
        for (int g = 0; g < G; ++g) dot[g] = 0.0f;
        if (t < t1) {
            float kv[EPL];
#pragma unroll
            for (int e = 0; e < EPL; ++e) kv[e] = ld(kbase + t * cstride_t + e);
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < EPL; ++e) dot[g] = fmaf(qv[g][e], kv[e], dot[g]);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float s = group_sum<LPR>(dot[g]);
            if (j == 0) sc[g][t - t0] = t < t1 ? s : -INFINITY;
        }
    }
    __syncthreads();
    // per-head max / exp / sum (wave w handles heads w, w+4, ...)
    const int wave = tid >> 6, lane = tid & 63;
    for (int g = wave; g < G; g += 4) {
        float m = -INFINITY;
        for (int k = lane; k < kAttnChunk; k += 64) m = fmaxf(m, sc[g][k]);
        m = wave_max(m);
        float l = 0.0f;
        for (int k = lane; k < kAttnChunk; k += 64) {
            const float p = sc[g][k] == -INFINITY ? 0.0f : fexp(sc[g][k] - m);
            sc[g][k] = p;
            l += p;
        }
        l = wave_sum(l);
        if (lane == 0) {
            stat[g][0] = m;
            stat[g][1] = l;
        }
    }
    __syncthreads();
    // weighted sums of V and K
    float cacc[G][EPL], kacc[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) cacc[g][e] = kacc[g][e] = 0.0f;
    for (int64_t t = t0 + grp; t < t1; t += RG) {
        float kv[EPL], vv[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            kv[e] = ld(kbase + t * cstride_t + e);
            vv[e] = ld(vbase + t * cstride_t + e);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float p = sc[g][t - t0];
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                cacc[g][e] = fmaf(p, vv[e], cacc[g][e]);
                kacc[g][e] = fmaf(p, kv[e], kacc[g][e]);
            }
        }
    }
    // reduce the RPW row groups of each wave (lanes j, j+LPR, ...)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float c = cacc[g][e], k = kacc[g][e];
#pragma unroll
            for (int off = LPR; off < 64; off <<= 1) {
                c += __shfl_xor(c, off, 64);
                k += __shfl_xor(k, off, 64);
            }
            cacc[g][e] = c;
            kacc[g][e] = k;
        }
    if (lane < LPR) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                red[wave][g * HD + d0 + e] = cacc[g][e];
                red[wave][G * HD + g * HD + d0 + e] = kacc[g][e];
            }
    }
    __syncthreads();
    // partial record: [m(G) | l(G) | c(G*HD) | kctx(G*HD)]
    const int rec = 2 * G + 2 * G * HD;
    float* out = ws + (((int64_t)b * KVH + kvh) * nchunks + chunk) * rec;
    for (int k = tid; k < 2 * G * HD; k += blockDim.x)
        out[2 * G + k] = red[0][k] + red[1][k] + red[2][k] + red[3][k];
    if (tid < G) {
        out[tid] = stat[tid][0];
        out[G + tid] = stat[tid][1];
    }
    (void)RPW;
}

template <typename T, int G>
__global__ void __launch_bounds__(256)
gqa_combine_kernel(const float* __restrict__ ws, T* __restrict__ c_out, T* __restrict__ k_out,
                   int nchunks, int QH, int KVH, int HD) {
    const int kvh = blockIdx.x;
    const int64_t b = blockIdx.y;
    const int rec = 2 * G + 2 * G * HD;
    const float* base = ws + ((int64_t)b * KVH + kvh) * nchunks * rec;
    for (int k = threadIdx.x; k < G * HD; k += blockDim.x) {
        const int g = k / HD, d = k % HD;
        float M = -INFINITY;
        for (int c = 0; c < nchunks; ++c) M = fmaxf(M, base[c * rec + g]);
        float L = 0.0f, C = 0.0f, K = 0.0f;
        for (int c = 0; c < nchunks; ++c) {
            const float* r = base + c * rec;
            if (r[g] == -INFINITY) continue;
            const float w = fexp(r[g] - M);
            L = fmaf(r[G + g], w, L);
            C = fmaf(r[2 * G + g * HD + d], w, C);
            K = fmaf(r[2 * G + G * HD + g * HD + d], w, K);
        }
        const float inv = 1.0f / L;
        const int64_t o = (b * QH + kvh * G + g) * HD + d;
        st(c_out + o, C * inv);
        st(k_out + o, K * inv);
    }
}

// ------------------------------------------------------------------ add + LayerNorm
// out = LN(a + b) * gamma + beta over rows of N (biased variance, eps inside
// the root, as torch.nn.LayerNorm); one wavefront per row.
template <typename T>
__global__ void __launch_bounds__(256)
add_layernorm_kernel(const T* __restrict__ a, const T* __restrict__ bsrc,
                     const float* __restrict__ gamma, const float* __restrict__ beta,
                     T* __restrict__ out, int64_t rows, int N, float eps) {
    const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    constexpr int kMax = 32;  // N <= 64 * 32
    float x[kMax];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kMax; ++k) {
        const int c = lane + 64 * k;
        x[k] = 0.0f;
        if (c < N) {
            x[k] = ld(a + row * N + c) + (bsrc ? ld(bsrc + row * N + c) : 0.0f);
            s += x[k];
        }
    }
    const float mean = wave_sum(s) / N;
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < kMax; ++k) {
        const int c = lane + 64 * k;
        if (c < N) {
            const float dlt = x[k] - mean;
            v = fmaf(dlt, dlt, v);
        }
    }
    const float rstd = 1.0f / sqrtf(wave_sum(v) / N + eps);
#pragma unroll
    for (int k = 0; k < kMax; ++k) {
        const int c = lane + 64 * k;
        if (c < N) st(out + row * N + c, (x[k] - mean) * rstd * gamma[c] + beta[c]);
    }
}

// ------------------------------------------------------------------ temporal decode step
__device__ __forceinline__ void mm3d(const float A[9], const float B[9], float o[9]) {
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int c = 0; c < 3; ++c)
            o[3 * r + c] = fmaf(A[3 * r + 2], B[6 + c], fmaf(A[3 * r + 1], B[3 + c], A[3 * r] * B[c]));
}

template <typename T>
__global__ void __launch_bounds__(256)
decode_temporal_kernel(const T* __restrict__ depth, const T* __restrict__ prev,
                       const uint8_t* __restrict__ reset_now, const uint8_t* __restrict__ fire,
                       T* __restrict__ out, int64_t B, int64_t H, float beta, float eps) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= B * H) return;
    const int64_t b = e / H;
    float M[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) M[k] = ld(depth + e * 9 + k);
    if (prev != nullptr && reset_now[b] == 0) {
        float P[9], R[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) P[k] = ld(prev + e * 9 + k);
        mm3d(M, P, R);
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < 9; ++k) s = fmaf(R[k], R[k], s);
        const float inv = 1.0f / sqrtf(s * (1.0f / 9.0f) + 1e-6f);
#pragma unroll
        for (int k = 0; k < 9; ++k) M[k] = R[k] * inv;
    }
    if (fire != nullptr && fire[b] != 0) {
        float Gm[9];
#pragma unroll
        for (int r = 0; r < 3; ++r)
#pragma unroll
            for (int c = 0; c < 3; ++c)
                Gm[3 * r + c] = fmaf(M[6 + r], M[6 + c], fmaf(M[3 + r], M[3 + c], M[r] * M[c]));
        const float s = fmaxf((Gm[0] + Gm[4] + Gm[8]) * (1.0f / 3.0f), eps);
        float C[9], R[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            const float id = (k == 0 || k == 4 || k == 8) ? 1.0f : 0.0f;
            C[k] = id - 0.5f * beta * (Gm[k] / s - id);
        }
        mm3d(M, C, R);
#pragma unroll
        for (int k = 0; k < 9; ++k) M[k] = R[k];
    }
#pragma unroll
    for (int k = 0; k < 9; ++k) st(out + e * 9 + k, M[k]);
}

// ------------------------------------------------------------------ dispatch

template <typename T>
static int rope_dispatch(const void* qkv, void* q_out, void* kc, void* vc, const float* cosv,
                         const float* sinv, int64_t B, int64_t pos, int64_t QH, int64_t KVH,
                         int64_t HD, int64_t sb, int64_t stt, hipStream_t st) {
    const int64_t total = B * (QH + 2 * KVH) * HD;
    hipLaunchKernelGGL((rope_append_kernel<T>), dim3((unsigned)ceil_div(total, 256)), dim3(256), 0,
                       st, (const T*)qkv, (T*)q_out, (T*)kc, (T*)vc, cosv, sinv, B, pos, (int)QH,
                       (int)KVH, (int)HD, sb, stt);
    return launch_status("loom_rope_append");
}

template <typename T>
static int gqa_dispatch(const void* q, const void* kc, const void* vc, int64_t sb, int64_t stt,
                        void* c_out, void* k_out, float* ws, int64_t B, int64_t len, int64_t QH,
                        int64_t KVH, int64_t HD, hipStream_t st) {
    const int G = (int)(QH / KVH);
    const int nchunks = (int)ceil_div(len, kAttnChunk);
    const float scale = 1.0f / sqrtf((float)HD);
    dim3 grid(nchunks, (unsigned)KVH, (unsigned)B);
#define LOOM_GQA(E, GG, LPR)                                                                     \
    if (HD == E * LPR && G == GG) {                                                              \
        hipLaunchKernelGGL((gqa_partial_kernel<T, E, GG, LPR>), grid, dim3(256), 0, st, (const T*)q, \
                           (const T*)kc, (const T*)vc, sb, stt, ws, len, (int)QH, (int)KVH,       \
                           scale);                                                               \
        int rc = launch_status("loom_gqa_decode_attention");                                    \
        if (rc != LOOM_OK) return rc;                                                            \
        hipLaunchKernelGGL((gqa_combine_kernel<T, GG>), dim3((unsigned)KVH, (unsigned)B),        \
                           dim3(256), 0, st, ws, (T*)c_out, (T*)k_out, nchunks, (int)QH,         \
                           (int)KVH, (int)HD);                                                   \
        return launch_status("loom_gqa_decode_attention(combine)");                              \
    }
    LOOM_GQA(6, 4, 16)
    LOOM_GQA(6, 1, 16)
    LOOM_GQA(6, 2, 16)
    LOOM_GQA(6, 8, 16)
    LOOM_GQA(4, 4, 16)
    LOOM_GQA(8, 4, 16)
    LOOM_GQA(2, 4, 16)
    LOOM_GQA(4, 2, 16)
    LOOM_GQA(8, 2, 16)
    LOOM_GQA(1, 1, 8)
    LOOM_GQA(1, 2, 8)
    LOOM_GQA(1, 4, 8)
#undef LOOM_GQA
    set_error("gqa_decode_attention: unsupported head_dim %lld / group %d", (long long)HD, G);
    return LOOM_ERR_INVALID;
}

template <typename T>
static int ln_dispatch(const void* a, const void* b, const float* g, const float* be, void* out,
                       int64_t rows, int64_t N, float eps, hipStream_t st) {
    hipLaunchKernelGGL((add_layernorm_kernel<T>), dim3((unsigned)ceil_div(rows * 64, 256)),
                       dim3(256), 0, st, (const T*)a, (const T*)b, g, be, (T*)out, rows, (int)N,
                       eps);
    return launch_status("loom_add_layernorm");
}

template <typename T>
static int temporal_step_dispatch(const void* depth, const void* prev, const uint8_t* reset_now,
                                  const uint8_t* fire, void* out, int64_t B, int64_t H, float beta,
                                  float eps, hipStream_t st) {
    hipLaunchKernelGGL((decode_temporal_kernel<T>), dim3((unsigned)ceil_div(B * H, 256)), dim3(256),
                       0, st, (const T*)depth, (const T*)prev, reset_now, fire, (T*)out, B, H,
                       beta, eps);
    return launch_status("loom_tria_decode_temporal");
}

#define LOOM_DTYPE_SWITCH(dtype, FN, ...)               \
    switch (dtype) {                                    \
        case LOOM_F32: return FN<float>(__VA_ARGS__);   \
        case LOOM_BF16: return FN<bf16_t>(__VA_ARGS__); \
        case LOOM_F16: return FN<f16_t>(__VA_ARGS__);   \
    }                                                   \
    set_error("unsupported dtype %d", dtype);           \
    return LOOM_ERR_INVALID;

}  // namespace loom

using namespace loom;

extern "C" int64_t loom_gqa_workspace_bytes(int64_t B, int64_t max_len, int64_t QH, int64_t KVH,
                                            int64_t HD) {
    const int64_t G = QH / KVH;
    const int64_t nchunks = ceil_div(max_len, kAttnChunk);
    return B * KVH * nchunks * (2 * G + 2 * G * HD) * (int64_t)sizeof(float);
}

extern "C" int loom_rope_append(int dtype, const void* qkv, void* q_out, void* k_cache,
                                void* v_cache, const float* cos_table, const float* sin_table,
                                int64_t B, int64_t pos, int64_t QH, int64_t KVH, int64_t HD,
                                int64_t cache_stride_b, int64_t cache_stride_t, void* stream) {
    clear_error();
    LOOM_CHECK(qkv && q_out && k_cache && v_cache && cos_table && sin_table,
               "rope_append: null argument");
    LOOM_CHECK(HD % 2 == 0 && QH > 0 && KVH > 0 && pos >= 0, "rope_append: bad shape");
    LOOM_CHECK(cache_stride_t >= KVH * HD, "rope_append: cache row stride too small");
    if (B == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, rope_dispatch, qkv, q_out, k_cache, v_cache, cos_table, sin_table, B,
                      pos, QH, KVH, HD, cache_stride_b, cache_stride_t, (hipStream_t)stream)
}

extern "C" int loom_gqa_decode_attention(int dtype, const void* q, const void* k_cache,
                                         const void* v_cache, int64_t cache_stride_b,
                                         int64_t cache_stride_t, void* c_out, void* kctx_out,
                                         float* workspace, int64_t workspace_bytes, int64_t B,
                                         int64_t len, int64_t QH, int64_t KVH, int64_t HD,
                                         void* stream) {
    clear_error();
    LOOM_CHECK(q && k_cache && v_cache && c_out && kctx_out && workspace,
               "gqa_decode_attention: null argument");
    LOOM_CHECK(len >= 1 && KVH >= 1 && QH % KVH == 0 && QH / KVH <= kAttnMaxG,
               "gqa_decode_attention: bad shape len=%lld QH=%lld KVH=%lld", (long long)len,
               (long long)QH, (long long)KVH);
    LOOM_CHECK(workspace_bytes >= loom_gqa_workspace_bytes(B, len, QH, KVH, HD),
               "gqa_decode_attention: workspace too small (%lld bytes)", (long long)workspace_bytes);
    if (B == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, gqa_dispatch, q, k_cache, v_cache, cache_stride_b, cache_stride_t,
                      c_out, kctx_out, workspace, B, len, QH, KVH, HD, (hipStream_t)stream)
}

extern "C" int loom_add_layernorm(int dtype, const void* a, const void* b, const float* gamma,
                                  const float* beta, void* out, int64_t rows, int64_t N,
                                  float eps, void* stream) {
    clear_error();
    LOOM_CHECK(a && gamma && beta && out, "add_layernorm: null argument");
    LOOM_CHECK(N >= 1 && N <= 64 * 32, "add_layernorm: N=%lld outside [1, 2048]", (long long)N);
    if (rows == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, ln_dispatch, a, b, gamma, beta, out, rows, N, eps, (hipStream_t)stream)
}

extern "C" int loom_tria_decode_temporal(int dtype, const void* depth, const void* prev,
                                         const uint8_t* reset_now, const uint8_t* fire, void* out,
                                         int64_t B, int64_t H, float polarm_beta, float eps,
                                         void* stream) {
    clear_error();
    LOOM_CHECK(depth && out, "tria_decode_temporal: null argument");
    LOOM_CHECK(!prev || reset_now, "tria_decode_temporal: prev needs reset_now");
    LOOM_CHECK(polarm_beta >= 0.0f && polarm_beta < 1.0f,
               "PolARM beta must be finite and in [0, 1), got %g", (double)polarm_beta);
    if (B * H == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, temporal_step_dispatch, depth, prev, reset_now, fire, out, B, H,
                      polarm_beta, eps, (hipStream_t)stream)
}
