// Decode-step kernels for gfx950: RoPE + KV-cache append, GQA decode
// attention with the dual readout (A.V and A.K_roped), fused residual add +
// LayerNorm, and the decode-time temporal Tria update (+ PolARM on fires).
#include <cmath>
#include <type_traits>

#include "attn_tile.h"
#include "loom_common.h"
#include "depth_row.h"

namespace loom {

// ------------------------------------------------------------------ RoPE + append
// qkv row b = [q (QH*HD) | k (KVH*HD) | v (KVH*HD)].  q_out[b] = rope(q);
// cache_k[b, pos] = rope(k); cache_v[b, pos] = v.  cos/sin: fp32 [*, HD] tables
// already scaled by the YaRN attention factor.
template <typename T>
__global__ void __launch_bounds__(256)
rope_append_kernel(const T* __restrict__ qkv, T* __restrict__ q_out, T* __restrict__ kc,
                   T* __restrict__ vc, const float* __restrict__ cosv, const float* __restrict__ sinv,
                   int64_t B, int64_t pos, const int64_t* __restrict__ pos_dev, int QH, int KVH,
                   int HD, int64_t cstride_b, int64_t cstride_t, int64_t cstride_h) {
    if (pos_dev != nullptr) pos = *pos_dev;
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
            st(kc + b * cstride_b + pos * cstride_t + (hs - QH) * cstride_h + d, v);
    } else {
        const int kvh = hs - QH - KVH;
        st(vc + b * cstride_b + pos * cstride_t + kvh * cstride_h + d, ld(row + hs * HD + d));
    }
}

// ------------------------------------------------------------------ GQA attention
// Split over the sequence (flash-decoding): block (chunk, kvh, b) covers one
// of the row's nchunks equal slices of the positions (gqa_chunk_len) for the
// G query heads that share kv head kvh and
// publishes an unnormalised partial record (m, l, sum p*v, sum p*k) per head.
// One pass over K and V: each cache row is read once and feeds both the
// scores and the A.K readout.  gqa_merge_kernel, the next launch, merges each
// row's records and writes C = A.V and Kctx = A.K_roped (a separate launch is
// cheaper than an in-kernel last-block merge, whose device-coherent record
// stores, arrival atomic and record loads are three serial memory trips).
//
// FROM_QKV: q comes unroped from the step's qkv row; the block roped q
// itself, and the block that holds position pos also ropes this token's k,
// attends to it from registers and appends (k_roped, v) to the caches
// (RoPE + cache append + attention in one launch, the combine in the next).
//
// Mapping: LPR lanes per cache row (EPL = HD/LPR contiguous elements each);
// the block's NG = 256/LPR row groups take positions t0 + grp + NG*i.  A group
// scores kAttnBatch positions for all G heads at once, then folds them into an
// online softmax with one rescale per batch.  Scores are kept in log2 units
// (q is pre-scaled by log2(e)/sqrt(HD)) so every exponential is one v_exp_f32.
// Chunk blocks per (b, kv head) row: about 1.5 blocks per CU over the whole
// grid (fewer, longer chunks measured faster than one chunk per 256 positions:
// every block pays its record and its ramp-up), and no chunk shorter than
// kAttnMinChunk positions.  The workspace and the launch use the same count.
constexpr int kAttnMinChunk = 128;
static int gqa_nchunks(int64_t B, int64_t KVH, int64_t max_len) {
    const int64_t rows = B * KVH;
    int64_t nc = (3 * (int64_t)device_cus() / 2 + rows - 1) / rows;
    const int64_t cap = (max_len + kAttnMinChunk - 1) / kAttnMinChunk;
    nc = nc < cap ? nc : cap;
    return (int)(nc > 1 ? nc : 1);
}

// Positions per chunk block when a row of len positions is split over nchunks
// blocks: equal slices, rounded up to a whole 32-position wave step.
__host__ __device__ __forceinline__ int64_t gqa_chunk_len(int64_t len, int nchunks) {
    const int64_t c = (len + nchunks - 1) / nchunks;
    return (c + 31) / 32 * 32;
}
constexpr int kAttnMaxG = 8;
constexpr int kAttnBatch = 4;

template <typename T>
struct GqaArgs {
    const T* q;            // roped q [B, QH, HD], or the qkv rows [B, (QH + 2 KVH) HD]
    T* kc;
    T* vc;
    int64_t csb, cst, csh; // cache strides (elements) of b, t and kv head
    const float* cosv;     // FROM_QKV: RoPE tables [*, HD] (attention factor folded in)
    const float* sinv;
    T* q_out;              // FROM_QKV, optional: the roped q [B, QH, HD]
    float* rec;            // [B, KVH, nchunks, REC]
    T* c_out;              // [B, QH, HD] with row stride out_sb
    T* k_out;
    int64_t out_sb;
    int64_t len;           // attended positions (ignored when pos_dev is set)
    const int64_t* pos_dev;
    int QH, KVH;
    float qscale;
    int nchunks;           // chunk blocks per (b, kv head) in the grid (records per row)
    // optional depth read folded into the launch (bf16 MFMA form): grid slice
    // x == nchunks computes DepthAttn rows (b, kvh*G .. kvh*G+G-1)
    const T* dq;           // [QH, HD] learned queries of the depth slot, or null
    const T* dk;
    const T* dv;
    int64_t dsbt, dss;     // history strides (b, slot)
    T* dout;               // [B, QH, HD]
    int dS;
    float dscale;
    // optional second query over the same slots (the next sublayer's read):
    // its normalised read in fp32 and its log-sum-exp, for a later fold of
    // the one slot that read adds
    const T* dq2;          // [QH, HD] or null
    float* dpd;            // [B, QH, HD]
    float* dpl;            // [B, QH]
};

// element d of head h of a qkv row, roped for position pos (x*cos + rot(x)*sin)
template <typename T>
__device__ __forceinline__ float rope_elem(const T* head, const float* cr, const float* sr, int d,
                                           int HD) {
    const int half = HD / 2;
    const float rot = d < half ? -ld(head + d + half) : ld(head + d - half);
    return ld(head + d) * cr[d] + rot * sr[d];
}

// End of a GQA chunk block: merge the four waves' partials wred[w] = [m(G) |
// l(G) | c(G*HD) | k(G*HD)] into the chunk's record (unnormalised, scores in
// log2 units).  The records of a row are merged by gqa_merge_kernel, the next
// launch on the stream.
template <typename T, int G, int HD>
__device__ __forceinline__ void gqa_record(const GqaArgs<T>& a, float (*wred)[2 * G + 2 * G * HD],
                                           int64_t b, int kvh, int chunk, int nchunks) {
    constexpr int REC = 2 * G + 2 * G * HD;
    float* rec = a.rec + (((int64_t)b * a.KVH + kvh) * nchunks + chunk) * REC;
    for (int k = threadIdx.x; k < REC; k += blockDim.x) {
        const int g = k < 2 * G ? k % G : ((k - 2 * G) % (G * HD)) / HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, wred[w][g]);
        float acc = M;
        if (k >= G) {
            acc = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                if (wred[w][g] != -INFINITY) acc = fmaf(wred[w][k], __builtin_amdgcn_exp2f(wred[w][g] - M), acc);
        }
        rec[k] = acc;
    }
}

// Second pass of the split attention: thread per output element (b, head, d)
// merges the nact chunk records of its (b, kv head) into C = A.V and
// Kctx = A.K_roped (flash-decoding's combine), with kMergeBatch chunks' loads
// in flight at once.
constexpr int kMergeBatch = 16;

template <typename T>
__global__ void __launch_bounds__(256)
gqa_merge_kernel(const float* __restrict__ rec, int nchunks, int64_t len,
                 const int64_t* __restrict__ pos_dev, T* __restrict__ c_out, T* __restrict__ k_out,
                 int64_t out_sb, int B, int QH, int KVH, int HD) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= (int64_t)B * QH * HD) return;
    const int d = (int)(e % HD);
    const int h = (int)((e / HD) % QH);
    const int64_t b = e / ((int64_t)HD * QH);
    const int G = QH / KVH, kvh = h / G, g = h % G;
    const int REC = 2 * G + 2 * G * HD;
    // the records of a batch of chunks are requested before the position is
    // used (a record past the active chunks is read and then ignored: the
    // workspace holds nchunks records), so a merge of up to kMergeBatch chunks
    // is one memory round trip
    const float* recs = rec + (b * KVH + kvh) * (int64_t)nchunks * REC;
    float M = -INFINITY, L = 0.0f, C = 0.0f, K = 0.0f;
    auto batch = [&](int c0) {
        float m[kMergeBatch], l[kMergeBatch], cv[kMergeBatch], kv[kMergeBatch];
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
            const float* r = recs + (int64_t)(c0 + u < nchunks ? c0 + u : 0) * REC;
            m[u] = r[g];
            l[u] = r[G + g];
            cv[u] = r[2 * G + g * HD + d];
            kv[u] = r[2 * G + G * HD + g * HD + d];
        }
        __builtin_amdgcn_sched_barrier(0);   // the position's wait stays after the requests
        const int64_t n = pos_dev != nullptr ? *pos_dev + 1 : len;
        const int64_t clen = gqa_chunk_len(n, nchunks);
        const int nact = (int)((n + clen - 1) / clen);
        if (c0 >= nact) return false;
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
            if (c0 + u < nact) continue;
            m[u] = -INFINITY;
            l[u] = 0.0f;
            cv[u] = 0.0f;
            kv[u] = 0.0f;
        }
        float Mb = M;
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) Mb = fmaxf(Mb, m[u]);
        if (Mb == -INFINITY) return true;
        const float r0 = __builtin_amdgcn_exp2f(M - Mb);   // 0 while M is -inf
        L *= r0;
        C *= r0;
        K *= r0;
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
            if (m[u] == -INFINITY) continue;
            const float w = __builtin_amdgcn_exp2f(m[u] - Mb);
            L = fmaf(l[u], w, L);
            C = fmaf(cv[u], w, C);
            K = fmaf(kv[u], w, K);
        }
        M = Mb;
        return true;
    };
    if (batch(0))
        for (int c0 = kMergeBatch; c0 < nchunks; c0 += kMergeBatch)
            if (!batch(c0)) break;
    const float inv = 1.0f / L;
    const int64_t o = b * out_sb + h * HD + d;
    st(c_out + o, C * inv);
    st(k_out + o, K * inv);
}

template <typename T, int EPL, int G, int LPR, bool FROM_QKV>
__global__ void __launch_bounds__(256)
gqa_decode_kernel(GqaArgs<T> a) {
    constexpr int HD = EPL * LPR;
    constexpr int NG = 256 / LPR;          // row groups per block
    constexpr int REC = 2 * G + 2 * G * HD;
    __shared__ float wred[4][REC];
    const int chunk = blockIdx.x, kvh = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int nchunks = a.nchunks;
    const int tid = threadIdx.x, j = tid % LPR, grp = tid / LPR;
    const int wave = tid >> 6, lane = tid & 63;
    const int64_t len = a.pos_dev != nullptr ? *a.pos_dev + 1 : a.len;
    const int64_t pos = len - 1;
    const int64_t clen = gqa_chunk_len(len, nchunks);
    const int nact = (int)((len + clen - 1) / clen);
    if (chunk >= nact) return;                    // past the end: no record
    const int64_t t0 = (int64_t)chunk * clen;
    const int64_t t1 = t0 + clen < len ? t0 + clen : len;
    // FROM_QKV: the cache holds positions < pos; position pos comes from qkv
    // and is folded in by the one chunk that contains it
    const bool holds_pos = FROM_QKV && t1 == len;
    const int64_t tc = holds_pos ? pos : t1;
    const int d0 = j * EPL;
    const int QKV = (a.QH + 2 * a.KVH) * HD;

    float qv[G][EPL];
    if constexpr (FROM_QKV) {
        const T* qrow = a.q + b * QKV;
        const float* cr = a.cosv + pos * HD;
        const float* sr = a.sinv + pos * HD;
        const bool write_q = a.q_out != nullptr && chunk == 0 && grp == 0;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const float x = rope_elem(qrow + (kvh * G + g) * HD, cr, sr, d0 + e, HD);
                if (write_q) st(a.q_out + (b * a.QH + kvh * G + g) * HD + d0 + e, x);
                qv[g][e] = x * a.qscale;
            }
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < EPL; ++e)
                qv[g][e] = ld(a.q + (b * a.QH + kvh * G + g) * HD + d0 + e) * a.qscale;
    }

    const T* kbase = a.kc + b * a.csb + kvh * a.csh + d0;
    const T* vbase = a.vc + b * a.csb + kvh * a.csh + d0;
    float m[G], l[G], ac[G][EPL], ak[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) ac[g][e] = ak[g][e] = 0.0f;
    }
    // fold kAttnBatch positions (scores s[u], rows kv[u], vv[u]) into head g's state
    auto fold = [&](int g, const float* s, const bool* ok, float (*kv)[EPL], float (*vv)[EPL],
                    int nb) {
        float mx = m[g];
        for (int u = 0; u < nb; ++u) mx = fmaxf(mx, ok[u] ? s[u] : -INFINITY);
        if (mx == -INFINITY) return;
        const float corr = __builtin_amdgcn_exp2f(m[g] - mx);   // 0 when m was -inf
        float lsum = l[g] * corr;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            ac[g][e] *= corr;
            ak[g][e] *= corr;
        }
        for (int u = 0; u < nb; ++u) {
            const float p = ok[u] ? __builtin_amdgcn_exp2f(s[u] - mx) : 0.0f;
            lsum += p;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                ac[g][e] = fmaf(p, vv[u][e], ac[g][e]);
                ak[g][e] = fmaf(p, kv[u][e], ak[g][e]);
            }
        }
        l[g] = lsum;
        m[g] = mx;
    };
    for (int64_t base = t0 + grp; base < tc; base += NG * kAttnBatch) {
        float kv[kAttnBatch][EPL], vv[kAttnBatch][EPL];
        bool ok[kAttnBatch];
#pragma unroll
        for (int u = 0; u < kAttnBatch; ++u) {
            const int64_t t = base + (int64_t)NG * u;
            ok[u] = t < tc;
            const int64_t tr = ok[u] ? t : tc - 1;   // in-range row; its score is masked
            RowIO<T, EPL>::load(kbase + tr * a.cst, kv[u]);
            RowIO<T, EPL>::load(vbase + tr * a.cst, vv[u]);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s[kAttnBatch];
#pragma unroll
            for (int u = 0; u < kAttnBatch; ++u) {
                float dot = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; ++e) dot = fmaf(qv[g][e], kv[u][e], dot);
                s[u] = group_sum<LPR>(dot);
            }
            fold(g, s, ok, kv, vv, kAttnBatch);
        }
    }
    if constexpr (FROM_QKV) {
        if (holds_pos && grp == 0) {
            // this token: rope k, attend to it from registers, append (k, v)
            const T* krow = a.q + b * QKV + (a.QH + kvh) * HD;
            const T* vrow = a.q + b * QKV + (a.QH + a.KVH + kvh) * HD;
            const float* cr = a.cosv + pos * HD;
            const float* sr = a.sinv + pos * HD;
            float kn[1][EPL], vn[1][EPL];
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                kn[0][e] = rope_elem(krow, cr, sr, d0 + e, HD);
                vn[0][e] = ld(vrow + d0 + e);
            }
            // attend with k, v as stored (rounded to T), like every cached row
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                T kt, vt;
                st(&kt, kn[0][e]);
                st(&vt, vn[0][e]);
                kn[0][e] = ld(&kt);
                vn[0][e] = ld(&vt);
            }
            RowIO<T, EPL>::store(a.kc + b * a.csb + pos * a.cst + kvh * a.csh + d0, kn[0]);
            RowIO<T, EPL>::store(a.vc + b * a.csb + pos * a.cst + kvh * a.csh + d0, vn[0]);
            const bool one = true;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float dot = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; ++e) dot = fmaf(qv[g][e], kn[0][e], dot);
                const float s1 = group_sum<LPR>(dot);
                fold(g, &s1, &one, kn, vn, 1);
            }
        }
    }
    // merge the row groups of each wave (lanes j, j+LPR, ...), head by head
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float M = m[g];
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        const float f = (M == -INFINITY || m[g] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m[g] - M);
        float L = l[g] * f;
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) L += __shfl_xor(L, off, 64);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float c = ac[g][e] * f, k = ak[g][e] * f;
#pragma unroll
            for (int off = LPR; off < 64; off <<= 1) {
                c += __shfl_xor(c, off, 64);
                k += __shfl_xor(k, off, 64);
            }
            ac[g][e] = c;
            ak[g][e] = k;
        }
        m[g] = M;
        l[g] = L;
    }
    if (lane < LPR) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (lane == 0) {
                wred[wave][g] = m[g];
                wred[wave][G + g] = l[g];
            }
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                wred[wave][2 * G + g * HD + d0 + e] = ac[g][e];
                wred[wave][2 * G + G * HD + g * HD + d0 + e] = ak[g][e];
            }
        }
    }
    __syncthreads();
    gqa_record<T, G, HD>(a, wred, b, kvh, chunk, nchunks);
}

// ------------------------------------------------------------------ GQA attention on MFMA (bf16)
// Same contract, chunking and merge as gqa_decode_kernel, with the three
// products on v_mfma_f32_16x16x32_bf16 (A: 16 rows x 32 k, B: 32 k x 16
// columns; lane l holds row/column l%16, k = 8*(l/16)..+7; result element
// [4*(l/16)+r][l%16] in register r):
//   S^T = K Q^T    A = 16 cached K rows (16-byte loads straight from the cache),
//                  B = the G query heads (columns >= G are zero);
//   C   = P V      A = P (rows = heads, k = 32 positions, bf16 like the
//   Kctx= P K      reference's softmax output), B = V / K transposed through LDS.
// Each wave takes 32 positions at a time; the online softmax runs in the
// lanes holding S (lane l: head l%16), P and the rescale factors go to the
// accumulator lanes through LDS.  Scores are in log2 units.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMfTile = 32;   // positions per wave step

__device__ __forceinline__ f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Eight consecutive elements d0..d0+7 of a head, roped for one position
// (d0 a multiple of 8 and HD/2 a multiple of 8: the group never straddles
// the rotate-half boundary): 16-byte loads of x and its partner half.
__device__ __forceinline__ void rope8(const bf16_t* head, const float* cr, const float* sr, int d0,
                                      int HD, float out[8]) {
    const int half = HD / 2;
    float x[8], y[8], c[8], sn[8];
    Vec8<bf16_t>::load(head + d0, x);
    Vec8<bf16_t>::load(head + (d0 < half ? d0 + half : d0 - half), y);
    Vec8<float>::load(cr + d0, c);
    Vec8<float>::load(sr + d0, sn);
    const float sg = d0 < half ? -1.0f : 1.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = fmaf(x[e], c[e], sg * y[e] * sn[e]);
}

// Cache policy of the K / V stream loads (2: nontemporal; 0: default).
constexpr int kKvLoadPolicy = 2;

__device__ __forceinline__ f32x4_t mfma16(gqa_u4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Each wave takes 32 positions at a time.  Their K and V rows are loaded as
// whole 16-byte pieces in cache order (piece j of the tile: row j / (HD/8),
// piece j % (HD/8): 1 KB contiguous per load instruction when the position
// stride is HD), stored to the wave's LDS tiles row-major, and read back as
//   S^T = K Q^T      A = 16 K rows (16-byte reads), B = the G query heads;
//   C = P V, Kctx = P K   A = P straight from the score registers,
//                    B = 8 positions of one dimension per lane through the
//                    gfx950 transposing LDS read (ds_read_b64_tr_b16), in the
//                    score registers' position order (tile_tr_frag).
// The next tile's loads are in flight while a tile is computed; the waves
// never wait for each other inside the loop.
// 2 waves per SIMD (<= 256 VGPRs; the chunking makes about 1.5 blocks per CU):
// all chunk blocks of a decode step resident in one round
template <int HD, int G, bool FROM_QKV>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
gqa_mfma_kernel(GqaArgs<bf16_t> a) {
    constexpr int KK = HD / 32;            // 32-wide k-steps of a head
    constexpr int DT = HD / 16;            // 16-wide output tiles of a head
    constexpr int CPR = HD / 8;            // 16-byte pieces per row
    constexpr int NI = kMfTile * CPR / 64; // load instructions per tile (K or V)
    constexpr int REC = 2 * G + 2 * G * HD;
    struct Tiles {
        gqa_u4 k[kMfTile * CPR];           // K tile, row-major (swizzled pieces)
        gqa_u4 v[kMfTile * CPR];
    };
    constexpr int kTileBytes = 4 * (int)sizeof(Tiles);
    constexpr int kRedBytes = 4 * REC * (int)sizeof(float);
    __shared__ __align__(16) unsigned char lds[kTileBytes > kRedBytes ? kTileBytes : kRedBytes];
    const int chunk = blockIdx.x, kvh = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int nchunks = a.nchunks;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lq = lane >> 4;
    if (chunk == nchunks) {
        // the depth read of this step: rows (b, heads kvh*G ..), 16 lanes each
        if (tid < 16 * G) {
            const int row = (int)b * a.QH + kvh * G + (tid >> 4);
            if (a.dq2 != nullptr)
                depth_row_pair<bf16_t, HD / 16>(a.dq, a.dq2, a.dk, a.dv, a.dsbt, a.dss, a.dout,
                                                a.dpd, a.dpl, row, tid & 15, a.dS, a.QH, a.dscale);
            else
                depth_row<bf16_t, HD / 16>(a.dq, a.dk, a.dv, a.dsbt, a.dss, a.dout, nullptr, nullptr,
                                           row, tid & 15, a.dS, a.QH, a.dscale);
        }
        return;
    }
    const int64_t len = a.pos_dev != nullptr ? *a.pos_dev + 1 : a.len;
    const int64_t pos = len - 1;
    const int64_t clen = gqa_chunk_len(len, nchunks);
    const int nact = (int)((len + clen - 1) / clen);
    if (chunk >= nact) return;
    const int64_t t0 = (int64_t)chunk * clen;
    const int64_t t1 = t0 + clen < len ? t0 + clen : len;
    const int QKV = (a.QH + 2 * a.KVH) * HD;
    Tiles& tl = reinterpret_cast<Tiles*>(lds)[wave];
    const TileLane<CPR> tln(lq, lr);
    const int span = (int)(t1 - t0);         // positions of this chunk (< 2^31)

    const bf16_t* kb = a.kc + b * a.csb + kvh * a.csh;
    const bf16_t* vb = a.vc + b * a.csb + kvh * a.csh;
    const int nstep = (int)((t1 - t0 + 4 * kMfTile - 1) / (4 * kMfTile));
    // piece j = i*64 + lane of the tile at ts: row j / CPR (clamped in range,
    // masked below), piece j % CPR; the next tile's pieces are requested as
    // soon as this tile's are in LDS
    gqa_u4 kr[NI], vr[NI];
    // raw buffer views of this (b, kv head)'s rows < t1 (byte offsets fit 31 bits:
    // checked by the host)
    const int kv_bytes = (int)(t1 * a.cst * 2);
    const auto rk = __builtin_amdgcn_make_buffer_rsrc((void*)kb, (short)0, kv_bytes, kBufferDword3);
    const auto rv = __builtin_amdgcn_make_buffer_rsrc((void*)vb, (short)0, kv_bytes, kBufferDword3);
    auto load_kv = [&](int64_t ts) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int j = i * 64 + lane, row = j / CPR, c = j - row * CPR;
            int64_t t = ts + row;
            t = t < t1 ? t : t1 - 1;
            const int off = (int)(t * a.cst * 2) + 16 * c;
            kr[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, kKvLoadPolicy);
            vr[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, kKvLoadPolicy);
        }
    };
    // the first tile is requested before anything else of the block
    load_kv(t0 + wave * kMfTile);

    // FROM_QKV: the block holding pos appends this token's (k_roped, v) to the
    // caches and stages it in LDS; its attention takes that row from the
    // staged copy (store_kv below), so nothing in this launch depends on the
    // appended cache row
    const bf16_t* krow_new = a.q + b * QKV + (a.QH + kvh) * HD;
    const bf16_t* vrow_new = krow_new + a.KVH * HD;
    __shared__ uint4 knew[HD / 8], vnew[HD / 8];   // this token's (k_roped, v) as bf16
    if constexpr (FROM_QKV) {
        if (t1 == len && tid < HD / 8) {
            float x[8];
            rope8(krow_new, a.cosv + pos * HD, a.sinv + pos * HD, 8 * tid, HD, x);
            const uint4 kw = make_uint4(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]),
                                        pack_bf16x2(x[4], x[5]), pack_bf16x2(x[6], x[7]));
            const uint4 vw = *reinterpret_cast<const uint4*>(vrow_new + 8 * tid);
            *reinterpret_cast<uint4*>(a.kc + b * a.csb + pos * a.cst + kvh * a.csh + 8 * tid) = kw;
            *reinterpret_cast<uint4*>(a.vc + b * a.csb + pos * a.cst + kvh * a.csh + 8 * tid) = vw;
            knew[tid] = kw;
            vnew[tid] = vw;
        }
    }
    const gqa_u4* kn_lds = reinterpret_cast<const gqa_u4*>(knew);
    const gqa_u4* vn_lds = reinterpret_cast<const gqa_u4*>(vnew);
    // this wave's tile at ts into its LDS tiles; FROM_QKV: the row of this
    // token from the staged copy (the loaded value may predate the append)
    auto store_kv = [&](int64_t ts) {
        if constexpr (FROM_QKV) {
            if (pos >= ts && pos < ts + kMfTile) {   // wave-uniform: the tile holds the token
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    const int j = i * 64 + lane, row = j / CPR, c = j - row * CPR;
                    if (ts + row == pos) {
                        kr[i] = kn_lds[c];
                        vr[i] = vn_lds[c];
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int j = i * 64 + lane, row = j / CPR, c = j - row * CPR;
            const int slot = row * CPR + (c ^ kv_swz(row));
            tl.k[slot] = kr[i];
            tl.v[slot] = vr[i];
        }
    };
    // B operand of S^T: q of head lr, dims 32*kk + 8*lq .. +7, rounded to bf16
    uint4 qf[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = 0.0f;
        if (lr < G) {
            const int d0 = 32 * kk + 8 * lq;
            if constexpr (FROM_QKV) {
                rope8(a.q + b * QKV + (kvh * G + lr) * HD, a.cosv + pos * HD, a.sinv + pos * HD, d0,
                      HD, x);
                if (a.q_out != nullptr && chunk == 0 && wave == 0)
                    Vec8<bf16_t>::store(a.q_out + (b * a.QH + kvh * G + lr) * HD + d0, x);
            } else {
                Vec8<bf16_t>::load(a.q + (b * a.QH + kvh * G + lr) * HD + d0, x);
            }
        }
        qf[kk] = make_uint4(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]),
                            pack_bf16x2(x[4], x[5]), pack_bf16x2(x[6], x[7]));
    }
    float mh = -INFINITY, lh = 0.0f;       // running max / sum of head lr (lanes l%16 == head)
    f32x4_t accC[DT], accK[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) accC[dt] = accK[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (FROM_QKV) lds_barrier();   // the staged row is visible to every wave

    // every wave runs the same number of steps; a step past t1 is fully masked
    for (int it = 0; it < nstep; ++it) {
        const int64_t ts = t0 + wave * kMfTile + (int64_t)it * 4 * kMfTile;
        wave_lds_fence();                  // the previous tile's reads came first
        store_kv(ts);
        if (it + 1 < nstep) load_kv(ts + 4 * kMfTile);
        wave_lds_fence();
        // S^T[position 16*hf + 4*lq + r][head lr]
        f32x4_t sc[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            sc[hf] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; ++kk)
                sc[hf] = mfma16(tile_s_frag<CPR>(tl.k, tln, hf, kk), qf[kk], sc[hf]);
        }
        float mx = -INFINITY;
        float sv[2][4];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool ok = (int)(ts - t0) + 16 * hf + 4 * lq + r < span;
                sv[hf][r] = ok ? sc[hf][r] * a.qscale : -INFINITY;
                mx = fmaxf(mx, sv[hf][r]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(mh, mx);
        // nothing seen yet (mnew = -inf): keep the zero state; otherwise 0 on the first step
        const float corr = mnew == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(mh - mnew);
        float ls = 0.0f, pv[2][4];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pv[hf][r] = sv[hf][r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sv[hf][r] - mnew);
                ls += pv[hf][r];
            }
        ls += __shfl_xor(ls, 16, 64);
        ls += __shfl_xor(ls, 32, 64);
        lh = fmaf(lh, corr, ls);
        mh = mnew;
        // A operand of P V / P K straight from the score registers: head lr,
        // positions 4*lq + r and 16 + 4*lq + r (bf16 like the reference's
        // softmax output), matched by tile_tr_frag
        const uint4 pa = make_uint4(pack_bf16x2(pv[0][0], pv[0][1]), pack_bf16x2(pv[0][2], pv[0][3]),
                                    pack_bf16x2(pv[1][0], pv[1][1]), pack_bf16x2(pv[1][2], pv[1][3]));
        // rescale the accumulators (rows = heads 4*lq + r: their factors from
        // the lanes of those heads) and add P V, P K
        // (skipped when no head's max moved: every factor exactly 1)
        if (__any(corr != 1.0f)) {
            float cf[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) cf[r] = __shfl(corr, 4 * lq + r, 64);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    accC[dt][r] *= cf[r];
                    accK[dt][r] *= cf[r];
                }
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            accC[dt] = mfma16(pa, tile_tr_frag<CPR>(tl.v, tln, dt), accC[dt]);
            accK[dt] = mfma16(pa, tile_tr_frag<CPR>(tl.k, tln, dt), accK[dt]);
        }
    }
    __syncthreads();                       // every wave is done with its tiles (wred aliases them)
    // this wave's partials -> wred[wave] = [m | l | c | k] (unnormalised)
    float (*wred)[REC] = reinterpret_cast<float (*)[REC]>(lds);
    if (lq == 0 && lr < G) {
        wred[wave][lr] = mh;
        wred[wave][G + lr] = lh;
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int g = 4 * lq + r;
            if (g < G) {
                wred[wave][2 * G + g * HD + 16 * dt + lr] = accC[dt][r];
                wred[wave][2 * G + G * HD + g * HD + 16 * dt + lr] = accK[dt][r];
            }
        }
    __syncthreads();
    gqa_record<bf16_t, G, HD>(a, wred, b, kvh, chunk, nchunks);
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

// out = round(round(x / sqrt(mean(x^2) + eps)) * w) over rows of N, the
// RMSNorm of final_norm (loomformer.py:3460-3464: fp32 statistics, the
// normalised row rounded to the storage type, then the learned scale in it);
// one wavefront per row.
template <typename T>
__global__ void __launch_bounds__(256)
rms_norm_kernel(const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ out,
                int64_t rows, int N, float eps) {
    const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    constexpr int kMax = 32;  // N <= 64 * 32
    float v[kMax];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kMax; ++k) {
        const int c = lane + 64 * k;
        v[k] = c < N ? ld(x + row * N + c) : 0.0f;
        ss = fmaf(v[k], v[k], ss);
    }
    const float r = 1.0f / sqrtf(wave_sum(ss) / N + eps);
#pragma unroll
    for (int k = 0; k < kMax; ++k) {
        const int c = lane + 64 * k;
        if (c < N) {
            T nrm;
            st(&nrm, v[k] * r);
            st(out + row * N + c, ld(&nrm) * ld(w + c));
        }
    }
}

// Vector form for N % 8 == 0 (N <= 64*8*4): lane owns 8-element vectors
// lane, lane+64, ...; two wave reductions (mean, variance).
template <typename T, int NV>
__global__ void __launch_bounds__(256)
add_layernorm_vec_kernel(const T* __restrict__ a, const T* __restrict__ bsrc,
                         const float* __restrict__ gamma, const float* __restrict__ beta,
                         T* __restrict__ out, int64_t rows, int N, float eps) {
    const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int nvec = N >> 3;
    float x[NV][8];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int v = lane + 64 * k;
        if (v < nvec) {
            Vec8<T>::load(a + row * N + v * 8, x[k]);
            if (bsrc != nullptr) {
                float y[8];
                Vec8<T>::load(bsrc + row * N + v * 8, y);
#pragma unroll
                for (int e = 0; e < 8; ++e) x[k][e] += y[e];
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) s += x[k][e];
        }
    }
    const float mean = wave_sum(s) / N;
    float var = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k)
        if (lane + 64 * k < nvec) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float d = x[k][e] - mean;
                var = fmaf(d, d, var);
            }
        }
    const float rstd = 1.0f / sqrtf(wave_sum(var) / N + eps);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int v = lane + 64 * k;
        if (v < nvec) {
            float o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                o[e] = (x[k][e] - mean) * rstd * gamma[v * 8 + e] + beta[v * 8 + e];
            Vec8<T>::store(out + row * N + v * 8, o);
        }
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

// One (b, h) stream of the decode temporal step (loomformer.py:4053-4085):
// M = D unless the stream continues, then M = N(D . P) (N: rms normalisation
// with eps 1e-6 inside the root); on a fire, PolARM: G = M^T M,
// s = max(tr(G)/3, eps), M <- M (I - beta/2 (G/s - I)) (tria.py:128-139).
__device__ __forceinline__ void temporal_head(float M[9], const float P[9], bool cont, bool fires,
                                              float beta, float eps) {
    if (cont) {
        float R[9];
        mm3d(M, P, R);
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < 9; ++k) s = fmaf(R[k], R[k], s);
        const float inv = 1.0f / sqrtf(s * (1.0f / 9.0f) + 1e-6f);
#pragma unroll
        for (int k = 0; k < 9; ++k) M[k] = R[k] * inv;
    }
    if (fires) {
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
}

template <typename T>
__global__ void __launch_bounds__(256)
decode_temporal_kernel(const T* __restrict__ depth, const T* __restrict__ prev,
                       const uint8_t* __restrict__ reset_now, const uint8_t* __restrict__ fire,
                       T* __restrict__ out, int64_t B, int64_t H, float beta, float eps) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= B * H) return;
    const int64_t b = e / H;
    float M[9], P[9];
    const bool cont = prev != nullptr && reset_now[b] == 0;
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        M[k] = ld(depth + e * 9 + k);
        P[k] = cont ? ld(prev + e * 9 + k) : 0.0f;
    }
    temporal_head(M, P, cont, fire != nullptr && fire[b] != 0, beta, eps);
#pragma unroll
    for (int k = 0; k < 9; ++k) st(out + e * 9 + k, M[k]);
}

// The per-token Tria tail of a decode step, in two launches spread over the
// chip (one CU streams its share far slower than the whole device, so a
// launch with one block per batch row would be bound by 32 CUs):
//   decode_readout_heads_kernel, grid (H / kReadHeads, B), one thread per head:
//     the temporal step and PolARM (temporal_head), stored as the new document
//     state doc[b, h] (in place: each thread reads its head's previous state
//     before it writes it); then this block's part of the slot attention pool
//     over h (tria.py:1351-1389), an online-softmax record (m, l, sum p vec C)
//     of <score_w, vec C_h> over the stored (rounded) state, natural exponentials;
//   decode_readout_rows_kernel, grid (N / kReadCols, B): merges row b's
//     records into pooled, then proj Linear(9, 32) and kReadCols outputs of up
//     Linear(32, N) (tria.py:1436-1441).
// The readout feeds only the final-CA keys staged at a fire (tria.py:1576-1582),
// so with fire flags given and none set both launches stop after the state
// update and a_out is left as it is.
// pooled and z are rounded to T before use, as the unfused ops store them.
constexpr int kReadHeads = 256;
constexpr int kReadCols = 128;
constexpr int kReadRec = 11;           // m, l, acc[9]

template <typename T>
__global__ void __launch_bounds__(kReadHeads)
decode_readout_heads_kernel(const T* __restrict__ depth, const T* prev,
                            const uint8_t* __restrict__ reset_now, const uint8_t* __restrict__ fire,
                            T* doc, const T* __restrict__ score_w, float* __restrict__ rec, int H,
                            float beta, float eps) {
    __shared__ float red[kReadHeads / 64][kReadRec];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int64_t b = blockIdx.y;
    const int h = blockIdx.x * kReadHeads + tid;
    const bool cont = prev != nullptr && reset_now[b] == 0;
    const bool fires = fire != nullptr && fire[b] != 0;
    // every load unconditional (a lane past H reads head H-1, then drops it),
    // so all of them are in flight at once instead of one round trip each
    const int64_t e = (b * H + (h < H ? h : H - 1)) * 9;
    const T* pp = prev != nullptr ? prev : depth;
    float M[9], P[9], sw[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        M[k] = ld(depth + e + k);
        P[k] = ld(pp + e + k);
        sw[k] = ld(score_w + k);
    }
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        M[k] = h < H ? M[k] : 0.0f;
        P[k] = (cont && h < H) ? P[k] : 0.0f;
    }
    float m = -INFINITY, l = 0.0f, acc[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) acc[k] = 0.0f;
    if (h < H) {
        temporal_head(M, P, cont, fires, beta, eps);
        float sc = 0.0f;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            T rounded;
            st(&rounded, M[k]);
            doc[e + k] = rounded;
            acc[k] = ld(&rounded);
            sc = fmaf(acc[k], sw[k], sc);
        }
        m = sc;
        l = 1.0f;                          // one head: p = e^(sc - m) = 1
    }
    // the readout feeds only the keys staged at a fire: without one, stop here
    // (one flag per thread, OR over the block: one memory round trip)
    if (fire != nullptr) {
        int any = 0;
        for (int q = tid; q < (int)gridDim.y; q += kReadHeads) any |= fire[q] != 0;
        if (!__syncthreads_or(any)) return;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float mo = __shfl_xor(m, off, 64);
        const float lo = __shfl_xor(l, off, 64);
        const float mn = fmaxf(m, mo);
        const float ca = (m == -INFINITY) ? 0.0f : expf(m - mn);
        const float cb = (mo == -INFINITY) ? 0.0f : expf(mo - mn);
        l = l * ca + lo * cb;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            const float ao = __shfl_xor(acc[k], off, 64);
            acc[k] = acc[k] * ca + ao * cb;
        }
        m = mn;
    }
    if (lane == 0) {
        red[wid][0] = m;
        red[wid][1] = l;
#pragma unroll
        for (int k = 0; k < 9; ++k) red[wid][2 + k] = acc[k];
    }
    __syncthreads();
    if (tid < kReadRec) {
        float Mx = -INFINITY;
#pragma unroll
        for (int q = 0; q < kReadHeads / 64; ++q) Mx = fmaxf(Mx, red[q][0]);
        float v = 0.0f;
        if (tid == 0) {
            v = Mx;
        } else {
#pragma unroll
            for (int q = 0; q < kReadHeads / 64; ++q)
                if (red[q][0] != -INFINITY) v = fmaf(red[q][tid], expf(red[q][0] - Mx), v);
        }
        rec[(b * gridDim.x + blockIdx.x) * kReadRec + tid] = v;
    }
}

template <typename T>
__global__ void __launch_bounds__(kReadCols)
decode_readout_rows_kernel(const float* __restrict__ rec, int nrec, const T* __restrict__ proj_w,
                           const float* __restrict__ proj_b, const T* __restrict__ up_w,
                           const float* __restrict__ up_b, T* __restrict__ a_out, int N,
                           const uint8_t* __restrict__ fire) {
    constexpr int kMaxRec = kReadCols;     // records per row (H <= kReadHeads * kReadCols)
    __shared__ float rs[kMaxRec * kReadRec];
    __shared__ float xs[9];
    __shared__ float zs[32];
    const int tid = threadIdx.x;
    const int64_t b = blockIdx.y;
    const int n = blockIdx.x * kReadCols + tid;
    if (fire != nullptr) {                 // no fire: no key to stage, a_out is left as it is
        int any = 0;
        for (int q = tid; q < (int)gridDim.y; q += kReadCols) any |= fire[q] != 0;
        if (!__syncthreads_or(any)) return;
    }
    // every load first, unconditionally (clamped rows, so they are all in
    // flight at once): this row's records, the proj row of thread tid < 32 and
    // the up row of column n
    const float* rb = rec + b * nrec * kReadRec;
    const int tot = nrec * kReadRec;
    const float r0 = rb[min(tid, tot - 1)], r1 = rb[min(tid + kReadCols, tot - 1)];
    const int pt = min(tid, 31), nn = min(n, N - 1);
    float pw[9], uw[32];
#pragma unroll
    for (int k = 0; k < 9; ++k) pw[k] = ld(proj_w + pt * 9 + k);
    const float pbias = proj_b != nullptr ? proj_b[pt] : 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j += 8) Vec8<T>::load(up_w + (int64_t)nn * 32 + j, uw + j);
    const float ubias = up_b != nullptr ? up_b[nn] : 0.0f;
    if (tid < tot) rs[tid] = r0;
    if (tid + kReadCols < tot) rs[tid + kReadCols] = r1;
    for (int i = tid + 2 * kReadCols; i < tot; i += kReadCols) rs[i] = rb[i];
    __syncthreads();
    if (tid < 9) {
        float Mx = -INFINITY;
        for (int r = 0; r < nrec; ++r) Mx = fmaxf(Mx, rs[r * kReadRec]);
        float L = 0.0f, A = 0.0f;
        for (int r = 0; r < nrec; ++r) {
            const float* q = rs + r * kReadRec;
            if (q[0] == -INFINITY) continue;
            const float c = expf(q[0] - Mx);
            L = fmaf(q[1], c, L);
            A = fmaf(q[2 + tid], c, A);
        }
        T pooled;
        st(&pooled, A * (1.0f / L));
        xs[tid] = ld(&pooled);
    }
    __syncthreads();
    if (tid < 32) {
        float z = pbias;
#pragma unroll
        for (int k = 0; k < 9; ++k) z = fmaf(pw[k], xs[k], z);
        T zr;
        st(&zr, z);
        zs[tid] = ld(&zr);
    }
    __syncthreads();
    if (n < N) {
        float a = ubias;
#pragma unroll
        for (int j = 0; j < 32; ++j) a = fmaf(uw[j], zs[j], a);
        st(a_out + b * N + n, a);
    }
}

// ------------------------------------------------------------------ dispatch

template <typename T>
static int rope_dispatch(const void* qkv, void* q_out, void* kc, void* vc, const float* cosv,
                         const float* sinv, int64_t B, int64_t pos, const int64_t* pos_dev,
                         int64_t QH, int64_t KVH, int64_t HD, int64_t sb, int64_t stt,
                         int64_t sh, hipStream_t st) {
    const int64_t total = B * (QH + 2 * KVH) * HD;
    hipLaunchKernelGGL((rope_append_kernel<T>), dim3((unsigned)ceil_div(total, 256)), dim3(256), 0,
                       st, (const T*)qkv, (T*)q_out, (T*)kc, (T*)vc, cosv, sinv, B, pos, pos_dev,
                       (int)QH, (int)KVH, (int)HD, sb, stt, sh);
    return launch_status("loom_rope_append");
}

// A DepthAttn read (loomformer.py:3404-3429) to run with the attention launch.
struct DepthRead {
    const void* q;         // [QH, HD]
    const void* hk;
    const void* hv;
    int64_t sbt, ss, S;
    void* out;             // [B, QH, HD]
    const void* q2;        // optional second query (bf16 MFMA form only)
    float* part_d;         // [B, QH, HD]
    float* part_lse;       // [B, QH]
};

template <typename T> constexpr int dtype_code();
template <> constexpr int dtype_code<float>() { return LOOM_F32; }
template <> constexpr int dtype_code<bf16_t>() { return LOOM_BF16; }
template <> constexpr int dtype_code<f16_t>() { return LOOM_F16; }

template <typename T>
static int gqa_dispatch(bool from_qkv, const void* q, const void* kc, const void* vc, int64_t sb,
                        int64_t stt, int64_t sh, const float* cosv, const float* sinv, void* q_out,
                        void* c_out, void* k_out,
                        int64_t out_sb, float* ws, int64_t B, int64_t len, const int64_t* pos_dev,
                        int64_t QH, int64_t KVH, int64_t HD, hipStream_t st,
                        const DepthRead* depth = nullptr) {
    const int G = (int)(QH / KVH);
    const int nchunks = gqa_nchunks(B, KVH, len);
    // the depth read rides in the attention grid when the rows can take the
    // paired 4-byte loads of depth_row (else it is its own launch, after)
    const bool fuse_depth =
        depth != nullptr && depth->sbt % 2 == 0 && depth->ss % 2 == 0 &&
        ((((uintptr_t)depth->q | (uintptr_t)depth->hk | (uintptr_t)depth->hv |
           (uintptr_t)depth->out) % 8) == 0) && B * QH * 16 < ((int64_t)1 << 31);
    auto depth_after = [&]() -> int {
        if (depth == nullptr) return LOOM_OK;
        return loom_depth_attn_forward(dtype_code<T>(), depth->q, depth->hk, depth->hv, depth->sbt,
                                       depth->ss, depth->out, nullptr, nullptr, B, depth->S, QH,
                                       HD, st);
    };
    GqaArgs<T> a{};
    // after the chunk launch: the merge of its records, then (unless folded in)
    // the depth read
    auto finish = [&](bool depth_done) -> int {
        int rc = launch_status(from_qkv ? "loom_gqa_decode_step" : "loom_gqa_decode_attention");
        if (rc != LOOM_OK) return rc;
        hipLaunchKernelGGL((gqa_merge_kernel<T>), dim3((unsigned)ceil_div(B * QH * HD, 256)), dim3(256),
                           0, st, a.rec, nchunks, len, pos_dev, (T*)c_out, (T*)k_out, out_sb, (int)B,
                           (int)QH, (int)KVH, (int)HD);
        rc = launch_status(from_qkv ? "loom_gqa_decode_step(merge)" : "loom_gqa_decode_attention(merge)");
        return (rc != LOOM_OK || depth_done) ? rc : depth_after();
    };
    a.q = (const T*)q;
    a.kc = (T*)kc;
    a.vc = (T*)vc;
    a.csb = sb;
    a.cst = stt;
    a.csh = sh;
    a.cosv = cosv;
    a.sinv = sinv;
    a.q_out = (T*)q_out;
    a.rec = ws;
    a.c_out = (T*)c_out;
    a.k_out = (T*)k_out;
    a.out_sb = out_sb;
    a.len = len;
    a.pos_dev = pos_dev;
    a.QH = (int)QH;
    a.KVH = (int)KVH;
    a.qscale = kLog2e / sqrtf((float)HD);   // scores in log2 units
    a.nchunks = nchunks;
    dim3 grid(nchunks, (unsigned)KVH, (unsigned)B);
    if constexpr (std::is_same<T, bf16_t>::value) {
        // bf16: the MFMA form for head_dim 32/64/96/128 and groups 1/2/4/8
        dim3 mgrid = grid;
        if (fuse_depth) {
            a.dq = (const T*)depth->q;
            a.dk = (const T*)depth->hk;
            a.dv = (const T*)depth->hv;
            a.dsbt = depth->sbt;
            a.dss = depth->ss;
            a.dout = (T*)depth->out;
            a.dS = (int)depth->S;
            a.dscale = 1.0f / sqrtf((float)HD);
            a.dq2 = (const T*)depth->q2;
            a.dpd = depth->part_d;
            a.dpl = depth->part_lse;
            mgrid.x += 1;
        }
#define LOOM_GQA_MF(HDV, GG)                                                                      \
        if (HD == HDV && G == GG) {                                                              \
            if (from_qkv)                                                                         \
                hipLaunchKernelGGL((gqa_mfma_kernel<HDV, GG, true>), mgrid, dim3(256), 0, st, a); \
            else                                                                                  \
                hipLaunchKernelGGL((gqa_mfma_kernel<HDV, GG, false>), mgrid, dim3(256), 0, st, a); \
            return finish(fuse_depth);                                                            \
        }
        LOOM_GQA_MF(96, 4) LOOM_GQA_MF(96, 1) LOOM_GQA_MF(96, 2) LOOM_GQA_MF(96, 8)
        LOOM_GQA_MF(64, 4) LOOM_GQA_MF(64, 1) LOOM_GQA_MF(64, 2) LOOM_GQA_MF(64, 8)
        LOOM_GQA_MF(128, 4) LOOM_GQA_MF(128, 1) LOOM_GQA_MF(128, 2) LOOM_GQA_MF(128, 8)
        LOOM_GQA_MF(32, 4) LOOM_GQA_MF(32, 1) LOOM_GQA_MF(32, 2) LOOM_GQA_MF(32, 8)
#undef LOOM_GQA_MF
    }
#define LOOM_GQA(E, GG, LPR)                                                                    \
    if (HD == E * LPR && G == GG) {                                                             \
        if (from_qkv)                                                                           \
            hipLaunchKernelGGL((gqa_decode_kernel<T, E, GG, LPR, true>), grid, dim3(256), 0, st, a); \
        else                                                                                    \
            hipLaunchKernelGGL((gqa_decode_kernel<T, E, GG, LPR, false>), grid, dim3(256), 0, st, a); \
        return finish(false);                                                                   \
    }
    // head_dim 32/64/96/128 (16 lanes per row) and 8 (8 lanes), groups 1/2/4/8
    LOOM_GQA(6, 4, 16) LOOM_GQA(6, 1, 16) LOOM_GQA(6, 2, 16) LOOM_GQA(6, 8, 16)
    LOOM_GQA(4, 4, 16) LOOM_GQA(4, 1, 16) LOOM_GQA(4, 2, 16) LOOM_GQA(4, 8, 16)
    LOOM_GQA(8, 4, 16) LOOM_GQA(8, 1, 16) LOOM_GQA(8, 2, 16) LOOM_GQA(8, 8, 16)
    LOOM_GQA(2, 4, 16) LOOM_GQA(2, 1, 16) LOOM_GQA(2, 2, 16) LOOM_GQA(2, 8, 16)
    LOOM_GQA(1, 1, 8) LOOM_GQA(1, 2, 8) LOOM_GQA(1, 4, 8) LOOM_GQA(1, 8, 8)
#undef LOOM_GQA
    set_error("gqa_decode_attention: unsupported head_dim %lld / group %d", (long long)HD, G);
    return LOOM_ERR_INVALID;
}

template <typename T>
static int ln_dispatch(const void* a, const void* b, const float* g, const float* be, void* out,
                       int64_t rows, int64_t N, float eps, hipStream_t st) {
    const bool vec = N % 8 == 0 && N <= 64 * 8 * 4 &&
                     (((uintptr_t)a | (uintptr_t)b | (uintptr_t)out) & 15) == 0;
    if (vec) {
        const dim3 grid((unsigned)ceil_div(rows * 64, 256));
        const int nv = (int)ceil_div(N / 8, 64);
        if (nv <= 2)
            hipLaunchKernelGGL((add_layernorm_vec_kernel<T, 2>), grid, dim3(256), 0, st,
                               (const T*)a, (const T*)b, g, be, (T*)out, rows, (int)N, eps);
        else
            hipLaunchKernelGGL((add_layernorm_vec_kernel<T, 4>), grid, dim3(256), 0, st,
                               (const T*)a, (const T*)b, g, be, (T*)out, rows, (int)N, eps);
        return launch_status("loom_add_layernorm");
    }
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

template <typename T>
static int readout_dispatch(const void* depth, const void* prev, const uint8_t* reset_now,
                            const uint8_t* fire, void* doc, const void* score_w, const void* proj_w,
                            const float* proj_b, const void* up_w, const float* up_b, void* a_out,
                            float* ws, int64_t B, int64_t H, int64_t N, float beta, float eps,
                            hipStream_t st) {
    const int nrec = (int)ceil_div(H, kReadHeads);
    hipLaunchKernelGGL((decode_readout_heads_kernel<T>), dim3((unsigned)nrec, (unsigned)B),
                       dim3(kReadHeads), 0, st, (const T*)depth, (const T*)prev, reset_now, fire,
                       (T*)doc, (const T*)score_w, ws, (int)H, beta, eps);
    int rc = launch_status("loom_decode_tria_readout");
    if (rc != LOOM_OK) return rc;
    hipLaunchKernelGGL((decode_readout_rows_kernel<T>), dim3((unsigned)ceil_div(N, kReadCols), (unsigned)B),
                       dim3(kReadCols), 0, st, ws, nrec, (const T*)proj_w, proj_b, (const T*)up_w,
                       up_b, (T*)a_out, (int)N, fire);
    return launch_status("loom_decode_tria_readout");
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
    const int64_t nchunks = gqa_nchunks(B, KVH, max_len);
    return B * KVH * nchunks * (2 * G + 2 * G * HD) * (int64_t)sizeof(float);
}

extern "C" int loom_rope_append(int dtype, const void* qkv, void* q_out, void* k_cache,
                                void* v_cache, const float* cos_table, const float* sin_table,
                                int64_t B, int64_t pos, const int64_t* pos_dev, int64_t QH,
                                int64_t KVH, int64_t HD, int64_t cache_stride_b,
                                int64_t cache_stride_t, int64_t cache_stride_h, void* stream) {
    clear_error();
    LOOM_CHECK(qkv && q_out && k_cache && v_cache && cos_table && sin_table,
               "rope_append: null argument");
    LOOM_CHECK(HD % 2 == 0 && QH > 0 && KVH > 0 && pos >= 0, "rope_append: bad shape");
    LOOM_CHECK(cache_stride_t >= HD && cache_stride_h >= HD,
               "rope_append: cache strides smaller than a head row");
    if (B == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, rope_dispatch, qkv, q_out, k_cache, v_cache, cos_table, sin_table, B,
                      pos, pos_dev, QH, KVH, HD, cache_stride_b, cache_stride_t, cache_stride_h,
                      (hipStream_t)stream)
}

static int gqa_checks(const char* who, const void* k_cache, const void* v_cache,
                      int64_t cache_stride_b, int64_t cache_stride_t, int64_t cache_stride_h,
                      const void* workspace,
                      int64_t workspace_bytes, int64_t B, int64_t len, int64_t QH, int64_t KVH,
                      int64_t HD) {
    LOOM_CHECK(len >= 1 && KVH >= 1 && QH % KVH == 0 && QH / KVH <= kAttnMaxG,
               "%s: bad shape len=%lld QH=%lld KVH=%lld", who, (long long)len, (long long)QH,
               (long long)KVH);
    LOOM_CHECK(workspace_bytes >= loom_gqa_workspace_bytes(B, len, QH, KVH, HD),
               "%s: workspace too small (%lld bytes)", who, (long long)workspace_bytes);
    LOOM_CHECK(((uintptr_t)workspace & 255) == 0, "%s: workspace must be 256-byte aligned", who);
    // cache rows are read as 4-/8-byte words when each lane owns an even count
    // (the bf16 MFMA form reads 16-byte pieces: 16-byte aligned, strides multiples of 8)
    LOOM_CHECK(HD % 32 != 0 || ((((uintptr_t)k_cache | (uintptr_t)v_cache) & 15) == 0 &&
                                cache_stride_b % 8 == 0 && cache_stride_t % 8 == 0 &&
                                cache_stride_h % 8 == 0),
               "%s: caches must be 16-byte aligned with strides divisible by 8", who);
    LOOM_CHECK(cache_stride_t >= HD && cache_stride_h >= HD,
               "%s: cache strides smaller than a head row", who);
    // the MFMA form addresses the rows of one (b, kv head) with 31-bit byte offsets
    LOOM_CHECK(len * cache_stride_t * 2 < (1LL << 31),
               "%s: %lld positions at stride %lld exceed the 2 GiB per-head row span", who,
               (long long)len, (long long)cache_stride_t);
    return LOOM_OK;
}

extern "C" int loom_gqa_decode_attention(int dtype, const void* q, const void* k_cache,
                                         const void* v_cache, int64_t cache_stride_b,
                                         int64_t cache_stride_t, int64_t cache_stride_h,
                                         void* c_out, void* kctx_out,
                                         float* workspace, int64_t workspace_bytes, int64_t B,
                                         int64_t len, const int64_t* pos_dev, int64_t QH,
                                         int64_t KVH, int64_t HD, void* stream) {
    clear_error();
    LOOM_CHECK(q && k_cache && v_cache && c_out && kctx_out && workspace,
               "gqa_decode_attention: null argument");
    const int rc = gqa_checks("gqa_decode_attention", k_cache, v_cache, cache_stride_b,
                              cache_stride_t, cache_stride_h, workspace, workspace_bytes, B, len,
                              QH, KVH, HD);
    if (rc != LOOM_OK) return rc;
    if (B == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, gqa_dispatch, false, q, k_cache, v_cache, cache_stride_b,
                      cache_stride_t, cache_stride_h, nullptr, nullptr, nullptr, c_out, kctx_out,
                      QH * HD, workspace, B,
                      len, pos_dev, QH, KVH, HD, (hipStream_t)stream)
}

extern "C" int loom_gqa_decode_step(int dtype, const void* qkv, void* k_cache, void* v_cache,
                                    int64_t cache_stride_b, int64_t cache_stride_t,
                                    int64_t cache_stride_h, const float* cos_table,
                                    const float* sin_table, void* q_out,
                                    void* c_out, void* kctx_out, int64_t out_stride_b, float* workspace,
                                    int64_t workspace_bytes, int64_t B, int64_t len,
                                    const int64_t* pos_dev, int64_t QH, int64_t KVH, int64_t HD,
                                    void* stream) {
    clear_error();
    LOOM_CHECK(qkv && k_cache && v_cache && cos_table && sin_table && c_out && kctx_out &&
                   workspace,
               "gqa_decode_step: null argument");
    LOOM_CHECK(HD % 2 == 0 && out_stride_b >= QH * HD, "gqa_decode_step: bad head_dim / out stride");
    const int rc = gqa_checks("gqa_decode_step", k_cache, v_cache, cache_stride_b, cache_stride_t,
                              cache_stride_h, workspace, workspace_bytes, B, len, QH, KVH, HD);
    if (rc != LOOM_OK) return rc;
    if (B == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, gqa_dispatch, true, qkv, k_cache, v_cache, cache_stride_b,
                      cache_stride_t, cache_stride_h, cos_table, sin_table, q_out, c_out, kctx_out,
                      out_stride_b,
                      workspace, B, len, pos_dev, QH, KVH, HD, (hipStream_t)stream)
}

extern "C" int loom_gqa_decode_step_depth(int dtype, const void* qkv, void* k_cache, void* v_cache,
                                          int64_t cache_stride_b, int64_t cache_stride_t,
                                          int64_t cache_stride_h, const float* cos_table,
                                          const float* sin_table, void* q_out, void* c_out,
                                          void* kctx_out, int64_t out_stride_b, float* workspace,
                                          int64_t workspace_bytes, int64_t B, int64_t len,
                                          const int64_t* pos_dev, int64_t QH, int64_t KVH,
                                          int64_t HD, const void* depth_q, const void* hist_k,
                                          const void* hist_v, int64_t hist_stride_bt,
                                          int64_t hist_stride_s, int64_t S, void* depth_out,
                                          void* stream) {
    clear_error();
    LOOM_CHECK(qkv && k_cache && v_cache && cos_table && sin_table && c_out && kctx_out &&
                   workspace && depth_q && hist_k && hist_v && depth_out,
               "gqa_decode_step_depth: null argument");
    LOOM_CHECK(HD % 2 == 0 && out_stride_b >= QH * HD,
               "gqa_decode_step_depth: bad head_dim / out stride");
    LOOM_CHECK(S >= 1 && hist_stride_s >= QH * HD && hist_stride_bt >= S * hist_stride_s,
               "gqa_decode_step_depth: history strides (bt=%lld, s=%lld) overlap the [S,QH,HD] block",
               (long long)hist_stride_bt, (long long)hist_stride_s);
    const int rc = gqa_checks("gqa_decode_step_depth", k_cache, v_cache, cache_stride_b,
                              cache_stride_t, cache_stride_h, workspace, workspace_bytes, B, len,
                              QH, KVH, HD);
    if (rc != LOOM_OK) return rc;
    if (B == 0) return LOOM_OK;
    const DepthRead dr{depth_q, hist_k, hist_v, hist_stride_bt, hist_stride_s, S, depth_out,
                       nullptr, nullptr, nullptr};
    LOOM_DTYPE_SWITCH(dtype, gqa_dispatch, true, qkv, k_cache, v_cache, cache_stride_b,
                      cache_stride_t, cache_stride_h, cos_table, sin_table, q_out, c_out, kctx_out,
                      out_stride_b, workspace, B, len, pos_dev, QH, KVH, HD, (hipStream_t)stream,
                      &dr)
}

extern "C" int loom_gqa_decode_step_depth2(int dtype, const void* qkv, void* k_cache, void* v_cache,
                                           int64_t cache_stride_b, int64_t cache_stride_t,
                                           int64_t cache_stride_h, const float* cos_table,
                                           const float* sin_table, void* q_out, void* c_out,
                                           void* kctx_out, int64_t out_stride_b, float* workspace,
                                           int64_t workspace_bytes, int64_t B, int64_t len,
                                           const int64_t* pos_dev, int64_t QH, int64_t KVH,
                                           int64_t HD, const void* depth_q, const void* depth_q2,
                                           const void* hist_k, const void* hist_v,
                                           int64_t hist_stride_bt, int64_t hist_stride_s, int64_t S,
                                           void* depth_out, float* part_d, float* part_lse,
                                           void* stream) {
    clear_error();
    LOOM_CHECK(qkv && k_cache && v_cache && cos_table && sin_table && c_out && kctx_out &&
                   workspace && depth_q && depth_q2 && hist_k && hist_v && depth_out && part_d &&
                   part_lse,
               "gqa_decode_step_depth2: null argument");
    LOOM_CHECK(out_stride_b >= QH * HD, "gqa_decode_step_depth2: bad out stride");
    LOOM_CHECK(S >= 1 && hist_stride_s >= QH * HD && hist_stride_bt >= S * hist_stride_s,
               "gqa_decode_step_depth2: history strides (bt=%lld, s=%lld) overlap the [S,QH,HD] block",
               (long long)hist_stride_bt, (long long)hist_stride_s);
    const int64_t G = KVH > 0 ? QH / KVH : 0;
    LOOM_CHECK(dtype == LOOM_BF16 && (HD == 32 || HD == 64 || HD == 96 || HD == 128) &&
                   (G == 1 || G == 2 || G == 4 || G == 8) && hist_stride_bt % 2 == 0 &&
                   hist_stride_s % 2 == 0 &&
                   ((((uintptr_t)depth_q | (uintptr_t)depth_q2 | (uintptr_t)hist_k |
                      (uintptr_t)hist_v | (uintptr_t)depth_out | (uintptr_t)part_d) % 8) == 0) &&
                   B * QH * 16 < ((int64_t)1 << 31),
               "gqa_decode_step_depth2: needs the bf16 MFMA form (head_dim 32/64/96/128, group "
               "1/2/4/8, 8-byte aligned depth rows)");
    const int rc = gqa_checks("gqa_decode_step_depth2", k_cache, v_cache, cache_stride_b,
                              cache_stride_t, cache_stride_h, workspace, workspace_bytes, B, len,
                              QH, KVH, HD);
    if (rc != LOOM_OK) return rc;
    if (B == 0) return LOOM_OK;
    const DepthRead dr{depth_q, hist_k, hist_v, hist_stride_bt, hist_stride_s, S, depth_out,
                       depth_q2, part_d, part_lse};
    return gqa_dispatch<bf16_t>(true, qkv, k_cache, v_cache, cache_stride_b, cache_stride_t,
                                cache_stride_h, cos_table, sin_table, q_out, c_out, kctx_out,
                                out_stride_b, workspace, B, len, pos_dev, QH, KVH, HD,
                                (hipStream_t)stream, &dr);
}

// ---------------------------------------------------------------- step control
// Device-resident step state so a whole decode step is a fixed launch sequence
// (capturable in a HIP graph): pos_dev[0] = position of this step.

__global__ void decode_prologue_kernel(int64_t* __restrict__ ids, const int64_t* __restrict__ prompt,
                                       int64_t prompt_len, int64_t prompt_ld,
                                       int64_t* __restrict__ tokens, int64_t tokens_ld,
                                       const int64_t* __restrict__ pos_dev,
                                       const uint8_t* __restrict__ pending, uint8_t* __restrict__ fire,
                                       uint8_t* __restrict__ reset_now, int64_t carry_id,
                                       int64_t window, int64_t seq_len, int64_t B) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const int64_t pos = *pos_dev;
    int64_t id = ids[b];
    if (prompt != nullptr && pos < prompt_len) {
        id = prompt[b * prompt_ld + pos];
        ids[b] = id;
    }
    if (tokens != nullptr) tokens[b * tokens_ld + pos] = id;
    // hard fire for the next token (loomformer.py:4069-4073) or an explicit <CARRY> id
    const bool hard = (pos + 1 < seq_len) && ((pos + 1) % window == 0);
    fire[b] = (hard || (carry_id >= 0 && id == carry_id)) ? 1 : 0;
    reset_now[b] = pending[b];
}

// decode_prologue_kernel for row b (one block per row) followed by the
// embedding lookup of the step's token: h[b] = emb[ids[b]] (rows of N
// elements, copied as 16-byte pieces when N * sizeof(T) % 16 == 0).
template <typename T>
__global__ void __launch_bounds__(128)
decode_prologue_embed_kernel(int64_t* __restrict__ ids, const int64_t* __restrict__ prompt,
                             int64_t prompt_len, int64_t prompt_ld, int64_t* __restrict__ tokens,
                             int64_t tokens_ld, const int64_t* __restrict__ pos_dev,
                             const uint8_t* __restrict__ pending, uint8_t* __restrict__ fire,
                             uint8_t* __restrict__ reset_now, int64_t carry_id, int64_t window,
                             int64_t seq_len, const T* __restrict__ emb, T* __restrict__ h,
                             int64_t N, int64_t V) {
    __shared__ int64_t s_id;
    const int64_t b = blockIdx.x;
    if (threadIdx.x == 0) {
        const int64_t pos = *pos_dev;
        int64_t id = ids[b];
        if (prompt != nullptr && pos < prompt_len) {
            id = prompt[b * prompt_ld + pos];
            ids[b] = id;
        }
        if (tokens != nullptr) tokens[b * tokens_ld + pos] = id;
        const bool hard = (pos + 1 < seq_len) && ((pos + 1) % window == 0);
        fire[b] = (hard || (carry_id >= 0 && id == carry_id)) ? 1 : 0;
        reset_now[b] = pending[b];
        s_id = id < 0 ? 0 : (id >= V ? V - 1 : id);   // out-of-vocabulary ids read a valid row
    }
    __syncthreads();
    const T* src = emb + s_id * N;
    T* dst = h + b * N;
    if ((N * (int64_t)sizeof(T)) % 16 == 0) {
        const int64_t nv = N * (int64_t)sizeof(T) / 16;
        for (int64_t i = threadIdx.x; i < nv; i += blockDim.x)
            reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
    } else {
        for (int64_t i = threadIdx.x; i < N; i += blockDim.x) dst[i] = src[i];
    }
}

// The step's prologue in one launch (one block per batch row b): the position,
// the row's logits and its pending flag are requested together; the token id
// is prompt[b, pos] while pos < prompt_len, otherwise argmax(logits[b]) (first
// index on ties, as argmax_rows_vec_kernel) or, without logits, ids[b] as the
// caller wrote it; then ids, tokens, fire and reset_now as
// decode_prologue_kernel, and row id of the projection table copied into up to
// two destinations (table row = [seg 0 | seg 1]).  A gathered table row equals
// the projection of the gathered embedding row (the projection is linear in
// it), so the step's embedding lookup and its first projections cost one load
// round trip after the id.
template <typename T>
struct PrologueGatherArgs {
    const T* logits;          // [B, V] or null
    int64_t* ids;
    const int64_t* prompt;
    int64_t prompt_len, prompt_ld;
    int64_t* tokens;
    int64_t tokens_ld;
    const int64_t* pos_dev;
    const uint8_t* pending;
    uint8_t* fire;
    uint8_t* reset_now;
    int64_t carry_id, window, seq_len;
    const T* table;           // [V, row_len]
    int64_t row_len, V;
    T* dst[2];
    int64_t ld[2], n[2];
    bool vec;                 // table rows and destinations take 16-byte pieces
};

template <typename T, int VPT>
__global__ void __launch_bounds__(256)
decode_prologue_gather_kernel(PrologueGatherArgs<T> a) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    __shared__ int64_t s_id;
    const int64_t b = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t pos = *a.pos_dev;
    // the logits of the row, requested with the position (clamped, unconditional)
    const int nvec = (int)(a.V / 8);
    float vals[VPT > 0 ? VPT : 1][8];
    if constexpr (VPT > 0) {
        const T* x = a.logits + b * a.V;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int v = tid + 256 * i;
            Vec8<T>::load(x + 8 * (v < nvec ? v : nvec - 1), vals[i]);
        }
    }
    const uint8_t pend = a.pending[b];
    const bool from_prompt = a.prompt != nullptr && pos < a.prompt_len;   // block-uniform
    if (from_prompt) {
        if (tid == 0) s_id = a.prompt[b * a.prompt_ld + pos];
    } else if constexpr (VPT > 0) {
        float best = -INFINITY;
        int idx = (int)a.V;                  // NaN-free rows always replace this
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int v = tid + 256 * i;
            if (v >= nvec) continue;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (vals[i][e] > best) { best = vals[i][e]; idx = 8 * v + e; }   // increasing index
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ob = __shfl_xor(best, off, 64);
            const int oi = __shfl_xor(idx, off, 64);
            if (ob > best || (ob == best && oi < idx)) { best = ob; idx = oi; }
        }
        const int w = tid >> 6;
        if ((tid & 63) == 0) { bv[w] = best; bi[w] = idx; }
        __syncthreads();
        if (tid == 0) {
            for (int k = 1; k < 4; ++k)
                if (bv[k] > best || (bv[k] == best && bi[k] < idx)) { best = bv[k]; idx = bi[k]; }
            s_id = idx < a.V ? idx : 0;
        }
    } else {
        if (tid == 0) s_id = a.ids[b];
    }
    __syncthreads();
    const int64_t id = s_id;
    if (tid == 0) {
        a.ids[b] = id;
        if (a.tokens != nullptr) a.tokens[b * a.tokens_ld + pos] = id;
        const bool hard = (pos + 1 < a.seq_len) && ((pos + 1) % a.window == 0);
        a.fire[b] = (hard || (a.carry_id >= 0 && id == a.carry_id)) ? 1 : 0;
        a.reset_now[b] = pend;
    }
    // out-of-vocabulary ids read a valid row (callers validate prompt ids)
    const int64_t rid = id < 0 ? 0 : (id >= a.V ? a.V - 1 : id);
    const T* src = a.table + rid * a.row_len;
    if (a.vec) {
        const uint4* s4 = reinterpret_cast<const uint4*>(src);
        constexpr int E = 16 / (int)sizeof(T);
        const int n0 = (int)(a.n[0] / E), n1 = (int)(a.n[1] / E);
        for (int i = tid; i < n0 + n1; i += 256) {
            const uint4 v = s4[i];
            if (i < n0) reinterpret_cast<uint4*>(a.dst[0] + b * a.ld[0])[i] = v;
            else reinterpret_cast<uint4*>(a.dst[1] + b * a.ld[1])[i - n0] = v;
        }
    } else {
        for (int64_t i = tid; i < a.n[0] + a.n[1]; i += 256) {
            if (i < a.n[0]) a.dst[0][b * a.ld[0] + i] = src[i];
            else a.dst[1][b * a.ld[1] + i - a.n[0]] = src[i];
        }
    }
}

// Final-CA key append (tria.py:1576-1582) and end-of-step bookkeeping: if any
// row fires, the staged keys/values of every row are stored at slot ca_len and
// marked valid where that row fired; then pending = fire and pos += 1.
template <typename T>
__global__ void __launch_bounds__(256)
decode_epilogue_kernel(const T* __restrict__ stage_k, const T* __restrict__ stage_v,
                       T* __restrict__ ca_k, T* __restrict__ ca_v, uint8_t* __restrict__ ca_valid,
                       int64_t* __restrict__ ca_len, const uint8_t* __restrict__ fire,
                       uint8_t* __restrict__ pending, int64_t* __restrict__ pos_dev, int64_t B,
                       int64_t N, int64_t max_keys) {
    __shared__ int64_t slot;
    int a = 0;
    for (int64_t b = threadIdx.x; b < B; b += blockDim.x) a |= fire[b];
    if (threadIdx.x == 0) slot = *ca_len;
    const int any = __syncthreads_or(a);   // also orders slot's store before its reads
    if (any && slot < max_keys) {
        for (int64_t e = threadIdx.x; e < B * N; e += blockDim.x) {
            const int64_t b = e / N, d = e - b * N;
            ca_k[(b * max_keys + slot) * N + d] = stage_k[e];
            ca_v[(b * max_keys + slot) * N + d] = stage_v[e];
        }
        for (int64_t b = threadIdx.x; b < B; b += blockDim.x)
            ca_valid[b * max_keys + slot] = fire[b];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        if (any && slot < max_keys) *ca_len = slot + 1;
        *pos_dev += 1;
    }
    for (int64_t b = threadIdx.x; b < B; b += blockDim.x) pending[b] = fire[b];
}

// Greedy pick: ids[r] = argmax_v logits[r, v], the first index on ties
// (torch.argmax semantics); one block per row.
template <typename T>
__global__ void __launch_bounds__(256)
argmax_rows_kernel(const T* __restrict__ logits, int64_t V, int64_t* __restrict__ ids) {
    __shared__ float bv[4];
    __shared__ int64_t bi[4];
    const int64_t row = blockIdx.x;
    const T* x = logits + row * V;
    float best = -INFINITY;
    int64_t idx = V;                       // NaN-free rows always replace this
    for (int64_t v = threadIdx.x; v < V; v += blockDim.x) {
        const float f = ld(x + v);
        if (f > best || (f == best && v < idx)) { best = f; idx = v; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ob = __shfl_xor(best, off, 64);
        const int64_t oi = __shfl_xor(idx, off, 64);
        if (ob > best || (ob == best && oi < idx)) { best = ob; idx = oi; }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { bv[w] = best; bi[w] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < (int)(blockDim.x >> 6); ++k)
            if (bv[k] > best || (bv[k] == best && bi[k] < idx)) { best = bv[k]; idx = bi[k]; }
        ids[row] = idx < V ? idx : 0;
    }
}

// Same pick for rows of 8-element vectors (V % 8 == 0, 16-byte aligned rows of
// at most 256*8*VPT values): every thread requests all of its VPT vectors
// before it compares, so a row costs one memory round trip.
template <typename T, int VPT>
__global__ void __launch_bounds__(256)
argmax_rows_vec_kernel(const T* __restrict__ logits, int64_t V, int64_t* __restrict__ ids) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    const T* x = logits + (int64_t)blockIdx.x * V;
    const int nvec = (int)(V / 8);
    float vals[VPT][8];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {   // unconditional (clamped), so all are in flight at once
        const int v = threadIdx.x + 256 * i;
        Vec8<T>::load(x + 8 * (v < nvec ? v : nvec - 1), vals[i]);
    }
    float best = -INFINITY;
    int idx = (int)V;                      // NaN-free rows always replace this
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int v = threadIdx.x + 256 * i;
        if (v >= nvec) continue;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (vals[i][e] > best) { best = vals[i][e]; idx = 8 * v + e; }   // increasing index
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ob = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (ob > best || (ob == best && oi < idx)) { best = ob; idx = oi; }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { bv[w] = best; bi[w] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; ++k)
            if (bv[k] > best || (bv[k] == best && bi[k] < idx)) { best = bv[k]; idx = bi[k]; }
        ids[blockIdx.x] = idx < V ? idx : 0;
    }
}

template <typename T>
static int argmax_dispatch(const void* logits, int64_t rows, int64_t V, int64_t* ids,
                           hipStream_t st) {
    const bool vec = V % 8 == 0 && V <= 256 * 8 * 8 && ((uintptr_t)logits & 15) == 0;
#define LOOM_ARGMAX(VPT)                                                                        \
    if (vec && V <= 256 * 8 * (VPT)) {                                                          \
        hipLaunchKernelGGL((argmax_rows_vec_kernel<T, VPT>), dim3((unsigned)rows), dim3(256), 0, \
                           st, (const T*)logits, V, ids);                                       \
        return launch_status("loom_argmax_rows");                                               \
    }
    LOOM_ARGMAX(1) LOOM_ARGMAX(2) LOOM_ARGMAX(4) LOOM_ARGMAX(8)
#undef LOOM_ARGMAX
    hipLaunchKernelGGL((argmax_rows_kernel<T>), dim3((unsigned)rows), dim3(256), 0, st,
                       (const T*)logits, V, ids);
    return launch_status("loom_argmax_rows");
}

template <typename T>
static int epilogue_dispatch(const void* sk, const void* sv, void* ck, void* cv, uint8_t* valid,
                             int64_t* ca_len, const uint8_t* fire, uint8_t* pending,
                             int64_t* pos_dev, int64_t B, int64_t N, int64_t max_keys,
                             hipStream_t st) {
    hipLaunchKernelGGL((decode_epilogue_kernel<T>), dim3(1), dim3(256), 0, st, (const T*)sk,
                       (const T*)sv, (T*)ck, (T*)cv, valid, ca_len, fire, pending, pos_dev, B, N,
                       max_keys);
    return launch_status("loom_decode_epilogue");
}

extern "C" int loom_decode_prologue(int64_t* ids, const int64_t* prompt, int64_t prompt_len,
                                    int64_t prompt_ld, int64_t* tokens, int64_t tokens_ld,
                                    const int64_t* pos_dev, const uint8_t* pending, uint8_t* fire,
                                    uint8_t* reset_now, int64_t carry_id, int64_t window,
                                    int64_t seq_len, int64_t B, void* stream) {
    clear_error();
    LOOM_CHECK(ids && pos_dev && pending && fire && reset_now, "decode_prologue: null argument");
    LOOM_CHECK(window >= 1 && B >= 0, "decode_prologue: bad window/batch");
    LOOM_CHECK(!prompt || prompt_ld >= prompt_len, "decode_prologue: prompt row stride < length");
    if (B == 0) return LOOM_OK;
    hipLaunchKernelGGL(decode_prologue_kernel, dim3((unsigned)ceil_div(B, 256)), dim3(256), 0,
                       (hipStream_t)stream, ids, prompt, prompt_len, prompt_ld, tokens, tokens_ld,
                       pos_dev, pending, fire, reset_now, carry_id, window, seq_len, B);
    return launch_status("loom_decode_prologue");
}

template <typename T>
static int prologue_embed_dispatch(int64_t* ids, const int64_t* prompt, int64_t prompt_len,
                                   int64_t prompt_ld, int64_t* tokens, int64_t tokens_ld,
                                   const int64_t* pos_dev, const uint8_t* pending, uint8_t* fire,
                                   uint8_t* reset_now, int64_t carry_id, int64_t window,
                                   int64_t seq_len, const void* emb, void* h, int64_t N, int64_t V,
                                   int64_t B, hipStream_t st) {
    hipLaunchKernelGGL((decode_prologue_embed_kernel<T>), dim3((unsigned)B), dim3(128), 0, st, ids,
                       prompt, prompt_len, prompt_ld, tokens, tokens_ld, pos_dev, pending, fire,
                       reset_now, carry_id, window, seq_len, (const T*)emb, (T*)h, N, V);
    return launch_status("loom_decode_prologue_embed");
}

extern "C" int loom_decode_prologue_embed(int dtype, int64_t* ids, const int64_t* prompt,
                                          int64_t prompt_len, int64_t prompt_ld, int64_t* tokens,
                                          int64_t tokens_ld, const int64_t* pos_dev,
                                          const uint8_t* pending, uint8_t* fire,
                                          uint8_t* reset_now, int64_t carry_id, int64_t window,
                                          int64_t seq_len, const void* emb, void* h, int64_t N,
                                          int64_t V, int64_t B, void* stream) {
    clear_error();
    LOOM_CHECK(ids && pos_dev && pending && fire && reset_now && emb && h,
               "decode_prologue_embed: null argument");
    LOOM_CHECK(window >= 1 && B >= 0 && N >= 1 && V >= 1, "decode_prologue_embed: bad shape");
    LOOM_CHECK(!prompt || prompt_ld >= prompt_len, "decode_prologue_embed: prompt row stride < length");
    LOOM_CHECK((((uintptr_t)emb | (uintptr_t)h) & 15) == 0,
               "decode_prologue_embed: emb and h must be 16-byte aligned");
    if (B == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, prologue_embed_dispatch, ids, prompt, prompt_len, prompt_ld, tokens,
                      tokens_ld, pos_dev, pending, fire, reset_now, carry_id, window, seq_len, emb,
                      h, N, V, B, (hipStream_t)stream)
}

template <typename T>
static int prologue_gather_dispatch(const PrologueGatherArgs<T>& a0, int64_t B, hipStream_t st) {
    PrologueGatherArgs<T> a = a0;
    const int64_t V = a.V;
    const bool vec = a.logits != nullptr && V % 8 == 0 && V <= 256 * 8 * 8 &&
                     ((uintptr_t)a.logits & 15) == 0;
    LOOM_CHECK(a.logits == nullptr || vec,
               "decode_prologue_gather: logits need V %% 8 == 0, V <= 16384 and 16-byte alignment");
    constexpr int E = 16 / (int)sizeof(T);
    a.vec = ((uintptr_t)a.table & 15) == 0 && a.row_len % E == 0 && a.n[0] % E == 0 &&
            (a.n[1] == 0 || (((uintptr_t)a.dst[1] & 15) == 0 && a.ld[1] % E == 0)) &&
            ((uintptr_t)a.dst[0] & 15) == 0 && a.ld[0] % E == 0 && a.n[1] % E == 0;
    const dim3 grid((unsigned)B), blk(256);
    if (a.logits == nullptr) hipLaunchKernelGGL((decode_prologue_gather_kernel<T, 0>), grid, blk, 0, st, a);
    else if (V <= 256 * 8) hipLaunchKernelGGL((decode_prologue_gather_kernel<T, 1>), grid, blk, 0, st, a);
    else if (V <= 256 * 8 * 2) hipLaunchKernelGGL((decode_prologue_gather_kernel<T, 2>), grid, blk, 0, st, a);
    else if (V <= 256 * 8 * 4) hipLaunchKernelGGL((decode_prologue_gather_kernel<T, 4>), grid, blk, 0, st, a);
    else hipLaunchKernelGGL((decode_prologue_gather_kernel<T, 8>), grid, blk, 0, st, a);
    return launch_status("loom_decode_prologue_gather");
}

template <typename T>
static int prologue_gather_typed(const void* logits, int64_t* ids, const int64_t* prompt,
                                 int64_t prompt_len, int64_t prompt_ld, int64_t* tokens,
                                 int64_t tokens_ld, const int64_t* pos_dev, const uint8_t* pending,
                                 uint8_t* fire, uint8_t* reset_now, int64_t carry_id,
                                 int64_t window, int64_t seq_len, const void* table,
                                 int64_t row_len, int64_t V, void* dst0, int64_t ld0, int64_t n0,
                                 void* dst1, int64_t ld1, int64_t n1, int64_t B, hipStream_t st) {
    PrologueGatherArgs<T> a{};
    a.logits = (const T*)logits; a.ids = ids; a.prompt = prompt; a.prompt_len = prompt_len;
    a.prompt_ld = prompt_ld; a.tokens = tokens; a.tokens_ld = tokens_ld; a.pos_dev = pos_dev;
    a.pending = pending; a.fire = fire; a.reset_now = reset_now; a.carry_id = carry_id;
    a.window = window; a.seq_len = seq_len; a.table = (const T*)table; a.row_len = row_len;
    a.V = V; a.dst[0] = (T*)dst0; a.ld[0] = ld0; a.n[0] = n0; a.dst[1] = (T*)dst1;
    a.ld[1] = ld1; a.n[1] = n1;
    return prologue_gather_dispatch<T>(a, B, st);
}

extern "C" int loom_decode_prologue_gather(int dtype, const void* logits, int64_t* ids,
                                           const int64_t* prompt, int64_t prompt_len,
                                           int64_t prompt_ld, int64_t* tokens, int64_t tokens_ld,
                                           const int64_t* pos_dev, const uint8_t* pending,
                                           uint8_t* fire, uint8_t* reset_now, int64_t carry_id,
                                           int64_t window, int64_t seq_len, const void* table,
                                           int64_t row_len, int64_t V, void* dst0, int64_t ld0,
                                           int64_t n0, void* dst1, int64_t ld1, int64_t n1,
                                           int64_t B, void* stream) {
    clear_error();
    LOOM_CHECK(ids && pos_dev && pending && fire && reset_now && table && dst0,
               "decode_prologue_gather: null argument");
    LOOM_CHECK(window >= 1 && B >= 0 && V >= 1 && n0 >= 1 && n1 >= 0 && n0 + n1 == row_len &&
                   ld0 >= n0 && (n1 == 0 || (dst1 != nullptr && ld1 >= n1)),
               "decode_prologue_gather: bad shape (n0 + n1 must equal row_len)");
    LOOM_CHECK(!prompt || prompt_ld >= prompt_len, "decode_prologue_gather: prompt row stride < length");
    if (B == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, prologue_gather_typed, logits, ids, prompt, prompt_len, prompt_ld,
                      tokens, tokens_ld, pos_dev, pending, fire, reset_now, carry_id, window,
                      seq_len, table, row_len, V, dst0, ld0, n0, dst1, ld1, n1, B,
                      (hipStream_t)stream)
}

extern "C" int loom_argmax_rows(int dtype, const void* logits, int64_t rows, int64_t V,
                                int64_t* ids, void* stream) {
    clear_error();
    LOOM_CHECK(logits && ids && V >= 1 && rows >= 0, "argmax_rows: bad arguments");
    if (rows == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, argmax_dispatch, logits, rows, V, ids, (hipStream_t)stream)
}

extern "C" int loom_decode_epilogue(int dtype, const void* stage_k, const void* stage_v,
                                    void* ca_k, void* ca_v, uint8_t* ca_valid, int64_t* ca_len,
                                    const uint8_t* fire, uint8_t* pending, int64_t* pos_dev,
                                    int64_t B, int64_t N, int64_t max_keys, void* stream) {
    clear_error();
    LOOM_CHECK(stage_k && stage_v && ca_k && ca_v && ca_valid && ca_len && fire && pending &&
                   pos_dev,
               "decode_epilogue: null argument");
    LOOM_DTYPE_SWITCH(dtype, epilogue_dispatch, stage_k, stage_v, ca_k, ca_v, ca_valid, ca_len,
                      fire, pending, pos_dev, B, N, max_keys, (hipStream_t)stream)
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

template <typename T>
static int rms_dispatch(const void* x, const void* w, void* out, int64_t rows, int64_t N,
                        float eps, hipStream_t st) {
    hipLaunchKernelGGL((rms_norm_kernel<T>), dim3((unsigned)ceil_div(rows * 64, 256)), dim3(256),
                       0, st, (const T*)x, (const T*)w, (T*)out, rows, (int)N, eps);
    return launch_status("loom_rms_norm");
}

extern "C" int loom_rms_norm(int dtype, const void* x, const void* weight, void* out,
                             int64_t rows, int64_t N, float eps, void* stream) {
    clear_error();
    LOOM_CHECK(x && weight && out, "rms_norm: null argument");
    LOOM_CHECK(N >= 1 && N <= 64 * 32, "rms_norm: N=%lld outside [1, 2048]", (long long)N);
    LOOM_CHECK(rows >= 0, "rms_norm: rows=%lld", (long long)rows);
    if (rows == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, rms_dispatch, x, weight, out, rows, N, eps, (hipStream_t)stream)
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

extern "C" int64_t loom_decode_tria_readout_workspace_bytes(int64_t B, int64_t H) {
    return B * ceil_div(H, kReadHeads) * kReadRec * (int64_t)sizeof(float);
}

extern "C" int loom_decode_tria_readout(int dtype, const void* depth, const void* prev,
                                        const uint8_t* reset_now, const uint8_t* fire, void* doc,
                                        const void* score_w, const void* proj_w,
                                        const float* proj_b, const void* up_w, const float* up_b,
                                        void* a_out, float* workspace, int64_t workspace_bytes,
                                        int64_t B, int64_t H, int64_t N, float polarm_beta,
                                        float eps, void* stream) {
    clear_error();
    LOOM_CHECK(depth && doc && score_w && proj_w && up_w && a_out && workspace,
               "decode_tria_readout: null argument");
    LOOM_CHECK(!prev || reset_now, "decode_tria_readout: prev needs reset_now");
    LOOM_CHECK(polarm_beta >= 0.0f && polarm_beta < 1.0f,
               "PolARM beta must be finite and in [0, 1), got %g", (double)polarm_beta);
    LOOM_CHECK(H >= 1 && H <= (int64_t)kReadHeads * kReadCols && N >= 1 && B >= 0 &&
                   N < ((int64_t)1 << 31) && B < 65536,
               "decode_tria_readout: bad shape B=%lld H=%lld N=%lld (H <= %d)", (long long)B,
               (long long)H, (long long)N, kReadHeads * kReadCols);
    LOOM_CHECK(((uintptr_t)up_w & 15) == 0, "decode_tria_readout: up weight must be 16-byte aligned");
    LOOM_CHECK(workspace_bytes >= loom_decode_tria_readout_workspace_bytes(B, H),
               "decode_tria_readout: workspace of %lld bytes, %lld needed", (long long)workspace_bytes,
               (long long)loom_decode_tria_readout_workspace_bytes(B, H));
    if (B == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, readout_dispatch, depth, prev, reset_now, fire, doc, score_w, proj_w,
                      proj_b, up_w, up_b, a_out, workspace, B, H, N, polarm_beta, eps,
                      (hipStream_t)stream)
}
