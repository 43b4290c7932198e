// Causal GQA attention over a chunk of prompt tokens, for prefilling the
// decode state in chunks (Model._forward_chunked, loomformer.py:3788-3883,
// runs the stack chunk by chunk; GroupedQueryCausalSelfAttention attends each
// chunk's queries to the cached keys of earlier chunks plus the chunk's own,
// :3215-3332).
//
// Token t of the chunk sits at position start + t.  One call:
//   1. ropes q and k of every token (YaRN tables as in the decode step),
//      writes the roped q [B, T, QH, HD] and appends (k_roped, v) at rows
//      start .. start+T-1 of the caches;
//   2. attends every (token, q head) to cache rows 0 .. start + t with an fp32
//      softmax and writes both readouts, C = A.V and Kctx = A.K_roped.
// The caches take the decode engine's strides (batch, position, kv head).
//
// bf16 with head_dim 32/64/96/128 runs on MFMA: a block holds 4 (query tile
// of 16 positions, head) pairs of one kv head, streams 32 cached rows per step
// through LDS once for all four (K as stored for the scores, K and V
// transposed for the two readouts), and keeps one online softmax per query
// column.  Other dtypes / head sizes take a 16-lanes-per-row VALU kernel, one
// block per (token, kv head).
#include <cmath>

#include "attn_tile.h"
#include "loom_common.h"

namespace loom {

template <typename T>
struct PrefillArgs {
    const T* q;            // roped q [B, T, QH, HD]
    const T* kc;
    const T* vc;
    int64_t csb, cst, csh;
    T* c_out;              // [B, T, QH*HD] rows at out_ld
    T* k_out;
    int64_t out_ld;
    int64_t start;         // position of token 0 of the chunk
    int Tc, QH, KVH;
    float qscale;          // log2(e) / sqrt(HD): scores in log2 units
};

template <typename T>
__global__ void __launch_bounds__(256)
prefill_rope_append_kernel(const T* __restrict__ qkv, int64_t qkv_ld, T* __restrict__ q_out,
                           T* __restrict__ kc, T* __restrict__ vc, const float* __restrict__ cosv,
                           const float* __restrict__ sinv, int64_t B, int64_t Tc, int64_t start,
                           int QH, int KVH, int HD, int64_t csb, int64_t cst, int64_t csh) {
    const int heads = QH + 2 * KVH;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= B * Tc * heads * HD) return;
    const int d = (int)(id % HD);
    const int hs = (int)((id / HD) % heads);
    const int64_t bt = id / ((int64_t)HD * heads);
    const int64_t b = bt / Tc, t = bt - b * Tc;
    const int64_t pos = start + t;
    const T* row = qkv + bt * qkv_ld;
    const int half = HD / 2;
    if (hs < QH + KVH) {
        const T* x = row + hs * HD;
        const float rot = d < half ? -ld(x + d + half) : ld(x + d - half);
        const float v = ld(x + d) * cosv[pos * HD + d] + rot * sinv[pos * HD + d];
        if (hs < QH)
            st(q_out + (bt * QH + hs) * HD + d, v);
        else
            st(kc + b * csb + pos * cst + (hs - QH) * csh + d, v);
    } else {
        const int kvh = hs - QH - KVH;
        st(vc + b * csb + pos * cst + kvh * csh + d, ld(row + hs * HD + d));
    }
}

// Same contract, one thread per 8 consecutive dims of one head of one token
// (head_dim a multiple of 16, so a group never straddles the rotate-half
// boundary and its partner group is whole too): 16-byte loads of x, its
// partner and the two table rows, one 16-byte store.  The rotation is the
// scalar kernel's fma(x, cos, rot * sin) to the bit.
template <typename T>
__global__ void __launch_bounds__(256)
prefill_rope_append8_kernel(const T* __restrict__ qkv, int64_t qkv_ld, T* __restrict__ q_out,
                            T* __restrict__ kc, T* __restrict__ vc, const float* __restrict__ cosv,
                            const float* __restrict__ sinv, int total, int Tc, int64_t start, int QH,
                            int KVH, int HD, int64_t csb, int64_t cst, int64_t csh) {
    const int id = blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const int P = HD >> 3, heads = QH + 2 * KVH;
    const int bt = id / (heads * P);
    const int rem = id - bt * heads * P;
    const int hs = rem / P, d0 = (rem - hs * P) * 8;
    const int b = bt / Tc, t = bt - b * Tc;
    const int64_t pos = start + t;
    const T* head = qkv + (int64_t)bt * qkv_ld + hs * HD;
    float v[8];
    if (hs < QH + KVH) {
        const int half = HD >> 1;
        float x[8], y[8], c[8], sn[8];
        Vec8<T>::load(head + d0, x);
        Vec8<T>::load(head + (d0 < half ? d0 + half : d0 - half), y);
        Vec8<float>::load(cosv + pos * HD + d0, c);
        Vec8<float>::load(sinv + pos * HD + d0, sn);
        const float sg = d0 < half ? -1.0f : 1.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = fmaf(x[e], c[e], (sg * y[e]) * sn[e]);
        if (hs < QH)
            Vec8<T>::store(q_out + ((int64_t)bt * QH + hs) * HD + d0, v);
        else
            Vec8<T>::store(kc + b * csb + pos * cst + (hs - QH) * csh + d0, v);
    } else {
        Vec8<T>::load(head + d0, v);
        Vec8<T>::store(vc + b * csb + pos * cst + (hs - QH - KVH) * csh + d0, v);
    }
}

// ------------------------------------------------------------------ VALU form
// Block (t, kvh, b): 256 / LPR row groups of LPR lanes (HD = EPL * LPR); group
// r takes cache rows r, r + NG, ... up to the token's position, in batches of
// 4 rows per load round, and keeps an online softmax per head of the group;
// the groups are merged through shuffles and LDS.
template <typename T, int EPL, int G, int LPR>
__global__ void __launch_bounds__(256)
gqa_prefill_kernel(PrefillArgs<T> a) {
    constexpr int HD = EPL * LPR;
    constexpr int NG = 256 / LPR;
    constexpr int NB = 4;
    constexpr int REC = 2 * G + 2 * G * HD;
    __shared__ float wred[4][REC];
    const int t = blockIdx.x, kvh = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int tid = threadIdx.x, j = tid % LPR, grp = tid / LPR;
    const int wave = tid >> 6, lane = tid & 63;
    const int64_t pos = a.start + t;
    const int d0 = j * EPL;
    const int64_t bt = b * a.Tc + t;

    float qv[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        RowIO<T, EPL>::load(a.q + (bt * a.QH + kvh * G + g) * HD + d0, qv[g]);
#pragma unroll
        for (int e = 0; e < EPL; ++e) qv[g][e] *= a.qscale;
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
    for (int64_t base = grp; base <= pos; base += (int64_t)NG * NB) {
        float kv[NB][EPL], vv[NB][EPL];
        bool ok[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int64_t r = base + (int64_t)NG * u;
            ok[u] = r <= pos;
            const int64_t rr = ok[u] ? r : pos;      // in range; masked below
            RowIO<T, EPL>::load(kbase + rr * a.cst, kv[u]);
            RowIO<T, EPL>::load(vbase + rr * a.cst, vv[u]);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s[NB];
            float mx = m[g];
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                float dot = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; ++e) dot = fmaf(qv[g][e], kv[u][e], dot);
                s[u] = group_sum<LPR>(dot);
                if (ok[u]) mx = fmaxf(mx, s[u]);
            }
            const float corr = __builtin_amdgcn_exp2f(m[g] - mx);   // 0 when m was -inf
            float ls = l[g] * corr;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                ac[g][e] *= corr;
                ak[g][e] *= corr;
            }
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const float p = ok[u] ? __builtin_amdgcn_exp2f(s[u] - mx) : 0.0f;
                ls += p;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    ac[g][e] = fmaf(p, vv[u][e], ac[g][e]);
                    ak[g][e] = fmaf(p, kv[u][e], ak[g][e]);
                }
            }
            l[g] = ls;
            m[g] = mx;
        }
    }
    // groups of one wave (lanes j, j+LPR, ...), head by head; a group that saw
    // no row keeps m = -inf and contributes nothing
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float M = m[g];
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        const float f = m[g] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[g] - M);
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
    // merge the 4 waves: thread i -> (head, dim) pairs
    for (int i = tid; i < G * HD; i += 256) {
        const int g = i / HD, d = i - g * HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, wred[w][g]);
        float L = 0.0f, c = 0.0f, k = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float mw = wred[w][g];
            const float f = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
            L = fmaf(wred[w][G + g], f, L);
            c = fmaf(wred[w][2 * G + g * HD + d], f, c);
            k = fmaf(wred[w][2 * G + G * HD + g * HD + d], f, k);
        }
        const float inv = 1.0f / L;
        const int64_t o = bt * a.out_ld + (int64_t)(kvh * G + g) * HD + d;
        st(a.c_out + o, c * inv);
        st(a.k_out + o, k * inv);
    }
}

// ------------------------------------------------------------------ MFMA form (bf16)
// v_mfma_f32_16x16x32_bf16 (A: 16 rows x 32 k, B: 32 k x 16 columns; lane l
// holds row/column l%16, k = 8*(l/16)..+7; result [4*(l/16)+r][l%16] in r):
//   S^T = K Q^T   A = 16 cached rows (16-byte reads of the row-major K tile),
//                 B = 16 query positions of one head
//   C   = P V     A = P (rows = query positions, k = 32 cached rows, bf16)
//   Kctx= P K         straight from the score registers,
//                 B = V / K through the transposing LDS read in the score
//                 registers' row order (tile_tr_frag, attn_tile.h).
// Block (x, y, b): y = kvh * HSPLIT + part; wave w takes head
// kvh*G + part*GP + w%GP and query tile x*QTB + w/GP (16 positions each).
// The block streams 64 cached rows per step into two LDS buffers: the next
// tile's loads are in flight while a tile is computed and land in the other
// buffer, one block barrier per step.  A step is two 32-row sub-tiles under
// one softmax update (at 1920 cached rows 74.4 -> 68.5 us against 32-row
// steps; 96 and 128 rows measured slower, 86-88 us, from register pressure).
// Two query tiles per wave (each K / V fragment read feeding two MFMAs)
// measured 12-14% slower: with 2048 query-tile x head items at the prefill's
// chunk shape a wave per SIMD is left, and the latency it no longer hides
// costs more than the halved LDS reads save.
typedef __bf16 bf16x8_p __attribute__((ext_vector_type(8)));
typedef float f32x4_p __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_p mfma16p(uint4 x, uint4 y, f32x4_p c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_p, x),
                                                   __builtin_bit_cast(bf16x8_p, y), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_p mfma16p(gqa_u4 x, uint4 y, f32x4_p c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_p, x),
                                                   __builtin_bit_cast(bf16x8_p, y), c, 0, 0, 0);
}

__device__ __forceinline__ void lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Block barrier over LDS filled by loads straight into LDS: this wave's
// loads but the last N have landed and its LDS reads have completed, then
// s_barrier.  The asm's memory clobber keeps the compiler from moving memory
// accesses across it; a workgroup fence would also wait for the N loads.
template <int N>
__device__ __forceinline__ void dma_barrier() {
    wait_vmcnt<N>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

constexpr int kPfSub = 2;     // 32-row sub-tiles per step (one softmax update per step)
constexpr int kPfRows = 32 * kPfSub;   // cached rows per step

// Two waves per SIMD (<= 256 VGPRs; the grid of a 128-token chunk has two
// per SIMD).  The file is built with -amdgpu-mfma-vgpr-form, so the
// accumulators sit in ordinary VGPRs, where the per-step rescale multiplies
// them in place (in AGPRs each would be copied out and back, 144 VALU
// operations per step)
template <int HD, int GP, int HSPLIT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
gqa_prefill_mfma_kernel(PrefillArgs<bf16_t> a) {
    constexpr int KK = HD / 32;
    constexpr int DT = HD / 16;
    constexpr int CPR = HD / 8;                 // 16-byte pieces per row
    constexpr int QTB = 4 / GP;                 // query tiles per block
    constexpr int G = GP * HSPLIT;
    constexpr int SUB = kPfSub, R = kPfRows;
    static_assert(CPR % 4 == 0 && R == 64, "a tile is CPR loads of 64 pieces, split evenly over the 4 waves");
    constexpr int GPW = CPR / 4;                // loads per tensor per wave and step
    // LDS rows of CPR pieces, piece c of row r at c ^ kv_swz(r); three stages
    // (tile t in stage t % 3) as separate arrays, so that a wait for one
    // stage's loads never covers another stage's reads
    constexpr int PITCH = CPR;
    __shared__ __align__(16) gqa_u4 K0[R * PITCH], K1[R * PITCH], K2[R * PITCH];
    __shared__ __align__(16) gqa_u4 V0[R * PITCH], V1[R * PITCH], V2[R * PITCH];
    __shared__ float cr[4][16];                           // per-column rescale of a step
    auto kst = [&](auto s_) -> gqa_u4* {
        constexpr int S = decltype(s_)::value;
        return S == 0 ? K0 : S == 1 ? K1 : K2;
    };
    auto vst = [&](auto s_) -> gqa_u4* {
        constexpr int S = decltype(s_)::value;
        return S == 0 ? V0 : S == 1 ? V1 : V2;
    };
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lq = lane >> 4;
    // work item (query tiles, head group, row) in query-tile-fastest order; the
    // query tiles of one (row, kv head) read the same K/V rows, so they share
    // an XCD and its L2
    const int ntile = (a.Tc + 16 * QTB - 1) / (16 * QTB), ngrp = a.KVH * HSPLIT;
    const int w = xcd_contiguous((int)blockIdx.x, (int)gridDim.x);
    const int bx = w % ntile, by = (w / ntile) % ngrp;
    const int kvh = by / HSPLIT, part = by % HSPLIT;
    const int64_t b = w / (ntile * ngrp);
    const int head = kvh * G + part * GP + wave % GP;
    const int qlast_blk = min((bx + 1) * QTB * 16, a.Tc) - 1;
    const int64_t kmax = a.start + qlast_blk;                    // last cached row the block reads
    const int nsteps = (int)((kmax + R) / R);
    const int q0 = (bx * QTB + wave / GP) * 16;                  // first query of the wave's tile
    // this lane's query column (lr): its position; a column past the chunk
    // attends to row 0 only (finite, never stored)
    const int qcol = q0 + lr;
    const int qpos32 = qcol < a.Tc ? (int)a.start + qcol : 0;    // positions fit 31 bits (host check)
    const int wave_qpos0 = (int)a.start + q0;                    // position of the wave's first query
    const int64_t wave_kmax = q0 < a.Tc ? a.start + min(q0 + 15, a.Tc - 1) : -1;
    const TileLane<CPR, PITCH, true> tl(lq, lr);

    const bf16_t* kb = a.kc + b * a.csb + kvh * a.csh;
    const bf16_t* vb = a.vc + b * a.csb + kvh * a.csh;
    // one step's tiles go from the caches straight into LDS, 16 bytes a lane:
    // load g (0..CPR-1) of a tensor fills LDS pieces 64g .. 64g+63 of the
    // stage, lane l piece 64g + l = row * CPR + p, which holds piece
    // p ^ kv_swz(row) of the row; wave w issues g = w, w+4, ...  Reads go
    // through buffer resources that end after row kmax: rows past it land as
    // zero (positions after every query of the block, masked out), so a load
    // needs no clamp and its offset is a per-lane constant plus the step's rows.
    const int kv_bytes = (int)((kmax + 1) * a.cst * 2);
    const auto rk = __builtin_amdgcn_make_buffer_rsrc((void*)kb, (short)0, kv_bytes, kBufferDword3);
    const auto rv = __builtin_amdgcn_make_buffer_rsrc((void*)vb, (short)0, kv_bytes, kBufferDword3);
    const uint32_t row_bytes = (uint32_t)(a.cst * 2);
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    uint32_t voff[GPW];
#pragma unroll
    for (int j = 0; j < GPW; ++j) {
        const int p = 64 * (wv + 4 * j) + lane, row = p / CPR, c = p % CPR;
        voff[j] = (uint32_t)row * row_bytes + (uint32_t)(c ^ kv_swz(row)) * 16u;
    }
    auto load_tile = [&](auto s_, int64_t r0) {     // 2 * GPW loads of this wave
        const uint32_t base = (uint32_t)r0 * row_bytes;
#pragma unroll
        for (int j = 0; j < GPW; ++j) {
            dma16(rk, kst(s_) + 64 * (wv + 4 * j), voff[j] + base, 0);
            dma16(rv, vst(s_) + 64 * (wv + 4 * j), voff[j] + base, 0);
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    // B operand of S^T: q of query column lr, dims 32*kk + 8*lq .. +7; loaded
    // first and complete before the loop (a register loaded ahead of a loop
    // whose own loads stay in flight would be waited for inside it, and that
    // wait would also drain the tile prefetches)
    uint4 qf[KK];
    {
        const int qrow = qcol < a.Tc ? qcol : a.Tc - 1;
        const bf16_t* qp = a.q + ((b * a.Tc + qrow) * a.QH + head) * HD;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
            qf[kk] = *reinterpret_cast<const uint4*>(qp + 32 * kk + 8 * lq);
    }
    load_tile(S0{}, 0);
    load_tile(S1{}, R);
    dma_barrier<2 * GPW>();                 // q and tile 0 (tile 1 may be in flight)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
        asm volatile("" : "+v"(qf[kk].x), "+v"(qf[kk].y), "+v"(qf[kk].z), "+v"(qf[kk].w));

    float mh = -INFINITY, lh = 0.0f;      // running max / sum of query column lr
    f32x4_p accC[DT], accK[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) accC[dt] = accK[dt] = f32x4_p{0.f, 0.f, 0.f, 0.f};

    // step it computes tile it from stage it % 3 and requests tile it+2 into
    // stage (it+2) % 3 (tile it-1's, read by every wave before the previous
    // barrier), then waits for tile it+1 and passes one barrier.  Every step
    // requests a tile (rows past kmax land as zero), so the loads in flight
    // are the same on every path and each wait is a constant.  A step is SUB
    // sub-tiles of 32 rows under one softmax update.
    auto step = [&](auto s_, int it) {
        constexpr int cur = decltype(s_)::value;
        const gqa_u4* tk = kst(s_);
        const gqa_u4* tv = vst(s_);
        const int64_t r0 = (int64_t)it * R;
        load_tile(std::integral_constant<int, (cur + 2) % 3>{}, r0 + 2 * R);
        const bool active = r0 <= wave_kmax;                 // wave-uniform
        if (active) {
            // sub-tile u: rows 32u .. 32u + 31 of the step (tile rows from 32u on);
            // S^T[row 32u + 16*hf + 4*lq + r][query column lr], unscaled
            f32x4_p sc[SUB][2];
#pragma unroll
            for (int u = 0; u < SUB; ++u)
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    sc[u][hf] = f32x4_p{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kk = 0; kk < KK; ++kk)
                        sc[u][hf] = mfma16p(tile_s_frag<CPR>(tk + u * 32 * PITCH, tl, hf, kk), qf[kk],
                                            sc[u][hf]);
                }
            // rows after a column's position are masked only in the steps that
            // reach the wave's first query (the scale is applied inside the
            // exponent: the maximum of the scaled scores is the scaled maximum)
            float sv[SUB][2][4];
            float mx = -INFINITY;
            if ((int)r0 + R - 1 <= wave_qpos0) {     // wave-uniform
#pragma unroll
                for (int u = 0; u < SUB; ++u)
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            sv[u][hf][r] = sc[u][hf][r];
                            mx = fmaxf(mx, sv[u][hf][r]);
                        }
            } else {
#pragma unroll
                for (int u = 0; u < SUB; ++u)
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int row = (int)r0 + 32 * u + 16 * hf + 4 * lq + r;
                            sv[u][hf][r] = row <= qpos32 ? sc[u][hf][r] : -INFINITY;
                            mx = fmaxf(mx, sv[u][hf][r]);
                        }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mnew = fmaxf(mh, mx * a.qscale);    // finite: row 0 is seen at step 0
            const float corr = __builtin_amdgcn_exp2f(mh - mnew);
            float ls = 0.0f, pv[SUB][2][4];
#pragma unroll
            for (int u = 0; u < SUB; ++u)
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        // a masked score gives exp2(-inf) = 0
                        pv[u][hf][r] = __builtin_amdgcn_exp2f(fmaf(sv[u][hf][r], a.qscale, -mnew));
                        ls += pv[u][hf][r];
                    }
            ls += __shfl_xor(ls, 16, 64);
            ls += __shfl_xor(ls, 32, 64);
            lh = fmaf(lh, corr, ls);
            mh = mnew;
            // A operands of P V / P K straight from the score registers: query
            // column lr, positions 32u + 4*lq + r and 32u + 16 + 4*lq + r (bf16
            // like the reference's softmax output), matched by tile_tr_frag
            uint4 pa[SUB];
#pragma unroll
            for (int u = 0; u < SUB; ++u)
                pa[u] = make_uint4(pack_bf16x2(pv[u][0][0], pv[u][0][1]), pack_bf16x2(pv[u][0][2], pv[u][0][3]),
                                   pack_bf16x2(pv[u][1][0], pv[u][1][1]), pack_bf16x2(pv[u][1][2], pv[u][1][3]));
            // the accumulator rows are query columns 4*lq + r: their rescale
            // from the lanes that hold those columns, through LDS (measured
            // faster here than four cross-lane permutes); skipped when no
            // column's max moved (every factor exactly 1)
            if (__any(corr != 1.0f)) {
                if (lq == 0) cr[wave][lr] = corr;
                wave_lds_fence();
                float cf[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) cf[r] = cr[wave][4 * lq + r];
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        accC[dt][r] *= cf[r];
                        accK[dt][r] *= cf[r];
                    }
                wave_lds_fence();              // cr is rewritten next step
            }
#pragma unroll
            for (int u = 0; u < SUB; ++u)
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    accC[dt] = mfma16p(pa[u], tile_tr_frag<CPR>(tv + u * 32 * PITCH, tl, dt), accC[dt]);
                    accK[dt] = mfma16p(pa[u], tile_tr_frag<CPR>(tk + u * 32 * PITCH, tl, dt), accK[dt]);
                }
        }
        dma_barrier<2 * GPW>();             // tile it+1 landed (tile it+2 may be in flight)
    };
    // a multiple of 3 steps (steps past kmax compute nothing)
    for (int it = 0; it < nsteps; it += 3) {
        step(S0{}, it);
        step(S1{}, it + 1);
        step(S2{}, it + 2);
    }
    wait_vmcnt<0>();                        // no load into LDS outlives the loop
    // normalise: the sum of query column c lives in lanes with lr == c
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int col = 4 * lq + r;
        const int qi = q0 + col;
        const float lsum = __shfl(lh, col, 64);
        if (qi >= a.Tc) continue;
        const float inv = 1.0f / lsum;
        const int64_t o = (b * a.Tc + qi) * a.out_ld + (int64_t)head * HD;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            a.c_out[o + 16 * dt + lr].x = f32_to_bf16(accC[dt][r] * inv);
            a.k_out[o + 16 * dt + lr].x = f32_to_bf16(accK[dt][r] * inv);
        }
    }
}

template <typename T>
static int rope_append_dispatch(const void* qkv, int64_t qkv_ld, void* kc, void* vc, int64_t csb,
                                int64_t cst, int64_t csh, const float* cosv, const float* sinv,
                                void* q_out, int64_t B, int64_t Tc, int64_t start, int64_t QH,
                                int64_t KVH, int64_t HD, hipStream_t st) {
    const int64_t total = B * Tc * (QH + 2 * KVH) * HD;
    // 16-byte groups: every row base and stride a multiple of 8 elements
    // (16 bytes for 16-bit types, 32 for fp32) and 16-byte aligned pointers
    const bool vec = HD % 16 == 0 && total / 8 < (1LL << 31) && qkv_ld % 8 == 0 && csb % 8 == 0 &&
                     cst % 8 == 0 && csh % 8 == 0 &&
                     (((uintptr_t)qkv | (uintptr_t)kc | (uintptr_t)vc | (uintptr_t)q_out |
                       (uintptr_t)cosv | (uintptr_t)sinv) & 15) == 0;
    if (vec)
        hipLaunchKernelGGL((prefill_rope_append8_kernel<T>), dim3((unsigned)ceil_div(total / 8, 256)),
                           dim3(256), 0, st, (const T*)qkv, qkv_ld, (T*)q_out, (T*)kc, (T*)vc, cosv,
                           sinv, (int)(total / 8), (int)Tc, start, (int)QH, (int)KVH, (int)HD, csb,
                           cst, csh);
    else
        hipLaunchKernelGGL((prefill_rope_append_kernel<T>), dim3((unsigned)ceil_div(total, 256)),
                           dim3(256), 0, st, (const T*)qkv, qkv_ld, (T*)q_out, (T*)kc, (T*)vc, cosv,
                           sinv, B, Tc, start, (int)QH, (int)KVH, (int)HD, csb, cst, csh);
    return launch_status("loom_gqa_prefill (rope/append)");
}

int prefill_rope_append(int dtype, const void* qkv, int64_t qkv_ld, void* kc, void* vc,
                        int64_t csb, int64_t cst, int64_t csh, const float* cosv,
                        const float* sinv, void* q_out, int64_t B, int64_t Tc, int64_t start,
                        int64_t QH, int64_t KVH, int64_t HD, hipStream_t st) {
    switch (dtype) {
        case LOOM_F32:
            return rope_append_dispatch<float>(qkv, qkv_ld, kc, vc, csb, cst, csh, cosv, sinv, q_out,
                                               B, Tc, start, QH, KVH, HD, st);
        case LOOM_BF16:
            return rope_append_dispatch<bf16_t>(qkv, qkv_ld, kc, vc, csb, cst, csh, cosv, sinv, q_out,
                                                B, Tc, start, QH, KVH, HD, st);
        case LOOM_F16:
            return rope_append_dispatch<f16_t>(qkv, qkv_ld, kc, vc, csb, cst, csh, cosv, sinv, q_out,
                                               B, Tc, start, QH, KVH, HD, st);
    }
    set_error("prefill rope/append: unsupported dtype %d", dtype);
    return LOOM_ERR_INVALID;
}

// qkv null: q_out already holds the chunk's roped q and the caches its rows
template <typename T>
static int prefill_dispatch(const void* qkv, int64_t qkv_ld, void* kc, void* vc, int64_t csb,
                            int64_t cst, int64_t csh, const float* cosv, const float* sinv,
                            void* q_out, void* c_out, void* k_out, int64_t out_ld, int64_t B,
                            int64_t Tc, int64_t start, int64_t QH, int64_t KVH, int64_t HD,
                            hipStream_t st) {
    if (qkv != nullptr) {
        const int rc = rope_append_dispatch<T>(qkv, qkv_ld, kc, vc, csb, cst, csh, cosv, sinv, q_out,
                                               B, Tc, start, QH, KVH, HD, st);
        if (rc != LOOM_OK) return rc;
    }
    PrefillArgs<T> a{};
    a.q = (const T*)q_out;
    a.kc = (const T*)kc;
    a.vc = (const T*)vc;
    a.csb = csb;
    a.cst = cst;
    a.csh = csh;
    a.c_out = (T*)c_out;
    a.k_out = (T*)k_out;
    a.out_ld = out_ld;
    a.start = start;
    a.Tc = (int)Tc;
    a.QH = (int)QH;
    a.KVH = (int)KVH;
    a.qscale = kLog2e / sqrtf((float)HD);
    const int G = (int)(QH / KVH);
    if constexpr (std::is_same<T, bf16_t>::value) {
        // the MFMA form addresses a (row, kv head)'s cache rows with 32-bit
        // byte offsets, up to four tiles past the chunk's last position
        const bool mf_ok = (HD == 32 || HD == 64 || HD == 96 || HD == 128) &&
                           (G == 1 || G == 2 || G == 4 || G == 8) &&
                           (start + Tc + 4 * kPfRows) * cst * 2 < ((int64_t)1 << 31);
        if (mf_ok) {
#define LOOM_PF_MF(HDV)                                                                          \
            if (HD == HDV) {                                                                     \
                if (G == 4) {                                                                    \
                    const dim3 g((unsigned)(ceil_div(Tc, 16) * KVH * B));                \
                    hipLaunchKernelGGL((gqa_prefill_mfma_kernel<HDV, 4, 1>), g, dim3(256), 0, st, a); \
                } else if (G == 8) {                                                             \
                    const dim3 g((unsigned)(ceil_div(Tc, 16) * KVH * 2 * B));            \
                    hipLaunchKernelGGL((gqa_prefill_mfma_kernel<HDV, 4, 2>), g, dim3(256), 0, st, a); \
                } else if (G == 2) {                                                             \
                    const dim3 g((unsigned)(ceil_div(Tc, 32) * KVH * B));                \
                    hipLaunchKernelGGL((gqa_prefill_mfma_kernel<HDV, 2, 1>), g, dim3(256), 0, st, a); \
                } else {                                                                         \
                    const dim3 g((unsigned)(ceil_div(Tc, 64) * KVH * B));                \
                    hipLaunchKernelGGL((gqa_prefill_mfma_kernel<HDV, 1, 1>), g, dim3(256), 0, st, a); \
                }                                                                                \
                return launch_status("loom_gqa_prefill");                                       \
            }
            LOOM_PF_MF(96) LOOM_PF_MF(64) LOOM_PF_MF(128) LOOM_PF_MF(32)
#undef LOOM_PF_MF
        }
    }
    dim3 grid((unsigned)Tc, (unsigned)KVH, (unsigned)B);
#define LOOM_PF(E, GG, LPR)                                                                     \
    if (HD == E * LPR && G == GG) {                                                             \
        hipLaunchKernelGGL((gqa_prefill_kernel<T, E, GG, LPR>), grid, dim3(256), 0, st, a);     \
        return launch_status("loom_gqa_prefill");                                               \
    }
    LOOM_PF(6, 4, 16) LOOM_PF(6, 1, 16) LOOM_PF(6, 2, 16) LOOM_PF(6, 8, 16)
    LOOM_PF(4, 4, 16) LOOM_PF(4, 1, 16) LOOM_PF(4, 2, 16) LOOM_PF(4, 8, 16)
    LOOM_PF(8, 4, 16) LOOM_PF(8, 1, 16) LOOM_PF(8, 2, 16) LOOM_PF(8, 8, 16)
    LOOM_PF(2, 4, 16) LOOM_PF(2, 1, 16) LOOM_PF(2, 2, 16) LOOM_PF(2, 8, 16)
    LOOM_PF(1, 1, 8) LOOM_PF(1, 2, 8) LOOM_PF(1, 4, 8) LOOM_PF(1, 8, 8)
#undef LOOM_PF
    set_error("gqa_prefill: unsupported head_dim %lld / group %d", (long long)HD, G);
    return LOOM_ERR_INVALID;
}

}  // namespace loom

using namespace loom;

extern "C" int loom_gqa_prefill(int dtype, const void* qkv, int64_t qkv_ld, void* k_cache,
                                void* v_cache, int64_t cache_stride_b, int64_t cache_stride_t,
                                int64_t cache_stride_h, const float* cos_table,
                                const float* sin_table, void* q_out, void* c_out, void* kctx_out,
                                int64_t out_ld, int64_t B, int64_t T, int64_t start,
                                int64_t cache_len, int64_t QH, int64_t KVH, int64_t HD,
                                void* stream) {
    clear_error();
    LOOM_CHECK(k_cache && v_cache && cos_table && sin_table && q_out && c_out && kctx_out,
               "gqa_prefill: null argument");
    LOOM_CHECK(B >= 0 && T >= 0 && start >= 0 && KVH >= 1 && QH % KVH == 0 && HD % 2 == 0,
               "gqa_prefill: bad shape B=%lld T=%lld start=%lld QH=%lld KVH=%lld HD=%lld",
               (long long)B, (long long)T, (long long)start, (long long)QH, (long long)KVH,
               (long long)HD);
    LOOM_CHECK((qkv == nullptr || qkv_ld >= (QH + 2 * KVH) * HD) && out_ld >= QH * HD,
               "gqa_prefill: row strides smaller than the rows");
    LOOM_CHECK(cache_stride_t >= HD && cache_stride_h >= HD,
               "gqa_prefill: cache strides smaller than a head row");
    LOOM_CHECK(T <= (1 << 20), "gqa_prefill: chunk of %lld tokens too long", (long long)T);
    LOOM_CHECK(start + T < (1LL << 31), "gqa_prefill: positions beyond 2^31");
    LOOM_CHECK(ceil_div(T, 16) * QH * B <= (1LL << 23),
               "gqa_prefill: %lld rows x %lld tokens x %lld heads exceed one launch", (long long)B,
               (long long)T, (long long)QH);
    LOOM_CHECK(start + T <= cache_len,
               "gqa_prefill: positions %lld..%lld beyond the cache capacity %lld", (long long)start,
               (long long)(start + T - 1), (long long)cache_len);
    // the vector forms read 16-byte pieces of rows
    LOOM_CHECK(HD % 32 != 0 ||
                   ((((uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)q_out) & 15) == 0 &&
                    cache_stride_b % 8 == 0 && cache_stride_t % 8 == 0 && cache_stride_h % 8 == 0),
               "gqa_prefill: caches must be 16-byte aligned with strides divisible by 8");
    if (B == 0 || T == 0) return LOOM_OK;
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case LOOM_F32:
            return prefill_dispatch<float>(qkv, qkv_ld, k_cache, v_cache, cache_stride_b,
                                           cache_stride_t, cache_stride_h, cos_table, sin_table,
                                           q_out, c_out, kctx_out, out_ld, B, T, start, QH, KVH,
                                           HD, st);
        case LOOM_BF16:
            return prefill_dispatch<bf16_t>(qkv, qkv_ld, k_cache, v_cache, cache_stride_b,
                                            cache_stride_t, cache_stride_h, cos_table, sin_table,
                                            q_out, c_out, kctx_out, out_ld, B, T, start, QH, KVH,
                                            HD, st);
        case LOOM_F16:
            return prefill_dispatch<f16_t>(qkv, qkv_ld, k_cache, v_cache, cache_stride_b,
                                           cache_stride_t, cache_stride_h, cos_table, sin_table,
                                           q_out, c_out, kctx_out, out_ld, B, T, start, QH, KVH,
                                           HD, st);
    }
    set_error("gqa_prefill: unsupported dtype %d", dtype);
    return LOOM_ERR_INVALID;
}
