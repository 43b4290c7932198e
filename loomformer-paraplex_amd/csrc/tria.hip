// Tria carriers for gfx950: local 3x3 operator construction, depth
// composition, gate slot mix, slot attention pool, temporal carry, PolARM and
// the sparse final cross-attention.  All math is fp32 in registers.
//
// 3x3 matrices are stored row-major, 9 values per element ([..., 3, 3]).
// Streaming kernels stage each block's slice of 3x3 matrices through LDS so
// global traffic is whole coalesced rows; per-thread LDS reads have stride 9
// words (odd), which spreads consecutive lanes over distinct banks.
#include <cmath>

#include "loom_common.h"
#include "paraplex_math.h"
#include "tria_math.h"

namespace loom {

constexpr int kTriaThreads = 256;

// Copy n9 = rows*9 contiguous values between global memory and LDS with
// coalesced accesses: whole 16-byte pieces (8 values of a 16-bit type, 4 of
// fp32) when the slice is 16-byte aligned and a whole number of pieces, single
// values otherwise.
// The same copy in two halves, so that loads issued between them stay in
// flight while the records are waited for: issue() requests the block's
// pieces (all of them before the first LDS store: one memory round trip per
// block; nontemporally, each record is read once), commit() writes them to
// LDS as fp32 (an unaligned slice is loaded and written value by value there).
template <typename T, int REC = kTriaThreads>
struct StageIn {
    static constexpr int V = 16 / (int)sizeof(T);
    // pieces per thread when the block stages REC records of 9
    static constexpr int kPer = (REC * 9 / V + kTriaThreads - 1) / kTriaThreads;
    u32x4 w[kPer];
    bool vec;
    __device__ __forceinline__ void issue(const T* src, int n9) {
        vec = ((uintptr_t)src & 15) == 0 && n9 % V == 0;
        if (!vec) return;
#pragma unroll
        for (int r = 0; r < kPer; ++r) {
            const int c = threadIdx.x + r * kTriaThreads;
            if (c < n9 / V) w[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + c);
        }
    }
    __device__ __forceinline__ void commit(float* lds, const T* src, int n9) const {
        if (!vec) {
            for (int k = threadIdx.x; k < n9; k += blockDim.x) lds[k] = ld(src + k);
            return;
        }
#pragma unroll
        for (int r = 0; r < kPer; ++r) {
            const int c = threadIdx.x + r * kTriaThreads;
            if (c >= n9 / V) continue;
            float v[V];
            if constexpr (V == 8) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const T lo{(uint16_t)(w[r][k] & 0xffffu)}, hi{(uint16_t)(w[r][k] >> 16)};
                    v[2 * k] = ld(&lo);
                    v[2 * k + 1] = ld(&hi);
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) v[k] = __uint_as_float(w[r][k]);
            }
#pragma unroll
            for (int e = 0; e < V; ++e) lds[c * V + e] = v[e];
        }
    }
};
template <typename T, int REC = kTriaThreads>
__device__ __forceinline__ void stage_in(float* lds, const T* src, int n9) {
    StageIn<T, REC> s;
    s.issue(src, n9);
    s.commit(lds, src, n9);
}
template <typename T>
__device__ __forceinline__ void stage_out(T* dst, const float* lds, int n9) {
    constexpr int V = 16 / (int)sizeof(T);
    if (((uintptr_t)dst & 15) == 0 && n9 % V == 0) {
        for (int c = threadIdx.x; c < n9 / V; c += blockDim.x) {
            float v[V];
#pragma unroll
            for (int e = 0; e < V; ++e) v[e] = lds[c * V + e];
            // the staged records are written once: nontemporal 16-byte stores
            u32x4 x;
            if constexpr (V == 8) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    T lo, hi;
                    st(&lo, v[2 * k]);
                    st(&hi, v[2 * k + 1]);
                    x[k] = (uint32_t)lo.x | ((uint32_t)hi.x << 16);
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) x[k] = __float_as_uint(v[k]);
            }
            __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(dst) + c);
        }
        return;
    }
    for (int k = threadIdx.x; k < n9; k += blockDim.x) st(dst + k, lds[k]);
}

// MODE 0: init (pre = M); 1: step (pre = M @ carry_prev[e]);
// 2: seeded init (pre = M @ seed[b,h] where t == 0 and valid[b], else M).
// SCALE: rms(pre) is written to scale_out (the reference API's third output,
// read only by its backward); the inference form leaves it out, 4 B per
// element less, and profiles under its own name.
template <typename T, int MODE, bool GATE, int AXIS, bool SCALE>
__global__ void __launch_bounds__(kTriaThreads)
tria_depth_kernel(const T* __restrict__ r, const T* __restrict__ i_, const T* __restrict__ o,
                  const T* __restrict__ prev, const T* __restrict__ seed,
                  const uint8_t* __restrict__ valid, const T* __restrict__ w,
                  T* __restrict__ carry_out, T* __restrict__ p_out, float* __restrict__ scale_out,
                  int64_t n, int64_t T_, int64_t H, float alpha) {
    __shared__ float tile[kTriaThreads * 9];
    const int64_t e0 = (int64_t)blockIdx.x * kTriaThreads;
    const int cnt = (int)((n - e0) < kTriaThreads ? (n - e0) : kTriaThreads);
    const int64_t e = e0 + threadIdx.x;
    const bool live = threadIdx.x < cnt;
    if constexpr (MODE == 1) {
        stage_in(tile, prev + e0 * 9, cnt * 9);
        __syncthreads();
    }
    float pre[9];
    if (live) {
        float mt[9];
        carrier9<AXIS>(ld(r + e), ld(i_ + e), ld(o + e), alpha, mt);
        if constexpr (MODE == 1) {
            float cp[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) cp[k] = tile[threadIdx.x * 9 + k];
            mm3(mt, cp, pre);
        } else if constexpr (MODE == 2) {
            const int64_t h = e % H;
            const int64_t bt = e / H;
            const int64_t t = bt % T_;
            const int64_t b = bt / T_;
            if (t == 0 && valid[b] != 0) {
                float sd[9];
#pragma unroll
                for (int k = 0; k < 9; ++k) sd[k] = ld(seed + (b * H + h) * 9 + k);
                mm3(mt, sd, pre);
            } else {
#pragma unroll
                for (int k = 0; k < 9; ++k) pre[k] = mt[k];
            }
        } else {
#pragma unroll
            for (int k = 0; k < 9; ++k) pre[k] = mt[k];
        }
        const float sc = rms9(pre);
        const float inv = 1.0f / sc;
#pragma unroll
        for (int k = 0; k < 9; ++k) pre[k] *= inv;
        if constexpr (SCALE) scale_out[e] = sc;
        if constexpr (GATE) {
            float p = 0.0f;
#pragma unroll
            for (int k = 0; k < 9; ++k) p = fmaf(pre[k], ld(w + k), p);
            st(p_out + e, p);
        }
    }
    if (carry_out != nullptr) {
        if constexpr (MODE == 1) __syncthreads();  // everyone has read tile
        if (live) {
#pragma unroll
            for (int k = 0; k < 9; ++k) tile[threadIdx.x * 9 + k] = pre[k];
        }
        __syncthreads();
        stage_out(carry_out + e0 * 9, tile, cnt * 9);
    }
}

// The Paraplex pointwise chain and the block's Tria depth op in one pass over
// a [B, T, H] sequence (the sequence form of ParaplexFFN's core, loomformer.py:
// 2856-2885, followed by _tria_depth_op, :3588-3617): per element the phase
// I from beta (+ bias) and the previous token's base phase (the carried trace
// at t = 0), O = (R + A*I) * G(A), then the carrier of (R, I, O) as the
// separate ops would read them back (I and O rounded to the storage type) and
// its composition with the carried record.  I is never stored; O goes out for
// W2, and the base phase of the sequence's last token as the next trace.
// Same staging of the 9-value records as tria_depth_kernel.
constexpr int kPxTriaPerThread = 2;   // elements per thread of paraplex_tria_kernel

template <typename T>
struct PxTriaArgs {
    const T* r;            // R [B, T, H]
    const T* gsrc;         // the amplitude source (R itself, or gate_proj(u))
    const T* beta;         // beta_linear [B, T, H] (bias not added)
    const float* bias;     // [H]
    const T* trace;        // [B, H] base phase of the token before t = 0
    const float* trace_w;  // [H]
    const T* prev;         // MODE 1: carried records [B, T, H, 9]
    const T* seed;         // MODE 2: [B, H, 9] for t == 0 where valid[b]
    const uint8_t* valid;
    const T* w;            // GATE: [9]
    T* act;                // O [B, T, H]
    T* next_trace;         // [B, H]
    T* carry_out;          // [B, T, H, 9]
    T* p_out;              // GATE: [B, T, H]
    int T_, H;
    int64_t n;
    float m, alpha;
};

// Each thread computes EPT elements: with PAIR the two consecutive elements
// 2 tid and 2 tid + 1 (EPT == 2, H even, the element operands aligned to two
// elements), whose operands load and store as one word each; otherwise
// elements tid + 256 u.  MODE 1: the block's carried records are requested
// first and every element operand before they are waited for, so a block
// makes one memory round trip before its math.
template <typename T, int MODE, bool GATE, int AXIS, bool SAME_GATE, int EPT, bool PAIR>
__global__ void __launch_bounds__(kTriaThreads)
paraplex_tria_kernel(PxTriaArgs<T> a) {
    static_assert(!PAIR || EPT == 2, "paired elements are two per thread");
    constexpr int REC = kTriaThreads * EPT;
    __shared__ float tile[REC * 9];
    const int64_t e0 = (int64_t)blockIdx.x * REC;
    const int cnt = (int)((a.n - e0) < REC ? (a.n - e0) : REC);
    StageIn<T, REC> stg;
    if constexpr (MODE == 1) stg.issue(a.prev + e0 * 9, cnt * 9);
    // every operand of the thread's elements requested before any store (an
    // output may alias them as far as the compiler knows, so a later load
    // would wait for the earlier stores), at clamped indices; the gate
    // weights once
    float wv[9];
    if constexpr (GATE) {
#pragma unroll
        for (int k = 0; k < 9; ++k) wv[k] = ld(a.w + k);
    }
    auto elem = [](int u) {
        return PAIR ? 2 * (int)threadIdx.x + u : (int)threadIdx.x + u * kTriaThreads;
    };
    float xr[EPT], bl[EPT], bp[EPT], tr[EPT], gs[EPT], bias_u[EPT], tw_u[EPT];
    int t_u[EPT], h_u[EPT];
    int64_t b_u[EPT];
    if constexpr (PAIR) {
        // cnt is even (n is): a pair is whole, and a pair lies in one row (h even)
        const int i0 = elem(0);
        const int64_t e = e0 + (i0 < cnt ? i0 : cnt - 2);
        const int64_t bt = e / a.H;
        const int h = (int)(e - bt * a.H);
        const int t = (int)(bt % a.T_);
        const int64_t b = bt / a.T_;
        RowIO<T, 2>::load(a.r + e, xr);
        RowIO<T, 2>::load(a.beta + e, bl);
        RowIO<T, 2>::load(a.beta + (t > 0 ? e - a.H : e), bp);   // the previous token's beta
        RowIO<T, 2>::load(a.trace + b * a.H + h, tr);            // the carried phase (t == 0)
        if constexpr (SAME_GATE) {
            gs[0] = gs[1] = 0.0f;
        } else {
            RowIO<T, 2>::load(a.gsrc + e, gs);
        }
        RowIO<float, 2>::load(a.bias + h, bias_u);
        RowIO<float, 2>::load(a.trace_w + h, tw_u);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            t_u[u] = t;
            h_u[u] = h + u;
            b_u[u] = b;
        }
    } else {
#pragma unroll
        for (int u = 0; u < EPT; ++u) {
            const int idx = elem(u);
            const int64_t e = e0 + (idx < cnt ? idx : cnt - 1);
            const int64_t bt = e / a.H;
            const int h = (int)(e - bt * a.H);
            const int t = (int)(bt % a.T_);
            const int64_t b = bt / a.T_;
            xr[u] = ld(a.r + e);
            bl[u] = ld(a.beta + e);
            bp[u] = ld(a.beta + (t > 0 ? e - a.H : e));   // the previous token's beta
            tr[u] = ld(a.trace + b * a.H + h);              // the carried phase (t == 0)
            gs[u] = SAME_GATE ? 0.0f : ld(a.gsrc + e);
            bias_u[u] = a.bias[h];
            tw_u[u] = a.trace_w[h];
            t_u[u] = t;
            h_u[u] = h;
            b_u[u] = b;
        }
    }
    if constexpr (MODE == 1) {
        stg.commit(tile, a.prev + e0 * 9, cnt * 9);
        lds_barrier();
    }
    float pre[EPT][9];
    float act_u[EPT], s0_u[EPT], p_u[EPT];
#pragma unroll
    for (int u = 0; u < EPT; ++u) {
        const int idx = elem(u);
        const int64_t e = e0 + idx;
        if (idx < cnt) {
            const int h = h_u[u], t = t_u[u];
            const int64_t b = b_u[u];
            // Paraplex chain (as paraplex_chunk_kernel / paraplex_forward_kernel)
            const float x = xr[u];
            const float bv = bias_u[u];
            const float s0 = phase_of(bl[u] + bv);
            const float prevs = t == 0 ? tr[u] : phase_of(bp[u] + bv);
            const float raw = fmaf(prevs, tw_u[u], s0);
            const float sv = raw * frsq(fmaf(raw, raw, 1.0f));
            float amp, gate;
            softplus_gate<!std::is_same<T, bf16_t>::value>(SAME_GATE ? x : gs[u], a.m, amp, gate);
            const float act = fmaf(amp, sv, x) * gate;
            T ts, to;
            st(&ts, sv);
            st(&to, act);
            act_u[u] = act;
            s0_u[u] = s0;
            if constexpr (!PAIR) {
                a.act[e] = to;
                if (t == a.T_ - 1) st(a.next_trace + b * a.H + h, s0);
            }
            // Tria depth op on (R, I, O) as stored
            float mt[9];
            float* pr = pre[u];
            carrier9<AXIS>(x, ld(&ts), ld(&to), a.alpha, mt);
            if constexpr (MODE == 1) {
                float cp[9];
#pragma unroll
                for (int k = 0; k < 9; ++k) cp[k] = tile[idx * 9 + k];
                mm3(mt, cp, pr);
            } else if constexpr (MODE == 2) {
                if (t == 0 && a.valid[b] != 0) {
                    float sd[9];
#pragma unroll
                    for (int k = 0; k < 9; ++k) sd[k] = ld(a.seed + (b * a.H + h) * 9 + k);
                    mm3(mt, sd, pr);
                } else {
#pragma unroll
                    for (int k = 0; k < 9; ++k) pr[k] = mt[k];
                }
            } else {
#pragma unroll
                for (int k = 0; k < 9; ++k) pr[k] = mt[k];
            }
            const float inv = 1.0f / rms9(pr);
#pragma unroll
            for (int k = 0; k < 9; ++k) pr[k] *= inv;
            if constexpr (GATE) {
                float pv = 0.0f;
#pragma unroll
                for (int k = 0; k < 9; ++k) pv = fmaf(pr[k], wv[k], pv);
                p_u[u] = pv;
                if constexpr (!PAIR) st(a.p_out + e, pv);
            }
        }
    }
    if constexpr (PAIR) {
        if (elem(0) < cnt) {
            const int64_t e = e0 + elem(0);
            RowIO<T, 2>::store(a.act + e, act_u);
            if (t_u[0] == a.T_ - 1) RowIO<T, 2>::store(a.next_trace + b_u[0] * a.H + h_u[0], s0_u);
            if constexpr (GATE) RowIO<T, 2>::store(a.p_out + e, p_u);
        }
    }
    if constexpr (MODE == 1) lds_barrier();  // everyone has read tile
#pragma unroll
    for (int u = 0; u < EPT; ++u) {
        const int idx = elem(u);
        if (idx < cnt) {
#pragma unroll
            for (int k = 0; k < 9; ++k) tile[idx * 9 + k] = pre[u][k];
        }
    }
    lds_barrier();
    stage_out(a.carry_out + e0 * 9, tile, cnt * 9);
}

template <typename T>
__global__ void __launch_bounds__(kTriaThreads)
gate_slot_mix_kernel(const T* __restrict__ carry, const T* __restrict__ w, T* __restrict__ p,
                     int64_t n) {
    __shared__ float tile[kTriaThreads * 9];
    const int64_t e0 = (int64_t)blockIdx.x * kTriaThreads;
    const int cnt = (int)((n - e0) < kTriaThreads ? (n - e0) : kTriaThreads);
    stage_in(tile, carry + e0 * 9, cnt * 9);
    __syncthreads();
    if (threadIdx.x < cnt) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 9; ++k) acc = fmaf(tile[threadIdx.x * 9 + k], ld(w + k), acc);
        st(p + e0 + threadIdx.x, acc);
    }
}

// One block per row: softmax over H of <score_w, vec C_h>; each thread keeps
// an online (max, sum, 9-slot) state over its h's, then the block merges.
template <typename T>
__global__ void __launch_bounds__(kTriaThreads)
slot_pool_kernel(const T* __restrict__ carry, const T* __restrict__ score_w,
                 T* __restrict__ pooled, T* __restrict__ lse, int64_t H) {
    __shared__ float red[kTriaThreads / 64][11];
    const int64_t row = blockIdx.x;
    const T* base = carry + row * H * 9;
    float sw[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) sw[k] = ld(score_w + k);
    float m = -INFINITY, l = 0.0f, acc[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) acc[k] = 0.0f;
    for (int64_t h = threadIdx.x; h < H; h += blockDim.x) {
        float c[9];
        float sc = 0.0f;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            c[k] = ld(base + h * 9 + k);
            sc = fmaf(c[k], sw[k], sc);
        }
        const float mn = fmaxf(m, sc);
        const float corr = expf(m - mn);
        const float pe = expf(sc - mn);
        l = l * corr + pe;
#pragma unroll
        for (int k = 0; k < 9; ++k) acc[k] = fmaf(pe, c[k], acc[k] * corr);
        m = mn;
    }
    // merge across the wave
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
    const int wid = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        red[wid][0] = m;
        red[wid][1] = l;
#pragma unroll
        for (int k = 0; k < 9; ++k) red[wid][2 + k] = acc[k];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int nw = blockDim.x >> 6;
        float M = -INFINITY;
        for (int q = 0; q < nw; ++q) M = fmaxf(M, red[q][0]);
        float L = 0.0f, A[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
        for (int q = 0; q < nw; ++q) {
            if (red[q][0] == -INFINITY) continue;
            const float c = expf(red[q][0] - M);
            L = fmaf(red[q][1], c, L);
            for (int k = 0; k < 9; ++k) A[k] = fmaf(red[q][2 + k], c, A[k]);
        }
        const float inv = 1.0f / L;
        for (int k = 0; k < 9; ++k) st(pooled + row * 9 + k, A[k] * inv);
        if (lse != nullptr) st(lse + row, logf(L) + M);
    }
}

// One thread per (b,h) stream, sequential over T.  The loads of the next
// kPrefetch local matrices are issued before the current one is consumed.
constexpr int kPrefetch = 4;

template <typename T, bool FULL>
__global__ void __launch_bounds__(kTriaThreads)
temporal_carry_kernel(const T* __restrict__ depth, const uint8_t* __restrict__ reset,
                      const T* __restrict__ initial, const uint8_t* __restrict__ init_valid,
                      T* __restrict__ endpoint, float* __restrict__ end_f32,
                      float* __restrict__ doc, float* __restrict__ scale_out, int64_t B, int64_t T_,
                      int64_t H) {
    const int64_t sid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (sid >= B * H) return;
    const int64_t b = sid / H;
    const int64_t h = sid - b * H;
    float acc[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    bool have = false;
    if (initial != nullptr) {
        have = init_valid == nullptr || init_valid[b] != 0;
        if (have) {
#pragma unroll
            for (int k = 0; k < 9; ++k) acc[k] = ld(initial + sid * 9 + k);
        }
    }
    const int64_t step = H * 9;
    const T* p = depth + (b * T_ * H + h) * 9;
    float buf[kPrefetch][9];
#pragma unroll
    for (int u = 0; u < kPrefetch; ++u)
        if (u < T_) {
#pragma unroll
            for (int k = 0; k < 9; ++k) buf[u][k] = ld(p + u * step + k);
        }
    for (int64_t t0 = 0; t0 < T_; t0 += kPrefetch) {
#pragma unroll
        for (int u = 0; u < kPrefetch; ++u) {
            const int64_t t = t0 + u;
            if (t < T_) {
                float loc[9], pre[9];
#pragma unroll
                for (int k = 0; k < 9; ++k) loc[k] = buf[u][k];
                const int64_t tn = t + kPrefetch;
                if (tn < T_) {
#pragma unroll
                    for (int k = 0; k < 9; ++k) buf[u][k] = ld(p + tn * step + k);
                }
                const bool restart = !have || reset[b * T_ + t] != 0;
                if (restart) {
#pragma unroll
                    for (int k = 0; k < 9; ++k) pre[k] = loc[k];
                } else {
                    mm3(loc, acc, pre);
                }
                const float sc = rms9(pre);
                const float inv = 1.0f / sc;
#pragma unroll
                for (int k = 0; k < 9; ++k) acc[k] = pre[k] * inv;
                have = true;
                if constexpr (FULL) {
                    const int64_t e = (b * T_ + t) * H + h;
                    if (doc != nullptr) {
#pragma unroll
                        for (int k = 0; k < 9; ++k) doc[e * 9 + k] = acc[k];
                    }
                    if (scale_out != nullptr) scale_out[e] = sc;
                }
            }
        }
    }
    if constexpr (!FULL) {
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            if (endpoint != nullptr) st(endpoint + sid * 9 + k, acc[k]);
            if (end_f32 != nullptr) end_f32[sid * 9 + k] = acc[k];
        }
    }
}

// Endpoint of the temporal carry with each chain's first T-1 steps split over
// four lanes of a wave (lanes c, c+16, c+32, c+48 hold chain c's quarters): a
// quarter composes its steps as the sequential form does (restart on a reset,
// normalised after every product), the quarters are combined later ones on
// the left, r = q3 (x) q2 (x) q1 (x) q0 with q (x) r = q when q saw a reset,
// else normalise(q r), and quarter 0's lane takes the last step from r as the
// sequential form does.  The normalisation divides by a positive scalar, so r
// has the direction of the sequential state before the last step; only the
// last normalisation sets the magnitude (the eps inside the rms matters there
// when a product is small, so it stays a sequential step).  At the chunked
// prefill's B x H = 98304 chains the sequential form runs 128-step dependency
// chains at 1.5 waves per SIMD.
// One step's 9-element carrier records of CH adjacent chains (h, h+1, ..),
// as floats: with 16-bit storage and CH = 2 the pair's 36 bytes start on a
// 4-byte boundary (h even, H even), so they load as nine dwords instead of
// eighteen 2-byte loads.
template <typename T, int CH>
__device__ __forceinline__ void load_records(const T* p, float (&v)[CH][9]) {
    if constexpr (CH == 2 && sizeof(T) == 2) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            const uint32_t x = w[k];
            T lo, hi;
            lo.x = (uint16_t)(x & 0xffffu);
            hi.x = (uint16_t)(x >> 16);
            const int e0 = 2 * k, e1 = 2 * k + 1;
            v[e0 / 9][e0 % 9] = ld(&lo);
            v[e1 / 9][e1 % 9] = ld(&hi);
        }
    } else {
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int k = 0; k < 9; ++k) v[c][k] = ld(p + c * 9 + k);
    }
}

// Endpoint of the temporal carry with each chain's first T-1 steps split over
// four lanes of a wave (lanes c, c+16, c+32, c+48 hold chain group c's
// quarters; a lane carries CH adjacent chains, which share b and so their
// resets): a quarter composes its steps as the sequential form does (restart
// on a reset, normalised after every product), the quarters are combined
// later ones on the left, r = q3 (x) q2 (x) q1 (x) q0 with q (x) r = q when q
// saw a reset, else normalise(q r), and quarter 0's lane takes the last step
// from r as the sequential form does.  The normalisation divides by a
// positive scalar, so r has the direction of the sequential state before the
// last step; only the last normalisation sets the magnitude (the eps inside
// the rms matters there when a product is small, so it stays a sequential
// step).  At the chunked prefill's B x H = 98304 chains the sequential form
// runs 128-step dependency chains at 1.5 waves per SIMD.
template <typename T, int CH>
__global__ void __launch_bounds__(kTriaThreads)
temporal_endpoint_quarters_kernel(const T* __restrict__ depth, const uint8_t* __restrict__ reset,
                                  const T* __restrict__ initial, const uint8_t* __restrict__ init_valid,
                                  T* __restrict__ endpoint, float* __restrict__ end_f32, int64_t B,
                                  int64_t T_, int64_t H) {
    const int lane = threadIdx.x & 63, qt = lane >> 4;
    const int64_t groups = B * H / CH;              // H % CH == 0 (host check)
    const int64_t gid = (((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6) * 16 + (lane & 15);
    const bool live = gid < groups;
    // no early exit: the whole wave takes part in the combining shuffles
    const int64_t c0 = (live ? gid : groups - 1) * CH;   // first chain (b, h) of the group
    const int64_t b = c0 / H, h = c0 - b * H;
    const int64_t L = (T_ + 3) / 4;
    const int64_t t_begin = min((int64_t)qt * L, T_ - 1), t_end = min(t_begin + L, T_ - 1);
    float acc[CH][9];
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int k = 0; k < 9; ++k) acc[c][k] = 0.0f;
    bool have = false;
    bool cut = qt == 0;     // this quarter's result ignores everything before it
    if (qt == 0 && initial != nullptr && (init_valid == nullptr || init_valid[b] != 0)) {
        load_records<T, CH>(initial + c0 * 9, acc);
        have = true;
    }
    const int64_t step = H * 9;
    const T* p = depth + (b * T_ * H + h) * 9;
    float buf[kPrefetch][CH][9];
#pragma unroll
    for (int u = 0; u < kPrefetch; ++u)
        if (t_begin + u < t_end) load_records<T, CH>(p + (t_begin + u) * step, buf[u]);
    for (int64_t t0 = t_begin; t0 < t_end; t0 += kPrefetch) {
#pragma unroll
        for (int u = 0; u < kPrefetch; ++u) {
            const int64_t t = t0 + u;
            if (t < t_end) {
                float loc[CH][9];
#pragma unroll
                for (int c = 0; c < CH; ++c)
#pragma unroll
                    for (int k = 0; k < 9; ++k) loc[c][k] = buf[u][c][k];
                const int64_t tn = t + kPrefetch;
                if (tn < t_end) load_records<T, CH>(p + tn * step, buf[u]);
                const bool rs = reset[b * T_ + t] != 0;
                cut = cut || rs;
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    float pre[9];
                    if (!have || rs) {
#pragma unroll
                        for (int k = 0; k < 9; ++k) pre[k] = loc[c][k];
                    } else {
                        mm3(loc[c], acc[c], pre);
                    }
                    const float inv = 1.0f / rms9(pre);
#pragma unroll
                    for (int k = 0; k < 9; ++k) acc[c][k] = pre[k] * inv;
                }
                have = true;
            }
        }
    }
    // quarter 0's lane combines: q1, q2, q3 in order, each from its lane
    float r[CH][9];
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int k = 0; k < 9; ++k) r[c][k] = acc[c][k];
    bool have_r = have;
#pragma unroll
    for (int j = 1; j < 4; ++j) {
        float qv[CH][9];
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int k = 0; k < 9; ++k) qv[c][k] = __shfl(acc[c][k], lane + 16 * j, 64);
        const int qcut = __shfl((int)cut, lane + 16 * j, 64);
        const int qhave = __shfl((int)have, lane + 16 * j, 64);
        if (qt == 0 && qhave) {
            have_r = true;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                if (qcut) {
#pragma unroll
                    for (int k = 0; k < 9; ++k) r[c][k] = qv[c][k];
                } else {
                    float pre[9];
                    mm3(qv[c], r[c], pre);
                    const float inv = 1.0f / rms9(pre);
#pragma unroll
                    for (int k = 0; k < 9; ++k) r[c][k] = pre[k] * inv;
                }
            }
        }
    }
    // the last step
    {
        const int64_t tl = T_ - 1;
        float loc[CH][9];
        load_records<T, CH>(p + tl * step, loc);
        const bool rl = reset[b * T_ + tl] != 0;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            float pre[9];
            if (!have_r || rl) {
#pragma unroll
                for (int k = 0; k < 9; ++k) pre[k] = loc[c][k];
            } else {
                mm3(loc[c], r[c], pre);
            }
            const float inv = 1.0f / rms9(pre);
#pragma unroll
            for (int k = 0; k < 9; ++k) r[c][k] = pre[k] * inv;
        }
    }
    if (qt == 0 && live) {
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                if (endpoint != nullptr) st(endpoint + (c0 + c) * 9 + k, r[c][k]);
                if (end_f32 != nullptr) end_f32[(c0 + c) * 9 + k] = r[c][k];
            }
    }
}

// The last block of a chunk in the chunked prefill in one pass: the Paraplex
// chain and the Tria depth step of paraplex_tria_kernel (carried records in,
// no gate) for every (b, t, h), and the temporal carry endpoint over the
// chunk's tokens of the carries it produces (rounded to the storage type, as
// temporal_endpoint_quarters_kernel reads them back), so the carries are
// never stored (the sequence of loomformer.py:2856-2885, :3588-3617 and the
// chunk endpoint of :3834-3850).
// Block: batch row b, 64 CH hidden columns (lane l takes columns h0 + CH l ..
// + CH - 1; with CH = 2 a pair's 16-bit operands and 9-value records load as
// words: 127-128 us at the prefill's [32, 128, 3072] in bf16, against 141-142
// with one column per lane and 5 waves per SIMD); wave q takes quarter q of
// the tokens.  Over its quarter a lane runs the
// per-element chain token by token, the next tokens' operands in flight, and
// composes the temporal quarter as the endpoint kernel's lane does (restart
// on a reset, normalised after every product) from the same rounded values;
// wave 0 then combines the four quarters in the endpoint kernel's order and
// takes the last token's step, so the endpoint is the same bits.
template <typename T>
struct PxTriaEndArgs {
    const T* r;            // R [B, T, H]
    const T* gsrc;         // the amplitude source (R itself, or gate_proj(u))
    const T* beta;         // beta_linear [B, T, H]
    const float* bias;     // [H]
    const T* trace;        // [B, H]
    const float* trace_w;  // [H]
    const T* prev;         // carried depth records [B, T, H, 9]
    const uint8_t* reset;  // [B, T]
    const T* initial;      // [B, H, 9] temporal state before t = 0, or null
    const uint8_t* init_valid;
    T* act;                // O [B, T, H]
    T* next_trace;         // [B, H]
    T* endpoint;           // [B, H, 9]
    float* end_f32;        // [B, H, 9] or null
    int T_, H;
    float m, alpha;
};

constexpr int kPxEndPrefetch = 2;   // tokens of operands in flight per lane
constexpr int kPxEndCols = 2;       // hidden columns per lane

// Operands of CH adjacent columns held as the words loaded (16-bit types
// stay packed until used, so the loads of a prefetched token are not waited
// for where they are issued): CH elements, and their CH 9-value records.
// With CH = 2 and 16-bit types the pair and its 36 record bytes are 4-byte
// aligned (h even), so they load as one and nine dwords.
template <typename T, int CH>
struct RawCols {
    static constexpr bool WORDS = CH == 2 || sizeof(T) == 4;
    static constexpr int NW = WORDS ? (int)sizeof(T) * CH / 4 : CH;
    uint32_t w[NW];
    __device__ __forceinline__ void load(const T* p) {
        if constexpr (WORDS) {
#pragma unroll
            for (int k = 0; k < NW; ++k) w[k] = reinterpret_cast<const uint32_t*>(p)[k];
        } else {
#pragma unroll
            for (int k = 0; k < CH; ++k) w[k] = p[k].x;
        }
    }
    __device__ __forceinline__ void to_float(float v[CH]) const {
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            if constexpr (sizeof(T) == 4) {
                v[e] = __uint_as_float(w[e]);
            } else {
                const uint32_t x = WORDS ? (e % 2 == 0 ? (w[e / 2] & 0xffffu) : (w[e / 2] >> 16)) : w[e];
                const T y{(uint16_t)x};
                v[e] = ld(&y);
            }
        }
    }
};
template <typename T, int CH>
struct RawRecs {
    static constexpr bool WORDS = CH == 2 || sizeof(T) == 4;
    static constexpr int NW = WORDS ? (int)sizeof(T) * 9 * CH / 4 : 9 * CH;
    uint32_t w[NW];
    __device__ __forceinline__ void load(const T* p) {
        if constexpr (WORDS) {
#pragma unroll
            for (int k = 0; k < NW; ++k) w[k] = reinterpret_cast<const uint32_t*>(p)[k];
        } else {
#pragma unroll
            for (int k = 0; k < NW; ++k) w[k] = p[k].x;
        }
    }
    __device__ __forceinline__ void to_float(float (&v)[CH][9]) const {
#pragma unroll
        for (int e = 0; e < 9 * CH; ++e) {
            if constexpr (sizeof(T) == 4) {
                v[e / 9][e % 9] = __uint_as_float(w[e]);
            } else {
                const uint32_t x = WORDS ? (e % 2 == 0 ? (w[e / 2] & 0xffffu) : (w[e / 2] >> 16)) : w[e];
                const T y{(uint16_t)x};
                v[e / 9][e % 9] = ld(&y);
            }
        }
    }
};

template <typename T, int AXIS, bool SAME_GATE, int CH>
__global__ void __launch_bounds__(kTriaThreads)
paraplex_tria_endpoint_kernel(PxTriaEndArgs<T> a) {
    constexpr int PF = kPxEndPrefetch;
    constexpr int REC = CH * 9 + 2;              // a lane's quarter state: CH records, have, cut
    __shared__ float xch[4][REC][64];            // quarters' states, [0] the last token's records
    const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
    const int T_ = a.T_, H = a.H;
    const int64_t b = blockIdx.y;
    const int hc = (blockIdx.x * 64 + lane) * CH; // this lane's first column (H % CH == 0)
    const bool live = hc < H;
    const int h = live ? hc : H - CH;            // clamped: loads stay in range
    const int L = (T_ + 3) / 4;
    const int ta = min(q * L, T_), tb = min(ta + L, T_);
    const int64_t row0 = b * (int64_t)T_;        // token index of (b, 0)
    float bv[CH], tw[CH];
    RowIO<float, CH>::load(a.bias + h, bv);
    RowIO<float, CH>::load(a.trace_w + h, tw);
    // the base phase of the token before ta: the carried trace, or that token's beta
    float prevs[CH];
    {
        float v[CH];
        if (ta == 0) {
            RowIO<T, CH>::load(a.trace + b * H + h, prevs);
        } else {
            RowIO<T, CH>::load(a.beta + (row0 + ta - 1) * H + h, v);
#pragma unroll
            for (int c = 0; c < CH; ++c) prevs[c] = phase_of(v[c] + bv[c]);
        }
    }
    // quarter state, as temporal_endpoint_quarters_kernel's lane keeps it
    float acc[CH][9];
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int k = 0; k < 9; ++k) acc[c][k] = 0.0f;
    bool have = false, cut = q == 0;
    if (q == 0 && a.initial != nullptr && (a.init_valid == nullptr || a.init_valid[b] != 0)) {
        load_records<T, CH>(a.initial + (b * H + h) * 9, acc);
        have = true;
    }
    float last[CH][9];                            // the chunk's last carries (wave holding T-1)
    // operands of token t into ring slot p
    RawCols<T, CH> xr[PF], bl[PF], gs[PF];
    RawRecs<T, CH> cp[PF];
    auto fetch = [&](int p, int t) {
        const int64_t e = (row0 + t) * H + h;
        xr[p].load(a.r + e);
        bl[p].load(a.beta + e);
        if constexpr (!SAME_GATE) gs[p].load(a.gsrc + e);
        cp[p].load(a.prev + e * 9);
    };
#pragma unroll
    for (int p = 0; p < PF; ++p)
        if (ta + p < tb) fetch(p, ta + p);
    for (int t0 = ta; t0 < tb; t0 += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int t = t0 + p;
            if (t >= tb) break;
            float x[CH], be[CH], g[CH], cpv[CH][9];
            xr[p].to_float(x);
            bl[p].to_float(be);
            if constexpr (SAME_GATE) {
#pragma unroll
                for (int c = 0; c < CH; ++c) g[c] = x[c];
            } else {
                gs[p].to_float(g);
            }
            cp[p].to_float(cpv);
            // the slot's values unpacked into registers of their own before
            // its refill is issued
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                asm volatile("" : "+v"(x[c]), "+v"(be[c]), "+v"(g[c]));
#pragma unroll
                for (int k = 0; k < 9; ++k) asm volatile("" : "+v"(cpv[c][k]));
            }
            if (t + PF < tb) fetch(p, t + PF);
            float ao[CH], s0v[CH], cr[CH][9];
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const float s0 = phase_of(be[c] + bv[c]);
                const float raw = fmaf(prevs[c], tw[c], s0);
                const float sv = raw * frsq(fmaf(raw, raw, 1.0f));
                float amp, gate;
                softplus_gate<!std::is_same<T, bf16_t>::value>(g[c], a.m, amp, gate);
                const float act = fmaf(amp, sv, x[c]) * gate;
                ao[c] = act;
                s0v[c] = s0;
                prevs[c] = s0;
                float mt[9], pr[9];
                carrier9<AXIS>(x[c], round_to<T>(sv), round_to<T>(act), a.alpha, mt);
                mm3(mt, cpv[c], pr);
                const float inv = 1.0f / rms9(pr);
#pragma unroll
                for (int k = 0; k < 9; ++k) cr[c][k] = round_to<T>(pr[k] * inv);
            }
            const int64_t e = (row0 + t) * H + h;
            if (live) {
                RowIO<T, CH>::store(a.act + e, ao);
                if (t == T_ - 1) RowIO<T, CH>::store(a.next_trace + b * H + h, s0v);
            }
            if (t == T_ - 1) {
#pragma unroll
                for (int c = 0; c < CH; ++c)
#pragma unroll
                    for (int k = 0; k < 9; ++k) last[c][k] = cr[c][k];
            } else {
                const bool rs = a.reset[row0 + t] != 0;
                cut = cut || rs;
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    float pre[9];
                    if (!have || rs) {
#pragma unroll
                        for (int k = 0; k < 9; ++k) pre[k] = cr[c][k];
                    } else {
                        mm3(cr[c], acc[c], pre);
                    }
                    const float inv = 1.0f / rms9(pre);
#pragma unroll
                    for (int k = 0; k < 9; ++k) acc[c][k] = pre[k] * inv;
                }
                have = true;
            }
        }
    }
    // quarters 1..3 (and the last token's records, from the wave that holds
    // T-1) to wave 0 through LDS
    const int qlast = (T_ - 1) / L;
    if (q > 0) {
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int k = 0; k < 9; ++k) xch[q][c * 9 + k][lane] = acc[c][k];
        xch[q][9 * CH][lane] = have ? 1.0f : 0.0f;
        xch[q][9 * CH + 1][lane] = cut ? 1.0f : 0.0f;
    }
    if (q == qlast && q > 0) {
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int k = 0; k < 9; ++k) xch[0][c * 9 + k][lane] = last[c][k];
    }
    __syncthreads();
    if (q != 0) return;
    if (qlast > 0) {
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int k = 0; k < 9; ++k) last[c][k] = xch[0][c * 9 + k][lane];
    }
    float rr[CH][9];
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int k = 0; k < 9; ++k) rr[c][k] = acc[c][k];
    bool have_r = have;
#pragma unroll
    for (int j = 1; j < 4; ++j) {
        if (xch[j][9 * CH][lane] == 0.0f) continue;   // quarter j saw no step
        have_r = true;
        const bool qcut = xch[j][9 * CH + 1][lane] != 0.0f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            float qv[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) qv[k] = xch[j][c * 9 + k][lane];
            if (qcut) {
#pragma unroll
                for (int k = 0; k < 9; ++k) rr[c][k] = qv[k];
            } else {
                float pre[9];
                mm3(qv, rr[c], pre);
                const float inv = 1.0f / rms9(pre);
#pragma unroll
                for (int k = 0; k < 9; ++k) rr[c][k] = pre[k] * inv;
            }
        }
    }
    // the last step
    const bool rl = a.reset[row0 + T_ - 1] != 0;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        float pre[9];
        if (!have_r || rl) {
#pragma unroll
            for (int k = 0; k < 9; ++k) pre[k] = last[c][k];
        } else {
            mm3(last[c], rr[c], pre);
        }
        const float inv = 1.0f / rms9(pre);
#pragma unroll
        for (int k = 0; k < 9; ++k) rr[c][k] = pre[k] * inv;
    }
    if (live) {
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                st(a.endpoint + (b * H + h + c) * 9 + k, rr[c][k]);
                if (a.end_f32 != nullptr) a.end_f32[(b * H + h + c) * 9 + k] = rr[c][k];
            }
    }
}

template <typename T>
__global__ void __launch_bounds__(kTriaThreads)
polarm_kernel(const T* __restrict__ in, T* __restrict__ out, const uint8_t* __restrict__ mask,
              int64_t n, int64_t per_mask, float beta, float eps) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    float M[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) M[k] = ld(in + e * 9 + k);
    if (mask == nullptr || mask[e / per_mask] != 0) polarm9(M, beta, eps);
#pragma unroll
    for (int k = 0; k < 9; ++k) st(out + e * 9 + k, M[k]);
}

// One block per query row: scores over the K keys (one wave per key at a
// time, lanes over D), masked softmax in LDS, then out = sum_j w_j v_j.
constexpr int kCaMaxK = 1024;

// k/v row j of batch b at b*kv_stride_b + j*D; allowed row r at r*allowed_stride.
// With a residual, out = residual + gamma * attention (TriaFinalCrossAttention
// adds gamma*out to its input, tria.py:1556-1557, :1593-1595).
template <typename T>
__global__ void __launch_bounds__(256)
final_ca_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                int64_t kv_stride_b, const uint8_t* __restrict__ allowed, int64_t allowed_stride,
                const T* __restrict__ residual, float gamma, T* __restrict__ out,
                float* __restrict__ lse, int64_t T_, int64_t K, const int64_t* __restrict__ k_dev,
                int64_t D, float scale) {
    __shared__ float wts[kCaMaxK];
    __shared__ float red[2];
    if (k_dev != nullptr) K = *k_dev < K ? *k_dev : K;   // graph replay: key count on the device
    const int64_t row = blockIdx.x;
    const int64_t b = row / T_;
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const T* qr = q + row * D;
    for (int64_t j = wid; j < K; j += nw) {
        float s = -INFINITY;
        if (allowed[row * allowed_stride + j]) {
            const T* kr = k + b * kv_stride_b + j * D;
            float dot = 0.0f;
            for (int64_t d = lane; d < D; d += 64) dot = fmaf(ld(qr + d), ld(kr + d), dot);
            s = wave_sum(dot) * scale;
        }
        if (lane == 0) wts[j] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float mx = -INFINITY;
        for (int64_t j = 0; j < K; ++j) mx = fmaxf(mx, wts[j]);
        float sum = 0.0f;
        if (mx == -INFINITY) {
            for (int64_t j = 0; j < K; ++j) wts[j] = 0.0f;
        } else {
            for (int64_t j = 0; j < K; ++j) {
                const float e = (wts[j] == -INFINITY) ? 0.0f : expf(wts[j] - mx);
                wts[j] = e;
                sum += e;
            }
            const float inv = 1.0f / sum;
            for (int64_t j = 0; j < K; ++j) wts[j] *= inv;
        }
        red[0] = mx;
        red[1] = sum;
    }
    __syncthreads();
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
        float a = 0.0f;
        for (int64_t j = 0; j < K; ++j) a = fmaf(wts[j], ld(v + b * kv_stride_b + j * D + d), a);
        if (residual != nullptr) a = ld(residual + row * D + d) + gamma * a;
        st(out + row * D + d, a);
    }
    if (lse != nullptr && threadIdx.x == 0)
        lse[row] = red[0] == -INFINITY ? -INFINITY : red[0] + logf(red[1]);
}

// Vector form for D % 8 == 0, D <= 1536 and 16-byte aligned rows: q is held as
// 8-element chunks (lane l: chunks l, l+64, l+128), keys are scored by the
// waves two at a time with 16-byte loads, wave 0 forms the softmax with its
// lanes over the keys, and P.V runs one 8-element chunk per thread with the
// key loop unrolled so several value rows are in flight.
constexpr int kCaChunks = 3;   // 8-element chunks of q per lane (D <= 3*64*8)

template <typename T>
__global__ void __launch_bounds__(256)
final_ca_vec_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                    int64_t kv_stride_b, const uint8_t* __restrict__ allowed,
                    int64_t allowed_stride, const T* __restrict__ residual, float gamma,
                    T* __restrict__ out, float* __restrict__ lse, int64_t T_, int64_t K,
                    const int64_t* __restrict__ k_dev, int D, float scale) {
    __shared__ float wts[kCaMaxK];
    __shared__ float red[2];
    if (k_dev != nullptr) K = *k_dev < K ? *k_dev : K;   // graph replay: key count on the device
    const int64_t row = blockIdx.x;
    const int64_t b = row / T_;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int nch = D / 8;
    float qf[kCaChunks][8];
#pragma unroll
    for (int c = 0; c < kCaChunks; ++c) {
        const int ch = lane + 64 * c;
        if (ch < nch) Vec8<T>::load(q + row * D + ch * 8, qf[c]);
        else
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[c][e] = 0.0f;
    }
    const T* kb = k + b * kv_stride_b;
    for (int64_t j0 = wid; j0 < K; j0 += 8) {            // keys j0 and j0 + 4 per wave
        float dot[2] = {0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t j = j0 + 4 * u;
            if (j >= K) continue;
#pragma unroll
            for (int c = 0; c < kCaChunks; ++c) {
                const int ch = lane + 64 * c;
                if (ch >= nch) continue;
                float kv[8];
                Vec8<T>::load(kb + j * D + ch * 8, kv);
#pragma unroll
                for (int e = 0; e < 8; ++e) dot[u] = fmaf(qf[c][e], kv[e], dot[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t j = j0 + 4 * u;
            const float s = wave_sum(dot[u]) * scale;
            if (lane == 0 && j < K) wts[j] = allowed[row * allowed_stride + j] ? s : -INFINITY;
        }
    }
    __syncthreads();
    if (wid == 0) {
        float mx = -INFINITY;
        for (int64_t j = lane; j < K; j += 64) mx = fmaxf(mx, wts[j]);
        mx = wave_max(mx);
        float sum = 0.0f;
        for (int64_t j = lane; j < K; j += 64) {
            const float e = (mx == -INFINITY || wts[j] == -INFINITY) ? 0.0f : fexp(wts[j] - mx);
            wts[j] = e;
            sum += e;
        }
        sum = wave_sum(sum);
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (int64_t j = lane; j < K; j += 64) wts[j] *= inv;
        if (lane == 0) {
            red[0] = mx;
            red[1] = sum;
        }
    }
    __syncthreads();
    const T* vb = v + b * kv_stride_b;
    for (int ch = threadIdx.x; ch < nch; ch += blockDim.x) {
        float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        int64_t j = 0;
        for (; j + 4 <= K; j += 4) {
            float vv[4][8];
#pragma unroll
            for (int u = 0; u < 4; ++u) Vec8<T>::load(vb + (j + u) * D + ch * 8, vv[u]);
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int e = 0; e < 8; ++e) a[e] = fmaf(wts[j + u], vv[u][e], a[e]);
        }
        for (; j < K; ++j) {
            float vv[8];
            Vec8<T>::load(vb + j * D + ch * 8, vv);
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = fmaf(wts[j], vv[e], a[e]);
        }
        if (residual != nullptr) {
            float rr[8];
            Vec8<T>::load(residual + row * D + ch * 8, rr);
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = rr[e] + gamma * a[e];
        }
        Vec8<T>::store(out + row * D + ch * 8, a);
    }
    if (lse != nullptr && threadIdx.x == 0)
        lse[row] = red[0] == -INFINITY ? -INFINITY : red[0] + logf(red[1]);
}

// Short key lists (16-bit types, K <= kCaRowKeys, D % 8 == 0, D <= 1024): every load of the
// row is issued before any arithmetic, so the row costs one memory round trip.
// 512 threads.  Scores: wave w holds keys w + 8i (lane l: 8-element chunks l
// and l + 64 of q and of each key).  P.V: thread t takes chunk t % 128 for the
// keys t/128 + 4i; its value rows are loaded together with the keys, and the
// four key subsets are summed through LDS.
constexpr int kCaRowKeys = 64;

// eight 16-bit elements held as one 16-byte word, to fp32
template <typename T>
__device__ __forceinline__ void unpack8(const uint4 w, float v[8]) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const T lo{(uint16_t)(u[k] & 0xffffu)}, hi{(uint16_t)(u[k] >> 16)};
        v[2 * k] = ld(&lo);
        v[2 * k + 1] = ld(&hi);
    }
}

template <typename T>
__global__ void __launch_bounds__(512)
final_ca_row_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                    int64_t kv_stride_b, const uint8_t* __restrict__ allowed,
                    int64_t allowed_stride, const T* __restrict__ residual, float gamma,
                    T* __restrict__ out, float* __restrict__ lse, int64_t T_, int64_t K,
                    const int64_t* __restrict__ k_dev, int D, float scale) {
    constexpr int KW = kCaRowKeys / 8, KS = kCaRowKeys / 4;
    __shared__ float wts[kCaRowKeys];
    __shared__ float part[4][128][9];      // [subset][chunk][8] (+1: bank spread)
    __shared__ float red[2];
    // every load first and none waiting on the device key count: keys and
    // values of all K slots the cache holds (slots past the count are read and
    // masked), q and the residual as raw words, the key mask
    const int64_t Kcap = K;
    const int64_t row = blockIdx.x;
    const int64_t b = row / T_;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int nch = D / 8;
    const T* kb = k + b * kv_stride_b;
    const T* vb = v + b * kv_stride_b;
    uint4 qw[2], kr[KW][2], vr[KS], rw;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int ch = min(lane + 64 * c, nch - 1);
        qw[c] = *reinterpret_cast<const uint4*>(q + row * D + ch * 8);
#pragma unroll
        for (int i = 0; i < KW; ++i) {
            const int64_t j = wid + 8 * i;
            if (j < Kcap) kr[i][c] = *reinterpret_cast<const uint4*>(kb + j * D + ch * 8);
        }
    }
    const int c2 = tid & 127, s2 = tid >> 7;
    {
        const int cc = min(c2, nch - 1);
#pragma unroll
        for (int i = 0; i < KS; ++i) {
            const int64_t j = s2 + 4 * i;
            if (j < Kcap) vr[i] = *reinterpret_cast<const uint4*>(vb + j * D + cc * 8);
        }
    }
    const uint8_t al = (wid == 0 && lane < Kcap) ? allowed[row * allowed_stride + lane] : 0;
    if (residual != nullptr)
        rw = *reinterpret_cast<const uint4*>(residual + row * D + min(tid, nch - 1) * 8);
    if (k_dev != nullptr) K = *k_dev < Kcap ? *k_dev : Kcap;
    float qf[2][8];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        if (lane + 64 * c < nch) {
            unpack8<T>(qw[c], qf[c]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[c][e] = 0.0f;
        }
    }
    const bool ok = wid == 0 && lane < K && al != 0;
    float rr[8];
    if (residual != nullptr) unpack8<T>(rw, rr);
#pragma unroll
    for (int i = 0; i < KW; ++i) {
        const int64_t j = wid + 8 * i;
        float dot = 0.0f;
        if (j < K) {
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                if (lane + 64 * c >= nch) continue;
                float kv[8];
                unpack8<T>(kr[i][c], kv);
#pragma unroll
                for (int e = 0; e < 8; ++e) dot = fmaf(qf[c][e], kv[e], dot);
            }
        }
        const float sc = wave_sum(dot) * scale;
        if (lane == 0 && j < K) wts[j] = sc;
    }
    __syncthreads();
    if (wid == 0) {
        const float sv = ok ? wts[lane] : -INFINITY;
        const float mx = wave_max(sv);
        const float e = (mx == -INFINITY || sv == -INFINITY) ? 0.0f : fexp(sv - mx);
        const float sum = wave_sum(e);
        if (lane < K) wts[lane] = sum > 0.0f ? e / sum : 0.0f;
        if (lane == 0) {
            red[0] = mx;
            red[1] = sum;
        }
    }
    __syncthreads();
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (c2 < nch) {
#pragma unroll
        for (int i = 0; i < KS; ++i) {
            const int64_t j = s2 + 4 * i;
            if (j >= K) continue;
            float vv[8];
            unpack8<T>(vr[i], vv);
            const float w = wts[j];
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = fmaf(w, vv[e], a[e]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) part[s2][c2][e] = a[e];
    }
    __syncthreads();
    if (tid < nch) {
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = part[0][tid][e] + part[1][tid][e] + part[2][tid][e] + part[3][tid][e];
        if (residual != nullptr) {
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = rr[e] + gamma * a[e];
        }
        Vec8<T>::store(out + row * D + tid * 8, a);
    }
    if (lse != nullptr && tid == 0)
        lse[row] = red[0] == -INFINITY ? -INFINITY : red[0] + logf(red[1]);
}

// ---------------------------------------------------------------- dispatch

template <typename T>
static int tria_depth_dispatch(const void* r, const void* i, const void* o, const void* prev,
                               const void* seed, const uint8_t* valid, const void* w,
                               void* carry_out, void* p_out, float* scale_out, int64_t B,
                               int64_t T_, int64_t H, float alpha, int axis, hipStream_t st) {
    const int64_t n = B * T_ * H;
    const dim3 grid((unsigned)ceil_div(n, kTriaThreads)), blk(kTriaThreads);
    const int mode = prev ? 1 : (seed ? 2 : 0);
    const bool gate = w != nullptr;
#define LOOM_TD_S(M, G, A, S)                                                               \
    hipLaunchKernelGGL((tria_depth_kernel<T, M, G, A, S>), grid, blk, 0, st, (const T*)r,  \
                       (const T*)i, (const T*)o, (const T*)prev, (const T*)seed, valid,    \
                       (const T*)w, (T*)carry_out, (T*)p_out, scale_out, n, T_, H, alpha)
#define LOOM_TD(M, G, A)                                     \
    if (scale_out != nullptr) { LOOM_TD_S(M, G, A, true); }  \
    else { LOOM_TD_S(M, G, A, false); }
#define LOOM_TD_AXIS(M, G)                        \
    switch (axis) {                               \
        case 0: LOOM_TD(M, G, 0); break;          \
        case 1: LOOM_TD(M, G, 1); break;          \
        default: LOOM_TD(M, G, 2); break;         \
    }
    if (mode == 0) { if (gate) { LOOM_TD_AXIS(0, true) } else { LOOM_TD_AXIS(0, false) } }
    else if (mode == 1) { if (gate) { LOOM_TD_AXIS(1, true) } else { LOOM_TD_AXIS(1, false) } }
    else { if (gate) { LOOM_TD_AXIS(2, true) } else { LOOM_TD_AXIS(2, false) } }
#undef LOOM_TD_AXIS
#undef LOOM_TD
#undef LOOM_TD_S
    return launch_status("loom_tria_depth_forward");
}

template <typename T, bool PAIR>
static int px_tria_dispatch(const PxTriaArgs<T>& a, int mode, bool gate, bool same, int axis,
                            hipStream_t st) {
    constexpr int EPT = kPxTriaPerThread;
    const dim3 grid((unsigned)ceil_div(a.n, kTriaThreads * EPT)), blk(kTriaThreads);
#define LOOM_PT(M, G, A, S) \
    hipLaunchKernelGGL((paraplex_tria_kernel<T, M, G, A, S, EPT, PAIR>), grid, blk, 0, st, a)
#define LOOM_PT_AXIS(M, G, S)                     \
    switch (axis) {                               \
        case 0: LOOM_PT(M, G, 0, S); break;       \
        case 1: LOOM_PT(M, G, 1, S); break;       \
        default: LOOM_PT(M, G, 2, S); break;      \
    }
#define LOOM_PT_SAME(M, G)                                          \
    if (same) { LOOM_PT_AXIS(M, G, true) } else { LOOM_PT_AXIS(M, G, false) }
    if (mode == 0) { if (gate) { LOOM_PT_SAME(0, true) } else { LOOM_PT_SAME(0, false) } }
    else if (mode == 1) { if (gate) { LOOM_PT_SAME(1, true) } else { LOOM_PT_SAME(1, false) } }
    else { if (gate) { LOOM_PT_SAME(2, true) } else { LOOM_PT_SAME(2, false) } }
#undef LOOM_PT_SAME
#undef LOOM_PT_AXIS
#undef LOOM_PT
    return launch_status("loom_paraplex_tria_forward");
}

template <typename T>
static int px_tria_typed(const void* r, const void* gsrc, const void* beta, const float* bias,
                         const void* trace, const float* trace_w, float m, const void* prev,
                         const void* seed, const uint8_t* valid, const void* w, void* act,
                         void* next_trace, void* carry_out, void* p_out, int64_t B, int64_t T_,
                         int64_t H, float alpha, int axis, hipStream_t st) {
    PxTriaArgs<T> a{};
    a.r = (const T*)r; a.gsrc = (const T*)gsrc; a.beta = (const T*)beta; a.bias = bias;
    a.trace = (const T*)trace; a.trace_w = trace_w; a.prev = (const T*)prev;
    a.seed = (const T*)seed; a.valid = valid; a.w = (const T*)w; a.act = (T*)act;
    a.next_trace = (T*)next_trace; a.carry_out = (T*)carry_out; a.p_out = (T*)p_out;
    a.T_ = (int)T_; a.H = (int)H; a.n = B * T_ * H; a.m = m; a.alpha = alpha;
    const int mode = prev ? 1 : (seed ? 2 : 0);
    // element pairs move as one word: H even, the per-element operands
    // aligned to two elements, bias and trace_w to two floats
    auto al = [](const void* p, size_t n) { return p == nullptr || (uintptr_t)p % n == 0; };
    const size_t two = 2 * sizeof(T);
    const bool pair = H % 2 == 0 && al(r, two) && al(gsrc, two) && al(beta, two) && al(trace, two) &&
                      al(act, two) && al(next_trace, two) && al(p_out, two) && al(bias, 8) &&
                      al(trace_w, 8);
    if (pair) return px_tria_dispatch<T, true>(a, mode, w != nullptr, gsrc == r, axis, st);
    return px_tria_dispatch<T, false>(a, mode, w != nullptr, gsrc == r, axis, st);
}

template <typename T>
static int px_tria_end_typed(const void* r, const void* gsrc, const void* beta, const float* bias,
                             const void* trace, const float* trace_w, float m, const void* prev,
                             const uint8_t* reset, const void* initial, const uint8_t* init_valid,
                             void* act, void* next_trace, void* endpoint, float* end_f32, int64_t B,
                             int64_t T_, int64_t H, float alpha, int axis, hipStream_t st) {
    // element pairs and record pairs move as words
    auto al = [](const void* p, size_t n) { return p == nullptr || (uintptr_t)p % n == 0; };
    const size_t two = 2 * sizeof(T);
    LOOM_CHECK(al(r, two) && al(gsrc, two) && al(beta, two) && al(trace, two) && al(act, two) &&
                   al(next_trace, two) && al(prev, 4) && al(initial, 4) && al(endpoint, 4) &&
                   al(bias, 8) && al(trace_w, 8),
               "paraplex_tria_endpoint: element operands must be aligned to two elements "
               "(bias and trace_w to two floats)");
    PxTriaEndArgs<T> a{};
    a.r = (const T*)r; a.gsrc = (const T*)gsrc; a.beta = (const T*)beta; a.bias = bias;
    a.trace = (const T*)trace; a.trace_w = trace_w; a.prev = (const T*)prev; a.reset = reset;
    a.initial = (const T*)initial; a.init_valid = init_valid; a.act = (T*)act;
    a.next_trace = (T*)next_trace; a.endpoint = (T*)endpoint; a.end_f32 = end_f32;
    a.T_ = (int)T_; a.H = (int)H; a.m = m; a.alpha = alpha;
    constexpr int CH = kPxEndCols;
    const dim3 grid((unsigned)ceil_div(H, 64 * CH), (unsigned)B), blk(kTriaThreads);
    const bool same = gsrc == r;
#define LOOM_PE(A)                                                                                  \
    if (same)                                                                                       \
        hipLaunchKernelGGL((paraplex_tria_endpoint_kernel<T, A, true, CH>), grid, blk, 0, st, a);   \
    else                                                                                            \
        hipLaunchKernelGGL((paraplex_tria_endpoint_kernel<T, A, false, CH>), grid, blk, 0, st, a);
    switch (axis) {
        case 0: LOOM_PE(0) break;
        case 1: LOOM_PE(1) break;
        default: LOOM_PE(2) break;
    }
#undef LOOM_PE
    return launch_status("loom_paraplex_tria_endpoint_forward");
}

#define LOOM_DTYPE_SWITCH(dtype, FN, ...)                            \
    switch (dtype) {                                                 \
        case LOOM_F32: return FN<float>(__VA_ARGS__);                \
        case LOOM_BF16: return FN<bf16_t>(__VA_ARGS__);              \
        case LOOM_F16: return FN<f16_t>(__VA_ARGS__);                \
    }                                                                \
    set_error("unsupported dtype %d", dtype);                        \
    return LOOM_ERR_INVALID;

template <typename T>
static int gate_mix_dispatch(const void* carry, const void* w, void* p, int64_t n, hipStream_t st) {
    hipLaunchKernelGGL((gate_slot_mix_kernel<T>), dim3((unsigned)ceil_div(n, kTriaThreads)),
                       dim3(kTriaThreads), 0, st, (const T*)carry, (const T*)w, (T*)p, n);
    return launch_status("loom_gate_slot_mix_forward");
}

template <typename T>
static int slot_pool_dispatch(const void* carry, const void* sw, void* pooled, void* lse,
                              int64_t rows, int64_t H, hipStream_t st) {
    hipLaunchKernelGGL((slot_pool_kernel<T>), dim3((unsigned)rows), dim3(kTriaThreads), 0, st,
                       (const T*)carry, (const T*)sw, (T*)pooled, (T*)lse, H);
    return launch_status("loom_slot_attention_pool_forward");
}

template <typename T>
static int temporal_dispatch(bool full, const void* depth, const uint8_t* reset, const void* initial,
                             const uint8_t* valid, void* endpoint, float* end32, float* doc,
                             float* scale, int64_t B, int64_t T_, int64_t H, hipStream_t st) {
    const dim3 grid((unsigned)ceil_div(B * H, kTriaThreads)), blk(kTriaThreads);
    if (full)
        hipLaunchKernelGGL((temporal_carry_kernel<T, true>), grid, blk, 0, st, (const T*)depth,
                           reset, (const T*)nullptr, nullptr, (T*)nullptr, nullptr, doc, scale,
                           B, T_, H);
    else
    {
        // 16 groups of chains per wave, four lanes each; 16-bit records two
        // chains per lane when H is even and the tensors 4-byte aligned
        bool pair = false;
        if constexpr (sizeof(T) == 2) {
            pair = H % 2 == 0 && (((uintptr_t)depth | (uintptr_t)initial) & 3) == 0;
            if (pair)
                hipLaunchKernelGGL((temporal_endpoint_quarters_kernel<T, 2>),
                                   dim3((unsigned)ceil_div(B * H / 2, kTriaThreads / 4)), blk, 0, st,
                                   (const T*)depth, reset, (const T*)initial, valid, (T*)endpoint,
                                   end32, B, T_, H);
        }
        if (!pair)
            hipLaunchKernelGGL((temporal_endpoint_quarters_kernel<T, 1>),
                               dim3((unsigned)ceil_div(B * H, kTriaThreads / 4)), blk, 0, st,
                               (const T*)depth, reset, (const T*)initial, valid, (T*)endpoint, end32, B,
                               T_, H);
    }
    return launch_status(full ? "loom_temporal_carry_forward" : "loom_temporal_carry_endpoint_forward");
}

template <typename T>
static int polarm_dispatch(const void* in, void* out, const uint8_t* mask, int64_t n,
                           int64_t per_mask, float beta, float eps, hipStream_t st) {
    hipLaunchKernelGGL((polarm_kernel<T>), dim3((unsigned)ceil_div(n, kTriaThreads)),
                       dim3(kTriaThreads), 0, st, (const T*)in, (T*)out, mask, n, per_mask, beta,
                       eps);
    return launch_status("loom_polarm_forward");
}

template <typename T>
static int final_ca_dispatch(const void* q, const void* k, const void* v, int64_t kv_stride_b,
                             const uint8_t* allowed, int64_t allowed_stride, const void* residual,
                             float gamma, void* out, float* lse, int64_t B, int64_t T_, int64_t K,
                             const int64_t* k_dev, int64_t D, float scale, hipStream_t st) {
    const bool vec = D % 8 == 0 && D <= kCaChunks * 64 * 8 && kv_stride_b % 8 == 0 &&
                     (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out |
                       (uintptr_t)residual) & 15) == 0;
    if constexpr (sizeof(T) == 2) {
        if (vec && K <= kCaRowKeys && D <= 1024) {
            hipLaunchKernelGGL((final_ca_row_kernel<T>), dim3((unsigned)(B * T_)), dim3(512), 0, st,
                               (const T*)q, (const T*)k, (const T*)v, kv_stride_b, allowed,
                               allowed_stride, (const T*)residual, gamma, (T*)out, lse, T_, K,
                               k_dev, (int)D, scale);
            return launch_status("loom_final_ca_sparse_forward");
        }
    }
    if (vec)
        hipLaunchKernelGGL((final_ca_vec_kernel<T>), dim3((unsigned)(B * T_)), dim3(256), 0, st,
                           (const T*)q, (const T*)k, (const T*)v, kv_stride_b, allowed,
                           allowed_stride, (const T*)residual, gamma, (T*)out, lse, T_, K, k_dev,
                           (int)D, scale);
    else
        hipLaunchKernelGGL((final_ca_kernel<T>), dim3((unsigned)(B * T_)), dim3(256), 0, st,
                           (const T*)q, (const T*)k, (const T*)v, kv_stride_b, allowed, allowed_stride,
                           (const T*)residual, gamma, (T*)out, lse, T_, K, k_dev, D, scale);
    return launch_status("loom_final_ca_sparse_forward");
}

}  // namespace loom

using namespace loom;

extern "C" int loom_tria_depth_forward(int dtype, const void* r, const void* i, const void* o,
                                       const void* carry_prev, const void* seed,
                                       const uint8_t* seed_valid, const void* w, void* carry_out,
                                       void* p_out, float* scale_out, int64_t B, int64_t T,
                                       int64_t H, float alpha, int axis, void* stream) {
    clear_error();
    LOOM_CHECK(r && i && o, "tria: r, i, o are required");
    LOOM_CHECK(axis >= 0 && axis <= 2, "tria: axis must be 0(z), 1(x), or 2(y), got %d", axis);
    LOOM_CHECK(!(carry_prev && seed), "tria: carry_prev and seed are mutually exclusive");
    LOOM_CHECK(!seed || seed_valid, "tria: seed needs seed_valid");
    LOOM_CHECK(!w || p_out, "tria: gate weights need p_out");
    LOOM_CHECK(B >= 0 && T >= 0 && H >= 0, "tria: bad shape");
    if (B * T * H == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, tria_depth_dispatch, r, i, o, carry_prev, seed, seed_valid, w,
                      carry_out, p_out, scale_out, B, T, H, alpha, axis, (hipStream_t)stream)
}

extern "C" int loom_paraplex_tria_forward(int dtype, const void* p_real, const void* gate_src,
                                          const void* beta_linear, const float* bias,
                                          const void* trace, const float* trace_w, float m,
                                          const void* carry_prev, const void* seed,
                                          const uint8_t* seed_valid, const void* w, void* act,
                                          void* next_trace, void* carry_out, void* p_out,
                                          int64_t B, int64_t T, int64_t H, float alpha, int axis,
                                          void* stream) {
    clear_error();
    LOOM_CHECK(p_real && gate_src && beta_linear && bias && trace && trace_w && act && next_trace &&
                   carry_out,
               "paraplex_tria: a required tensor is null");
    LOOM_CHECK(axis >= 0 && axis <= 2, "paraplex_tria: axis must be 0(z), 1(x), or 2(y), got %d", axis);
    LOOM_CHECK(!(carry_prev && seed), "paraplex_tria: carry_prev and seed are mutually exclusive");
    LOOM_CHECK(!seed || seed_valid, "paraplex_tria: seed needs seed_valid");
    LOOM_CHECK(!w || p_out, "paraplex_tria: gate weights need p_out");
    LOOM_CHECK(B >= 0 && T >= 0 && H >= 0 && T < (1LL << 31) && H < (1LL << 31),
               "paraplex_tria: bad shape");
    // with T > 1 the block of a row's last token stores next_trace while the
    // block of its first token may still be reading trace
    LOOM_CHECK(T <= 1 || trace != (const void*)next_trace,
               "paraplex_tria: trace and next_trace must be distinct buffers when T > 1");
    if (B * T * H == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, px_tria_typed, p_real, gate_src, beta_linear, bias, trace, trace_w, m,
                      carry_prev, seed, seed_valid, w, act, next_trace, carry_out, p_out, B, T, H,
                      alpha, axis, (hipStream_t)stream)
}

extern "C" int loom_paraplex_tria_endpoint_forward(int dtype, const void* p_real,
                                                   const void* gate_src, const void* beta_linear,
                                                   const float* bias, const void* trace,
                                                   const float* trace_w, float m,
                                                   const void* carry_prev, const uint8_t* reset,
                                                   const void* initial,
                                                   const uint8_t* initial_valid, void* act,
                                                   void* next_trace, void* endpoint,
                                                   float* endpoint_f32, int64_t B, int64_t T,
                                                   int64_t H, float alpha, int axis, void* stream) {
    clear_error();
    LOOM_CHECK(p_real && gate_src && beta_linear && bias && trace && trace_w && carry_prev && reset &&
                   act && next_trace && endpoint,
               "paraplex_tria_endpoint: a required tensor is null");
    LOOM_CHECK(axis >= 0 && axis <= 2, "paraplex_tria_endpoint: axis must be 0(z), 1(x), or 2(y), got %d",
               axis);
    LOOM_CHECK(B >= 0 && B < 65536 && T >= 1 && T < (1LL << 31) && H >= 0 && H < (1LL << 31) &&
                   H % 2 == 0,
               "paraplex_tria_endpoint: bad shape (B < 65536, T >= 1, H even)");
    LOOM_CHECK(T <= 1 || trace != (const void*)next_trace,
               "paraplex_tria_endpoint: trace and next_trace must be distinct buffers when T > 1");
    if (B * H == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, px_tria_end_typed, p_real, gate_src, beta_linear, bias, trace, trace_w,
                      m, carry_prev, reset, initial, initial_valid, act, next_trace, endpoint,
                      endpoint_f32, B, T, H, alpha, axis, (hipStream_t)stream)
}

extern "C" int loom_gate_slot_mix_forward(int dtype, const void* carry, const void* w, void* p,
                                          int64_t n, void* stream) {
    clear_error();
    LOOM_CHECK(carry && w && p && n >= 0, "gate_slot_mix: bad arguments");
    if (n == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, gate_mix_dispatch, carry, w, p, n, (hipStream_t)stream)
}

extern "C" int loom_slot_attention_pool_forward(int dtype, const void* carry, const void* score_w,
                                                void* pooled, void* lse, int64_t rows, int64_t H,
                                                void* stream) {
    clear_error();
    LOOM_CHECK(carry && score_w && pooled && rows >= 0 && H >= 1,
               "slot_attention_pool: bad arguments");
    if (rows == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, slot_pool_dispatch, carry, score_w, pooled, lse, rows, H,
                      (hipStream_t)stream)
}

extern "C" int loom_temporal_carry_forward(int dtype, const void* depth, const uint8_t* reset,
                                           float* doc, float* scale, int64_t B, int64_t T,
                                           int64_t H, void* stream) {
    clear_error();
    LOOM_CHECK(depth && reset && B >= 0 && T >= 1 && H >= 0, "temporal_carry: bad arguments");
    if (B * H == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, temporal_dispatch, true, depth, reset, nullptr, nullptr, nullptr,
                      nullptr, doc, scale, B, T, H, (hipStream_t)stream)
}

extern "C" int loom_temporal_carry_endpoint_forward(int dtype, const void* depth,
                                                    const uint8_t* reset, const void* initial,
                                                    const uint8_t* initial_valid, void* endpoint,
                                                    float* endpoint_f32, int64_t B, int64_t T,
                                                    int64_t H, void* stream) {
    clear_error();
    LOOM_CHECK(depth && reset && B >= 0 && H >= 0, "temporal_carry_endpoint: bad arguments");
    LOOM_CHECK(T >= 1, "temporal carry needs at least one token");
    if (B * H == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, temporal_dispatch, false, depth, reset, initial, initial_valid,
                      endpoint, endpoint_f32, nullptr, nullptr, B, T, H, (hipStream_t)stream)
}

extern "C" int loom_polarm_forward(int dtype, const void* in, void* out, const uint8_t* mask,
                                   int64_t n, int64_t per_mask, float beta, float eps,
                                   void* stream) {
    clear_error();
    LOOM_CHECK(in && out && n >= 0 && per_mask >= 1, "polarm: bad arguments");
    LOOM_CHECK(beta >= 0.0f && beta < 1.0f, "PolARM beta must be finite and in [0, 1), got %g",
               (double)beta);
    if (n == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, polarm_dispatch, in, out, mask, n, per_mask, beta, eps,
                      (hipStream_t)stream)
}

extern "C" int loom_final_ca_sparse_forward(int dtype, const void* q, const void* k, const void* v,
                                            const uint8_t* allowed, void* out, float* lse,
                                            int64_t B, int64_t T, int64_t K, int64_t D,
                                            float scale, void* stream) {
    clear_error();
    LOOM_CHECK(q && k && v && allowed && out, "final_ca_sparse: null tensor argument");
    LOOM_CHECK(K >= 1 && K <= kCaMaxK, "final_ca_sparse: K=%lld outside [1, %d]", (long long)K,
               kCaMaxK);
    if (B * T == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, final_ca_dispatch, q, k, v, K * D, allowed, K, nullptr, 0.0f, out, lse,
                      B, T, K, nullptr, D, scale, (hipStream_t)stream)
}

extern "C" int loom_final_ca_sparse_strided(int dtype, const void* q, const void* k, const void* v,
                                            int64_t kv_stride_b, const uint8_t* allowed,
                                            int64_t allowed_stride, const void* residual,
                                            float gamma, void* out, float* lse, int64_t B,
                                            int64_t T, int64_t K, const int64_t* k_dev, int64_t D,
                                            float scale, void* stream) {
    clear_error();
    LOOM_CHECK(q && k && v && allowed && out, "final_ca_sparse: null tensor argument");
    LOOM_CHECK(K >= (k_dev ? 0 : 1) && K <= kCaMaxK, "final_ca_sparse: K=%lld outside [1, %d]",
               (long long)K, kCaMaxK);
    LOOM_CHECK(kv_stride_b >= K * D && allowed_stride >= K, "final_ca_sparse: strides too small");
    if (B * T == 0) return LOOM_OK;
    LOOM_DTYPE_SWITCH(dtype, final_ca_dispatch, q, k, v, kv_stride_b, allowed, allowed_stride,
                      residual, gamma, out, lse, B, T, K, k_dev, D, scale, (hipStream_t)stream)
}
