// Fused Paraplex pointwise chain, phase_sin and PvPowLU for gfx950.
//
// paraplex_forward: one thread owns VEC consecutive hidden units h of one
// batch row and walks a chunk of TC consecutive tokens.  The previous-token
// phase I_base[t-1] is carried in registers from the previous iteration, so
// the only extra HBM read is one beta row per chunk (1/TC overhead).  Loads
// and stores are whole 16-byte vectors, so a wavefront touches 64*16 = 1 KiB
// of contiguous memory per tensor and per token.  Aligned rows (H % 8 == 0)
// go to paraplex_chunk_kernel, whose blocks each cover one (row, chunk) so
// that addressing and loop control are scalar; the rest to
// paraplex_forward_kernel.
#include <type_traits>

#include "loom_common.h"
#include "paraplex_math.h"

namespace loom {

// VEC elements held as the raw words loaded from memory (16-bit types stay
// packed, so a prefetched row costs VEC/2 registers instead of VEC).
template <typename T, int VEC>
struct RawVec {
    static constexpr int NW = (int)((sizeof(T) * VEC + 3) / 4);
    uint32_t w[NW];
    __device__ __forceinline__ void load(const T* p) {
        if constexpr (sizeof(T) * VEC % 16 == 0) {
#pragma unroll
            for (int k = 0; k < NW / 4; ++k) {
                const uint4 v = reinterpret_cast<const uint4*>(p)[k];
                w[4 * k] = v.x; w[4 * k + 1] = v.y; w[4 * k + 2] = v.z; w[4 * k + 3] = v.w;
            }
        } else if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int k = 0; k < NW; ++k) w[k] = __float_as_uint(p[k]);
        } else if constexpr (VEC == 1) {
            w[0] = p->x;                       // one 16-bit element
        } else {
            static_assert(sizeof(T) * VEC % 16 == 0, "RawVec: unsupported width");
        }
    }
    __device__ __forceinline__ void to_float(float v[VEC]) const {
        if constexpr (sizeof(T) == 2 && VEC == 1) {
            const T one{(uint16_t)w[0]};
            v[0] = ld(&one);
            return;
        }
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            if constexpr (sizeof(T) == 4) {
                v[k] = __uint_as_float(w[k]);
            } else if constexpr (std::is_same<T, bf16_t>::value) {
                v[2 * k] = __uint_as_float(w[k] << 16);
                v[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
            } else {
                T lo{(uint16_t)(w[k] & 0xffffu)}, hi{(uint16_t)(w[k] >> 16)};
                v[2 * k] = ld(&lo);
                v[2 * k + 1] = ld(&hi);
            }
        }
    }
};

template <typename T, int VEC>
struct VecIO {
    __device__ __forceinline__ static void load(const T* p, float v[VEC]) {
        if constexpr (VEC == 8) {
            Vec8<T>::load(p, v);
        } else {
#pragma unroll
            for (int k = 0; k < VEC; ++k) v[k] = ld(p + k);
        }
    }
    __device__ __forceinline__ static void store(T* p, const float v[VEC]) {
        if constexpr (VEC == 8) {
            Vec8<T>::store(p, v);
        } else {
#pragma unroll
            for (int k = 0; k < VEC; ++k) st(p + k, v[k]);
        }
    }
    // write-once outputs of the chain (nontemporal where the row is one 16-byte vector)
    __device__ __forceinline__ static void store_nt(T* p, const float v[VEC]) {
        if constexpr (VEC == 8 && std::is_same<T, bf16_t>::value)
            Vec8<T>::store_nt(p, v);
        else
            store(p, v);
    }
};

constexpr int kPxPrefetch = 2;   // tokens of R / beta (/ gate_src) in flight per thread
constexpr int kPxUnrolled = 16;  // longest token chunk; a full chunk runs unrolled

template <typename T, int VEC, bool SAME_GATE, bool HAS_RESET>
__global__ void __launch_bounds__(256)
paraplex_forward_kernel(const T* __restrict__ p_real, const T* __restrict__ gate_src,
                        const T* __restrict__ beta_lin, const float* __restrict__ bias,
                        const T* __restrict__ trace, const float* __restrict__ trace_w,
                        const uint8_t* __restrict__ reset, const float* __restrict__ anchor,
                        T* __restrict__ act, T* __restrict__ s_out, T* __restrict__ next_trace,
                        float* __restrict__ anchor_snap, int B, int T_, int H, int nchunks, int TC,
                        float m) {
    constexpr int PF = kPxPrefetch;
    // 32-bit index math: the host guarantees B*nchunks*(H/VEC) < 2^31
    const unsigned gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid == 0 && anchor_snap != nullptr) anchor_snap[0] = anchor[0];
    const unsigned HV = (unsigned)H / VEC;
    if (gid >= (unsigned)B * (unsigned)nchunks * HV) return;
    const unsigned hv = gid % HV;
    const unsigned rest = gid / HV;
    const unsigned chunk = rest % (unsigned)nchunks;
    const unsigned b = rest / (unsigned)nchunks;
    const int h0 = (int)hv * VEC;
    const int t0 = (int)chunk * TC;
    if (t0 >= T_) return;
    const int n = (t0 + TC < T_ ? t0 + TC : T_) - t0;

    float bv[VEC], tw[VEC], prev[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        bv[k] = bias[h0 + k];
        tw[k] = trace_w[h0 + k];
    }
    const int64_t base0 = ((int64_t)b * T_ + t0) * H + h0;
    if (t0 == 0) {
        VecIO<T, VEC>::load(trace + (int64_t)b * H + h0, prev);
    } else {
        float bl[VEC];
        VecIO<T, VEC>::load(beta_lin + base0 - H, bl);
#pragma unroll
        for (int k = 0; k < VEC; ++k) prev[k] = phase_of(bl[k] + bv[k]);
    }
    const T* pr = p_real + base0;
    const T* pg = gate_src + base0;
    const T* pb = beta_lin + base0;
    T* po = act + base0;
    T* ps = s_out + base0;
    const uint8_t* prs = HAS_RESET ? reset + (int64_t)b * T_ + t0 : nullptr;
    // ring of PF prefetched tokens; slot p holds token it0 + p
    RawVec<T, VEC> rr[PF], rb[PF], rg[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        if (p < n) {
            rr[p].load(pr + (int64_t)p * H);
            rb[p].load(pb + (int64_t)p * H);
            if constexpr (!SAME_GATE) rg[p].load(pg + (int64_t)p * H);
        }
    }
    for (int it0 = 0; it0 < n; it0 += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int it = it0 + p;
            if (it >= n) break;
            float r[VEC], bl[VEC], g[VEC];
            rr[p].to_float(r);
            rb[p].to_float(bl);
            if constexpr (!SAME_GATE) rg[p].to_float(g);
            if (it + PF < n) {
                // issue token it+PF's loads ahead of this token's math, at raised
                // wave priority so the loads of all waves go out early
                __builtin_amdgcn_s_setprio(3);
                rr[p].load(pr + (int64_t)PF * H);
                rb[p].load(pb + (int64_t)PF * H);
                if constexpr (!SAME_GATE) rg[p].load(pg + (int64_t)PF * H);
                __builtin_amdgcn_s_setprio(0);
            }
            const bool rs = HAS_RESET && prs[it] != 0;
            float so[VEC], ao[VEC];
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const float s0 = phase_of(bl[k] + bv[k]);
                const float raw = rs ? s0 : fmaf(prev[k], tw[k], s0);
                const float sv = raw * frsq(fmaf(raw, raw, 1.0f));
                float amp, gate;
                softplus_gate<!std::is_same<T, bf16_t>::value>(SAME_GATE ? r[k] : g[k], m, amp, gate);
                so[k] = sv;
                ao[k] = fmaf(amp, sv, r[k]) * gate;
                prev[k] = s0;
            }
            VecIO<T, VEC>::store_nt(ps, so);
            VecIO<T, VEC>::store_nt(po, ao);
            pr += H; pb += H; pg += H; po += H; ps += H;
        }
    }
    if (t0 + n == T_) VecIO<T, VEC>::store(next_trace + (int64_t)b * H + h0, prev);
}

// Eight elements as 16-byte raw-buffer pieces (one for 16-bit types, two for
// fp32).  `soff` is a scalar byte offset shared by the wave, `voff` the lane's.
// The chain reads R / beta once and writes I / O once: nontemporal loads and
// stores (over three rotated PX operand sets 38.0-38.8 us against 39.4-40.0 us
// with default-policy loads; a plain two-in two-out copy of the same bytes
// runs at 33.2-34.5 us nontemporal, 37-38 us default).
constexpr int kBufCoherent = 0;
constexpr int kBufStream = 2;      // nontemporal
template <typename T>
__device__ __forceinline__ void buf_load8(RawVec<T, 8>& v, __amdgpu_buffer_rsrc_t r,
                                          uint32_t voff, uint32_t soff) {
#pragma unroll
    for (int q = 0; q < RawVec<T, 8>::NW / 4; ++q) {
        const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(voff + 16 * q), (int)soff,
                                                              kBufStream);
        v.w[4 * q] = x.x; v.w[4 * q + 1] = x.y; v.w[4 * q + 2] = x.z; v.w[4 * q + 3] = x.w;
    }
}
// Eight outputs packed into the 16-byte pieces a store writes.
template <typename T>
struct Packed8 {
    static constexpr int NQ = sizeof(T) == 4 ? 2 : 1;
    u32x4 q[NQ];
};
template <typename T>
__device__ __forceinline__ Packed8<T> pack8(const float v[8]) {
    Packed8<T> x;
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int q = 0; q < 2; ++q)
            x.q[q] = (u32x4){__float_as_uint(v[4 * q]), __float_as_uint(v[4 * q + 1]),
                             __float_as_uint(v[4 * q + 2]), __float_as_uint(v[4 * q + 3])};
    } else {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if constexpr (std::is_same<T, bf16_t>::value) {
                w[k] = pack_bf16x2(v[2 * k], v[2 * k + 1]);
            } else {
                T lo, hi;
                st(&lo, v[2 * k]);
                st(&hi, v[2 * k + 1]);
                w[k] = (uint32_t)lo.x | ((uint32_t)hi.x << 16);
            }
        }
        x.q[0] = (u32x4){w[0], w[1], w[2], w[3]};
    }
    return x;
}
// 16-byte raw-buffer stores take their whole offset in the VGPR operand and a
// constant-zero soffset.  A VALU write to the data registers of a store wider
// than 8 bytes, issued in the next cycle, can reach memory in place of the
// stored data (the ">8-byte store data" hazard).  The compiler's hazard
// recognizer inserts the wait state for this hazard only when soffset is not a
// register; with the token offset in an SGPR soffset it placed such writes
// back to back after the store, and a few lanes of the first dword then held
// the next instruction's result.  With soffset = 0 the wait states are
// inserted (one v_add per token forms the offset).
template <typename T>
__device__ __forceinline__ void buf_store8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                           const Packed8<T>& x) {
#pragma unroll
    for (int q = 0; q < Packed8<T>::NQ; ++q)
        __builtin_amdgcn_raw_buffer_store_b128(x.q[q], r, (int)(voff + soff + 16 * q), 0,
                                               sizeof(T) == 2 ? kBufStream : kBufCoherent);
}

// The same chain with one block per (batch row, token chunk, run of hidden
// units): the chunk bounds, the token loop and the reset flags are uniform
// across the block, and every tensor access is a raw-buffer access over the
// chunk's slice with the lane's 32-bit byte offset (its hidden units) and a
// scalar token offset, so the loop spends no vector instructions on
// addresses or loop control.  The host guarantees H % 8 == 0, 16-byte
// aligned tensors and TC * H * sizeof(T) < 2^31.
template <typename T, bool SAME_GATE, bool HAS_RESET, int TCU>
__global__ void __launch_bounds__(256)
paraplex_chunk_kernel(const T* __restrict__ p_real, const T* __restrict__ gate_src,
                      const T* __restrict__ beta_lin, const float* __restrict__ bias,
                      const T* __restrict__ trace, const float* __restrict__ trace_w,
                      const uint8_t* __restrict__ reset, const float* __restrict__ anchor,
                      T* __restrict__ act, T* __restrict__ s_out, T* __restrict__ next_trace,
                      float* __restrict__ anchor_snap, int T_, int H, int TC, float m) {
    constexpr int VEC = 8;
    constexpr int PF = kPxPrefetch;
    const int b = blockIdx.z;
    const int t0 = blockIdx.y * TC;
    const int n = min(TC, T_ - t0);
    const int h0 = (blockIdx.x * blockDim.x + threadIdx.x) * VEC;
    if ((blockIdx.x | blockIdx.y | blockIdx.z | threadIdx.x) == 0 && anchor_snap != nullptr)
        anchor_snap[0] = anchor[0];
    if (h0 >= H) return;

    float bv[VEC], tw[VEC], prev[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        bv[k] = bias[h0 + k];
        tw[k] = trace_w[h0 + k];
    }
    const int64_t base0 = ((int64_t)b * T_ + t0) * H;
    if (t0 == 0) {
        VecIO<T, VEC>::load(trace + (int64_t)b * H + h0, prev);
    } else {
        float bl[VEC];
        VecIO<T, VEC>::load(beta_lin + base0 - H + h0, bl);
#pragma unroll
        for (int k = 0; k < VEC; ++k) prev[k] = phase_of(bl[k] + bv[k]);
    }
    const uint32_t step = (uint32_t)H * (uint32_t)sizeof(T);
    const uint32_t bytes = (uint32_t)n * step;
    const uint32_t voff = (uint32_t)h0 * (uint32_t)sizeof(T);
    const auto rR = __builtin_amdgcn_make_buffer_rsrc((void*)(p_real + base0), (short)0, (int)bytes, kBufferDword3);
    const auto rG = __builtin_amdgcn_make_buffer_rsrc((void*)(gate_src + base0), (short)0, (int)bytes, kBufferDword3);
    const auto rB = __builtin_amdgcn_make_buffer_rsrc((void*)(beta_lin + base0), (short)0, (int)bytes, kBufferDword3);
    const auto rA = __builtin_amdgcn_make_buffer_rsrc((void*)(act + base0), (short)0, (int)bytes, kBufferDword3);
    const auto rS = __builtin_amdgcn_make_buffer_rsrc((void*)(s_out + base0), (short)0, (int)bytes, kBufferDword3);
    const uint8_t* prs = HAS_RESET ? reset + (int64_t)b * T_ + t0 : nullptr;

    RawVec<T, VEC> rr[PF], rb[PF], rg[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        if (p < n) {
            buf_load8<T>(rr[p], rR, voff, p * step);
            buf_load8<T>(rb[p], rB, voff, p * step);
            if constexpr (!SAME_GATE) buf_load8<T>(rg[p], rG, voff, p * step);
        }
    }
    // token `it` from ring slot p; with `refill`, token it+PF's loads go out
    // ahead of the math (at raised wave priority, so every wave's loads issue early)
    auto token = [&](int p, int it, bool refill) {
        float r[VEC], bl[VEC], g[VEC];
        rr[p].to_float(r);
        rb[p].to_float(bl);
        if constexpr (!SAME_GATE) rg[p].to_float(g);
        // unpacked into registers of their own before the refill is issued, so
        // the load lands in the slot's registers with no copies
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            asm volatile("" : "+v"(r[k]), "+v"(bl[k]));
            if constexpr (!SAME_GATE) asm volatile("" : "+v"(g[k]));
        }
        if (refill) {
            __builtin_amdgcn_s_setprio(3);
            buf_load8<T>(rr[p], rR, voff, (it + PF) * step);
            buf_load8<T>(rb[p], rB, voff, (it + PF) * step);
            if constexpr (!SAME_GATE) buf_load8<T>(rg[p], rG, voff, (it + PF) * step);
            __builtin_amdgcn_s_setprio(0);
        }
        const bool rs = HAS_RESET && prs[it] != 0;
        float so[VEC], ao[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            const float s0 = phase_of(bl[k] + bv[k]);
            const float raw = rs ? s0 : fmaf(prev[k], tw[k], s0);
            const float sv = raw * frsq(fmaf(raw, raw, 1.0f));
            float amp, gate;
            softplus_gate<!std::is_same<T, bf16_t>::value>(SAME_GATE ? r[k] : g[k], m, amp, gate);
            so[k] = sv;
            ao[k] = fmaf(amp, sv, r[k]) * gate;
            prev[k] = s0;
        }
        buf_store8<T>(rS, voff, it * step, pack8<T>(so));
        buf_store8<T>(rA, voff, it * step, pack8<T>(ao));
    };
    if constexpr (TCU > 0) {
        if (n == TCU) {
            // a whole chunk as straight-line code: the ring slots are fixed
            // registers and every wait covers exactly the loads it needs
#pragma unroll
            for (int it = 0; it < TCU; ++it) token(it % PF, it, it + PF < TCU);
            if (t0 + n == T_) VecIO<T, VEC>::store(next_trace + (int64_t)b * H + h0, prev);
            return;
        }
    }
    // every slot is refilled while PF more tokens follow the group, so the
    // ring registers are overwritten in place; the last one or two groups
    // refill only what is left
    int it0 = 0;
    for (; it0 + 2 * PF <= n; it0 += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) token(p, it0 + p, true);
    }
    for (; it0 < n; it0 += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            if (it0 + p >= n) break;
            token(p, it0 + p, it0 + p + PF < n);
        }
    }
    if (t0 + n == T_) VecIO<T, VEC>::store(next_trace + (int64_t)b * H + h0, prev);
}

template <typename T, int VEC>
__global__ void __launch_bounds__(256)
phase_sin_kernel(const T* __restrict__ beta, T* __restrict__ out, int64_t nvec) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec;
         i += (int64_t)gridDim.x * blockDim.x) {
        float v[VEC];
        VecIO<T, VEC>::load(beta + i * VEC, v);
#pragma unroll
        for (int k = 0; k < VEC; ++k) v[k] = phase_of(v[k]);
        VecIO<T, VEC>::store(out + i * VEC, v);
    }
}

template <typename T, int VEC>
__global__ void __launch_bounds__(256)
pvpowlu_kernel(const T* __restrict__ x1, const T* __restrict__ x2, T* __restrict__ out,
               int64_t nvec, float m) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec;
         i += (int64_t)gridDim.x * blockDim.x) {
        float a[VEC], g[VEC];
        VecIO<T, VEC>::load(x1 + i * VEC, a);
        VecIO<T, VEC>::load(x2 + i * VEC, g);
#pragma unroll
        for (int k = 0; k < VEC; ++k) a[k] *= powlu_gate(g[k], m);
        VecIO<T, VEC>::store(out + i * VEC, a);
    }
}

static bool aligned16(const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

template <typename T, int VEC>
static int launch_paraplex(const void* p_real, const void* gate_src, const void* beta_lin,
                           const float* bias, const void* trace, const float* trace_w,
                           const uint8_t* reset, const float* anchor, void* act, void* s,
                           void* next_trace, float* anchor_snap, int64_t B, int64_t T_,
                           int64_t H, float m, hipStream_t stream) {
    // Tokens per thread: the longest run of t, up to kPxUnrolled, that still
    // gives every SIMD at least 3 waves (enough to hide memory latency behind
    // the math).  Longer runs mean fewer per-chunk restarts (each reads one
    // more beta row, 1/TC of the beta stream).
    const int64_t HV = H / VEC;
    const bool same = gate_src == p_real;
    auto kern = same ? (reset ? paraplex_forward_kernel<T, VEC, true, true>
                              : paraplex_forward_kernel<T, VEC, true, false>)
                     : (reset ? paraplex_forward_kernel<T, VEC, false, true>
                              : paraplex_forward_kernel<T, VEC, false, false>);
    const int64_t simds = 4 * (int64_t)device_cus();
    int TC = kPxUnrolled;
    while (TC > 1 && B * ceil_div(T_, TC) * HV < 3 * 64 * simds) --TC;
    const int64_t nchunks = ceil_div(T_, TC);
    if (VEC == 8 && nchunks <= 65535 && B <= 65535 &&
        (int64_t)TC * H * (int64_t)sizeof(T) < ((int64_t)1 << 31)) {
        // one block per (b, chunk, run of hidden units): the widest block of
        // 1-4 waves that splits the row's waves evenly
        const int64_t waves = ceil_div(HV, 64);
        const int w = waves % 4 == 0 ? 4 : waves % 3 == 0 ? 3 : waves % 2 == 0 ? 2 : (waves < 4 ? (int)waves : 4);
        const dim3 grid((unsigned)ceil_div(HV, 64 * w), (unsigned)nchunks, (unsigned)B);
        // a full chunk of 16-bit rows runs as straight-line code (fp32 keeps
        // the loop: unrolled, its registers would allow only 2 waves per SIMD)
        auto ck = same ? (reset ? paraplex_chunk_kernel<T, true, true, 0> : paraplex_chunk_kernel<T, true, false, 0>)
                       : (reset ? paraplex_chunk_kernel<T, false, true, 0> : paraplex_chunk_kernel<T, false, false, 0>);
        if (TC == kPxUnrolled && sizeof(T) == 2)
            ck = same ? (reset ? paraplex_chunk_kernel<T, true, true, kPxUnrolled>
                               : paraplex_chunk_kernel<T, true, false, kPxUnrolled>)
                      : (reset ? paraplex_chunk_kernel<T, false, true, kPxUnrolled>
                               : paraplex_chunk_kernel<T, false, false, kPxUnrolled>);
        hipLaunchKernelGGL(ck, grid, dim3(64 * w), 0, stream, (const T*)p_real,
                           (const T*)gate_src, (const T*)beta_lin, bias, (const T*)trace, trace_w,
                           reset, anchor, (T*)act, (T*)s, (T*)next_trace, anchor_snap, (int)T_,
                           (int)H, TC, m);
        return launch_status("loom_paraplex_forward");
    }
    const int64_t total = B * nchunks * HV;
    LOOM_CHECK(total < ((int64_t)1 << 31) && T_ < ((int64_t)1 << 31) && H < ((int64_t)1 << 31),
               "paraplex: %lld x %lld x %lld exceeds the 32-bit thread index", (long long)B,
               (long long)T_, (long long)H);
    const int threads = 256;
    const int64_t blocks = ceil_div(total, threads);
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(threads), 0, stream,
                       (const T*)p_real, (const T*)gate_src, (const T*)beta_lin, bias,
                       (const T*)trace, trace_w, reset, anchor, (T*)act, (T*)s, (T*)next_trace,
                       anchor_snap, (int)B, (int)T_, (int)H, (int)nchunks, TC, m);
    return launch_status("loom_paraplex_forward");
}

template <typename T>
static int dispatch_paraplex(const void* p_real, const void* gate_src, const void* beta_lin,
                             const float* bias, const void* trace, const float* trace_w,
                             const uint8_t* reset, const float* anchor, void* act, void* s,
                             void* next_trace, float* anchor_snap, int64_t B, int64_t T_,
                             int64_t H, float m, hipStream_t stream) {
    const bool vec = (H % 8 == 0) && aligned16(p_real) && aligned16(gate_src) &&
                     aligned16(beta_lin) && aligned16(trace) && aligned16(act) &&
                     aligned16(s) && aligned16(next_trace);
    if (vec)
        return launch_paraplex<T, 8>(p_real, gate_src, beta_lin, bias, trace, trace_w, reset,
                                     anchor, act, s, next_trace, anchor_snap, B, T_, H, m, stream);
    return launch_paraplex<T, 1>(p_real, gate_src, beta_lin, bias, trace, trace_w, reset, anchor,
                                 act, s, next_trace, anchor_snap, B, T_, H, m, stream);
}

template <typename T>
static int dispatch_elementwise(int which, const void* a, const void* b, void* out, int64_t n,
                                float m, hipStream_t stream) {
    const bool vec = (n % 8 == 0) && aligned16(a) && aligned16(b) && aligned16(out);
    const int threads = 256;
    const int64_t nvec = vec ? n / 8 : n;
    int64_t blocks = ceil_div(nvec, threads);
    if (blocks > 256 * 64) blocks = 256 * 64;
    if (which == 0) {
        if (vec)
            hipLaunchKernelGGL((phase_sin_kernel<T, 8>), dim3(blocks), dim3(threads), 0, stream,
                               (const T*)a, (T*)out, nvec);
        else
            hipLaunchKernelGGL((phase_sin_kernel<T, 1>), dim3(blocks), dim3(threads), 0, stream,
                               (const T*)a, (T*)out, nvec);
        return launch_status("loom_phase_sin_forward");
    }
    if (vec)
        hipLaunchKernelGGL((pvpowlu_kernel<T, 8>), dim3(blocks), dim3(threads), 0, stream,
                           (const T*)a, (const T*)b, (T*)out, nvec, m);
    else
        hipLaunchKernelGGL((pvpowlu_kernel<T, 1>), dim3(blocks), dim3(threads), 0, stream,
                           (const T*)a, (const T*)b, (T*)out, nvec, m);
    return launch_status("loom_pvpowlu_forward");
}

}  // namespace loom

using namespace loom;

extern "C" int loom_paraplex_forward(int dtype, const void* p_real, const void* gate_src,
                                     const void* beta_linear, const float* bias,
                                     const void* trace, const float* trace_w,
                                     const uint8_t* reset, const float* anchor, void* act,
                                     void* s, void* next_trace, float* anchor_snapshot,
                                     int64_t B, int64_t T, int64_t H, float m, void* stream) {
    clear_error();
    LOOM_CHECK(B > 0 && T > 0 && H > 0, "paraplex: empty tensors are unsupported");
    LOOM_CHECK(p_real && gate_src && beta_linear && bias && trace && trace_w && act && s &&
                   next_trace,
               "paraplex: null tensor argument");
    LOOM_CHECK((anchor == nullptr) == (anchor_snapshot == nullptr),
               "paraplex: anchor and anchor_snapshot must be given together");
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case LOOM_F32:
            return dispatch_paraplex<float>(p_real, gate_src, beta_linear, bias, trace, trace_w,
                                            reset, anchor, act, s, next_trace, anchor_snapshot, B,
                                            T, H, m, st);
        case LOOM_BF16:
            return dispatch_paraplex<bf16_t>(p_real, gate_src, beta_linear, bias, trace, trace_w,
                                             reset, anchor, act, s, next_trace, anchor_snapshot,
                                             B, T, H, m, st);
        case LOOM_F16:
            return dispatch_paraplex<f16_t>(p_real, gate_src, beta_linear, bias, trace, trace_w,
                                            reset, anchor, act, s, next_trace, anchor_snapshot, B,
                                            T, H, m, st);
    }
    set_error("paraplex: unsupported dtype %d", dtype);
    return LOOM_ERR_INVALID;
}

extern "C" int loom_phase_sin_forward(int dtype, const void* beta, void* out, int64_t n,
                                      void* stream) {
    clear_error();
    LOOM_CHECK(n >= 0 && beta && out, "phase_sin: bad arguments");
    if (n == 0) return LOOM_OK;
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case LOOM_F32: return dispatch_elementwise<float>(0, beta, beta, out, n, 0.f, st);
        case LOOM_BF16: return dispatch_elementwise<bf16_t>(0, beta, beta, out, n, 0.f, st);
        case LOOM_F16: return dispatch_elementwise<f16_t>(0, beta, beta, out, n, 0.f, st);
    }
    set_error("phase_sin: unsupported dtype %d", dtype);
    return LOOM_ERR_INVALID;
}

extern "C" int loom_pvpowlu_forward(int dtype, const void* x1, const void* x2, void* out,
                                    int64_t n, float m, void* stream) {
    clear_error();
    LOOM_CHECK(n >= 0 && x1 && x2 && out, "pvpowlu: bad arguments");
    if (n == 0) return LOOM_OK;
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case LOOM_F32: return dispatch_elementwise<float>(1, x1, x2, out, n, m, st);
        case LOOM_BF16: return dispatch_elementwise<bf16_t>(1, x1, x2, out, n, m, st);
        case LOOM_F16: return dispatch_elementwise<f16_t>(1, x1, x2, out, n, m, st);
    }
    set_error("pvpowlu: unsupported dtype %d", dtype);
    return LOOM_ERR_INVALID;
}
