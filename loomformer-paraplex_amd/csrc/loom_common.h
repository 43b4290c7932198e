// Shared device/host helpers for the LoomFormer gfx950 library.
//
// All arithmetic is fp32 in registers; tensors are fp32, bf16 or fp16 in HBM.
// Conversions to bf16 round to nearest-even (the same rounding torch uses for
// .to(torch.bfloat16)).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/loom_hip.h"

namespace loom {

// ------------------------------------------------------------------ errors
void set_error(const char* fmt, ...);
void clear_error();
int launch_status(const char* what);
// compute units of the current device; threads of `kernel` it keeps resident
int device_cus();
int64_t resident_threads(const void* kernel, int block);
// the chunked prefill's RoPE + cache append of a qkv chunk (prefill.hip):
// q_out [B*Tc, QH*HD] roped, k roped and v into the caches at positions
// start .. start + Tc - 1
int prefill_rope_append(int dtype, const void* qkv, int64_t qkv_ld, void* kc, void* vc,
                        int64_t csb, int64_t cst, int64_t csh, const float* cosv,
                        const float* sinv, void* q_out, int64_t B, int64_t Tc, int64_t start,
                        int64_t QH, int64_t KVH, int64_t HD, hipStream_t st);

#define LOOM_CHECK(cond, ...)            \
    do {                                 \
        if (!(cond)) {                   \
            ::loom::set_error(__VA_ARGS__); \
            return LOOM_ERR_INVALID;     \
        }                                \
    } while (0)

// ------------------------------------------------------------------ dtypes
struct bf16_t { uint16_t x; };
struct f16_t { uint16_t x; };

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}

// Round to nearest-even with gfx950's v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Dword 3 of a gfx9 raw-buffer descriptor (untyped 32-bit data format).
constexpr int kBufferDword3 = 0x00020000;

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Barrier for LDS traffic only: waits for this wave's LDS operations, not
// for its outstanding global loads (which __syncthreads would also drain).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Wait until at most N of this wave's vector-memory operations are in flight
// (loads straight into LDS included).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// 16 bytes per lane from a raw buffer straight into LDS (lane l lands at
// lds + 16*l; lds wave-uniform); an offset past the buffer's end lands zeros
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, const void* lds, uint32_t voff,
                                      uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, voff, soff, 0, 0);
}

// two floats -> packed bf16 pair (low = a), one conversion instruction
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

template <typename T> struct Cvt;
template <> struct Cvt<float> {
    __device__ __forceinline__ static float load(const float* p) { return *p; }
    __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
};
template <> struct Cvt<bf16_t> {
    __device__ __forceinline__ static float load(const bf16_t* p) { return bf16_to_f32(p->x); }
    __device__ __forceinline__ static void store(bf16_t* p, float v) { p->x = f32_to_bf16(v); }
};
template <> struct Cvt<f16_t> {
    __device__ __forceinline__ static float load(const f16_t* p) {
        return __half2float(__ushort_as_half(p->x));
    }
    __device__ __forceinline__ static void store(f16_t* p, float v) {
        // the fp32 value first, then its rounding to half: kept opaque so the
        // compiler cannot fold a preceding multiply or fma into a mixed-precision
        // instruction that rounds the exact product to half in one step (a
        // different result wherever the fp32 rounding decides the half one)
        __asm__("" : "+v"(v));
        p->x = __half_as_ushort(__float2half_rn(v));
    }
};

template <typename T> __device__ __forceinline__ float ld(const T* p) { return Cvt<T>::load(p); }
template <typename T> __device__ __forceinline__ void st(T* p, float v) { Cvt<T>::store(p, v); }

// x rounded to the storage type T and back (the identity for fp32)
template <typename T> __device__ __forceinline__ float round_to(float x) {
    if constexpr (std::is_same<T, float>::value) {
        return x;
    } else {
        T t;
        st(&t, x);
        return ld(&t);
    }
}

// Vector of 8 elements (16 B for 16-bit types, 32 B for fp32) loaded/stored
// as whole 16-byte transactions.
template <typename T> struct Vec8;
template <> struct Vec8<float> {
    __device__ __forceinline__ static void load(const float* p, float v[8]) {
        const float4 a = *reinterpret_cast<const float4*>(p);
        const float4 b = *reinterpret_cast<const float4*>(p + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    __device__ __forceinline__ static void store(float* p, const float v[8]) {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
};
template <typename T16> struct Vec8_16 {
    __device__ __forceinline__ static void load(const T16* p, float v[8]) {
        const uint4 a = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            T16 lo{(uint16_t)(w[k] & 0xffffu)}, hi{(uint16_t)(w[k] >> 16)};
            v[2 * k] = Cvt<T16>::load(&lo);
            v[2 * k + 1] = Cvt<T16>::load(&hi);
        }
    }
    __device__ __forceinline__ static void store(T16* p, const float v[8]) {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            T16 lo, hi;
            Cvt<T16>::store(&lo, v[2 * k]);
            Cvt<T16>::store(&hi, v[2 * k + 1]);
            w[k] = (uint32_t)lo.x | ((uint32_t)hi.x << 16);
        }
        *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    }
};
template <> struct Vec8<bf16_t> : Vec8_16<bf16_t> {
    __device__ __forceinline__ static void store(bf16_t* p, const float v[8]) {
        *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                  pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
    }
    // write-once output: one nontemporal 16-byte store
    __device__ __forceinline__ static void store_nt(bf16_t* p, const float v[8]) {
        const u32x4 w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                         pack_bf16x2(v[6], v[7])};
        __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
    }
};
template <> struct Vec8<f16_t> : Vec8_16<f16_t> {};

// EPL contiguous elements of one row, moved as 4- or 8-byte words (the
// caller guarantees 4-byte alignment of p for 16-bit types, 8 for fp32).
template <typename T, int EPL>
struct RowIO {
    __device__ __forceinline__ static void load(const T* p, float v[EPL]) {
        if constexpr (sizeof(T) == 2 && EPL % 2 == 0) {
#pragma unroll
            for (int k = 0; k < EPL / 2; ++k) {
                const uint32_t w = reinterpret_cast<const uint32_t*>(p)[k];
                T lo{(uint16_t)(w & 0xffffu)}, hi{(uint16_t)(w >> 16)};
                v[2 * k] = ld(&lo);
                v[2 * k + 1] = ld(&hi);
            }
        } else if constexpr (sizeof(T) == 4 && EPL % 2 == 0) {
#pragma unroll
            for (int k = 0; k < EPL / 2; ++k) {
                const float2 w = reinterpret_cast<const float2*>(p)[k];
                v[2 * k] = w.x;
                v[2 * k + 1] = w.y;
            }
        } else {
#pragma unroll
            for (int k = 0; k < EPL; ++k) v[k] = ld(p + k);
        }
    }
    __device__ __forceinline__ static void store(T* p, const float v[EPL]) {
        if constexpr (sizeof(T) == 2 && EPL % 2 == 0) {
#pragma unroll
            for (int k = 0; k < EPL / 2; ++k) {
                T lo, hi;
                st(&lo, v[2 * k]);
                st(&hi, v[2 * k + 1]);
                reinterpret_cast<uint32_t*>(p)[k] = (uint32_t)lo.x | ((uint32_t)hi.x << 16);
            }
        } else if constexpr (sizeof(T) == 4 && EPL % 2 == 0) {
#pragma unroll
            for (int k = 0; k < EPL / 2; ++k)
                reinterpret_cast<float2*>(p)[k] = make_float2(v[2 * k], v[2 * k + 1]);
        } else {
#pragma unroll
            for (int k = 0; k < EPL; ++k) st(p + k, v[k]);
        }
    }
};

// EPL elements of one row held as the raw words loaded from memory (16-bit
// types stay packed two to a register until to_float); p must be 4-byte
// aligned when EPL is even.
template <typename T, int EPL>
struct RawRow {
    static constexpr bool kPairs = sizeof(T) == 4 || EPL % 2 == 0;
    static constexpr int NW = sizeof(T) == 4 ? EPL : (kPairs ? EPL / 2 : EPL);
    uint32_t w[NW];
    __device__ __forceinline__ void load(const T* p) {
        if constexpr (kPairs) {
            const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
            for (int k = 0; k < NW; ++k) w[k] = q[k];
        } else {
            const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
            for (int k = 0; k < NW; ++k) w[k] = q[k];
        }
    }
    // Streaming form of load for rows read exactly once: the nontemporal hint
    // keeps them from displacing reused lines in the caches.
    __device__ __forceinline__ void load_nt(const T* p) {
        if constexpr (kPairs) {
            const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
            for (int k = 0; k < NW; ++k) w[k] = __builtin_nontemporal_load(q + k);
        } else {
            const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
            for (int k = 0; k < NW; ++k) w[k] = __builtin_nontemporal_load(q + k);
        }
    }
    // Hide the words' values from the compiler (no instruction is emitted), so a
    // later to_float recomputes the unpacking instead of keeping an earlier
    // unpacked copy alive in registers.
    __device__ __forceinline__ void opaque() {
#pragma unroll
        for (int k = 0; k < NW; ++k) asm volatile("" : "+v"(w[k]));
    }
    __device__ __forceinline__ void to_float(float v[EPL]) const {
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            if constexpr (sizeof(T) == 4) {
                v[k] = __uint_as_float(w[k]);
            } else if constexpr (!kPairs) {
                const T one{(uint16_t)w[k]};
                v[k] = ld(&one);
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

// ------------------------------------------------------------------ fast math
// Built directly on the gfx950 transcendental instructions (v_exp_f32 = 2^x,
// v_log_f32 = log2 x, v_sin_f32 = sin(2*pi*x), v_rsq_f32, v_rcp_f32,
// v_sqrt_f32); each is accurate to about one ulp over the ranges used here.
// Position in the work order of block L of a 1-D launch of n blocks, such
// that each XCD works through one contiguous share of that order: blocks are
// dealt round-robin to the 8 XCDs (block L runs on XCD L % 8), so XCD k's
// blocks L = 8*slot + k take work items k*(n/8) + min(k, n%8) + slot.  Work
// items next to each other in the order then share an L2.
__device__ __forceinline__ int xcd_contiguous(int L, int n) {
    const int k = L & 7, slot = L >> 3;
    return k * (n >> 3) + min(k, n & 7) + slot;
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float flog2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float frsq(float x) { return __builtin_amdgcn_rsqf(x); }
__device__ __forceinline__ float fsqrt(float x) { return __builtin_amdgcn_sqrtf(x); }
// sin(2*pi*r) for |r| <= 0.25 (one quarter turn)
__device__ __forceinline__ float fsin_turns(float r) { return __builtin_amdgcn_sinf(r); }

// log1p(t) for t in [0, 1]: log(u) corrected by the rounding of u = 1 + t
// (the classic Goldberg correction), so small t keep full relative accuracy.
__device__ __forceinline__ float flog1p_unit(float t) {
    const float u = 1.0f + t;
    const float du = u - 1.0f;
    const float l = flog2(u) * kLn2;
    // when u rounds to 1, du == 0 and log1p(t) ~= t
    return du == 0.0f ? t : l * (t / du);
}

// softplus with torch's threshold (x > 20 -> x); log1p(exp(x)) otherwise,
// evaluated as max(x,0) + log1p(exp(-|x|)) to keep it accurate for x < 0.
__device__ __forceinline__ float fsoftplus(float x) {
    if (x > 20.0f) return x;
    const float t = fexp(-fabsf(x));
    return fmaxf(x, 0.0f) + flog1p_unit(t);
}

// ------------------------------------------------------------------ wave ops
// Lane permutations inside a 16-lane DPP row (VALU only, no LDS traffic):
// quad_perm [1,0,3,2] and [2,3,0,1] pair lanes at distance 1 and 2, the
// half-row mirror pairs the two quads of each 8-lane half, the row mirror pairs
// the two halves.  Each is an involution, so after k steps every lane of an
// aligned group of 2^k lanes holds the group's reduction.
constexpr int kDppQuad1032 = 0xB1, kDppQuad2301 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

// (every source lane of these permutations lies in the same row, so none is
// out of range; the "old" operand is the lane's own value regardless)
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    const int b = __builtin_bit_cast(int, v);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(b, b, CTRL, 0xF, 0xF, false));
}

// sum over aligned groups of G lanes (G a power of two <= 64)
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (G >= 2) v += dpp<kDppQuad1032>(v);
    if constexpr (G >= 4) v += dpp<kDppQuad2301>(v);
    if constexpr (G >= 8) v += dpp<kDppHalfMirror>(v);
    if constexpr (G >= 16) v += dpp<kDppMirror>(v);
    if constexpr (G >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (G >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}
template <int G>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (G >= 2) v = fmaxf(v, dpp<kDppQuad1032>(v));
    if constexpr (G >= 4) v = fmaxf(v, dpp<kDppQuad2301>(v));
    if constexpr (G >= 8) v = fmaxf(v, dpp<kDppHalfMirror>(v));
    if constexpr (G >= 16) v = fmaxf(v, dpp<kDppMirror>(v));
    if constexpr (G >= 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
    if constexpr (G >= 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// whole-wave reductions: rows by DPP, then the four row results by readlane
__device__ __forceinline__ float wave_sum(float v) {
    v = group_sum<16>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = group_max<16>(v);
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace loom
