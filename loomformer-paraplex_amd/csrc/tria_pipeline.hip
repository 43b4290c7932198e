// Tria path of the chunked sequence forward: per-token depth composition
// through L layers, the boundary-to-boundary temporal carry and PolARM at
// fires, producing the document keys the Tria readout pools.
//
// Restates the Tria part of Model._forward_chunked (loomformer.py:3788-3883):
//   boundaries are the grid positions (t+1) % W == 0 (never t = T-1,
//   :3802-3805) plus, with explicit <CARRY> fires, every position where any
//   row fires (:3797-3801, :3811-3815); chunks run from one boundary to the
//   next ([cW, min(cW+W, T)) on the grid alone) and the last one ends at T-1;
//   a row's fire at a boundary t is (grid(t) & ~reset[t+1]) | explicit[t]
//   (hard_fire & ~next_is_reset | explicit_fire, :3808-3810), and every
//   boundary emits a key for every row with that fire as its validity;
//   layer l of token t uses axis l % 3: C_1 = N(T_1), C_l = N(T_l C_{l-1})
//   (_block_core :3588-3617; tria_init / tria_step, tria.py:814-910), and the
//   first token of chunk c >= 1 starts from the seed when it is valid
//   (tria_init_seed, tria.py:835-844);
//   the temporal endpoint runs acc = N(D_t acc) over the chunk, restarting at
//   document resets and at a seeded first token
//   (temporal_carry_endpoint_reference, tria.py:1089-1123);
//   at a boundary the state becomes polarm(state) where the fire is valid
//   (tria.py:128-139) and is the boundary's document key.
//
// Work split.  N is a positive rescale, so every carry is a positive multiple
// of the plain product of its local matrices, and the seed enters a chunk only
// through its first token's layer-1 product: D_s(seeded) ~ D_s seed.  Hence
//   endpoint_c ~ E_c seed,   E_c = N(D_{e-1} ... N(D_s))   (unseeded),
// the reassociation the reference's own scan relies on (temporal_carry_pytorch,
// tria.py:1044-1085, valid while no local RMS falls below sqrt(eps); the
// operators built here are rotations times (I + K) with |K| <= alpha, whose RMS
// stays near 1/sqrt(3)).
//   tria_chunk_kernel: one thread per (b, chunk, h) composes all L layers of
//     each of its tokens in registers and folds them into E_c, streaming the
//     r, i, o stacks once (12 B per token-layer); nothing per layer touches HBM.
//   tria_chunk_scan_kernel: one thread per (b, h) runs the short sequential
//     scan over chunks: state = E_c (restart) or N(E_c state), PolARM at valid
//     fires, keys out, and the seeded first-token rows of the optional
//     per-token depth output.  Seeded or not, the next chunk's endpoint is
//     N(E_c state) unless a document starts inside it: a seeded first token
//     restarts the endpoint at D_s ~ D_s(unseeded) state, an unseeded one
//     continues from state.
#include <cmath>
#include <vector>

#include "loom_common.h"
#include "tria_math.h"

namespace loom {

constexpr int kChunkThreads = 256;

struct TriaChunkArgs {
    const void* r;
    const void* i;
    const void* o;
    int64_t layer_stride;      // elements between consecutive layers' [B,T,H] slices
    int L;
    const uint8_t* reset;      // [B,T] or null
    float* E;                  // [B, NC, 9, H] chunk products (slot-major, coalesced in h)
    uint8_t* restarted;        // [B, NC]: a reset lies inside the chunk
    void* depth_out;           // [B,T,H,9] dtype or null
    float* keys;               // [B, K, H, 9] fp32
    const int32_t* cend;       // [NC] exclusive chunk ends, or null: the grid [cW, min(cW+W, T))
    const uint8_t* efire;      // [B,T] explicit fires or null
    uint8_t* key_valid;        // [B, K] or null
    int64_t B, T, H;
    int W, NC, HB, K;          // K = boundaries = keys: NC-1, or NC when T-1 is one
    float alpha, polarm_beta, eps;
};

// First position and length of chunk c.
__device__ __forceinline__ void chunk_span(const TriaChunkArgs& a, int c, int64_t& s, int& nt) {
    if (a.cend != nullptr) {
        s = c == 0 ? 0 : a.cend[c - 1];
        nt = (int)(a.cend[c] - s);
    } else {
        s = (int64_t)c * a.W;
        nt = (int)((a.T - s) < a.W ? (a.T - s) : a.W);
    }
}

// C <- T(r,i,o) C.  A token's first layer starts from C = I, for which the
// product is exactly T (every term is a multiply by 1 or an add of 0), so one
// branch-free body serves both tria_init and tria_step.
template <int AXIS>
__device__ __forceinline__ void tria_mul(float r, float i, float o, float alpha, float C[9]) {
    float mt[9], pre[9];
    carrier9_fast<AXIS>(r, i, o, alpha, mt);
    mm3(mt, C, pre);
#pragma unroll
    for (int k = 0; k < 9; ++k) C[k] = pre[k];
}

__device__ __forceinline__ void normalize9_fast(float C[9]) {
    const float inv = rms9_inv_fast(C);
#pragma unroll
    for (int k = 0; k < 9; ++k) C[k] *= inv;
}

// A pointer every lane of the wave holds, moved to scalar registers.
__device__ __forceinline__ const char* uniform_ptr(const char* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const char*)(((uint64_t)hi << 32) | lo);
}

// Raw buffer loads over one layer slice: the descriptor (base, byte size) is
// scalar and each lane adds only its 32-bit byte offset, so a load costs no
// vector address arithmetic.  Offsets past `bytes` read zero.
constexpr int kBufNT = 2;                   // cache policy: nontemporal (r, i, o are read once)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slice_rsrc(const char* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)uniform_ptr(base), (short)0, (int)bytes,
                                             kBufferDword3);
}
template <typename T> __device__ __forceinline__ float ld_buf(__amdgpu_buffer_rsrc_t r, uint32_t off);
template <> __device__ __forceinline__ float ld_buf<float>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kBufNT));
}
template <> __device__ __forceinline__ float ld_buf<bf16_t>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, kBufNT));
}
template <> __device__ __forceinline__ float ld_buf<f16_t>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __half2float(__ushort_as_half(__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, kBufNT)));
}

// Byte offsets of a layer slice: 32-bit when one slice is under 4 GiB (the
// loads then take a uniform 64-bit base and a 32-bit per-lane offset).
template <bool WIDE> struct SliceOff { using type = uint32_t; };
template <> struct SliceOff<true> { using type = uint64_t; };

// FULL: L % 3 == 0, every group has its three layers.
template <typename T, bool DOUT, bool FULL, bool WIDE>
__global__ void __launch_bounds__(kChunkThreads)
tria_chunk_kernel(TriaChunkArgs a) {
    using off_t = typename SliceOff<WIDE>::type;
    int64_t blk = blockIdx.x;
    const int hb = (int)(blk % a.HB);
    blk /= a.HB;
    const int c = (int)(blk % a.NC);
    const int64_t b = blk / a.NC;
    const int64_t h = (int64_t)hb * kChunkThreads + threadIdx.x;
    int64_t s;
    int nt;
    chunk_span(a, c, s, nt);
    const uint8_t* rst = a.reset != nullptr ? a.reset + b * a.T + s : nullptr;
    if (h == 0) {
        uint8_t any = 0;
        if (rst != nullptr)
            for (int t = 0; t < nt; ++t) any |= rst[t];
        a.restarted[b * a.NC + c] = any != 0;
    }
    if (h >= a.H) return;

    const char* rp = (const char*)a.r;
    const char* ip = (const char*)a.i;
    const char* op = (const char*)a.o;
    const int64_t row0 = (b * a.T + s) * a.H + h;       // (b, s, h) inside one layer slice
    const off_t off0 = (off_t)(row0 * (int64_t)sizeof(T));
    const off_t tstep = (off_t)(a.H * (int64_t)sizeof(T));
    const int64_t lstep = a.layer_stride * (int64_t)sizeof(T);
    const uint32_t slice_bytes = (uint32_t)(a.B * a.T * a.H * (int64_t)sizeof(T));
    const int G = (a.L + 2) / 3;                        // groups of 3 layers (axes 0, 1, 2)

    // Groups of 3 layers (axes 0, 1, 2) stream through two register buffers:
    // the loads of group j+1 are in flight while group j is composed.
    auto load_group = [&](float (&dst)[9], off_t toff, int g) {
#pragma unroll
        for (int ax = 0; ax < 3; ++ax) {
            const int l = 3 * g + ax;
            if (FULL || l < a.L) {
                const int64_t lb = (int64_t)l * lstep;
                if constexpr (WIDE) {
                    dst[3 * ax] = ld((const T*)(rp + lb + toff));
                    dst[3 * ax + 1] = ld((const T*)(ip + lb + toff));
                    dst[3 * ax + 2] = ld((const T*)(op + lb + toff));
                } else {
                    dst[3 * ax] = ld_buf<T>(slice_rsrc(rp + lb, slice_bytes), toff);
                    dst[3 * ax + 1] = ld_buf<T>(slice_rsrc(ip + lb, slice_bytes), toff);
                    dst[3 * ax + 2] = ld_buf<T>(slice_rsrc(op + lb, slice_bytes), toff);
                }
            }
        }
    };
    float C[9], acc[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        C[k] = (k % 4 == 0) ? 1.0f : 0.0f;
        acc[k] = 0.0f;
    }
    bool have = false;
    int t = 0, g = 0, j = 0;
    off_t toff = off0;                // offset of the group being loaded next
    int gl = 0;                       // its group index
    const int J = nt * G;
    auto advance_load = [&]() {
        if (++gl == G) { gl = 0; toff += tstep; }
    };
    // Compose group j from v (its loads were issued one group earlier), issue
    // group j+1's loads into nb first.  The chain is renormalised once per
    // group: N is a positive rescale, so this moves only where the 1e-6 inside
    // N enters, by a relative 1e-6 of a scale the token's final N removes.
    auto step = [&](float (&v)[9], float (&nb)[9]) {
        if (j + 1 < J) {
            load_group(nb, toff, gl);
            advance_load();
        }
        tria_mul<0>(v[0], v[1], v[2], a.alpha, C);
        if (FULL || 3 * g + 1 < a.L) tria_mul<1>(v[3], v[4], v[5], a.alpha, C);
        if (FULL || 3 * g + 2 < a.L) tria_mul<2>(v[6], v[7], v[8], a.alpha, C);
        normalize9_fast(C);
        if (++g == G) {  // token t composed through depth: D_t = C
            g = 0;
            if constexpr (DOUT) {
                T* d = (T*)a.depth_out + (row0 + (int64_t)t * a.H) * 9;
#pragma unroll
                for (int k = 0; k < 9; ++k) st(d + k, C[k]);
            }
            float pre[9];
            const bool restart = !have || (rst != nullptr && rst[t] != 0);
            if (restart) {
#pragma unroll
                for (int k = 0; k < 9; ++k) pre[k] = C[k];
            } else {
                mm3(C, acc, pre);
            }
            const float inv = rms9_inv_fast(pre);
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                acc[k] = pre[k] * inv;
                C[k] = (k % 4 == 0) ? 1.0f : 0.0f;
            }
            have = true;
            ++t;
        }
        ++j;
    };
    float va[9], vb[9];
    load_group(va, toff, gl);
    advance_load();
    while (true) {
        step(va, vb);
        if (j == J) break;
        step(vb, va);
        if (j == J) break;
    }
    float* e = a.E + ((b * a.NC + c) * 9) * a.H + h;
#pragma unroll
    for (int k = 0; k < 9; ++k) e[k * a.H] = acc[k];
}

template <typename T, bool DOUT>
__global__ void __launch_bounds__(kChunkThreads)
tria_chunk_scan_kernel(TriaChunkArgs a) {
    const int64_t sid = (int64_t)blockIdx.x * kChunkThreads + threadIdx.x;
    if (sid >= a.B * a.H) return;
    const int64_t b = sid / a.H;
    const int64_t h = sid - b * a.H;
    const int K = a.K;
    float S[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) S[k] = 0.0f;
    const float* e = a.E + (b * a.NC * 9) * a.H + h;
    float nx[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) nx[k] = e[k * a.H];
    for (int c = 0; c < K; ++c) {
        float Ec[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) Ec[k] = nx[k];
        if (c + 1 < K) {
            const float* en = e + (int64_t)(c + 1) * 9 * a.H;
#pragma unroll
            for (int k = 0; k < 9; ++k) nx[k] = en[k * a.H];
        }
        if (c == 0 || a.restarted[b * a.NC + c] != 0) {
#pragma unroll
            for (int k = 0; k < 9; ++k) S[k] = Ec[k];
        } else {
            // the chunk continues the state (seeded first token, or a plain
            // continuation when the previous boundary did not fire)
            float pre[9];
            mm3(Ec, S, pre);
            const float inv = 1.0f / rms9(pre);
#pragma unroll
            for (int k = 0; k < 9; ++k) S[k] = pre[k] * inv;
        }
        // boundary t = snext - 1; snext == T only for a fire at T-1
        int64_t snext;
        int nt;
        chunk_span(a, c, snext, nt);
        snext += nt;
        const bool next_reset = snext < a.T && a.reset != nullptr && a.reset[b * a.T + snext] != 0;
        const bool grid = a.cend == nullptr || (snext % a.W == 0 && snext < a.T);
        const bool valid = (grid && !next_reset) ||
                           (a.efire != nullptr && a.efire[b * a.T + snext - 1] != 0);
        if (valid) polarm9(S, a.polarm_beta, a.eps);
        float* kp = a.keys + ((b * K + c) * a.H + h) * 9;
#pragma unroll
        for (int k = 0; k < 9; ++k) kp[k] = S[k];
        if (a.key_valid != nullptr && h == 0) a.key_valid[b * K + c] = valid ? 1 : 0;
        if constexpr (DOUT) {
            // the next chunk's first token was seeded (seed_valid = fire &
            // ~reset there): D = N(T_L ... N(T_1 seed))
            if (valid && !next_reset && snext < a.T) {
                T* d = (T*)a.depth_out + ((b * a.T + snext) * a.H + h) * 9;
                float u[9], pre[9];
#pragma unroll
                for (int k = 0; k < 9; ++k) u[k] = ld(d + k);
                mm3(u, S, pre);
                const float inv = 1.0f / rms9(pre);
#pragma unroll
                for (int k = 0; k < 9; ++k) st(d + k, pre[k] * inv);
            }
        }
    }
}

template <typename T, bool DOUT, bool FULL>
static void launch_chunk(const TriaChunkArgs& a, dim3 grid, hipStream_t st) {
    const bool wide = a.B * a.T * a.H * (int64_t)sizeof(T) >= (1LL << 32);
    if (wide)
        hipLaunchKernelGGL((tria_chunk_kernel<T, DOUT, FULL, true>), grid, dim3(kChunkThreads), 0,
                           st, a);
    else
        hipLaunchKernelGGL((tria_chunk_kernel<T, DOUT, FULL, false>), grid, dim3(kChunkThreads), 0,
                           st, a);
}

template <typename T>
static int chunked_dispatch(TriaChunkArgs a, hipStream_t st) {
    const dim3 blk(kChunkThreads);
    const dim3 g1((unsigned)(a.B * a.NC * a.HB));
    const dim3 g2((unsigned)ceil_div(a.B * a.H, kChunkThreads));
    const bool full = a.L % 3 == 0;
    if (a.depth_out != nullptr) {
        if (full) launch_chunk<T, true, true>(a, g1, st);
        else launch_chunk<T, true, false>(a, g1, st);
        if (a.K > 0) hipLaunchKernelGGL((tria_chunk_scan_kernel<T, true>), g2, blk, 0, st, a);
    } else {
        if (full) launch_chunk<T, false, true>(a, g1, st);
        else launch_chunk<T, false, false>(a, g1, st);
        if (a.K > 0) hipLaunchKernelGGL((tria_chunk_scan_kernel<T, false>), g2, blk, 0, st, a);
    }
    return launch_status("loom_tria_chunked_forward");
}

// Workspace of NC chunks: E, the restart flags, the chunk ends.
static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }
static int64_t chunks_ws_bytes(int64_t B, int64_t H, int64_t NC) {
    return align256(B * NC * 9 * H * 4) + align256(B * NC) + align256(NC * 4);
}
static int64_t chunked_ws_bytes(int64_t B, int64_t T, int64_t H, int64_t W) {
    return chunks_ws_bytes(B, H, ceil_div(T, W));
}

// Chunk count of a boundary list: one chunk per boundary, plus the tail when
// T-1 is not a boundary.
static int64_t chunks_of(int64_t T, const int64_t* bounds, int64_t n_bounds) {
    return n_bounds + ((n_bounds == 0 || bounds[n_bounds - 1] != T - 1) ? 1 : 0);
}

static int chunked_dtype_dispatch(int dtype, const TriaChunkArgs& a, hipStream_t st) {
    switch (dtype) {
        case LOOM_F32: return chunked_dispatch<float>(a, st);
        case LOOM_BF16: return chunked_dispatch<bf16_t>(a, st);
        case LOOM_F16: return chunked_dispatch<f16_t>(a, st);
    }
    set_error("tria_chunked: unsupported dtype %d", dtype);
    return LOOM_ERR_INVALID;
}

}  // namespace loom

using namespace loom;

extern "C" int64_t loom_tria_chunked_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t W) {
    if (B < 0 || T < 1 || H < 0 || W < 1) return -1;
    return chunked_ws_bytes(B, T, H, W);
}

// Shape checks and argument block shared by both entry points.
static int chunked_args(TriaChunkArgs& a, const void* r, const void* i, const void* o,
                        int64_t layer_stride, int64_t L, const uint8_t* reset, float* keys,
                        void* depth_out, int64_t B, int64_t T, int64_t H, int64_t W, int64_t NC,
                        int64_t K, float alpha, float polarm_beta, float eps, void* ws,
                        int64_t ws_bytes) {
    LOOM_CHECK(r && i && o, "tria_chunked: null r/i/o");
    LOOM_CHECK(B >= 0 && T >= 1 && H >= 0 && L >= 1 && W >= 1,
               "tria_chunked: bad shape B=%lld T=%lld H=%lld L=%lld W=%lld", (long long)B,
               (long long)T, (long long)H, (long long)L, (long long)W);
    LOOM_CHECK(L <= 4096, "tria_chunked: L=%lld layers is beyond the supported 4096", (long long)L);
    LOOM_CHECK(W <= (1 << 20), "tria_chunked: window W=%lld too large", (long long)W);
    LOOM_CHECK(T < (1LL << 31), "tria_chunked: T=%lld too large", (long long)T);
    LOOM_CHECK(layer_stride >= B * T * H || L == 1,
               "tria_chunked: layer_stride %lld smaller than one [B,T,H] slice",
               (long long)layer_stride);
    LOOM_CHECK(polarm_beta >= 0.0f && polarm_beta < 1.0f,
               "PolARM beta must be finite and in [0, 1), got %g", (double)polarm_beta);
    LOOM_CHECK(K == 0 || keys != nullptr, "tria_chunked: keys output required (%lld boundaries)",
               (long long)K);
    LOOM_CHECK(ws != nullptr && ws_bytes >= chunks_ws_bytes(B, H, NC),
               "tria_chunked: workspace of %lld bytes, need %lld", (long long)ws_bytes,
               (long long)chunks_ws_bytes(B, H, NC));
    LOOM_CHECK(B * NC * ceil_div(H, kChunkThreads) < (1LL << 31), "tria_chunked: grid too large");
    a.r = r; a.i = i; a.o = o; a.layer_stride = layer_stride; a.L = (int)L; a.reset = reset;
    a.E = (float*)ws;
    a.restarted = (uint8_t*)ws + align256(B * NC * 9 * H * 4);
    a.depth_out = depth_out; a.keys = keys;
    a.B = B; a.T = T; a.H = H; a.W = (int)W; a.NC = (int)NC; a.K = (int)K;
    a.HB = (int)ceil_div(H, kChunkThreads);
    a.alpha = alpha; a.polarm_beta = polarm_beta; a.eps = eps;
    return LOOM_OK;
}

extern "C" int loom_tria_chunked_forward(int dtype, const void* r, const void* i, const void* o,
                                         int64_t layer_stride, int64_t L, const uint8_t* reset,
                                         float* keys, void* depth_out, void* ws, int64_t ws_bytes,
                                         int64_t B, int64_t T, int64_t H, int64_t W, float alpha,
                                         float polarm_beta, float eps, void* stream) {
    clear_error();
    LOOM_CHECK(T >= 1 && W >= 1, "tria_chunked: need T >= 1 and W >= 1");
    const int64_t NC = ceil_div(T, W);
    TriaChunkArgs a{};
    int rc = chunked_args(a, r, i, o, layer_stride, L, reset, keys, depth_out, B, T, H, W, NC, NC - 1,
                          alpha, polarm_beta, eps, ws, ws_bytes);
    if (rc != LOOM_OK || B * H == 0) return rc;
    return chunked_dtype_dispatch(dtype, a, (hipStream_t)stream);
}

extern "C" int64_t loom_tria_chunked_fires_workspace_bytes(int64_t B, int64_t T, int64_t H,
                                                           const int64_t* bounds, int64_t n_bounds) {
    if (B < 0 || T < 1 || H < 0 || n_bounds < 0 || (n_bounds > 0 && bounds == nullptr)) return -1;
    return chunks_ws_bytes(B, H, chunks_of(T, bounds, n_bounds));
}

extern "C" int loom_tria_chunked_forward_fires(int dtype, const void* r, const void* i,
                                               const void* o, int64_t layer_stride, int64_t L,
                                               const uint8_t* reset, const uint8_t* explicit_fire,
                                               const int64_t* bounds, int64_t n_bounds, float* keys,
                                               uint8_t* key_valid, void* depth_out, void* ws,
                                               int64_t ws_bytes, int64_t B, int64_t T, int64_t H,
                                               int64_t W, float alpha, float polarm_beta, float eps,
                                               void* stream) {
    clear_error();
    LOOM_CHECK(T >= 1 && W >= 1, "tria_chunked: need T >= 1 and W >= 1");
    LOOM_CHECK(n_bounds >= 0 && (n_bounds == 0 || bounds != nullptr), "tria_chunked: null boundary list");
    // the boundary list is the grid plus the explicit fire positions: sorted,
    // in range, and holding every grid position
    int64_t grid_seen = 0;
    for (int64_t k = 0; k < n_bounds; ++k) {
        LOOM_CHECK(bounds[k] >= 0 && bounds[k] < T, "tria_chunked: boundary %lld outside [0, %lld)",
                   (long long)bounds[k], (long long)T);
        LOOM_CHECK(k == 0 || bounds[k] > bounds[k - 1], "tria_chunked: boundaries must increase");
        grid_seen += ((bounds[k] + 1) % W == 0 && bounds[k] != T - 1) ? 1 : 0;
    }
    LOOM_CHECK(grid_seen == (T - 1) / W,
               "tria_chunked: the boundary list lacks %lld of the %lld grid positions (t+1) %% %lld == 0",
               (long long)((T - 1) / W - grid_seen), (long long)((T - 1) / W), (long long)W);
    const int64_t NC = chunks_of(T, bounds, n_bounds);
    TriaChunkArgs a{};
    int rc = chunked_args(a, r, i, o, layer_stride, L, reset, keys, depth_out, B, T, H, W, NC, n_bounds,
                          alpha, polarm_beta, eps, ws, ws_bytes);
    if (rc != LOOM_OK || B * H == 0) return rc;
    // exclusive chunk ends, uploaded to the workspace; the stream is synchronised
    // so the host array may go out of scope (the caller built the list on the host,
    // after a device-to-host read of the fire mask, as the reference does)
    std::vector<int32_t> ends((size_t)NC);
    for (int64_t k = 0; k < n_bounds; ++k) ends[(size_t)k] = (int32_t)(bounds[k] + 1);
    ends[(size_t)NC - 1] = (int32_t)T;
    int32_t* dend = (int32_t*)((uint8_t*)ws + align256(B * NC * 9 * H * 4) + align256(B * NC));
    hipStream_t st = (hipStream_t)stream;
    LOOM_CHECK(hipMemcpyAsync(dend, ends.data(), (size_t)NC * sizeof(int32_t), hipMemcpyHostToDevice, st) ==
                   hipSuccess && hipStreamSynchronize(st) == hipSuccess,
               "tria_chunked: chunk-end upload failed");
    a.cend = dend;
    a.efire = explicit_fire;
    a.key_valid = key_valid;
    return chunked_dtype_dispatch(dtype, a, st);
}
