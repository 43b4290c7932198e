// Row-major K / V tiles in LDS for the MFMA attention kernels (decode and
// prefill): 16-byte pieces of each row stored swizzled, read back as the A
// operand of S^T = K Q^T (16-byte reads of whole rows) and, through the gfx950
// transposing LDS read, as the B operand of C = P V and Kctx = P K.
#pragma once

#include "loom_common.h"

namespace loom {

// Piece swizzle: piece c of row r sits at c ^ kv_swz(r) (bits 1, 2 of r to
// bits 0, 1).  Chosen by timing both read forms on gfx950 over every 2-bit
// swizzle of 192-byte rows (HD = 96): a 16-byte fragment read takes 5.0 LDS
// cycles and a transposing read 2.6 (the 1024 and 512 bytes they move need
// 4 and 2), against 8.7 and 4.4 with the two bits crossed (bits 1, 2 to 1, 0)
// and 9.3 and 4.7 with unswizzled rows padded to 13 pieces.  The pieces of a
// row stay a permutation of 0..HD/8-1 (HD/8 a multiple of 4).
__device__ __forceinline__ int kv_swz(int r) { return ((r >> 1) & 1) | (((r >> 2) & 1) << 1); }

typedef short gqa_v4s __attribute__((ext_vector_type(4)));
typedef uint32_t gqa_u4 __attribute__((ext_vector_type(4)));   // a 16-byte piece as a native vector

// Lane constants of the fragment reads of a row-major tile (byte offsets
// within the tile), computed once per kernel so that every read is one LDS
// instruction with a compile-time offset:
//   s_off[hf]: the A operand of S^T = K Q^T, 16-byte read of row 16*hf + l%16,
//     piece 4*kk + l/16 -> s_off[hf] + 64*kk (the swizzle only touches the
//     piece's low two bits);
//   t_off[p][h]: tile_tr_frag's read h of dim tile dt with dt % 2 == p ->
//     t_off[p][h] + 64*(dt/2) (piece (2*dt + b) ^ kv_swz(row) is
//     4*(dt/2) + a lane constant for each parity of dt).
// PITCH: pieces per LDS row (CPR, or more to spread rows over the banks);
// SWZ: pieces stored at c ^ kv_swz(r) (else at c).
template <int CPR, int PITCH = CPR, bool SWZ = true>
struct TileLane {
    uint32_t s_off[2];
    uint32_t t_off[2][2];
    __device__ __forceinline__ TileLane(int lq, int lr) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const int row = 16 * hf + lr;
            s_off[hf] = (uint32_t)((row * PITCH + (SWZ ? lq ^ kv_swz(row) : lq)) * 16);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int row = 16 * h + 4 * lq + (lr >> 2);
            const int sw = SWZ ? kv_swz(row) : 0, b1 = (lr & 3) >> 1;
#pragma unroll
            for (int par = 0; par < 2; ++par) {
                const int q = ((par ^ (sw >> 1)) << 1) | (b1 ^ (sw & 1));
                t_off[par][h] = (uint32_t)((row * PITCH + q) * 16 + 8 * (lr & 1));
            }
        }
    }
};

// A operand of S^T (16 K rows x 32 dims of k-step kk) from a row-major tile
template <int CPR, int PITCH, bool SWZ>
__device__ __forceinline__ gqa_u4 tile_s_frag(const gqa_u4* tile, const TileLane<CPR, PITCH, SWZ>& L,
                                              int hf, int kk) {
    return *reinterpret_cast<const gqa_u4*>(reinterpret_cast<const char*>(tile) + L.s_off[hf] + 64 * kk);
}

// B fragment of 32 positions x 16 dims (dims 16*dt..) from a row-major tile,
// its 8 positions per lane in the order of a score tile's registers: lane
// group q (= l/16) gets rows 4q..4q+3 and 16+4q..16+4q+3 of dim 16*dt + l%16,
// the positions whose probabilities the lanes of group q hold after
// S^T = K Q^T (result register r of 16-row half hf is row 16*hf + 4q + r), so
// P feeds P V and P K straight from registers.  Two transposing 8-byte reads:
// lane r of a 16-lane group points at row k0 + r/4, dims 16*dt + 4*(r%4)..+3
// and receives rows k0..k0+3 of dim 16*dt + r (k0 = 16*h + 4q).
template <int CPR, int PITCH, bool SWZ>
__device__ __forceinline__ uint4 tile_tr_frag(const gqa_u4* tile, const TileLane<CPR, PITCH, SWZ>& L,
                                              int dt) {
    uint2 w[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const char* p = reinterpret_cast<const char*>(tile) + L.t_off[dt & 1][h] + 64 * (dt >> 1);
        w[h] = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                             (__attribute__((address_space(3))) gqa_v4s*)(p)));
    }
    return make_uint4(w[0].x, w[0].y, w[1].x, w[1].y);
}

// LDS ordering inside one wave (its LDS operations execute in order): keeps
// the compiler from moving LDS accesses across; no wait, no s_barrier.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

}  // namespace loom
