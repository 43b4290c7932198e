// Dense projections for gfx950: out[M,N] = epilogue(X[M,K] @ W[N,K]^T).
//
// bf16: MFMA v_mfma_f32_16x16x32_bf16, fp32 accumulation.  Block tile
// 128 (n) x 128 (m) x 64 (k), four waves each owning a 64x64 sub-tile as 4x4
// MFMA tiles.  The MFMA A operand is the weight tile (rows n), the B operand
// the activation tile (columns m), so each lane's four accumulator values are
// four consecutive n of one output row m (one 8-byte store).  Both tiles are
// K-contiguous in LDS with rows padded to 144 B, so the 16-byte fragment reads
// of 16 consecutive rows fall in distinct banks.
//
// fp32/fp16: SIMT tile 64x64x16, 4x4 outputs per thread, fp32 FMA.
//
// "Gather" mode is the grouped W_imag product of ParaplexFFN: the activation
// row of hidden group g is the concatenation of sector slices
// [Q_g | Kctx_g | C_g | U | D_g] (head sectors) or [Q_g | Kctx | C | U | D]
// (open sectors); the loader reads each 8-element piece from its sector, so
// the packed matrix is never written to HBM.
#include <atomic>
#include <cmath>
#include <type_traits>
#include <utility>

#include "depth_row.h"
#include "loom_common.h"
#include "paraplex_math.h"
#include "tria_math.h"

namespace loom {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf(uint16_t x) { return bf16_to_f32(x); }
__device__ __forceinline__ float round_bf(float x) { return bf16_to_f32(f32_to_bf16(x)); }

struct GemmArgs {
    const void* X;
    int64_t ldx;
    const void* W;
    int64_t ldw;
    const float* bias;
    const void* gate_p;
    float gate_alpha;
    const void* residual;
    void* out;
    int64_t ldc;
    int64_t M, N, K;
    // gather mode (beta space)
    const void* src[5];  // Q, Kctx, C, U, D  (each [M, Nm] row-major)
    int64_t Nm, HD, Hq;
    int open;
    const uint4* Uf;     // head sectors: fragment-major copy of U (the skinny form reads its
                         // sector from it), or null
    // big kernel only (not gather): a second input along K, k >= K1 reading
    // X2 / W2 at k - K1 (X2 null: one input), and split-K, the K range in
    // nsplit equal parts with fp32 sums to partial[(split*M + m)*ldp + n] and
    // no epilogue (partial null: the epilogue, nsplit 1)
    const void* X2;
    int64_t ldx2;
    const void* W2;
    int64_t ldw2, K1;
    float* partial;
    int64_t ldp;
    int nsplit;
    // big kernel only (not gather, no gate or residual): columns N1 .. N-1 of
    // the launch are a second product of the same X with weight rows Wb
    // (stride ldwb), written to outb (stride ldcb) with bias biasb, so two
    // projections of one activation share a launch; tiles never straddle N1
    // (N1 0: one product)
    int64_t N1;
    const void* Wb;
    int64_t ldwb;
    void* outb;
    int64_t ldcb;
    const float* biasb;
    // big kernel with 96-column wave tiles only: the first product's columns
    // are the heads [q (QH) | k (KVH) | v (KVH)] of 96; with rope.q set its
    // epilogue applies RoPE to q and k and writes q to rope.q ([M, QH*96]),
    // k and v into the caches at position start + m % Tc of row b = m / Tc,
    // instead of writing out
    struct RopeOut {
        void* q;
        void* kc;
        void* vc;
        int64_t csb, cst, csh;     // cache strides (elements) of b, t and kv head
        const float* cosv;         // [*, 96] fp32 tables (attention factor folded in)
        const float* sinv;
        int64_t Tc, start;
        int QH, KVH;
    } rope;
};

// Element offset of packed column kk of group g, and which source it is in.
__device__ __forceinline__ const void* gather_ptr(const GemmArgs& a, int64_t m, int64_t kk,
                                                  int64_t g, int elem_size) {
    int s;
    int64_t col;
    const int64_t HD = a.HD, Nm = a.Nm;
    if (!a.open) {
        if (kk < HD) { s = 0; col = g * HD + kk; }
        else if (kk < 2 * HD) { s = 1; col = g * HD + kk - HD; }
        else if (kk < 3 * HD) { s = 2; col = g * HD + kk - 2 * HD; }
        else if (kk < 3 * HD + Nm) { s = 3; col = kk - 3 * HD; }
        else { s = 4; col = g * HD + kk - 3 * HD - Nm; }
    } else {
        if (kk < HD) { s = 0; col = g * HD + kk; }
        else if (kk < HD + Nm) { s = 1; col = kk - HD; }
        else if (kk < HD + 2 * Nm) { s = 2; col = kk - HD - Nm; }
        else if (kk < HD + 3 * Nm) { s = 3; col = kk - HD - 2 * Nm; }
        else { s = 4; col = kk - HD - 3 * Nm; }
    }
    // the source picked by masks over constant indices, so the pointers stay
    // in scalar registers: an array indexed by a per-lane value is read from
    // memory, and the wait for that read also drains the operand loads in
    // flight (a select chain is folded back into such a read)
    uintptr_t base = 0;
#pragma unroll
    for (int i = 0; i < 5; ++i) base |= (uintptr_t)a.src[i] & (uintptr_t)(-(intptr_t)(s == i));
    return (const char*)base + (m * Nm + col) * elem_size;
}

template <typename T>
__device__ __forceinline__ float epilogue(const GemmArgs& a, int64_t m, int64_t n, float v) {
    if (a.gate_p != nullptr) v *= 1.0f + a.gate_alpha * ld((const T*)a.gate_p + m * a.ldc + n);
    if (a.bias != nullptr) v += a.bias[n];
    if (a.residual != nullptr) v += ld((const T*)a.residual + m * a.ldc + n);
    return v;
}

// ------------------------------------------------------------------ MFMA bf16

constexpr int MB_M = 128, MB_N = 128, MB_K = 64;

template <bool GATHER>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_bf16_mfma_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t Ws[2][MB_N * MB_K];
    __shared__ __attribute__((aligned(16))) uint16_t Xs[2][MB_M * MB_K];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1;
    const int64_t n0 = (int64_t)blockIdx.x * MB_N;
    const int64_t m0 = (int64_t)blockIdx.y * MB_M;
    const int64_t g = GATHER ? n0 / a.Hq : 0;
    const uint16_t* W = (const uint16_t*)a.W;
    const uint16_t* X = (const uint16_t*)a.X;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Tiles are 64 k per row (128 B) with the 16-byte chunk c of row r stored at
    // chunk c ^ ((r >> 1) & 7): the 16 rows of a fragment read and the two rows
    // of 8 chunks in a 16-lane store each cover all 64 banks once.
    auto lds_off = [](int r, int c) { return r * MB_K + ((c ^ ((r >> 1) & 7)) << 3); };
    auto load_tiles = [&](int64_t k0, uint4 (&wr)[4], uint4 (&xr)[4]) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int chunk = tid + c * 256;
            const int row = chunk >> 3;
            const int64_t k = k0 + (chunk & 7) * 8;
            const int64_t n = n0 + row;
            const int64_t m = m0 + row;
            uint4 wv = make_uint4(0, 0, 0, 0), xv = make_uint4(0, 0, 0, 0);
            if (n < a.N && k < a.K) wv = *reinterpret_cast<const uint4*>(W + n * a.ldw + k);
            if (m < a.M && k < a.K) {
                if constexpr (GATHER)
                    xv = *reinterpret_cast<const uint4*>(gather_ptr(a, m, k, g, 2));
                else
                    xv = *reinterpret_cast<const uint4*>(X + m * a.ldx + k);
            }
            wr[c] = wv;
            xr[c] = xv;
        }
    };
    auto store_tiles = [&](int buf, const uint4 (&wr)[4], const uint4 (&xr)[4]) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int chunk = tid + c * 256;
            const int off = lds_off(chunk >> 3, chunk & 7);
            *reinterpret_cast<uint4*>(&Ws[buf][off]) = wr[c];
            *reinterpret_cast<uint4*>(&Xs[buf][off]) = xr[c];
        }
    };
    const int fr = lane & 15;          // fragment row
    const int fc = lane >> 4;          // fragment 8-element chunk within a 32-wide k-step
    auto compute = [&](int buf) {
#pragma unroll
        for (int kk = 0; kk < MB_K / 32; ++kk) {
            bf16x8 af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                af[i] = *reinterpret_cast<const bf16x8*>(&Ws[buf][lds_off(wn * 64 + i * 16 + fr, 4 * kk + fc)]);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                bf[j] = *reinterpret_cast<const bf16x8*>(&Xs[buf][lds_off(wm * 64 + j * 16 + fr, 4 * kk + fc)]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };
    // Barrier for the LDS tiles only: the global loads of later k-tiles stay in
    // flight (each is waited for where its registers are stored to LDS).
    auto lds_sync = []() {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };

    // k-tile t lives in LDS buffer t & 1; its global loads are issued one
    // k-step ahead and waited for where they are stored to LDS
    const int64_t nk = ceil_div(a.K, MB_K);
    uint4 wr[4], xr[4];
    load_tiles(0, wr, xr);
    store_tiles(0, wr, xr);
    lds_sync();
    for (int64_t kt = 0; kt < nk; ++kt) {
        const int cur = (int)(kt & 1);
        const bool more = kt + 1 < nk;
        if (more) load_tiles((kt + 1) * MB_K, wr, xr);
        compute(cur);
        if (more) store_tiles(cur ^ 1, wr, xr);
        lds_sync();
    }

    uint16_t* out = (uint16_t*)a.out;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t nb = n0 + wn * 64 + i * 16 + (lane >> 4) * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t m = m0 + wm * 64 + j * 16 + (lane & 15);
            if (m >= a.M) continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
                v[r] = (nb + r < a.N) ? epilogue<bf16_t>(a, m, nb + r, acc[i][j][r]) : 0.0f;
            uint16_t* op = out + m * a.ldc + nb;
            if (nb + 3 < a.N && ((uintptr_t)op & 7) == 0) {
                const uint32_t lo = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
                const uint32_t hi = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
                *reinterpret_cast<uint2*>(op) = make_uint2(lo, hi);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (nb + r < a.N) op[r] = f32_to_bf16(v[r]);
            }
        }
    }
}

// ------------------------------------------------------------------ big bf16 (M >= 256)
// Block tile 256 (m) x 128 (n), v_mfma_f32_16x16x32_bf16 with fp32
// accumulators.  BgCfg<WAVES, WGM, KH, WPE, NS> sets the waves of a block (WGM of
// them along m, so a wave owns a (256/WGM) x (128*WGM/WAVES) sub-tile), the
// 32-wide k-halves per pipeline stage (KH) and the waves per SIMD the register
// budget is sized for.  Operand tiles travel from global memory straight into
// LDS (buffer_load_dwordx4 ... lds, no register staging) through NS stages,
// each its own LDS array so the compiler's waits name exactly the stage they
// need: k-tiles t+1 .. t+NS-1 are in flight while t is computed.
//
// LDS layout of a stage: [k-half h][row][4 chunks of 8 k] (64 B rows), chunk c
// of row r stored at position c ^ bg_swz(r) = c ^ 2*(bit 3 of r).  gfx950
// serves a 16-byte ds_read one half-wave per cycle, 8 bytes per lane, from 128
// banks of 4 bytes, so the 32 lanes of a half-wave are conflict-free when their
// 16-byte pieces are distinct modulo 512 B.  A fragment read's half-wave takes
// chunks {0, 1} or {2, 3} of 16 rows; rows r and r + 8 lie 512 B apart, and the
// swizzle moves the second of them to the other two positions (measured: 4 LDS
// cycles per read, no bank-conflict cycles).  One DMA instruction of a wave fills 16
// rows of one k-half (lane l: row l/4, position l%4; the lane fetches the
// chunk the swizzle puts there), so its 32 k lie in one gather sector and the
// source and column offset are uniform (scalar) per instruction; per lane only
// a 32-bit row offset per 16-row group is held, and the k advance is the
// scalar soffset.  Requires K % (32 * KH * NS) == 0 (whole rounds of the
// stages).
__host__ __device__ constexpr int bg_swz(int r) { return ((r >> 3) & 1) << 1; }
// Full-line stages (no gather, 64 k per stage): a stage row is the whole
// 128-byte line [8 chunks of 8 k], chunk c of row r at position c ^ bg_swz8(r)
// = c ^ (r & 7).  One DMA instruction fills 8 whole rows (lane l: row l/8,
// position l%8), 8 full lines.  The swizzle was chosen by timing ds_read_b128
// fragment reads over 128-byte rows (a calibration kernel, 16-row x 4-chunk
// pattern): c ^ (r & 7) and c ^ ((r >> 1) & 7) read at the rate of a linear
// 1 KB read (2.7-2.9 ns per wave-read per CU), c ^ 2*((r >> 2) & 3) at 3.5
// (2-way), no swizzle at 7.0; the model that fits 64-byte rows (a half-wave's
// pieces distinct modulo 512 B) does not predict these.
__host__ __device__ constexpr int bg_swz8(int r) { return r & 7; }

template <int BM_, int BN_, int WAVES_, int WGM_, int KH_, int WPE_, int NS_>
struct BgCfg {
    static constexpr int BG_M = BM_, BG_N = BN_;               // block tile
    static constexpr int WAVES = WAVES_, WGM = WGM_, KH = KH_, WPE = WPE_, NS = NS_;
    static constexpr int BK = 32 * KH;                         // k per stage
    static constexpr int WTM = BG_M / WGM, WTN = BG_N / (WAVES / WGM);   // wave sub-tile
    static constexpr int FJ = WTM / 16, FI = WTN / 16;         // x and w fragments per k-step
    // DMA row groups per wave; W groups rounded up when BG_N / 16 does not
    // divide over the waves (the groups past BG_N fetch an in-range row into a
    // scratch LDS row nobody reads, so every wave issues the same count)
    static constexpr int XG = BG_M / 16 / WAVES, WG = (BG_N / 16 + WAVES - 1) / WAVES;
    static constexpr bool WPAD = WG * WAVES * 16 != BG_N;
    static constexpr int DMA = KH * (XG + WG);                 // DMA instructions per lane per stage
    static constexpr int LDS = NS * KH * (BG_M + BG_N) * 32 * 2 + (WPAD ? 1024 : 0);
    static_assert(WAVES % WGM == 0 && XG * WAVES * 16 == BG_M && WG >= 1 && (KH == 1 || KH == 2),
                  "big GEMM shape");
    static_assert(NS >= 3 && NS <= 6 && (NS - 1) * DMA < 64 && LDS <= 160 * 1024, "big GEMM stages");
};
using BgConf = BgCfg<256, 128, 8, 4, 2, 2, 3>;
// 128 x 128 tiles (four waves of 64 x 64, one 32-wide k-half per stage, four
// stages, two blocks per CU) and 128 x 256 tiles (eight waves of 64 x 64, 64 k
// per stage in three full-line stages: 8192 x 3072 x 768 52 us against 58-62
// with four 32-k stages): the smaller tile fills the CUs when the 256 x 128
// tiles leave many idle or end in a partial round, the wider one serves
// many-row products with N a multiple of 256
using BgSmall = BgCfg<128, 128, 4, 2, 1, 2, 4>;
using BgWide = BgCfg<128, 256, 8, 2, 2, 2, 3>;
// 256 x 192 tiles (eight waves of 64 x 96, four 32-k stages): at M = 4096 and
// N = 3072 they make 256 tiles, one round of the CUs, where 256 x 128 or
// 128 x 256 make 384 (a round and a half)
using BgTall = BgCfg<256, 192, 8, 4, 1, 2, 4>;
// 128 x 192 tiles of four waves of 64 x 96 (80 KB, two blocks per CU), for
// shared-tile mode (loom_gemm_shared_tiles): alone they are slower than
// 256 x 192 (4096 x 3072 x 768: 32.3 against 30.0 us; 1.4x the operand
// traffic per flop), but a block holds half a CU, so another stream's
// kernels run beside the product instead of waiting for a whole CU to drain
// (the chunked prefill: 63.8 -> 62.0 ms)
using BgTallS = BgCfg<128, 192, 4, 2, 1, 2, 4>;

// Source and element offset (within the source's row) of the 32 packed
// columns [kk, kk + 32) of group g in gather mode; they lie in one sector.
__device__ __forceinline__ void gather_half(const GemmArgs& a, int64_t kk, int64_t g,
                                            const void*& src, int64_t& col) {
    const int64_t HD = a.HD, Nm = a.Nm;
    if (!a.open) {                                   // [Q_g | Kctx_g | C_g | U | D_g]
        if (kk < HD) { src = a.src[0]; col = g * HD + kk; }
        else if (kk < 2 * HD) { src = a.src[1]; col = g * HD + kk - HD; }
        else if (kk < 3 * HD) { src = a.src[2]; col = g * HD + kk - 2 * HD; }
        else if (kk < 3 * HD + Nm) { src = a.src[3]; col = kk - 3 * HD; }
        else { src = a.src[4]; col = g * HD + kk - 3 * HD - Nm; }
    } else {                                         // [Q_g | Kctx | C | U | D]
        if (kk < HD) { src = a.src[0]; col = g * HD + kk; }
        else if (kk < HD + Nm) { src = a.src[1]; col = kk - HD; }
        else if (kk < HD + 2 * Nm) { src = a.src[2]; col = kk - HD - Nm; }
        else if (kk < HD + 3 * Nm) { src = a.src[3]; col = kk - HD - 2 * Nm; }
        else { src = a.src[4]; col = kk - HD - 3 * Nm; }
    }
}

// Scheduling hints of one k-step: NR fragment reads (and the first ND of them
// each preceded by a DMA request) spread evenly over NMM MFMAs, group GRP.
template <int NMM, int NR, int ND, int GRP, int Q>
__device__ __forceinline__ void bg_sched_step() {
    if constexpr (Q < ND) __builtin_amdgcn_sched_group_barrier(0x0020, 1, GRP);   // VMEM read
    __builtin_amdgcn_sched_group_barrier(0x0100, 1, GRP);                         // DS read
    constexpr int n = NMM * (Q + 1) / NR - NMM * Q / NR;
    if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x0008, n, GRP);    // MFMA
}
// f(integral_constant<int, s>) for s = 0 .. N-1, in order
template <class F, int... S>
__device__ __forceinline__ void bg_static_for_(F&& f, std::integer_sequence<int, S...>) {
    (f(std::integral_constant<int, S>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void bg_static_for(F&& f) {
    bg_static_for_(f, std::make_integer_sequence<int, N>{});
}
template <int NMM, int NR, int ND, int GRP, int... Q>
__device__ __forceinline__ void bg_interleave(std::integer_sequence<int, Q...>) {
    static_assert(ND <= NR, "more DMA requests than fragment reads");
    (bg_sched_step<NMM, NR, ND, GRP, Q>(), ...);
}

template <bool GATHER, class C>
__global__ void __launch_bounds__(64 * C::WAVES) __attribute__((amdgpu_waves_per_eu(C::WPE, C::WPE)))
gemm_bf16_big_kernel(GemmArgs a) {
    constexpr int BG_M = C::BG_M, BG_N = C::BG_N;
    constexpr int XH = BG_M * 32, WH = BG_N * 32;   // elements per k-half of a stage
    constexpr int KH = C::KH, FI = C::FI, FJ = C::FJ, XG = C::XG, WG = C::WG, DMA = C::DMA;
    constexpr int NS = C::NS;
    // full-line stages (bg_swz8) for the products without a gather at 64 k per
    // stage; XQ / WQ DMA slots per wave (8 rows each, else 16 rows of a k-half)
    constexpr bool FL = !GATHER && KH == 2;
    constexpr int XQ = FL ? 2 * XG : XG, WQ = FL ? 2 * WG : WG;
    // stage s: X_s, W_s (separate arrays, so a wait for one stage's DMA never
    // covers another's reads); arrays of stages >= NS are not referenced
    __shared__ __attribute__((aligned(16))) uint16_t X0[KH * XH], X1[KH * XH], X2[KH * XH],
        X3[NS > 3 ? KH * XH : 8], X4[NS > 4 ? KH * XH : 8], X5[NS > 5 ? KH * XH : 8];
    __shared__ __attribute__((aligned(16))) uint16_t W0[KH * WH], W1[KH * WH], W2[KH * WH],
        W3[NS > 3 ? KH * WH : 8], W4[NS > 4 ? KH * WH : 8], W5[NS > 5 ? KH * WH : 8];
    // landing rows of the padding W groups (BgCfg::WPAD), never read
    __shared__ __attribute__((aligned(16))) uint16_t Wpad[C::WPAD ? 512 : 8];
    auto xs = [&](auto s_) -> uint16_t* {
        constexpr int S = decltype(s_)::value;
        if constexpr (S == 0) return X0; else if constexpr (S == 1) return X1;
        else if constexpr (S == 2) return X2; else if constexpr (S == 3) return X3;
        else if constexpr (S == 4) return X4; else return X5;
    };
    auto ws = [&](auto s_) -> uint16_t* {
        constexpr int S = decltype(s_)::value;
        if constexpr (S == 0) return W0; else if constexpr (S == 1) return W1;
        else if constexpr (S == 2) return W2; else if constexpr (S == 3) return W3;
        else if constexpr (S == 4) return W4; else return W5;
    };
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % C::WGM, wn = wave / C::WGM;
    // Tile of this block.  Blocks are dispatched round-robin over the 8 XCDs
    // (block b runs on XCD b % 8), each with its own L2: when the m-tiles
    // split evenly, XCD x takes m-tiles [x*MT/8, (x+1)*MT/8) and walks the
    // n-tiles with its m-tiles innermost, so the tiles resident on one XCD at
    // a time share their X rows and a few W column blocks in its L2.
    const int64_t MT = ceil_div(a.M, BG_M), NT = ceil_div(a.N, BG_N);
    // split-K: block x takes split x / (MT*NT) of the K range, tile x % (MT*NT)
    const int64_t split = a.partial != nullptr ? (int64_t)blockIdx.x / (MT * NT) : 0;
    const int64_t b = (int64_t)blockIdx.x - split * MT * NT;
    const int64_t kspan = a.partial != nullptr ? a.K / a.nsplit : a.K;
    const int64_t kbase = split * kspan;
    int64_t mt, nt;
    if (MT % 8 == 0) {
        const int64_t mpx = MT / 8, li = b / 8;
        mt = (b % 8) * mpx + li % mpx;
        nt = li / mpx;
    } else {
        mt = b / NT;
        nt = b % NT;
    }
    int64_t n0 = nt * BG_N;
    const int64_t m0 = mt * BG_M;
    bool seg_b = false;
    if (!GATHER && a.N1 > 0) {               // block-uniform: this tile's product
        if (n0 >= a.N1) {
            seg_b = true;
            n0 -= a.N1;
            a.N -= a.N1;
            a.W = a.Wb; a.ldw = a.ldwb; a.out = a.outb; a.ldc = a.ldcb; a.bias = a.biasb;
            a.gate_p = nullptr; a.residual = nullptr;     // the first product's only
        } else {
            a.N = a.N1;
        }
    }
    const int64_t g = GATHER ? n0 / a.Hq : 0;
    const int64_t ldx = GATHER ? a.Nm : a.ldx;

    // DMA slots: X 16-row groups XG*wave + q, W groups WG*wave + q, each for
    // every k-half; lane: row 16*group + lane/4, chunk (lane%4) ^ bg_swz(row);
    // rows past M / N read the last row (their results are not stored)
    // (full-line stages: X groups of 8 rows XQ*wave + q, lane: row 8*group +
    // lane/8, chunk (lane%8) ^ bg_swz8(row))
    auto slot_row = [&](int q, int per) {
        return FL ? 8 * (per * wave + q) + (lane >> 3) : 16 * (per * wave + q) + (lane >> 2);
    };
    auto slot_pos = [&](int r) { return FL ? (lane & 7) ^ bg_swz8(r) : (lane & 3) ^ bg_swz(r); };
    uint32_t xv[XQ], wv[WQ];
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
        const int r = slot_row(q, XQ);
        const int64_t rr = m0 + r < a.M ? r : a.M - 1 - m0;
        xv[q] = (uint32_t)((rr * ldx + 8 * slot_pos(r)) * 2);
    }
#pragma unroll
    for (int q = 0; q < WQ; ++q) {
        const int r = slot_row(q, WQ);
        const int64_t rr = n0 + r < a.N ? r : a.N - 1 - n0;
        wv[q] = (uint32_t)((rr * a.ldw + 8 * slot_pos(r)) * 2);
    }
    const auto rw = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint16_t*)a.W + n0 * a.ldw),
                                                      (short)0, 0x7fffffff, kBufferDword3);
    const auto rx = __builtin_amdgcn_make_buffer_rsrc(
        GATHER ? (void*)nullptr : (void*)((const uint16_t*)a.X + m0 * a.ldx), (short)0, 0x7fffffff,
        kBufferDword3);
    // second input (k >= K1): its own row offsets and descriptors
    const bool dual = !GATHER && a.X2 != nullptr;
    const int64_t K1 = dual ? a.K1 : a.K;
    uint32_t xv2[XQ], wv2[WQ];
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
        const int r = slot_row(q, XQ);
        const int64_t rr = m0 + r < a.M ? r : a.M - 1 - m0;
        xv2[q] = dual ? (uint32_t)((rr * a.ldx2 + 8 * slot_pos(r)) * 2) : 0u;
    }
#pragma unroll
    for (int q = 0; q < WQ; ++q) {
        const int r = slot_row(q, WQ);
        const int64_t rr = n0 + r < a.N ? r : a.N - 1 - n0;
        wv2[q] = dual ? (uint32_t)((rr * a.ldw2 + 8 * slot_pos(r)) * 2) : 0u;
    }
    const auto rw2 = __builtin_amdgcn_make_buffer_rsrc(
        dual ? (void*)((const uint16_t*)a.W2 + n0 * a.ldw2) : (void*)nullptr, (short)0, 0x7fffffff,
        kBufferDword3);
    const auto rx2 = __builtin_amdgcn_make_buffer_rsrc(
        dual ? (void*)((const uint16_t*)a.X2 + m0 * a.ldx2) : (void*)nullptr, (short)0, 0x7fffffff,
        kBufferDword3);
    // the DMA requests of the stage holding k-tile k0 / C::BK, one instruction
    // per call of dma_one(q), q < DMA (so they can be spread over the MFMAs)
    auto dma_one = [&](int q, int64_t k0, uint16_t* Xs, uint16_t* Ws) {
        if constexpr (FL) {
            const bool second = k0 >= K1;           // uniform: K1 is a multiple of the stage k
            const uint32_t sk = (uint32_t)((second ? k0 - K1 : k0) * 2);
            if (q < XQ)
                dma16(second ? rx2 : rx, Xs + 8 * (XQ * wave + q) * 64, second ? xv2[q] : xv[q], sk);
            else
            {
                const int gw = WQ * wave + q - XQ;
                uint16_t* dst = Ws + 8 * gw * 64;
                if constexpr (C::WPAD) dst = 8 * gw < BG_N ? dst : Wpad;
                dma16(second ? rw2 : rw, dst, second ? wv2[q - XQ] : wv[q - XQ], sk);
            }
            return;
        }
        const int h = q / (XG + WG), p = q % (XG + WG);
        const int64_t k = k0 + 32 * h;
        const bool second = !GATHER && k >= K1;     // uniform: K1 is a multiple of the stage k
        const uint32_t sk = (uint32_t)((second ? k - K1 : k) * 2);
        if (p < XG) {
            auto rxh = second ? rx2 : rx;
            uint32_t sx = sk;
            if constexpr (GATHER) {
                const void* src;
                int64_t col;
                gather_half(a, k, g, src, col);
                rxh = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint16_t*)src + m0 * a.Nm),
                                                        (short)0, 0x7fffffff, kBufferDword3);
                sx = (uint32_t)(col * 2);
            }
            dma16(rxh, Xs + h * XH + 16 * (XG * wave + p) * 32, second ? xv2[p] : xv[p], sx);
        } else {
            const int w = p - XG;
            const int gw = WG * wave + w;
            uint16_t* dst = Ws + h * WH + 16 * gw * 32;
            if constexpr (C::WPAD) dst = 16 * gw < BG_N ? dst : Wpad;
            dma16(second ? rw2 : rw, dst, second ? wv2[w] : wv[w], sk);
        }
    };
    auto issue = [&](int64_t k0, uint16_t* Xs, uint16_t* Ws) {
#pragma unroll
        for (int q = 0; q < DMA; ++q) dma_one(q, k0, Xs, Ws);
    };

    f32x4 acc[FI][FJ];
#pragma unroll
    for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // fragment of k-step kk: row base + 16*i + fr of half kk, chunk fc at its
    // swizzled position (bg_swz(row) = bg_swz(fr) for every tile: bases are
    // multiples of 16)
    const int fr = lane & 15, fc = lane >> 4;
    const int lo = fr * 32 + ((fc ^ bg_swz(fr)) << 3);
    // full-line stages: k-step kk of row fr at chunk 4*kk + fc
    const int lo8[2] = {fr * 64 + ((fc ^ bg_swz8(fr)) << 3), fr * 64 + (((4 + fc) ^ bg_swz8(fr)) << 3)};
    struct Frags {
        bf16x8 w[FI], x[FJ];
    };
    auto read = [&](Frags& f, const uint16_t* Xs, const uint16_t* Ws, int kk) {
        if constexpr (FL) {
#pragma unroll
            for (int i = 0; i < FI; ++i)
                f.w[i] = *reinterpret_cast<const bf16x8*>(&Ws[(wn * C::WTN + i * 16) * 64 + lo8[kk]]);
#pragma unroll
            for (int j = 0; j < FJ; ++j)
                f.x[j] = *reinterpret_cast<const bf16x8*>(&Xs[(wm * C::WTM + j * 16) * 64 + lo8[kk]]);
            return;
        }
#pragma unroll
        for (int i = 0; i < FI; ++i)
            f.w[i] = *reinterpret_cast<const bf16x8*>(&Ws[kk * WH + (wn * C::WTN + i * 16) * 32 + lo]);
#pragma unroll
        for (int j = 0; j < FJ; ++j)
            f.x[j] = *reinterpret_cast<const bf16x8*>(&Xs[kk * XH + (wm * C::WTM + j * 16) * 32 + lo]);
    };
    // MFMAs of x-fragments [j0, j1) (the fragments of a half die after it)
    auto mma = [&](const Frags& f, auto j0_, auto j1_) {
        constexpr int j0 = decltype(j0_)::value, j1 = decltype(j1_)::value;
#pragma unroll
        for (int j = j0; j < j1; ++j)
#pragma unroll
            for (int i = 0; i < FI; ++i)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.w[i], f.x[j], acc[i][j], 0, 0, 0);
    };
    using I0 = std::integral_constant<int, 0>;
    using IH = std::integral_constant<int, FJ / 2>;
    using IF = std::integral_constant<int, FJ>;
    constexpr int NR = FI + FJ;        // fragment reads per k-step
    constexpr int NM = FI * FJ;        // MFMAs per k-step
    using T_ = std::true_type;
    using F_ = std::false_type;
    using SEQ = std::make_integer_sequence<int, NR>;

    // Tile t lives in stage t % NS; all NS stages are requested up front and
    // tile t+NS into t's stage as soon as every wave has read t (nk = K / BK
    // is a multiple of NS).  Straight-line code per stage, so every wait is a
    // constant.  Iteration t (f0 = the first k-step of t, already in
    // registers):
    //   KH = 2: read k-step 1 of t; MFMAs of k-step 0; wait for tile t+1's DMA
    //           and every wave's reads of t (barrier); request tile t+NS into
    //           t's stage; read k-step 0 of t+1 (f0); MFMAs of k-step 1.
    //   KH = 1: MFMAs of the first half of the x-fragments; wait and barrier;
    //           request tile t+NS; read tile t+1 (f1); the second half; f0 = f1.
    const int64_t nk = kspan / C::BK;
    bg_static_for<NS>([&](auto s_) { issue(kbase + decltype(s_)::value * C::BK, xs(s_), ws(s_)); });
    wait_vmcnt<(NS - 1) * DMA>();
    __builtin_amdgcn_s_barrier();
    Frags f0, f1;
    read(f0, X0, W0, 0);
    // S: stage of tile t; NEXT: tile t+1 exists; OUT: tiles after t+1 that
    // may still be in flight at its wait; ISSUE: tile t+NS exists
    auto iter = [&](auto s_, auto next_, auto out_, auto issue_, int64_t t) {
        constexpr int S = decltype(s_)::value, OUT = decltype(out_)::value;
        constexpr bool NEXT = decltype(next_)::value, ISSUE = decltype(issue_)::value;
        uint16_t* Xc = xs(s_);
        uint16_t* Wc = ws(s_);
        const uint16_t* Xn = xs(std::integral_constant<int, (S + 1) % NS>{});
        const uint16_t* Wn = ws(std::integral_constant<int, (S + 1) % NS>{});
        if constexpr (KH == 2) {
            read(f1, Xc, Wc, 1);
            mma(f0, I0{}, IF{});
            bg_interleave<NM, NR, 0, 0>(SEQ{});
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (NEXT) {
                wait_vmcnt<OUT * DMA>();
                __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's reads of t landed
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (ISSUE) issue(kbase + (t + NS) * C::BK, Xc, Wc);
                read(f0, Xn, Wn, 0);
            }
            mma(f1, I0{}, IF{});
            if constexpr (NEXT) bg_interleave<NM, NR, ISSUE ? DMA : 0, 1>(SEQ{});
            __builtin_amdgcn_sched_barrier(0);
        } else {
            mma(f0, I0{}, IH{});
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (NEXT) {
                wait_vmcnt<OUT * DMA>();
                __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's reads of t landed
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (ISSUE) issue(kbase + (t + NS) * C::BK, Xc, Wc);
                read(f1, Xn, Wn, 0);
            }
            mma(f0, IH{}, IF{});
            if constexpr (NEXT) bg_interleave<NM - NM / 2, NR, ISSUE ? DMA : 0, 1>(SEQ{});
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (NEXT) f0 = f1;
        }
    };
    for (int64_t t = 0; t < nk - NS; t += NS) {
        bg_static_for<NS>([&](auto s_) {
            iter(s_, T_{}, std::integral_constant<int, NS - 2>{}, T_{}, t + decltype(s_)::value);
        });
    }
    bg_static_for<NS>([&](auto s_) {
        constexpr int S = decltype(s_)::value;
        iter(s_, std::bool_constant<(S < NS - 1)>{}, std::integral_constant<int, (S < NS - 1 ? NS - 2 - S : 0)>{},
             F_{}, nk - NS + S);
    });

    // epilogue: output group gi = (i, j) holds the 4 consecutive columns
    // gcol(gi) = ncol + 16i .. +3 of row grow(gi) = mrow + 16j; its bias
    // operand depends on i only.  Whole tiles take straight-line code with
    // 8-byte stores (one variant per gate / residual combination, chosen once
    // per block); edge tiles check every element.
    constexpr int NG = FI * FJ;
    constexpr int NB = FI;
    const int64_t mrow = m0 + wm * C::WTM + (lane & 15);
    const int64_t ncol = n0 + wn * C::WTN + (lane >> 4) * 4;
    auto scol = [&](int sl) -> int64_t { return ncol + 16 * sl; };
    auto gslot = [&](int gi) -> int { return gi / FJ; };
    auto gcol = [&](int gi) -> int64_t { return scol(gslot(gi)); };
    auto grow = [&](int gi) -> int64_t { return mrow + 16 * (gi % FJ); };
    auto gval = [&](int gi, int r) -> float { return acc[gi / FJ][gi % FJ][r]; };
    // Staged stores: a wave's finished tile goes to a wave-private LDS region,
    // row-major with its 16-byte pieces permuted within each row, and each
    // lane then stores 16 contiguous bytes of a row, so the output leaves in
    // row runs instead of 16 rows of 32 or 64 bytes per store (the
    // 8-byte-per-lane form made the bf16 epilogue of 4096 x 3072 x 768 take
    // 30.4 against 26.2 us with row runs).  The regions are carved out of the
    // stage arrays, X arrays first, after one barrier (every wave has read its
    // last stage).
    auto stage_region = [&](auto bytes_) -> uint16_t* {
        constexpr int BYTES = decltype(bytes_)::value;
        constexpr int RX = KH * XH * 2 / BYTES, RW = KH * WH * 2 / BYTES;
        uint16_t* reg = nullptr;
        int q = wave;
        bg_static_for<NS>([&](auto s_) {
            if (reg == nullptr) {
                if (q < RX) reg = xs(s_) + q * (BYTES / 2);
                else q -= RX;
            }
        });
        bg_static_for<NS>([&](auto s_) {
            if (reg == nullptr) {
                if (q < RW) reg = ws(s_) + q * (BYTES / 2);
                else q -= RW;
            }
        });
        return reg;
    };
    // regions of BYTES for every wave
    constexpr int REG2 = C::WTM * C::WTN * 2, REG4 = 2 * REG2;
    constexpr bool FIT2 = NS * (KH * XH * 2 / REG2 + KH * WH * 2 / REG2) >= C::WAVES;
    constexpr bool FIT4 = NS * (KH * XH * 2 / REG4 + KH * WH * 2 / REG4) >= C::WAVES;
    static_assert(FIT2 && C::WTN % 32 == 0, "staging regions");
    if constexpr (!GATHER && C::WTN == 96) {
        if (a.rope.q != nullptr && !seg_b) {
            // the wave's 96 columns are one head; column d's rotation partner
            // d +- 48 sits in fragment i +- 3 of the same lane and register.
            // As the unfused path: the product rounded to bf16, then
            // fma(x, cos, (sign * partner) * sin), rounded on the store
            const GemmArgs::RopeOut& ro = a.rope;
            const int hd = (int)((n0 + wn * 96) / 96);
            const int dl = (lane >> 4) * 4;
            const bool rot = hd < ro.QH + ro.KVH;
            // the destination row of output row m (q row, or the cache row of its position)
            auto row_dst = [&](int64_t m) -> uint16_t* {
                const int64_t b = m / ro.Tc, pos = ro.start + (m - b * ro.Tc);
                if (hd < ro.QH) return (uint16_t*)ro.q + m * (int64_t)(ro.QH * 96) + hd * 96;
                if (rot) return (uint16_t*)ro.kc + b * ro.csb + pos * ro.cst + (hd - ro.QH) * ro.csh;
                return (uint16_t*)ro.vc + b * ro.csb + pos * ro.cst + (hd - ro.QH - ro.KVH) * ro.csh;
            };
            // staged (16-byte row pieces) when the block's rows are all in range
            // and every destination row is 16-byte aligned
            const bool st16 = m0 + BG_M <= a.M && ((ro.csb | ro.cst | ro.csh) & 7) == 0 &&
                              (((uintptr_t)ro.q | (uintptr_t)ro.kc | (uintptr_t)ro.vc) & 15) == 0;
            uint16_t* reg = nullptr;
            if (st16) {
                __syncthreads();            // every wave is done with the stages
                reg = stage_region(std::integral_constant<int, REG2>{});
            }
#pragma unroll
            for (int j = 0; j < FJ; ++j) {
                const int64_t m = mrow + 16 * j;
                if (m >= a.M) continue;
                const int64_t pos = ro.start + (m - (m / ro.Tc) * ro.Tc);
                uint16_t* dst = st16 ? nullptr : row_dst(m);
                float4 cv[FI], sv[FI];
#pragma unroll
                for (int i = 0; i < FI; ++i) {
                    cv[i] = rot ? *reinterpret_cast<const float4*>(ro.cosv + pos * 96 + 16 * i + dl)
                                : make_float4(1.f, 1.f, 1.f, 1.f);
                    sv[i] = rot ? *reinterpret_cast<const float4*>(ro.sinv + pos * 96 + 16 * i + dl)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
                for (int i = 0; i < FI; ++i) {
                    const int ip = i < 3 ? i + 3 : i - 3;
                    const float sg = i < 3 ? -1.0f : 1.0f;
                    const float c4[4] = {cv[i].x, cv[i].y, cv[i].z, cv[i].w};
                    const float s4[4] = {sv[i].x, sv[i].y, sv[i].z, sv[i].w};
                    float v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float x = round_bf(acc[i][j][r]), y = round_bf(acc[ip][j][r]);
                        v[r] = rot ? fmaf(x, c4[r], (sg * y) * s4[r]) : x;
                    }
                    const uint2 w = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
                    if (st16) {
                        const int rl = 16 * j + (lane & 15), cl = 16 * i + dl;
                        *reinterpret_cast<uint2*>(reg + rl * 96 + 8 * ((cl >> 3) ^ ((rl >> 1) & 3)) + (cl & 7)) = w;
                    } else {
                        *reinterpret_cast<uint2*>(dst + 16 * i + dl) = w;
                    }
                }
            }
            if (st16) {
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int it = 0; it < C::WTM * 12 / 64; ++it) {
                    const int c = it * 64 + lane, row = c / 12, pc = c % 12;
                    *reinterpret_cast<uint4*>(row_dst(m0 + wm * C::WTM + row) + 8 * pc) =
                        *reinterpret_cast<const uint4*>(reg + row * 96 + 8 * (pc ^ ((row >> 1) & 3)));
                }
            }
            return;
        }
    }
    if (a.partial != nullptr) {
        // split-K: raw fp32 sums of this split, 16-byte stores where all four
        // columns are in range
        float* part = a.partial + split * a.M * a.ldp;
        if constexpr (FIT4) {
            if (m0 + BG_M <= a.M && n0 + BG_N <= a.N && (a.ldp & 3) == 0 && ((uintptr_t)part & 15) == 0) {
                // whole tile, staged: piece p (4 floats) of row r at p ^ (r & 15)
                __syncthreads();
                float* reg = reinterpret_cast<float*>(stage_region(std::integral_constant<int, REG4>{}));
                constexpr int PR = C::WTN / 4;          // 16-byte pieces of a wave-tile row
#pragma unroll
                for (int gi = 0; gi < NG; ++gi) {
                    const int rl = 16 * (gi % FJ) + (lane & 15);
                    const int pc = 4 * gslot(gi) + (lane >> 4);
                    *reinterpret_cast<float4*>(reg + rl * C::WTN + 4 * (pc ^ (rl & 15))) =
                        make_float4(gval(gi, 0), gval(gi, 1), gval(gi, 2), gval(gi, 3));
                }
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                __builtin_amdgcn_wave_barrier();
                float* orow = part + (m0 + wm * C::WTM) * a.ldp + n0 + wn * C::WTN;
#pragma unroll
                for (int it = 0; it < C::WTM * PR / 64; ++it) {
                    const int c = it * 64 + lane, row = c / PR, pc = c % PR;
                    *reinterpret_cast<float4*>(orow + row * a.ldp + 4 * pc) =
                        *reinterpret_cast<const float4*>(reg + row * C::WTN + 4 * (pc ^ (row & 15)));
                }
                return;
            }
        }
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
            const int64_t nb = gcol(gi), m = grow(gi);
            if (m >= a.M || nb >= a.N) continue;
            float* po = part + m * a.ldp + nb;
            if (nb + 3 < a.N && ((a.ldp | nb) & 3) == 0) {
                *reinterpret_cast<float4*>(po) = make_float4(gval(gi, 0), gval(gi, 1), gval(gi, 2), gval(gi, 3));
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (nb + r < a.N) po[r] = gval(gi, r);
            }
        }
        return;
    }
    uint16_t* out = (uint16_t*)a.out;
    const uint16_t* gp = (const uint16_t*)a.gate_p;
    const uint16_t* rs = (const uint16_t*)a.residual;
    const int64_t ldc = a.ldc;
    const bool whole = m0 + BG_M <= a.M && n0 + BG_N <= a.N && (ldc & 3) == 0 &&
                       (((uintptr_t)out | (uintptr_t)gp | (uintptr_t)rs) & 7) == 0 &&
                       ((uintptr_t)a.bias & 15) == 0;
    auto bf4 = [](uint2 w, float (&x)[4]) {
        x[0] = __uint_as_float(w.x << 16); x[1] = __uint_as_float(w.x & 0xffff0000u);
        x[2] = __uint_as_float(w.y << 16); x[3] = __uint_as_float(w.y & 0xffff0000u);
    };
    // whole tiles staged (bf16 piece p of row r at p ^ ((r >> 1) & 3))
    const bool staged = whole && (((uintptr_t)out & 15) == 0) && (ldc & 7) == 0;
    auto whole_tile = [&](auto gate_, auto res_) {
        constexpr bool GATE = decltype(gate_)::value, RES = decltype(res_)::value;
        uint16_t* reg = nullptr;
        if (staged) {
            __syncthreads();                // every wave is done with the stages
            reg = stage_region(std::integral_constant<int, REG2>{});
        }
        // every operand of the wave's outputs requested before the first store
        // (an output may alias them as far as the compiler knows, so a load
        // after a store would wait for it: one round trip per group)
        float4 bv[NB];
        uint2 gw[NG], rw[NG];
#pragma unroll
        for (int sl = 0; sl < NB; ++sl)
            bv[sl] = a.bias != nullptr ? *reinterpret_cast<const float4*>(a.bias + scol(sl))
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
            const int64_t e = grow(gi) * ldc + gcol(gi);
            if constexpr (GATE) gw[gi] = *reinterpret_cast<const uint2*>(gp + e);
            if constexpr (RES) rw[gi] = *reinterpret_cast<const uint2*>(rs + e);
        }
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
            const int64_t e = grow(gi) * ldc + gcol(gi);
            const float4 b4 = bv[gslot(gi)];
            const float bias4[4] = {b4.x, b4.y, b4.z, b4.w};
            float v[4], gv[4], rv[4];
            if constexpr (GATE) bf4(gw[gi], gv);
            if constexpr (RES) bf4(rw[gi], rv);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                v[r] = gval(gi, r);
                if constexpr (GATE) v[r] *= 1.0f + a.gate_alpha * gv[r];
                v[r] += bias4[r];
                if constexpr (RES) v[r] += rv[r];
            }
            const uint2 w = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
            if (staged) {
                const int rl = 16 * (gi % FJ) + (lane & 15);             // row of the wave tile
                const int cl = 16 * gslot(gi) + (lane >> 4) * 4;         // column of the wave tile
                *reinterpret_cast<uint2*>(reg + rl * C::WTN + 8 * ((cl >> 3) ^ ((rl >> 1) & 3)) + (cl & 7)) = w;
            } else {
                *reinterpret_cast<uint2*>(out + e) = w;
            }
        }
        if (staged) {
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
            constexpr int PR = C::WTN / 8;  // 16-byte pieces of a wave-tile row
            uint16_t* orow = out + (m0 + wm * C::WTM) * ldc + n0 + wn * C::WTN;
#pragma unroll
            for (int it = 0; it < C::WTM * PR / 64; ++it) {
                const int c = it * 64 + lane, row = c / PR, pc = c % PR;
                const uint4 v = *reinterpret_cast<const uint4*>(reg + row * C::WTN + 8 * (pc ^ ((row >> 1) & 3)));
                *reinterpret_cast<uint4*>(orow + row * ldc + 8 * pc) = v;
            }
        }
    };
    if (whole) {
        if (gp == nullptr && rs == nullptr) whole_tile(F_{}, F_{});
        else if (gp != nullptr && rs == nullptr) whole_tile(T_{}, F_{});
        else if (gp == nullptr && rs != nullptr) whole_tile(F_{}, T_{});
        else whole_tile(T_{}, T_{});
        return;
    }
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        const int64_t nb = gcol(gi), m = grow(gi);
        if (nb >= a.N || m >= a.M) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (nb + r >= a.N) continue;
            const int64_t e = m * ldc + nb + r;
            float v = gval(gi, r);
            if (gp != nullptr) v *= 1.0f + a.gate_alpha * bf16_to_f32(gp[e]);
            if (a.bias != nullptr) v += a.bias[nb + r];
            if (rs != nullptr) v += bf16_to_f32(rs[e]);
            out[e] = f32_to_bf16(v);
        }
    }
}

// ------------------------------------------------------------------ skinny bf16 (M <= 64)
// Decode-shaped products: the weight is streamed once and dominates traffic.
// Block = 16 weight rows (one MFMA n-tile) x all M rows (MT m-tiles of 16);
// its four waves split K into contiguous quarters.  Fragments are loaded
// straight from global memory in the MFMA operand layout (lane l: row l%16,
// 8 consecutive k at 8*(l/16)), kUnroll k-steps at a time so each lane keeps
// several 16-byte weight loads in flight.  The four partial tiles are summed
// through LDS and the epilogue is applied by all 256 threads.
// Main loop of the skinny product for the 16 columns starting at n0: every
// wave accumulates its k-range, the partial tiles land in red[] (summed by the
// caller's epilogue after the barrier).
// dl (gather, head sectors): the D sector comes from LDS rows dl + m*HD.
template <int MT, bool GATHER, int NW, int UN>
__device__ __forceinline__ void skinny_mainloop(const GemmArgs& a, int64_t n0,
                                                float (&red)[NW][MT][4][64],
                                                const uint16_t* dl = nullptr) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t g = GATHER ? n0 / a.Hq : 0;
    const int fr = lane & 15, fk = (lane >> 4) * 8;
    const uint16_t* W = (const uint16_t*)a.W;
    const uint16_t* X = (const uint16_t*)a.X;
    // k range of this wave, in whole 32-wide steps
    const int64_t nsteps = ceil_div(a.K, 32);
    const int64_t per = ceil_div(nsteps, NW);
    const int64_t s_begin = wave * per;
    const int64_t s_end = s_begin + per < nsteps ? s_begin + per : nsteps;
    const int64_t n = n0 + fr;
    const bool nvalid = n < a.N;

    f32x4 acc[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int64_t s0 = s_begin; s0 < s_end; s0 += UN) {
        uint4 wv[UN];
        uint4 xv[UN][MT];
#pragma unroll
        for (int u = 0; u < UN; ++u) {
            const int64_t k = (s0 + u) * 32 + fk;
            const bool kin = (s0 + u) < s_end && k < a.K;
            wv[u] = (kin && nvalid) ? *reinterpret_cast<const uint4*>(W + n * a.ldw + k)
                                    : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < MT; ++j) {
                const int64_t m = j * 16 + fr;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (kin && m < a.M) {
                    if constexpr (GATHER) {
                        // a 32-wide step lies in one sector (HD % 32 == 0 with Uf)
                        const int64_t ku = k - 3 * a.HD;
                        if (a.Uf != nullptr && ku >= 0 && ku < a.Nm)
                            v = a.Uf[(j * (a.Nm >> 5) + (ku >> 5)) * 64 + (threadIdx.x & 63)];
                        else if (dl != nullptr && ku >= a.Nm)   // head sectors: D from LDS
                            v = *reinterpret_cast<const uint4*>(dl + m * a.HD + (ku - a.Nm));
                        else
                            v = *reinterpret_cast<const uint4*>(gather_ptr(a, m, k, g, 2));
                    } else {
                        v = *reinterpret_cast<const uint4*>(X + m * a.ldx + k);
                    }
                }
                xv[u][j] = v;
            }
        }
#pragma unroll
        for (int u = 0; u < UN; ++u)
#pragma unroll
            for (int j = 0; j < MT; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8, wv[u]), __builtin_bit_cast(bf16x8, xv[u][j]), acc[j],
                    0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][j][r][lane] = acc[j][r];
    __syncthreads();
}

// Sum of the NW partial tiles for output (row mi, column nn) of the block:
// accumulator element of (m, nn) sits in lane m%16 + 16*(nn/4), register nn%4.
template <int MT, int NW>
__device__ __forceinline__ float skinny_sum(const float (&red)[NW][MT][4][64], int mi, int nn) {
    const int j = mi >> 4, ml = mi & 15;
    const int ln = ml + 16 * (nn >> 2), r = nn & 3;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += red[w][j][r][ln];
    return v;
}

template <int MT, bool GATHER, int NW, int UN>
__global__ void __launch_bounds__(NW * 64)
gemm_bf16_skinny_kernel(GemmArgs a) {
    __shared__ float red[NW][MT][4][64];
    const int64_t n0 = (int64_t)blockIdx.x * 16;
    skinny_mainloop<MT, GATHER, NW, UN>(a, n0, red);
    uint16_t* out = (uint16_t*)a.out;
    for (int o = threadIdx.x; o < MT * 256; o += NW * 64) {
        const int nn = o & 15, mi = o >> 4;       // mi in [0, 16*MT)
        const int64_t m = mi, nidx = n0 + nn;
        if (m >= a.M || nidx >= a.N) continue;
        const float v = skinny_sum<MT, NW>(red, mi, nn);
        out[m * a.ldc + nidx] = f32_to_bf16(epilogue<bf16_t>(a, m, nidx, v));
    }
}

// ------------------------------------------------------------------ fused decode FFN core
// One decode token of the Paraplex FFN and the Tria depth op in one launch
// (bf16): the beta-space gather product, then per output (b, h) in the
// epilogue the fused pointwise chain (phase, trace combine with the carried
// phase, softplus, PvPowLU; loomformer.py:2533-2560) and the Tria carrier
// composed onto the previous depth carry with its gate mix (tria.py:890-978).
// beta and I never leave registers.
struct FfnArgs {
    GemmArgs g;                 // beta space: out unused
    const uint16_t* R;          // p_real [M, H]
    const uint16_t* G;          // amplitude source [M, H]: R, or gate_proj(u)
    const float* ib;            // w1_imag_bias [H]
    uint16_t* trace;            // [M, H]: previous phase in, this token's phase out
    const float* tw;            // [H]
    float m;
    uint16_t* act;              // [M, H]
    uint16_t* s;                // [M, H] or null
    const uint16_t* prev;       // [M, H, 9] (mode 1)
    const uint16_t* seed;       // [M, H, 9] (mode 2)
    const uint8_t* valid;       // [M] (mode 2)
    const uint16_t* gate_w;     // [9] or null
    uint16_t* carry;            // [M, H, 9]
    uint16_t* p;                // [M, H] (with gate_w)
    float alpha;
    int mode, axis;
    uint16_t* actf;             // fragment-major copy of act, or null
    // optional depth read of the block's head computed in the launch (head
    // sectors): D = DepthAttn over history slots 0..dS-1, into LDS for the
    // gather and, by the first column block of each head, into src[4]
    const uint16_t* dq;         // [QH, HD] queries of the slot, or null
    const uint16_t* dk;
    const uint16_t* dv;
    int64_t dsbt, dss;
    int dS;
    float dscale;
    DepthRms drms;
    // optional: the read over slots 0..dS-2 (normalised fp32 rows [M, QH, HD]
    // and their log-sum-exp [M, QH]); the launch folds in slot dS-1 only
    const float* dpd;
    const float* dpl;
};


// cp: the carried (or seed) record of element e, loaded by the caller with
// the rest of the epilogue's operands; used when carry_in is set.
template <int AXIS>
__device__ __forceinline__ void ffn_tria(const FfnArgs& f, int64_t e, float r, float i, float o,
                                         const float (&cp)[9], bool carry_in) {
    float mt[9], pre[9];
    carrier9<AXIS>(r, i, o, f.alpha, mt);
    if (carry_in) {
        mm3(mt, cp, pre);
    } else {
#pragma unroll
        for (int k = 0; k < 9; ++k) pre[k] = mt[k];
    }
    const float inv = 1.0f / rms9(pre);
#pragma unroll
    for (int k = 0; k < 9; ++k) pre[k] *= inv;
    if (f.gate_w != nullptr) {
        float pv = 0.0f;
#pragma unroll
        for (int k = 0; k < 9; ++k) pv = fmaf(pre[k], bf(f.gate_w[k]), pv);
        f.p[e] = f32_to_bf16(pv);
    }
#pragma unroll
    for (int k = 0; k < 9; ++k) f.carry[e * 9 + k] = f32_to_bf16(pre[k]);
}

// DE > 0: the depth read is part of the launch (head_dim = 16*DE, DR: fixed-
// RMS q/k/v); the column blocks of a head then sit on one XCD (block b takes
// head b % QH, so with 8 heads each XCD's L2 serves one head's history rows to
// the head's blocks).
template <int MT, int NW, int UN, int DE = 0, bool DR = false>
__global__ void __launch_bounds__(NW * 64)
ffn_decode_kernel(FfnArgs f) {
    __shared__ float red[NW][MT][4][64];
    __shared__ __align__(16) uint16_t dsh[DE > 0 ? MT * 16 * 16 * DE : 8];   // D rows of the head
    const int64_t H = f.g.N;
    int64_t n0 = (int64_t)blockIdx.x * 16;
    const int QH = DE > 0 ? (int)(H / f.g.Hq) : 1;
    const int g = (int)(blockIdx.x % QH), t = (int)(blockIdx.x / QH);
    if constexpr (DE > 0) n0 = (int64_t)g * f.g.Hq + (int64_t)t * 16;
    // the depth read of the block's head (before the main loop: with the first
    // weight loads held across it the 16-wave block runs out of registers)
    auto depth = [&]() {
      if constexpr (DE > 0) {
        // M*16 rows (b, j) over NW*64 threads: up to 512 rows, so a 4-wave
        // block takes two rounds
        for (int row = (int)threadIdx.x; row < f.g.M * 16; row += NW * 64) {
            const int b = row >> 4, j = row & 15;
            uint16_t o16[DE];
            if (!DR && f.dpd != nullptr) {
                // the earlier slots' part of the read comes in; fold in slot dS-1
                const int r = b * QH + g;
                const int64_t off = (int64_t)b * f.dsbt + (int64_t)(f.dS - 1) * f.dss + g * 16 * DE + j * DE;
                float qv[DE], kn[DE], vn[DE], pd[DE], out[DE];
                RowIO<bf16_t, DE>::load((const bf16_t*)f.dq + g * 16 * DE + j * DE, qv);
                RowIO<bf16_t, DE>::load((const bf16_t*)f.dk + off, kn);
                RowIO<bf16_t, DE>::load((const bf16_t*)f.dv + off, vn);
                RowIO<float, DE>::load(f.dpd + (int64_t)r * 16 * DE + j * DE, pd);
                depth_fold_last<DE>(qv, kn, vn, pd, f.dpl[r], f.dscale, out);
#pragma unroll
                for (int k = 0; k < DE; ++k) o16[k] = f32_to_bf16(out[k]);
            } else {
                float qv[DE], acc[DE], m, l;
                depth_row_core<bf16_t, DE, 4, DR, false>(
                    (const bf16_t*)f.dq, (const bf16_t*)f.dk, (const bf16_t*)f.dv, f.dsbt, f.dss,
                    b * QH + g, j, f.dS, QH, f.dscale, f.drms, qv, acc, m, l);
                const float inv_l = 1.0f / l;
#pragma unroll
                for (int k = 0; k < DE; ++k) o16[k] = f32_to_bf16(acc[k] * inv_l);
            }
#pragma unroll
            for (int k = 0; k < DE; ++k) dsh[b * 16 * DE + j * DE + k] = o16[k];
            if (t == 0) {
                uint16_t* dg = (uint16_t*)f.g.src[4] + (int64_t)b * f.g.Nm + (int64_t)g * 16 * DE + j * DE;
#pragma unroll
                for (int k = 0; k < DE; ++k) dg[k] = o16[k];
            }
        }
        __syncthreads();
      }
    };
    // The epilogue's operands of this thread's elements (kIt of the block's
    // 16 x MT*16 outputs) do not depend on the product: they are requested
    // first, at clamped indices, and arrive during the depth read and the main
    // loop (the carried record is read whether or not it is used, from R's
    // first elements without one)
    constexpr int kIt = (MT * 256 + NW * 64 - 1) / (NW * 64);
    uint16_t e_cr[kIt][9], e_tr[kIt], e_x[kIt], e_g[kIt];
    float e_ib[kIt], e_tw[kIt];
    uint8_t e_valid[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int o0 = (int)threadIdx.x + it * NW * 64;
        const int o = o0 < MT * 256 ? o0 : MT * 256 - 1;
        const int64_t mc = (o >> 4) < f.g.M ? (o >> 4) : f.g.M - 1;
        const int64_t hc = n0 + (o & 15) < H ? n0 + (o & 15) : H - 1;
        const int64_t e = mc * H + hc;
        const uint16_t* src = f.mode == 1 ? f.prev + e * 9 : f.mode == 2 ? f.seed + e * 9 : f.R;
#pragma unroll
        for (int k = 0; k < 9; ++k) e_cr[it][k] = src[k];
        e_tr[it] = f.trace[e];
        e_x[it] = f.R[e];
        e_g[it] = f.G[e];
        e_ib[it] = f.ib[hc];
        e_tw[it] = f.tw[hc];
        e_valid[it] = f.mode == 2 ? f.valid[mc] : 0;
    }
    if constexpr (DE > 0) {
        depth();
        skinny_mainloop<MT, true, NW, UN>(f.g, n0, red, dsh);
    } else {
        skinny_mainloop<MT, true, NW, UN>(f.g, n0, red);
    }
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int o = (int)threadIdx.x + it * NW * 64;
        const int nn = o & 15, mi = o >> 4;
        const int64_t m = mi, h = n0 + nn;
        if (o >= MT * 256 || m >= f.g.M || h >= H) continue;
        const int64_t e = m * H + h;
        const bool carry_in = f.mode == 1 || (f.mode == 2 && e_valid[it] != 0);
        float cp[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) cp[k] = bf(e_cr[it][k]);
        const float tr = bf(e_tr[it]);
        const float x = bf(e_x[it]);
        const float gsrc = f.G == f.R ? x : bf(e_g[it]);
        const float beta = skinny_sum<MT, NW>(red, mi, nn);
        // Paraplex pointwise, one token: prev phase = the carried trace
        const float s0 = phase_of(beta + e_ib[it]);
        const float raw = fmaf(tr, e_tw[it], s0);
        const float sv = raw * frsq(fmaf(raw, raw, 1.0f));
        float amp, gate;
        softplus_gate<false>(gsrc, f.m, amp, gate);   // bf16 outputs (see softplus_gate)
        const float act = fmaf(amp, sv, x) * gate;
        f.trace[e] = f32_to_bf16(s0);
        f.act[e] = f32_to_bf16(act);
        if (f.actf != nullptr)
            f.actf[(((m >> 4) * (H >> 5) + (h >> 5)) * 64 + (m & 15) + 16 * ((h & 31) >> 3)) * 8 + (h & 7)] =
                f32_to_bf16(act);
        if (f.s != nullptr) f.s[e] = f32_to_bf16(sv);
        // Tria depth op on (r, i, o) = (R, I, O) as stored
        const float i_ = round_bf(sv), o_ = round_bf(act);
        switch (f.axis) {
            case 0: ffn_tria<0>(f, e, x, i_, o_, cp, carry_in); break;
            case 1: ffn_tria<1>(f, e, x, i_, o_, cp, carry_in); break;
            default: ffn_tria<2>(f, e, x, i_, o_, cp, carry_in); break;
        }
    }
}

// ------------------------------------------------------------------ fused decode projections
// Several decode projections in one launch (M <= 64, bf16):
//   * concat-K: out = X W^T + X2 W2^T (two activations, two weights, one
//     accumulator), e.g. attn_out + depth skip before LayerNorm;
//   * output segments: the N columns are split into up to 4 segments that
//     share the activations but have their own weight rows, output (and row
//     stride), bias and identity-anchored gate, e.g. [history kv | W_real].
// Same block shape as the skinny kernel: 16 output columns x all M rows per
// block, the four waves split the combined k-steps of X and X2.
struct LinSeg {
    const uint16_t* W;
    int64_t ldw;
    const uint16_t* W2;
    int64_t ldw2;
    void* out;
    int64_t ldc;
    const float* bias;
    const void* gate_p;
    int64_t gate_ld;
    float gate_alpha;
    int64_t n;
};

constexpr int kMaxSeg = 4;

struct LinArgs {
    const uint16_t* X;
    int64_t ldx, K;
    const uint16_t* X2;
    int64_t ldx2, K2;
    int64_t M;
    int nseg;
    int64_t nstart[kMaxSeg + 1];   // first global column of each segment
    LinSeg seg[kMaxSeg];
    // split-K (one segment): blockIdx.y takes k-steps [y*S/nsplit, (y+1)*S/nsplit)
    // and writes raw fp32 sums to partial[(y*M + m)*ldp + n]; no epilogue
    float* partial;
    int64_t ldp;
    int nsplit;
    const uint8_t* only_if;   // with only_if_n flags: the launch does nothing unless one is set
    int only_if_n;
    const uint4* Xf;          // fragment-major copies of X / X2 (or null): piece
    const uint4* X2f;         // (j*(K/32) + step)*64 + lane is the MFMA B fragment
};

template <int MT, int NW, int UN>
__global__ void __launch_bounds__(NW * 64)
gemm_bf16_skinny_multi_kernel(LinArgs a) {
    __shared__ float red[NW][MT][4][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (a.only_if != nullptr) {              // one flag per thread, OR over the block
        int any = 0;
        for (int i = tid; i < a.only_if_n; i += NW * 64) any |= a.only_if[i] != 0;
        if (!__syncthreads_or(any)) return;  // block-uniform
    }
    const int64_t ng = (int64_t)blockIdx.x * 16;
    int s = 0;
#pragma unroll
    for (int q = 1; q < kMaxSeg; ++q) s += (q < a.nseg && ng >= a.nstart[q]) ? 1 : 0;
    const LinSeg sg = a.seg[s];
    const int64_t n0 = ng - a.nstart[s];
    const int fr = lane & 15, fk = (lane >> 4) * 8;
    const int64_t n = n0 + fr;
    const bool nvalid = n < sg.n;
    const int64_t S1 = ceil_div(a.K, 32), S2 = ceil_div(a.K2, 32), S = S1 + S2;
    const int64_t sb = S * blockIdx.y / a.nsplit, se = S * (blockIdx.y + 1) / a.nsplit;
    const int64_t per = ceil_div(se - sb, NW);
    const int64_t s_begin = sb + wave * per;
    const int64_t s_end = s_begin + per < se ? s_begin + per : se;

    // the gate and bias operands of this thread's outputs, requested with the
    // main loop's loads (they do not depend on the product), at clamped indices
    // so no load waits inside a condition; selected in the epilogue
    constexpr int kIt = (MT * 256 + NW * 64 - 1) / (NW * 64);
    float graw[kIt], braw[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int o = tid + it * NW * 64;
        const int64_t m = o >> 4, nidx = n0 + (o & 15);
        const int64_t mc = m < a.M ? m : a.M - 1, nc = nidx < sg.n ? nidx : sg.n - 1;
        graw[it] = sg.gate_p != nullptr ? ld((const bf16_t*)sg.gate_p + mc * sg.gate_ld + nc) : 0.0f;
        braw[it] = sg.bias != nullptr ? sg.bias[nc] : 0.0f;
    }

    f32x4 acc[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int64_t s0 = s_begin; s0 < s_end; s0 += UN) {
        uint4 wv[UN];
        uint4 xv[UN][MT];
#pragma unroll
        for (int u = 0; u < UN; ++u) {
            const int64_t step = s0 + u;
            const bool first = step < S1;
            const int64_t k = (first ? step : step - S1) * 32 + fk;
            const bool kin = step < s_end && k < (first ? a.K : a.K2);
            const uint16_t* wrow = first ? sg.W + n * sg.ldw : sg.W2 + n * sg.ldw2;
            const uint16_t* xb = first ? a.X : a.X2;
            const int64_t ldx = first ? a.ldx : a.ldx2;
            const uint4* xf = first ? a.Xf : a.X2f;
            const int64_t fs = first ? step : step - S1, fS = first ? S1 : S2;
            wv[u] = (kin && nvalid) ? *reinterpret_cast<const uint4*>(wrow + k) : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < MT; ++j) {
                const int64_t m = j * 16 + fr;
                xv[u][j] = !(kin && m < a.M) ? make_uint4(0, 0, 0, 0)
                           : xf != nullptr ? xf[(j * fS + fs) * 64 + lane]
                                           : *reinterpret_cast<const uint4*>(xb + m * ldx + k);
            }
        }
#pragma unroll
        for (int u = 0; u < UN; ++u)
#pragma unroll
            for (int j = 0; j < MT; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8, wv[u]), __builtin_bit_cast(bf16x8, xv[u][j]), acc[j],
                    0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][j][r][lane] = acc[j][r];
    __syncthreads();
    uint16_t* out = (uint16_t*)sg.out;
    float gmul[kIt], badd[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int o = tid + it * NW * 64;
        const int64_t m = o >> 4, nidx = n0 + (o & 15);
        const bool ok = o < MT * 256 && m < a.M && nidx < sg.n && a.partial == nullptr;
        gmul[it] = (ok && sg.gate_p != nullptr) ? 1.0f + sg.gate_alpha * graw[it] : 1.0f;
        badd[it] = (ok && sg.bias != nullptr) ? braw[it] : 0.0f;
    }
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int o = tid + it * NW * 64;
        if (o >= MT * 256) break;
        const int nn = o & 15, mi = o >> 4;
        const int j = mi >> 4, ml = mi & 15;
        const int64_t m = mi, nidx = n0 + nn;
        if (m >= a.M || nidx >= sg.n) continue;
        const int ln = ml + 16 * (nn >> 2), r = nn & 3;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red[w][j][r][ln];
        if (a.partial != nullptr) {
            a.partial[((int64_t)blockIdx.y * a.M + m) * a.ldp + nidx] = v;
            continue;
        }
        v *= gmul[it];
        v += badd[it];
        out[m * sg.ldc + nidx] = f32_to_bf16(v);
    }
}

// ------------------------------------------------------------------ fp32 GEMV (M <= 8)
// Decode-shaped fp32 products: one wave per output column n, its lanes stride
// the row of W in 16-byte pieces (4 in flight per lane) against the MR
// activation rows, a wave reduction per row, the epilogue on lane 0.  The
// weight row is read once, whole lines at a time.
template <int MR, bool GATHER>
__global__ void __launch_bounds__(256)
gemv_f32_kernel(GemmArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= a.N) return;                         // whole wave
    const int64_t g = GATHER ? n / a.Hq : 0;
    const float* W = (const float*)a.W + n * a.ldw;
    const float* X = (const float*)a.X;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
    constexpr int U = 4;
    for (int64_t k0 = 4 * lane; k0 < a.K; k0 += 256 * U) {
        float4 w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t k = k0 + 256 * u;
            w[u] = k < a.K ? *reinterpret_cast<const float4*>(W + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (m >= a.M) break;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t k = k0 + 256 * u;
                if (k >= a.K) break;
                float4 x;
                if constexpr (GATHER)
                    x = *reinterpret_cast<const float4*>(gather_ptr(a, m, k, g, 4));
                else
                    x = *reinterpret_cast<const float4*>(X + m * a.ldx + k);
                acc[m] = fmaf(w[u].x, x.x, fmaf(w[u].y, x.y, fmaf(w[u].z, x.z, fmaf(w[u].w, x.w, acc[m]))));
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        if (m >= a.M) break;
        const float v = wave_sum(acc[m]);
        if (lane == 0) ((float*)a.out)[m * a.ldc + n] = epilogue<float>(a, m, n, v);
    }
}

template <bool GATHER>
static void launch_gemv_f32(const GemmArgs& a, hipStream_t st) {
    const dim3 grid((unsigned)ceil_div(a.N, 4));
    if (a.M <= 1) hipLaunchKernelGGL((gemv_f32_kernel<1, GATHER>), grid, dim3(256), 0, st, a);
    else if (a.M <= 2) hipLaunchKernelGGL((gemv_f32_kernel<2, GATHER>), grid, dim3(256), 0, st, a);
    else if (a.M <= 4) hipLaunchKernelGGL((gemv_f32_kernel<4, GATHER>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((gemv_f32_kernel<8, GATHER>), grid, dim3(256), 0, st, a);
}

// ------------------------------------------------------------------ SIMT

constexpr int SB_M = 64, SB_N = 64, SB_K = 16;

template <typename T, bool GATHER>
__global__ void __launch_bounds__(256)
gemm_simt_kernel(GemmArgs a) {
    __shared__ float As[SB_K][SB_M + 4];
    __shared__ float Bs[SB_K][SB_N + 4];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * SB_N;
    const int64_t m0 = (int64_t)blockIdx.y * SB_M;
    const int64_t g = GATHER ? n0 / a.Hq : 0;
    const T* X = (const T*)a.X;
    const T* W = (const T*)a.W;
    float acc[4][4] = {};
    const int lrow = tid >> 2, lk = (tid & 3) * 4;
    for (int64_t k0 = 0; k0 < a.K; k0 += SB_K) {
        const int64_t m = m0 + lrow, n = n0 + lrow;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t k = k0 + lk + e;
            float xv = 0.0f, wv = 0.0f;
            if (m < a.M && k < a.K) {
                if constexpr (GATHER)
                    xv = ld((const T*)gather_ptr(a, m, k, g, (int)sizeof(T)));
                else
                    xv = ld(X + m * a.ldx + k);
            }
            if (n < a.N && k < a.K) wv = ld(W + n * a.ldw + k);
            As[lk + e][lrow] = xv;
            Bs[lk + e][lrow] = wv;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < SB_K; ++k) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = As[k][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = Bs[k][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
    T* out = (T*)a.out;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + ty * 4 + i;
        if (m >= a.M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t n = n0 + tx * 4 + j;
            if (n < a.N) st(out + m * a.ldc + n, epilogue<T>(a, m, n, acc[i][j]));
        }
    }
}

// One thread per output; any shape / group width.
template <typename T, bool GATHER>
__global__ void __launch_bounds__(256)
gemm_naive_kernel(GemmArgs a) {
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= a.M * a.N) return;
    const int64_t n = id % a.N, m = id / a.N;
    const int64_t g = GATHER ? n / a.Hq : 0;
    float acc = 0.0f;
    for (int64_t k = 0; k < a.K; ++k) {
        float xv;
        if constexpr (GATHER)
            xv = ld((const T*)gather_ptr(a, m, k, g, (int)sizeof(T)));
        else
            xv = ld((const T*)a.X + m * a.ldx + k);
        acc = fmaf(xv, ld((const T*)a.W + n * a.ldw + k), acc);
    }
    st((T*)a.out + m * a.ldc + n, epilogue<T>(a, m, n, acc));
}

// Waves per block and k-steps in flight per wave for a skinny product of
// `steps` 32-wide k-steps and MT 16-row m-tiles: enough waves that each makes
// one pass (a single round of weight loads) where the registers allow it:
// 8 steps in flight only for one m-tile, 16 waves only up to 3 m-tiles.
static void skinny_shape(int64_t steps, int mt, int& nw, int& un) {
    un = 4;
    if (steps <= 16) nw = 4;
    else if (steps <= 32 || mt >= 4) nw = 8;
    else nw = 16;
    if (nw == 16 && mt == 1 && steps > 64) un = 8;
}

template <int MT, bool GATHER>
static void launch_skinny(const GemmArgs& a, dim3 grid, hipStream_t st) {
    int nw, un;
    skinny_shape(ceil_div(a.K, 32), MT, nw, un);
    if (nw == 4) {
        hipLaunchKernelGGL((gemm_bf16_skinny_kernel<MT, GATHER, 4, 4>), grid, dim3(256), 0, st, a);
    } else if (nw == 8) {
        hipLaunchKernelGGL((gemm_bf16_skinny_kernel<MT, GATHER, 8, 4>), grid, dim3(512), 0, st, a);
    } else if constexpr (MT <= 3) {
        if (un == 4 || MT > 1)
            hipLaunchKernelGGL((gemm_bf16_skinny_kernel<MT, GATHER, 16, 4>), grid, dim3(1024), 0, st, a);
        else
            hipLaunchKernelGGL((gemm_bf16_skinny_kernel<MT, GATHER, 16, (MT == 1 ? 8 : 4)>), grid,
                               dim3(1024), 0, st, a);
    }
}

// Tile configuration of a big bf16 product, from the 256 x 128 tile count t
// against the CU count c:
//   128 x 256 when N % 256 == 0 and t >= 3c/4 (8192 x 768 x 3072: 49.6
//     against 53.2 us; 8192 x 3072 x 768: 60.9 against 63.4 us; the chunked
//     prefill's 4096 x 1536 history projections);
//   256 x 128 otherwise, and 128 x 128 only where 256 x 128 cannot run (fewer
//     than 256 rows, K not a whole round of its stages).  Alone, 128 x 128 is
//     faster whenever 256 x 128 leaves CUs idle (4096 x 768 x 3072: 32.5
//     against 47.0 us), but inside the chunked prefill, beside the other
//     streams' kernels, choosing it there measured 74.4-75.2 ms against
//     73.5-74.0 ms (same box, alternating runs).
// K must fill whole rounds of the configuration's stages; gather tiles must
// not straddle a q-head group (Hq % BG_N == 0).
enum BigTile { kBigNone, kBigStd, kBigSmall, kBigWide, kBigTall, kBigTallS };
// shared-tile mode (loom_gemm_shared_tiles): process-wide
static std::atomic<int> g_shared_tiles{0};
template <class C>
static bool big_fits(int64_t M, int64_t K, bool gather, int64_t Hq) {
    return M >= C::BG_M && K % (C::NS * C::BK) == 0 && (!gather || Hq % C::BG_N == 0);
}
static BigTile big_tile(int64_t M, int64_t N, int64_t K, bool gather, int64_t Hq) {
    if (g_shared_tiles.load(std::memory_order_relaxed) != 0 && (gather || N % BgTallS::BG_N == 0) &&
        big_fits<BgTallS>(M, K, gather, Hq))
        return kBigTallS;
    const bool std_ok = big_fits<BgConf>(M, K, gather, Hq);
    const bool small_ok = big_fits<BgSmall>(M, K, gather, Hq);
    const bool wide_ok = !gather && N % BgWide::BG_N == 0 && big_fits<BgWide>(M, K, gather, Hq);
    if (!std_ok) return small_ok ? kBigSmall : (wide_ok ? kBigWide : kBigNone);
    const int64_t c = device_cus();
    const int64_t t = ceil_div(M, BgConf::BG_M) * ceil_div(N, BgConf::BG_N);
    // rounds of the CUs times the work of a tile (in 256 x 64 units): 256 x 192
    // where it takes fewer
    const bool tall_ok = N % BgTall::BG_N == 0 && big_fits<BgTall>(M, K, gather, Hq);
    const int64_t tt = ceil_div(M, BgTall::BG_M) * (N / BgTall::BG_N);
    if (tall_ok && ceil_div(tt, c) * 3 < ceil_div(t, c) * 2) return kBigTall;
    if (wide_ok && 4 * t >= 3 * c) return kBigWide;
    return kBigStd;
}
static int64_t big_tile_n(BigTile t) {
    return t == kBigSmall ? BgSmall::BG_N : t == kBigWide ? BgWide::BG_N : t == kBigTall ? BgTall::BG_N
         : t == kBigTallS ? BgTallS::BG_N : BgConf::BG_N;
}
template <bool GATHER, class C>
static void launch_big_cfg(const GemmArgs& a, int64_t nsplit, hipStream_t st) {
    const dim3 grid((unsigned)(ceil_div(a.N, C::BG_N) * ceil_div(a.M, C::BG_M) * nsplit));
    hipLaunchKernelGGL((gemm_bf16_big_kernel<GATHER, C>), grid, dim3(64 * C::WAVES), 0, st, a);
}
template <bool GATHER>
static void launch_big(const GemmArgs& a, BigTile tile, int64_t nsplit, hipStream_t st) {
    if (tile == kBigSmall) launch_big_cfg<GATHER, BgSmall>(a, nsplit, st);
    else if (tile == kBigTallS) launch_big_cfg<GATHER, BgTallS>(a, nsplit, st);
    else if constexpr (!GATHER) {
        if (tile == kBigWide) launch_big_cfg<GATHER, BgWide>(a, nsplit, st);
        else if (tile == kBigTall) launch_big_cfg<GATHER, BgTall>(a, nsplit, st);
        else launch_big_cfg<GATHER, BgConf>(a, nsplit, st);
    } else {
        if (tile == kBigTall) launch_big_cfg<GATHER, BgTall>(a, nsplit, st);
        else launch_big_cfg<GATHER, BgConf>(a, nsplit, st);
    }
}

template <typename T, bool GATHER>
static int run_gemm(const GemmArgs& a, hipStream_t st, const char* what) {
    if (a.M == 0 || a.N == 0) return LOOM_OK;
    if constexpr (sizeof(T) == 2 && std::is_same<T, bf16_t>::value) {
        bool sk = a.M <= 64 && a.K % 8 == 0 && a.ldw % 8 == 0 && ((uintptr_t)a.W & 15) == 0;
        if (GATHER)
            sk = sk && a.Hq % 16 == 0 && a.HD % 8 == 0 && a.Nm % 8 == 0 &&
                 ((uintptr_t)a.src[0] | (uintptr_t)a.src[1] | (uintptr_t)a.src[2] |
                  (uintptr_t)a.src[3] | (uintptr_t)a.src[4]) % 16 == 0;
        else
            sk = sk && a.ldx % 8 == 0 && ((uintptr_t)a.X & 15) == 0;
        if (sk) {
            const dim3 grid((unsigned)ceil_div(a.N, 16));
            switch ((int)ceil_div(a.M, 16)) {
                case 1: launch_skinny<1, GATHER>(a, grid, st); break;
                case 2: launch_skinny<2, GATHER>(a, grid, st); break;
                case 3: launch_skinny<3, GATHER>(a, grid, st); break;
                default: launch_skinny<4, GATHER>(a, grid, st); break;
            }
            return launch_status(what);
        }
        bool ok = a.K % 8 == 0;
        if (GATHER) ok = ok && a.Hq % MB_N == 0 && a.HD % 8 == 0 && a.Nm % 8 == 0;
        else ok = ok && a.ldx % 8 == 0 && ((uintptr_t)a.X & 15) == 0;
        ok = ok && a.ldw % 8 == 0 && ((uintptr_t)a.W & 15) == 0;
        if (GATHER)
            for (int s = 0; s < 5; ++s) ok = ok && ((uintptr_t)a.src[s] & 15) == 0;
        // many rows and whole rounds of k-stages: the DMA-staged tiles
        const BigTile tile = ok ? big_tile(a.M, a.N, a.K, GATHER, a.Hq) : kBigNone;
        if (tile != kBigNone) {
            launch_big<GATHER>(a, tile, 1, st);
            return launch_status(what);
        }
        if (ok) {
            dim3 grid((unsigned)ceil_div(a.N, MB_N), (unsigned)ceil_div(a.M, MB_M));
            hipLaunchKernelGGL((gemm_bf16_mfma_kernel<GATHER>), grid, dim3(256), 0, st, a);
            return launch_status(what);
        }
    }
    if constexpr (std::is_same<T, float>::value) {
        // few rows: the fp32 GEMV (16-byte pieces: K, ldw, ldx multiples of 4, aligned bases;
        // gather pieces stay inside one sector: head_dim and the model width multiples of 4)
        bool gv = a.M <= 8 && a.K % 4 == 0 && a.ldw % 4 == 0 && ((uintptr_t)a.W & 15) == 0;
        if (GATHER)
            gv = gv && a.HD % 4 == 0 && a.Nm % 4 == 0 &&
                 ((uintptr_t)a.src[0] | (uintptr_t)a.src[1] | (uintptr_t)a.src[2] |
                  (uintptr_t)a.src[3] | (uintptr_t)a.src[4]) % 16 == 0;
        else
            gv = gv && a.ldx % 4 == 0 && ((uintptr_t)a.X & 15) == 0;
        if (gv) {
            launch_gemv_f32<GATHER>(a, st);
            return launch_status(what);
        }
    }
    if (!GATHER || a.Hq % SB_N == 0) {
        dim3 grid((unsigned)ceil_div(a.N, SB_N), (unsigned)ceil_div(a.M, SB_M));
        hipLaunchKernelGGL((gemm_simt_kernel<T, GATHER>), grid, dim3(256), 0, st, a);
        return launch_status(what);
    }
    hipLaunchKernelGGL((gemm_naive_kernel<T, GATHER>), dim3((unsigned)ceil_div(a.M * a.N, 256)),
                       dim3(256), 0, st, a);
    return launch_status(what);
}

template <typename T>
static int linear_dispatch(const GemmArgs& a, hipStream_t st) {
    return run_gemm<T, false>(a, st, "loom_linear");
}

template <typename T>
static int beta_dispatch(const GemmArgs& a, void* r_pack, int64_t QH, hipStream_t st);

// Optional packed copy [QH, M, imag_in] (the reference's second output).
template <typename T>
__global__ void pack_kernel(GemmArgs a, T* __restrict__ pack, int64_t QH) {
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = QH * a.M * a.K;
    if (id >= total) return;
    const int64_t kk = id % a.K;
    const int64_t m = (id / a.K) % a.M;
    const int64_t g = id / (a.K * a.M);
    pack[id] = *(const T*)gather_ptr(a, m, kk, g, (int)sizeof(T));
}

template <typename T>
static int beta_dispatch(const GemmArgs& a, void* r_pack, int64_t QH, hipStream_t st) {
    if (r_pack != nullptr) {
        const int64_t total = QH * a.M * a.K;
        hipLaunchKernelGGL((pack_kernel<T>), dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st,
                           a, (T*)r_pack, QH);
        int rc = launch_status("loom_beta_forward(pack)");
        if (rc != LOOM_OK) return rc;
    }
    return run_gemm<T, true>(a, st, "loom_beta_forward");
}

}  // namespace loom

using namespace loom;

extern "C" int loom_linear(int dtype, const void* A, int64_t lda, const void* W, int64_t ldw,
                           const float* bias, const void* gate_p, float gate_alpha,
                           const void* residual, void* out, int64_t ldc, int64_t M, int64_t Nout,
                           int64_t K, void* stream) {
    clear_error();
    LOOM_CHECK(A && W && out, "linear: null tensor argument");
    LOOM_CHECK(M >= 0 && Nout >= 0 && K >= 1, "linear: bad shape M=%lld N=%lld K=%lld",
               (long long)M, (long long)Nout, (long long)K);
    LOOM_CHECK(lda >= K && ldw >= K && ldc >= Nout, "linear: row strides smaller than the rows");
    GemmArgs a{};
    a.X = A; a.ldx = lda; a.W = W; a.ldw = ldw; a.bias = bias; a.gate_p = gate_p;
    a.gate_alpha = gate_alpha; a.residual = residual; a.out = out; a.ldc = ldc;
    a.M = M; a.N = Nout; a.K = K;
    switch (dtype) {
        case LOOM_F32: return linear_dispatch<float>(a, (hipStream_t)stream);
        case LOOM_BF16: return linear_dispatch<bf16_t>(a, (hipStream_t)stream);
        case LOOM_F16: return linear_dispatch<f16_t>(a, (hipStream_t)stream);
    }
    set_error("linear: unsupported dtype %d", dtype);
    return LOOM_ERR_INVALID;
}

template <int MT>
static void launch_skinny_multi_mt(const LinArgs& a, dim3 grid, int64_t steps, hipStream_t st) {
    int nw, un;
    skinny_shape(steps, MT, nw, un);
    if (nw == 4) {
        hipLaunchKernelGGL((gemm_bf16_skinny_multi_kernel<MT, 4, 4>), grid, dim3(256), 0, st, a);
    } else if (nw == 8) {
        hipLaunchKernelGGL((gemm_bf16_skinny_multi_kernel<MT, 8, 4>), grid, dim3(512), 0, st, a);
    } else if constexpr (MT <= 3) {
        if (un == 4 || MT > 1)
            hipLaunchKernelGGL((gemm_bf16_skinny_multi_kernel<MT, 16, 4>), grid, dim3(1024), 0, st, a);
        else
            hipLaunchKernelGGL((gemm_bf16_skinny_multi_kernel<MT, 16, (MT == 1 ? 8 : 4)>), grid,
                               dim3(1024), 0, st, a);
    }
}

static void launch_skinny_multi(const LinArgs& a, dim3 grid, int mt, int64_t steps, hipStream_t st) {
    switch (mt) {
        case 1: launch_skinny_multi_mt<1>(a, grid, steps, st); break;
        case 2: launch_skinny_multi_mt<2>(a, grid, steps, st); break;
        case 3: launch_skinny_multi_mt<3>(a, grid, steps, st); break;
        default: launch_skinny_multi_mt<4>(a, grid, steps, st); break;
    }
}

// Fragment-major activation copies: whole 32-wide k-steps, 16-byte aligned.
static bool frag_ok(const loom_linear_multi_desc& d) {
    return (d.x_frag == nullptr || (d.k % 32 == 0 && ((uintptr_t)d.x_frag & 15) == 0)) &&
           (d.x2_frag == nullptr || (d.k2 > 0 && d.k2 % 32 == 0 && ((uintptr_t)d.x2_frag & 15) == 0));
}

// Host side of loom_linear_multi: one fused launch for bf16 when every piece
// is 16-byte aligned, otherwise (and for fp32 / fp16) one product per segment
// and input, the second input accumulated through the residual epilogue.
template <typename T>
static int linear_multi_dispatch(const loom_linear_multi_desc& d, hipStream_t st) {
    bool fused = std::is_same<T, bf16_t>::value && d.m <= 64 && d.k % 8 == 0 && d.ldx % 8 == 0 &&
                 ((uintptr_t)d.x & 15) == 0 && frag_ok(d);
    if (d.k2 > 0) fused = fused && d.k2 % 8 == 0 && d.ldx2 % 8 == 0 && ((uintptr_t)d.x2 & 15) == 0;
    for (int s = 0; s < d.nseg; ++s) {
        const loom_linear_segment& g = d.seg[s];
        fused = fused && g.ldw % 8 == 0 && ((uintptr_t)g.w & 15) == 0 && (s == d.nseg - 1 || g.n % 16 == 0);
        if (d.k2 > 0) fused = fused && g.ldw2 % 8 == 0 && ((uintptr_t)g.w2 & 15) == 0;
    }
    if (fused) {
        LinArgs a{};
        a.X = (const uint16_t*)d.x; a.ldx = d.ldx; a.K = d.k;
        a.X2 = (const uint16_t*)d.x2; a.ldx2 = d.ldx2; a.K2 = d.k2;
        a.M = d.m; a.nseg = d.nseg; a.nsplit = 1;
        a.only_if = d.only_if;
        a.only_if_n = (int)d.only_if_n;
        a.Xf = (const uint4*)d.x_frag;
        a.X2f = (const uint4*)d.x2_frag;
        int64_t ncols = 0;
        for (int s = 0; s < d.nseg; ++s) {
            const loom_linear_segment& g = d.seg[s];
            a.nstart[s] = ncols;
            a.seg[s] = LinSeg{(const uint16_t*)g.w, g.ldw, (const uint16_t*)g.w2, g.ldw2, g.out, g.ldc,
                              g.bias, g.gate_p, g.gate_ld, g.gate_alpha, g.n};
            ncols += ceil_div(g.n, 16) * 16;
        }
        for (int s = d.nseg; s <= kMaxSeg; ++s) a.nstart[s] = ncols;
        const dim3 grid((unsigned)(ncols / 16));
        const int64_t steps = ceil_div(d.k, 32) + ceil_div(d.k2, 32);
        launch_skinny_multi(a, grid, (int)ceil_div(d.m, 16), steps, st);
        return launch_status("loom_linear_multi");
    }
    if (std::is_same<T, bf16_t>::value && d.nseg == 2 && d.k2 == 0 && d.m > 64) {
        // two single-input segments on the DMA-staged tiles: one launch when the
        // first segment ends on a tile boundary (a gate on the first only)
        const loom_linear_segment& g0 = d.seg[0];
        const loom_linear_segment& g1 = d.seg[1];
        bool ok = g1.gate_p == nullptr && (g0.gate_p == nullptr || g0.gate_ld == g0.ldc) &&
                  d.k % 8 == 0 && d.ldx % 8 == 0 &&
                  ((uintptr_t)d.x & 15) == 0 && g0.ldw % 8 == 0 && g1.ldw % 8 == 0 &&
                  (((uintptr_t)g0.w | (uintptr_t)g1.w) & 15) == 0;
        const BigTile tile = ok ? big_tile(d.m, g0.n + g1.n, d.k, false, 0) : kBigNone;
        if (tile != kBigNone && g0.n % big_tile_n(tile) == 0) {
            GemmArgs a{};
            a.X = d.x; a.ldx = d.ldx; a.W = g0.w; a.ldw = g0.ldw; a.out = g0.out; a.ldc = g0.ldc;
            a.bias = g0.bias; a.gate_p = g0.gate_p; a.gate_alpha = g0.gate_alpha;
            a.M = d.m; a.N = g0.n + g1.n; a.K = d.k;
            a.N1 = g0.n; a.Wb = g1.w; a.ldwb = g1.ldw; a.outb = g1.out; a.ldcb = g1.ldc; a.biasb = g1.bias;
            launch_big<false>(a, tile, 1, st);
            return launch_status("loom_linear_multi");
        }
    }
    for (int s = 0; s < d.nseg; ++s) {
        const loom_linear_segment& g = d.seg[s];
        GemmArgs a{};
        a.X = d.x; a.ldx = d.ldx; a.W = g.w; a.ldw = g.ldw; a.out = g.out; a.ldc = g.ldc;
        a.M = d.m; a.N = g.n; a.K = d.k;
        if (d.k2 == 0) {
            // the many-row kernels read the gate at the output's row stride
            LOOM_CHECK(g.gate_p == nullptr || g.gate_ld == g.ldc,
                       "linear_multi: over 64 rows a gate needs the output's row stride (gate_ld %lld, ldc %lld)",
                       (long long)g.gate_ld, (long long)g.ldc);
            a.bias = g.bias; a.gate_p = g.gate_p; a.gate_alpha = g.gate_alpha;
            int rc = run_gemm<T, false>(a, st, "loom_linear_multi");
            if (rc != LOOM_OK) return rc;
            continue;
        }
        int rc = run_gemm<T, false>(a, st, "loom_linear_multi");
        if (rc != LOOM_OK) return rc;
        GemmArgs b = a;
        b.X = d.x2; b.ldx = d.ldx2; b.W = g.w2; b.ldw = g.ldw2; b.K = d.k2;
        b.bias = g.bias; b.residual = g.out;
        rc = run_gemm<T, false>(b, st, "loom_linear_multi");
        if (rc != LOOM_OK) return rc;
    }
    return LOOM_OK;
}

extern "C" int64_t loom_linear_multi_desc_bytes(void) { return (int64_t)sizeof(loom_linear_multi_desc); }

extern "C" int loom_linear_multi(int dtype, const loom_linear_multi_desc* d, void* stream) {
    clear_error();
    LOOM_CHECK(d != nullptr && d->x != nullptr, "linear_multi: null descriptor or input");
    LOOM_CHECK(d->only_if == nullptr || (d->only_if_n >= 1 && d->only_if_n <= 1024),
               "linear_multi: only_if_n=%lld outside [1, 1024]", (long long)d->only_if_n);
    LOOM_CHECK(d->nseg >= 1 && d->nseg <= kMaxSeg, "linear_multi: nseg=%d outside [1, %d]",
               (int)d->nseg, kMaxSeg);
    LOOM_CHECK(d->m >= 0 && d->k >= 1 && d->ldx >= d->k && d->k2 >= 0,
               "linear_multi: bad input shape");
    LOOM_CHECK(d->k2 == 0 || (d->x2 != nullptr && d->ldx2 >= d->k2),
               "linear_multi: second input missing or its stride is too small");
    for (int s = 0; s < d->nseg; ++s) {
        const loom_linear_segment& g = d->seg[s];
        LOOM_CHECK(g.w && g.out && g.n >= 1 && g.ldw >= d->k && g.ldc >= g.n,
                   "linear_multi: bad segment %d", s);
        LOOM_CHECK(d->k2 == 0 || (g.w2 && g.ldw2 >= d->k2), "linear_multi: segment %d lacks w2", s);
        LOOM_CHECK(d->k2 == 0 || g.gate_p == nullptr,
                   "linear_multi: the gate applies to single-input segments only");
        LOOM_CHECK(g.gate_p == nullptr || g.gate_ld >= g.n, "linear_multi: gate row stride too small");
    }
    if (d->m == 0) return LOOM_OK;
    switch (dtype) {
        case LOOM_F32: return linear_multi_dispatch<float>(*d, (hipStream_t)stream);
        case LOOM_BF16: return linear_multi_dispatch<bf16_t>(*d, (hipStream_t)stream);
        case LOOM_F16: return linear_multi_dispatch<f16_t>(*d, (hipStream_t)stream);
    }
    set_error("linear_multi: unsupported dtype %d", dtype);
    return LOOM_ERR_INVALID;
}

// ------------------------------------------------------------------ split-K + LayerNorm
constexpr int kMaxSplit = 8;

// out[m] = LN(sum_s partial[s, m] + bias) * gamma + beta; one wave per row,
// N <= 64 * 4 * kLnVec.
constexpr int kLnVec = 8;      // 256-column chunks per row: rows of up to 2048
// One block per row, one wave per 256-column chunk (KV waves), so a decode
// step's 32 rows spread over 32 CUs.  Every load of the row (all NS split
// partials, bias, gamma and beta) is issued before the first add; the row's
// sum and squared deviation are reduced over the waves through LDS.
template <typename T, int NS, int KV>
__global__ void __launch_bounds__(64 * KV)
splitk_ln_kernel(const float* __restrict__ partial, int64_t ldp,
                 const float* __restrict__ bias, const float* __restrict__ gamma,
                 const float* __restrict__ beta, T* __restrict__ out, int64_t ldo, int64_t rows,
                 int N, float eps, T* __restrict__ outf) {
    __shared__ float red[2][KV];
    const int64_t row = blockIdx.x;
    const int lane = threadIdx.x & 63, k = threadIdx.x >> 6;
    const int c = (lane + 64 * k) * 4;
    const bool in = c < N;
    // every load unconditional, at column 0 for lanes past N (their values are
    // never used), so all of a row's loads are in flight at once
    const int cl = in ? c : 0;
    float4 v[NS], bv, gv, ev;
#pragma unroll
    for (int sp = 0; sp < NS; ++sp)
        v[sp] = *reinterpret_cast<const float4*>(partial + (sp * rows + row) * ldp + cl);
    bv = *reinterpret_cast<const float4*>((bias != nullptr ? bias : gamma) + cl);
    if (bias == nullptr) bv = make_float4(0.f, 0.f, 0.f, 0.f);
    gv = *reinterpret_cast<const float4*>(gamma + cl);
    ev = *reinterpret_cast<const float4*>(beta + cl);
    float x[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
    for (int sp = 0; sp < NS; ++sp) {
        x[0] += v[sp].x; x[1] += v[sp].y; x[2] += v[sp].z; x[3] += v[sp].w;
    }
    float s = in ? (x[0] + x[1]) + (x[2] + x[3]) : 0.0f;
    s = wave_sum(s);
    if (lane == 0) red[0][k] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int q = 0; q < KV; ++q) tot += red[0][q];
    const float mean = tot / N;
    float var = 0.0f;
    if (in)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float dlt = x[e] - mean;
            var = fmaf(dlt, dlt, var);
        }
    var = wave_sum(var);
    if (lane == 0) red[1][k] = var;
    __syncthreads();
    float vt = 0.0f;
#pragma unroll
    for (int q = 0; q < KV; ++q) vt += red[1][q];
    const float rstd = frsq(vt / N + eps);
    if (!in) return;
    const float g[4] = {gv.x, gv.y, gv.z, gv.w};
    const float e4[4] = {ev.x, ev.y, ev.z, ev.w};
    T y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        st(&y[e], fmaf((x[e] - mean) * rstd, g[e], e4[e]));
        out[row * ldo + c + e] = y[e];
    }
    if (outf != nullptr) {
        // fragment-major copy: piece (row/16, c/32, row%16 + 16*((c%32)/8)), elements c%8 ..
        const int64_t piece = ((row >> 4) * (N >> 5) + (c >> 5)) * 64 + (row & 15) + 16 * ((c & 31) >> 3);
#pragma unroll
        for (int e = 0; e < 4; ++e) outf[piece * 8 + (c & 7) + e] = y[e];
    }
}

extern "C" int64_t loom_linear_ln_workspace_bytes(int64_t M, int64_t N) {
    return kMaxSplit * M * N * (int64_t)sizeof(float);
}

// LayerNorm of the ns split-K partial sums (+ bias) of d's product, one block per row
static int launch_splitk_ln(int64_t ns, const loom_linear_multi_desc* d, const float* workspace,
                            const float* gamma, const float* beta, float eps, void* out, int64_t ldo,
                            void* out_frag, hipStream_t st) {
    const loom_linear_segment& g = d->seg[0];
#define LOOM_SLN_KV(NS, KV)                                                                   \
    hipLaunchKernelGGL((splitk_ln_kernel<bf16_t, NS, KV>), dim3((unsigned)d->m), dim3(64 * (KV)), \
                       0, st, workspace, g.n, g.bias, gamma, beta, (bf16_t*)out, ldo, d->m,     \
                       (int)g.n, eps, (bf16_t*)out_frag);
#define LOOM_SLN(NS)                                                                          \
    case NS:                                                                                  \
        if (kv <= 1) { LOOM_SLN_KV(NS, 1) }                                                   \
        else if (kv == 2) { LOOM_SLN_KV(NS, 2) }                                              \
        else if (kv == 3) { LOOM_SLN_KV(NS, 3) }                                              \
        else if (kv == 4) { LOOM_SLN_KV(NS, 4) }                                              \
        else { LOOM_SLN_KV(NS, 8) }                                                           \
        break;
    const int kv = (int)ceil_div(g.n, 256);
    switch (ns) {
        LOOM_SLN(1) LOOM_SLN(2) LOOM_SLN(3) LOOM_SLN(4) LOOM_SLN(5) LOOM_SLN(6) LOOM_SLN(7)
        LOOM_SLN(8)
    }
#undef LOOM_SLN_KV
#undef LOOM_SLN
    return launch_status("loom_linear_ln(layernorm)");
}

extern "C" int loom_linear_ln(int dtype, const loom_linear_multi_desc* d, const float* gamma,
                              const float* beta, float eps, void* out, int64_t ldo, float* workspace,
                              int64_t workspace_bytes, void* out_frag, void* stream) {
    clear_error();
    LOOM_CHECK(d != nullptr && d->nseg == 1, "linear_ln: one output segment expected");
    LOOM_CHECK(gamma && beta && out, "linear_ln: null LayerNorm argument");
    const loom_linear_segment& g = d->seg[0];
    LOOM_CHECK(g.gate_p == nullptr, "linear_ln: no gate on a LayerNorm input");
    LOOM_CHECK(g.n >= 1 && g.n <= 64 * 4 * kLnVec && ldo >= g.n,
               "linear_ln: N=%lld outside [1, %d]", (long long)g.n, 64 * 4 * kLnVec);
    hipStream_t st = (hipStream_t)stream;
    // operands of the bf16 split-K forms (both read 16-byte pieces)
    bool aligned = dtype == LOOM_BF16 && d->k % 8 == 0 && d->ldx % 8 == 0 &&
                   ((uintptr_t)d->x & 15) == 0 && g.ldw % 8 == 0 && ((uintptr_t)g.w & 15) == 0 &&
                   g.n % 4 == 0 && workspace != nullptr && ((uintptr_t)workspace & 15) == 0 &&
                   ((((uintptr_t)gamma | (uintptr_t)beta | (uintptr_t)g.bias) & 15) == 0) &&
                   workspace_bytes >= loom_linear_ln_workspace_bytes(d->m, g.n);
    if (d->k2 > 0)
        aligned = aligned && d->k2 % 8 == 0 && d->ldx2 % 8 == 0 && ((uintptr_t)d->x2 & 15) == 0 &&
                  g.ldw2 % 8 == 0 && ((uintptr_t)g.w2 & 15) == 0;
    const bool fused = aligned && d->m >= 1 && d->m <= 64 && frag_ok(*d);
    LOOM_CHECK(out_frag == nullptr || (fused && g.n % 32 == 0 && ((uintptr_t)out_frag & 15) == 0),
               "linear_ln: out_frag needs the bf16 split-K form (m <= 64, aligned) and n %% 32 == 0");
    if (!fused) {
        // many rows: the DMA-staged MFMA tiles over both inputs (configuration as
        // big_tile picks it), split-K sums in the workspace, reduced with the bias
        // in the LayerNorm kernel.  Splits: whole rounds of the stages each;
        // fewest block rounds times (k per split + ~320, the measured fixed cost
        // of a block in k units).
        const int64_t K = d->k + d->k2;
        const BigTile tile = aligned ? big_tile(d->m, g.n, K, false, 0) : kBigNone;
        int64_t bm = BgConf::BG_M, bn = BgConf::BG_N, stage_k = BgConf::NS * BgConf::BK,
                half_k = BgConf::BK, per_cu = 1;
        if (tile == kBigSmall) {
            bm = BgSmall::BG_M; bn = BgSmall::BG_N; stage_k = BgSmall::NS * BgSmall::BK;
            half_k = BgSmall::BK; per_cu = 2;
        } else if (tile == kBigWide) {
            bm = BgWide::BG_M; bn = BgWide::BG_N; stage_k = BgWide::NS * BgWide::BK;
            half_k = BgWide::BK;
        } else if (tile == kBigTall) {
            bm = BgTall::BG_M; bn = BgTall::BG_N; stage_k = BgTall::NS * BgTall::BK;
            half_k = BgTall::BK;
        } else if (tile == kBigTallS) {
            // counted as one block per CU: in shared-tile mode the other
            // stream's kernels hold part of every CU (two splits at the
            // prefill's 4096 x 768 tails, measured faster than three)
            bm = BgTallS::BG_M; bn = BgTallS::BG_N; stage_k = BgTallS::NS * BgTallS::BK;
            half_k = BgTallS::BK;
        }
        const int64_t tiles = ceil_div(d->m, bm) * ceil_div(g.n, bn);
        int64_t ns = 0, best = 0;
        if (tile != kBigNone && d->k % half_k == 0)
            for (int64_t q = 1; q <= kMaxSplit; ++q) {
                if (K % (q * stage_k) != 0) continue;
                const int64_t cost = ceil_div(tiles * q, per_cu * (int64_t)device_cus()) * (K / q + 320);
                if (ns == 0 || cost < best) { ns = q; best = cost; }
            }
        if (ns > 0) {
            GemmArgs a{};
            a.X = d->x; a.ldx = d->ldx; a.W = g.w; a.ldw = g.ldw;
            a.X2 = d->k2 > 0 ? d->x2 : nullptr; a.ldx2 = d->ldx2; a.W2 = g.w2; a.ldw2 = g.ldw2;
            a.K1 = d->k;
            a.M = d->m; a.N = g.n; a.K = K;
            a.partial = workspace; a.ldp = g.n; a.nsplit = (int)ns;
            launch_big<false>(a, tile, ns, st);
            const int rc = launch_status("loom_linear_ln");
            if (rc != LOOM_OK) return rc;
            return launch_splitk_ln(ns, d, workspace, gamma, beta, eps, out, ldo, nullptr, st);
        }
        // y = product (+ bias) into seg.out, then LayerNorm of y
        int rc = loom_linear_multi(dtype, d, stream);
        if (rc != LOOM_OK) return rc;
        LOOM_CHECK(g.ldc == g.n && ldo == g.n, "linear_ln: the unfused path needs dense rows");
        return loom_add_layernorm(dtype, g.out, nullptr, gamma, beta, out, d->m, g.n, eps, stream);
    }
    if (d->m == 0) return LOOM_OK;
    LinArgs a{};
    a.X = (const uint16_t*)d->x; a.ldx = d->ldx; a.K = d->k;
    a.X2 = (const uint16_t*)d->x2; a.ldx2 = d->ldx2; a.K2 = d->k2;
    a.M = d->m; a.nseg = 1;
    a.Xf = (const uint4*)d->x_frag;
    a.X2f = (const uint4*)d->x2_frag;
    a.seg[0] = LinSeg{(const uint16_t*)g.w, g.ldw, (const uint16_t*)g.w2, g.ldw2, g.out, g.ldc,
                      nullptr, nullptr, 0, 0.0f, g.n};
    const int64_t ntiles = ceil_div(g.n, 16);
    for (int s2 = 0; s2 <= kMaxSeg; ++s2) a.nstart[s2] = s2 == 0 ? 0 : ntiles * 16;
    const int64_t steps = ceil_div(d->k, 32) + ceil_div(d->k2, 32);
    // about two blocks per CU, at most kSkinnyLnSplit k-splits (each split is
    // one more partial row the LayerNorm kernel reads: at N = 768, K = 1536 /
    // 3840, 4 splits measured 6.8 / 8.3 us per call against 7.3 / 8.7 with 8
    // and 7.5 / 11.0 with 2), at least 4 k-steps per split
    constexpr int64_t kSkinnyLnSplit = 4;
    int64_t ns = ceil_div(2 * (int64_t)device_cus(), ntiles);
    if (ns > kSkinnyLnSplit) ns = kSkinnyLnSplit;
    if (ns > steps / 4) ns = steps / 4 > 0 ? steps / 4 : 1;
    a.nsplit = (int)ns;
    a.partial = workspace;
    a.ldp = g.n;
    const dim3 grid((unsigned)ntiles, (unsigned)ns);
    launch_skinny_multi(a, grid, (int)ceil_div(d->m, 16), ceil_div(steps, ns), st);
    int rc = launch_status("loom_linear_ln");
    if (rc != LOOM_OK) return rc;
    return launch_splitk_ln(ns, d, workspace, gamma, beta, eps, out, ldo, out_frag, st);
}

extern "C" int64_t loom_ffn_decode_desc_bytes(void) { return (int64_t)sizeof(loom_ffn_decode_desc); }

template <int MT, int DE = 0, bool DR = false>
static void launch_ffn_mt(const FfnArgs& f, dim3 grid, hipStream_t st) {
    int nw, un;
    skinny_shape(ceil_div(f.g.K, 32), MT, nw, un);
    if (nw == 4) hipLaunchKernelGGL((ffn_decode_kernel<MT, 4, 4, DE, DR>), grid, dim3(256), 0, st, f);
    else if (nw == 8) hipLaunchKernelGGL((ffn_decode_kernel<MT, 8, 4, DE, DR>), grid, dim3(512), 0, st, f);
    else if constexpr (MT <= 3) hipLaunchKernelGGL((ffn_decode_kernel<MT, 16, 4, DE, DR>), grid, dim3(1024), 0, st, f);
}

// The depth read fused into the launch: rows <= 32 (MT <= 2), head_dim 64/96/128.
template <int MT>
static bool launch_ffn_depth(const FfnArgs& f, dim3 grid, bool rms, hipStream_t st) {
    if constexpr (MT <= 2) {
        switch (f.g.HD) {
            case 64: rms ? launch_ffn_mt<MT, 4, true>(f, grid, st) : launch_ffn_mt<MT, 4, false>(f, grid, st); return true;
            case 96: rms ? launch_ffn_mt<MT, 6, true>(f, grid, st) : launch_ffn_mt<MT, 6, false>(f, grid, st); return true;
            case 128: rms ? launch_ffn_mt<MT, 8, true>(f, grid, st) : launch_ffn_mt<MT, 8, false>(f, grid, st); return true;
        }
    }
    return false;
}

// The depth read of an ffn_decode descriptor as its own launch, into d_h.
static int ffn_depth_launch(int dtype, const loom_ffn_decode_desc* d, void* stream) {
    if (d->depth_rms != 0)
        return loom_depth_attn_forward_rms(dtype, d->depth_q, d->depth_k, d->depth_v, d->depth_sbt,
                                           d->depth_ss, (void*)d->d_h, nullptr, nullptr, d->M,
                                           d->depth_S, d->n_q_heads, d->head_dim, d->depth_qt,
                                           d->depth_kt, d->depth_vt, stream);
    return loom_depth_attn_forward(dtype, d->depth_q, d->depth_k, d->depth_v, d->depth_sbt,
                                   d->depth_ss, (void*)d->d_h, nullptr, nullptr, d->M, d->depth_S,
                                   d->n_q_heads, d->head_dim, stream);
}

extern "C" int loom_ffn_decode(int dtype, const loom_ffn_decode_desc* d, void* stream) {
    clear_error();
    LOOM_CHECK(d != nullptr, "ffn_decode: null descriptor");
    LOOM_CHECK(d->u && d->q_h && d->k_ctx_h && d->c_h && d->d_h && d->w_compact && d->p_real &&
                   d->imag_bias && d->trace && d->trace_w && d->act && d->carry_out,
               "ffn_decode: null tensor argument");
    LOOM_CHECK(d->axis >= 0 && d->axis <= 2, "ffn_decode: axis must be 0(z), 1(x), or 2(y), got %d",
               (int)d->axis);
    LOOM_CHECK(!(d->carry_prev && d->seed), "ffn_decode: carry_prev and seed are mutually exclusive");
    LOOM_CHECK(!d->seed || d->seed_valid, "ffn_decode: seed needs seed_valid");
    LOOM_CHECK(!d->gate_w || d->p_out, "ffn_decode: gate weights need p_out");
    LOOM_CHECK(d->M >= 0 && d->N > 0 && d->H > 0 && d->head_dim > 0 && d->n_q_heads > 0 &&
                   d->n_q_heads * d->head_dim == d->N && d->hidden_per_q_head * d->n_q_heads == d->H,
               "ffn_decode: bad shape");
    const int64_t want = d->open_sectors ? 4 * d->N + d->head_dim : d->N + 4 * d->head_dim;
    LOOM_CHECK(d->imag_in == want, "ffn_decode: imag_in=%lld, expected %lld", (long long)d->imag_in,
               (long long)want);
    LOOM_CHECK(d->depth_q == nullptr || (d->depth_k && d->depth_v && d->depth_S >= 1 &&
                                         d->depth_ss >= d->N && d->depth_sbt >= d->depth_S * d->depth_ss),
               "ffn_decode: depth read needs k/v history, S >= 1 and non-overlapping strides");
    LOOM_CHECK(d->depth_rms == 0 || (d->depth_qt > 0.0f && d->depth_kt > 0.0f && d->depth_vt > 0.0f),
               "ffn_decode: fixed-RMS depth targets must be > 0");
    if (d->M == 0) return LOOM_OK;
    const uintptr_t al = (uintptr_t)d->u | (uintptr_t)d->q_h | (uintptr_t)d->k_ctx_h |
                         (uintptr_t)d->c_h | (uintptr_t)d->d_h | (uintptr_t)d->w_compact;
    const bool fused = dtype == LOOM_BF16 && d->M <= 64 && d->imag_in % 8 == 0 &&
                       d->hidden_per_q_head % 16 == 0 && d->head_dim % 8 == 0 && d->N % 8 == 0 &&
                       (al & 15) == 0;
    if (fused) {
        FfnArgs f{};
        GemmArgs& a = f.g;
        a.W = d->w_compact; a.ldw = d->imag_in; a.M = d->M; a.N = d->H; a.K = d->imag_in;
        a.src[0] = d->q_h; a.src[1] = d->k_ctx_h; a.src[2] = d->c_h; a.src[3] = d->u; a.src[4] = d->d_h;
        a.Nm = d->N; a.HD = d->head_dim; a.Hq = d->hidden_per_q_head; a.open = d->open_sectors ? 1 : 0;
        a.X = d->u; a.ldx = d->N;
        f.R = (const uint16_t*)d->p_real; f.ib = d->imag_bias; f.trace = (uint16_t*)d->trace;
        f.G = (const uint16_t*)(d->gate_src ? d->gate_src : d->p_real);
        f.tw = d->trace_w; f.m = d->powlu_m; f.act = (uint16_t*)d->act; f.s = (uint16_t*)d->s;
        f.prev = (const uint16_t*)d->carry_prev; f.seed = (const uint16_t*)d->seed;
        f.valid = d->seed_valid; f.gate_w = (const uint16_t*)d->gate_w;
        f.carry = (uint16_t*)d->carry_out; f.p = (uint16_t*)d->p_out; f.alpha = d->alpha;
        f.mode = d->carry_prev ? 1 : (d->seed ? 2 : 0);
        f.axis = d->axis;
        LOOM_CHECK(d->act_frag == nullptr || d->H % 32 == 0, "ffn_decode: act_frag needs H %% 32 == 0");
        f.actf = (uint16_t*)d->act_frag;
        LOOM_CHECK(d->u_frag == nullptr || (!d->open_sectors && d->head_dim % 32 == 0 && d->N % 32 == 0 &&
                                           ((uintptr_t)d->u_frag & 15) == 0),
                   "ffn_decode: u_frag needs head sectors, head_dim and N multiples of 32, 16-byte alignment");
        a.Uf = (const uint4*)d->u_frag;
        const dim3 grid((unsigned)ceil_div(d->H, 16));
        hipStream_t st = (hipStream_t)stream;
        if (d->depth_q != nullptr) {
            // the depth read D of this sublayer: in the launch when it can be, else its own
            // launch first (D then comes from d_h as usual)
            const bool rms = d->depth_rms != 0;
            const bool fusable = !d->open_sectors && d->M <= 32 && d->H % 16 == 0 &&
                                 d->depth_sbt % 2 == 0 && d->depth_ss % 2 == 0 &&
                                 ((((uintptr_t)d->depth_q | (uintptr_t)d->depth_k | (uintptr_t)d->depth_v) & 7) == 0);
            if (fusable) {
                f.dq = (const uint16_t*)d->depth_q; f.dk = (const uint16_t*)d->depth_k;
                f.dv = (const uint16_t*)d->depth_v; f.dsbt = d->depth_sbt; f.dss = d->depth_ss;
                f.dS = d->depth_S; f.dscale = 1.0f / sqrtf((float)d->head_dim);
                f.drms = DepthRms{d->depth_qt, d->depth_kt, d->depth_vt};
                // the earlier slots' part, when given, for the plain read over two or more slots
                const bool part = !rms && d->depth_part_d != nullptr && d->depth_part_lse != nullptr &&
                                  d->depth_S >= 2 && ((uintptr_t)d->depth_part_d & 7) == 0;
                f.dpd = part ? d->depth_part_d : nullptr;
                f.dpl = part ? d->depth_part_lse : nullptr;
                const bool done = d->M <= 16 ? launch_ffn_depth<1>(f, grid, rms, st)
                                             : launch_ffn_depth<2>(f, grid, rms, st);
                if (done) return launch_status("loom_ffn_decode");
            }
            const int rc = ffn_depth_launch(dtype, d, stream);
            if (rc != LOOM_OK) return rc;
        }
        switch ((int)ceil_div(d->M, 16)) {
            case 1: launch_ffn_mt<1>(f, grid, st); break;
            case 2: launch_ffn_mt<2>(f, grid, st); break;
            case 3: launch_ffn_mt<3>(f, grid, st); break;
            default: launch_ffn_mt<4>(f, grid, st); break;
        }
        return launch_status("loom_ffn_decode");
    }
    LOOM_CHECK(d->beta && d->s, "ffn_decode: the unfused path needs the beta and s buffers");
    if (d->depth_q != nullptr) {
        const int rc0 = ffn_depth_launch(dtype, d, stream);
        if (rc0 != LOOM_OK) return rc0;
    }
    LOOM_CHECK(d->act_frag == nullptr, "ffn_decode: act_frag needs the fused bf16 path (M <= 64, aligned)");
    // (u_frag is only read, and u holds the same values: the unfused path reads u)
    int rc = loom_beta_forward(dtype, d->u, d->q_h, d->k_ctx_h, d->c_h, d->d_h, d->w_compact,
                               d->beta, nullptr, d->M, d->N, d->H, d->imag_in, d->hidden_per_q_head,
                               d->head_dim, d->n_q_heads, d->open_sectors, stream);
    if (rc != LOOM_OK) return rc;
    rc = loom_paraplex_forward(dtype, d->p_real, d->gate_src ? d->gate_src : d->p_real, d->beta,
                               d->imag_bias, d->trace,
                               d->trace_w, nullptr, nullptr, d->act, d->s, d->trace, nullptr, d->M,
                               1, d->H, d->powlu_m, stream);
    if (rc != LOOM_OK) return rc;
    return loom_tria_depth_forward(dtype, d->p_real, d->s, d->act, d->carry_prev, d->seed,
                                   d->seed_valid, d->gate_w, d->carry_out, d->p_out, nullptr, d->M,
                                   1, d->H, d->alpha, d->axis, stream);
}

extern "C" int loom_beta_forward(int dtype, const void* u, const void* q_h, const void* k_ctx_h,
                                 const void* c_h, const void* d_h, const void* w_compact,
                                 void* out, void* r_pack, int64_t M, int64_t N, int64_t H,
                                 int64_t imag_in, int64_t hidden_per_q_head, int64_t head_dim,
                                 int64_t n_q_heads, int open_sectors, void* stream) {
    clear_error();
    LOOM_CHECK(u && q_h && k_ctx_h && c_h && d_h && w_compact && out,
               "beta_space: null tensor argument");
    LOOM_CHECK(M >= 0 && N > 0 && H > 0 && head_dim > 0 && n_q_heads > 0, "beta_space: bad shape");
    LOOM_CHECK(n_q_heads * head_dim == N, "beta_space: n_q_heads*head_dim (%lld) != N (%lld)",
               (long long)(n_q_heads * head_dim), (long long)N);
    LOOM_CHECK(hidden_per_q_head * n_q_heads == H, "beta_space: hidden_per_q_head*n_q_heads != H");
    const int64_t want = open_sectors ? 4 * N + head_dim : N + 4 * head_dim;
    LOOM_CHECK(imag_in == want, "beta_space: imag_in=%lld, expected %lld", (long long)imag_in,
               (long long)want);
    LOOM_CHECK((N % 4) == 0 && (head_dim % 4) == 0 && (imag_in % 4) == 0,
               "maskpack path requires N, head_dim, IMAG_IN divisible by 4");
    GemmArgs a{};
    a.W = w_compact; a.ldw = imag_in; a.out = out; a.ldc = H; a.M = M; a.N = H; a.K = imag_in;
    a.src[0] = q_h; a.src[1] = k_ctx_h; a.src[2] = c_h; a.src[3] = u; a.src[4] = d_h;
    a.Nm = N; a.HD = head_dim; a.Hq = hidden_per_q_head; a.open = open_sectors ? 1 : 0;
    a.X = u; a.ldx = N;
    switch (dtype) {
        case LOOM_F32: return beta_dispatch<float>(a, r_pack, n_q_heads, (hipStream_t)stream);
        case LOOM_BF16: return beta_dispatch<bf16_t>(a, r_pack, n_q_heads, (hipStream_t)stream);
        case LOOM_F16: return beta_dispatch<f16_t>(a, r_pack, n_q_heads, (hipStream_t)stream);
    }
    set_error("beta_space: unsupported dtype %d", dtype);
    return LOOM_ERR_INVALID;
}

// The chunked prefill's projections of one hidden state for the next block:
// qkv = x w_qkv^T, then RoPE of q and k and the cache append of k and v
// (as loom_gqa_prefill's first step), and optionally the history projection
// hist_out = x w_hist^T.  bf16 with 96-wide heads and at least 256 rows: one
// launch of 256 x 192 tiles, the RoPE and the cache stores in its epilogue
// (each wave's 96 columns are one head) and the history columns as a second
// product of the same launch; qkv is never stored.  Otherwise the two
// products into qkv_scratch / hist_out and the separate RoPE + append launch.
extern "C" int loom_gemm_shared_tiles(int on) {
    return g_shared_tiles.exchange(on != 0 ? 1 : 0);
}

extern "C" int loom_prefill_qkv(int dtype, const void* x, int64_t ldx, const void* w_qkv,
                                const void* w_hist, void* hist_out, int64_t hist_ld, int64_t n_hist,
                                void* qkv_scratch, void* q_out, void* k_cache, void* v_cache,
                                int64_t cache_stride_b, int64_t cache_stride_t,
                                int64_t cache_stride_h, const float* cos_table,
                                const float* sin_table, int64_t B, int64_t T, int64_t start,
                                int64_t cache_len, int64_t K, int64_t QH, int64_t KVH, int64_t HD,
                                void* stream) {
    clear_error();
    LOOM_CHECK(x && w_qkv && qkv_scratch && q_out && k_cache && v_cache && cos_table && sin_table,
               "prefill_qkv: null argument");
    LOOM_CHECK(w_hist == nullptr || (hist_out != nullptr && n_hist >= 1 && hist_ld >= n_hist),
               "prefill_qkv: history projection without output or width");
    LOOM_CHECK(B >= 0 && T >= 0 && start >= 0 && K >= 1 && ldx >= K && KVH >= 1 && QH % KVH == 0 &&
                   HD >= 2 && HD % 2 == 0,
               "prefill_qkv: bad shape B=%lld T=%lld K=%lld QH=%lld KVH=%lld HD=%lld", (long long)B,
               (long long)T, (long long)K, (long long)QH, (long long)KVH, (long long)HD);
    LOOM_CHECK(cache_stride_t >= HD && cache_stride_h >= HD, "prefill_qkv: cache strides smaller than a head row");
    LOOM_CHECK(start + T <= cache_len && start + T < (1LL << 31),
               "prefill_qkv: positions %lld..%lld beyond the cache capacity %lld", (long long)start,
               (long long)(start + T - 1), (long long)cache_len);
    const int64_t M = B * T, QKV = (QH + 2 * KVH) * HD;
    if (M == 0) return LOOM_OK;
    hipStream_t st = (hipStream_t)stream;
    const uintptr_t a16 = (uintptr_t)x | (uintptr_t)w_qkv | (uintptr_t)w_hist | (uintptr_t)cos_table |
                          (uintptr_t)sin_table;
    const uintptr_t a8 = (uintptr_t)q_out | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)hist_out;
    const bool shared = g_shared_tiles.load(std::memory_order_relaxed) != 0;
    const bool fused = dtype == LOOM_BF16 && HD == 96 && QKV % BgTall::BG_N == 0 &&
                       (shared ? big_fits<BgTallS>(M, K, false, 0) : big_fits<BgTall>(M, K, false, 0)) &&
                       K % 8 == 0 && ldx % 8 == 0 &&
                       (a16 & 15) == 0 && (a8 & 7) == 0 && cache_stride_b % 4 == 0 &&
                       cache_stride_t % 4 == 0 && cache_stride_h % 4 == 0 &&
                       (w_hist == nullptr || hist_ld % 4 == 0);
    if (fused) {
        GemmArgs a{};
        a.X = x; a.ldx = ldx; a.W = w_qkv; a.ldw = K; a.out = qkv_scratch; a.ldc = QKV;
        a.M = M; a.N = QKV + (w_hist != nullptr ? n_hist : 0); a.K = K;
        if (w_hist != nullptr) {
            a.N1 = QKV; a.Wb = w_hist; a.ldwb = K; a.outb = hist_out; a.ldcb = hist_ld;
        }
        a.rope = GemmArgs::RopeOut{q_out, k_cache, v_cache, cache_stride_b, cache_stride_t,
                                   cache_stride_h, cos_table, sin_table, T, start, (int)QH, (int)KVH};
        if (shared) launch_big_cfg<false, BgTallS>(a, 1, st);
        else launch_big_cfg<false, BgTall>(a, 1, st);
        return launch_status("loom_prefill_qkv");
    }
    int rc = loom_linear(dtype, x, ldx, w_qkv, K, nullptr, nullptr, 0.0f, nullptr, qkv_scratch, QKV, M,
                         QKV, K, stream);
    if (rc != LOOM_OK) return rc;
    if (w_hist != nullptr) {
        rc = loom_linear(dtype, x, ldx, w_hist, K, nullptr, nullptr, 0.0f, nullptr, hist_out, hist_ld, M,
                         n_hist, K, stream);
        if (rc != LOOM_OK) return rc;
    }
    return prefill_rope_append(dtype, qkv_scratch, QKV, k_cache, v_cache, cache_stride_b,
                               cache_stride_t, cache_stride_h, cos_table, sin_table, q_out, B, T, start,
                               QH, KVH, HD, st);
}
