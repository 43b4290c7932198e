/*
 * loom_hip.h -- C ABI of libloom_hip.so, the gfx950 (MI355X) implementation of
 * LoomFormer's fused-kernel inference path.
 *
 * Every entry point replaces one function of the reference's CUDA extensions
 * (srose69/Loomformer-Paraplex, kernels/ *_launcher.cu and
 * kernels/tria/bindings.cpp); the reference citation is given per function.
 *
 * Conventions (shared by all entry points):
 *   - Plain pointers to device memory, element counts as int64_t; no tensor
 *     types.  Tensors are dense row-major unless a stride argument says
 *     otherwise.  The caller allocates every output (the reference launchers
 *     allocate with torch::empty; the Python mirror does that instead).
 *   - `dtype` is a loom_dtype and applies to the "activation" tensors named in
 *     each comment; parameters documented as float are always fp32.
 *   - bool tensors are 1 byte per element (uint8_t, 0 or 1).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = default stream).  No
 *     entry point synchronises the host or allocates device memory.
 *   - Return value: LOOM_OK, or a negative error code with a message readable
 *     through loom_last_error() (thread-local).  The Python mirror raises
 *     RuntimeError(message), like the reference's TORCH_CHECK.
 */
#ifndef LOOM_HIP_H
#define LOOM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum loom_dtype { LOOM_F32 = 0, LOOM_BF16 = 1, LOOM_F16 = 2 };

enum loom_status {
    LOOM_OK = 0,
    LOOM_ERR_INVALID = -1,     /* bad argument / unsupported shape or dtype */
    LOOM_ERR_LAUNCH = -2,      /* HIP reported an error for a launch */
};

/* Last error message of the calling thread ("" if none). */
const char* loom_last_error(void);
/* ABI version (bumped on any signature change). */
int loom_abi_version(void);

/* ---------------------------------------------------------------------------
 * Paraplex FFN
 * ------------------------------------------------------------------------ */

/* Fused Paraplex pointwise chain.  Replaces paraplex_forward_cuda
 * (kernels/paraplex/paraplex_launcher.cu:49) in eval mode.
 *   p_real, gate_src, beta_linear: [B,T,H] dtype (gate_src may equal p_real)
 *   bias, trace_w: [H] float;  trace: [B,H] dtype;  reset: [B,T] bool or NULL
 *   anchor: [1] float, copied to anchor_snapshot (eval: no EMA update)
 *   outputs act (=O), s (=I): [B,T,H] dtype; next_trace: [B,H] dtype (I_base
 *   at t = T-1).  m = powlu_m.
 */
int loom_paraplex_forward(int dtype, const void* p_real, const void* gate_src,
                          const void* beta_linear, const float* bias, const void* trace,
                          const float* trace_w, const uint8_t* reset, const float* anchor,
                          void* act, void* s, void* next_trace, float* anchor_snapshot,
                          int64_t B, int64_t T, int64_t H, float m, void* stream);

/* sin(pi/2 * beta / sqrt(1 + beta^2)), elementwise.  Replaces
 * phase_sin_forward_cuda (kernels/phase_sin/phase_sin_launcher.cu:11). */
int loom_phase_sin_forward(int dtype, const void* beta, void* out, int64_t n, void* stream);

/* x1 * max(x2,1e-12)^(m/(sqrt(x2)+1)) * sigmoid(x2), elementwise.  Replaces
 * pvpowlu_forward_cuda (kernels/pvpowlu/pvpowlu_launcher.cu:11). */
int loom_pvpowlu_forward(int dtype, const void* x1, const void* x2, void* out, int64_t n,
                         float m, void* stream);

/* Sector-gathered grouped W_imag product (no packed copy is materialised).
 * Replaces beta_forward_cuda (kernels/beta_space/beta_space_launcher.cu:225,
 * pack kernel beta_space_kernel.cuh:87 + cuBLAS strided-batched GEMM :57).
 *   u: [M,N]; q_h, k_ctx_h, c_h, d_h: [M, n_q_heads*head_dim] (= [M,N]);
 *   w_compact: [H, imag_in] with imag_in = N + 4*head_dim (head sectors) or
 *   4*N + head_dim (open sectors);  out: [M,H].  All dtype; fp32 accumulate.
 *   Group g (hidden rows [g*Hq,(g+1)*Hq), Hq = hidden_per_q_head) reads the
 *   activation row [Q_g | Kctx_g | C_g | U | D_g] (head) or
 *   [Q_g | Kctx | C | U | D] (open).
 *   If r_pack is not NULL the packed activations [n_q_heads, M, imag_in] are
 *   also written (the reference's second output). */
int loom_beta_forward(int dtype, const void* u, const void* q_h, const void* k_ctx_h,
                      const void* c_h, const void* d_h, const void* w_compact, void* out,
                      void* r_pack, int64_t M, int64_t N, int64_t H, int64_t imag_in,
                      int64_t hidden_per_q_head, int64_t head_dim, int64_t n_q_heads,
                      int open_sectors, void* stream);

/* Dense projection out[M,Nout] = epilogue(A[M,K] @ W[Nout,K]^T), fp32
 * accumulate (bf16 operands on MFMA).  Replaces the F.linear calls of the
 * path: ParaplexFFN w1_real (loomformer.py:2839) with the IdentityAnchoredGate
 * epilogue (tria.py:1287-1299), w2 (loomformer.py:2854), DepthAttn.project
 * (loomformer.py:3397), attention qkv/o (loomformer.py:3262, 3332), the Tria
 * readout and final cross-attention projections and the LM head.
 *   lda/ldw/ldc: row strides in elements.  bias: [Nout] float or NULL.
 *   gate_p: [M,Nout] dtype (row stride ldc) or NULL; when given the epilogue is
 *   acc * (1 + gate_alpha * gate_p) + bias, otherwise acc + bias.
 *   residual: [M,Nout] dtype (row stride ldc) or NULL; added last. */
int loom_linear(int dtype, const void* A, int64_t lda, const void* W, int64_t ldw,
                const float* bias, const void* gate_p, float gate_alpha, const void* residual,
                void* out, int64_t ldc, int64_t M, int64_t Nout, int64_t K, void* stream);

/* One output segment of loom_linear_multi: n columns with their own weight
 * rows, output, bias and identity-anchored gate. */
typedef struct {
    const void* w;        /* [n, k] rows multiplying x (row stride ldw) */
    int64_t ldw;
    const void* w2;       /* [n, k2] rows multiplying x2; NULL when k2 == 0 */
    int64_t ldw2;
    void* out;            /* [m, n] output (row stride ldc) */
    int64_t ldc;
    const float* bias;    /* [n] fp32 or NULL */
    const void* gate_p;   /* [m, n] dtype (row stride gate_ld; over 64 rows gate_ld == ldc) or NULL;
                             single-input only */
    int64_t gate_ld;
    float gate_alpha;
    int64_t n;
} loom_linear_segment;

typedef struct {
    const void* x;        /* [m, k] activations (row stride ldx) */
    int64_t ldx;
    int64_t k;
    const void* x2;       /* [m, k2] second activations or NULL (k2 = 0) */
    int64_t ldx2;
    int64_t k2;
    int64_t m;
    int32_t nseg;         /* 1..4 */
    loom_linear_segment seg[4];
    const uint8_t* only_if;   /* optional [only_if_n] device flags: when none is set the */
    int64_t only_if_n;        /* bf16 fused launch leaves every output untouched */
    const void* x_frag;   /* optional fragment-major copy of x (k % 32 == 0), else NULL */
    const void* x2_frag;  /* optional fragment-major copy of x2 (k2 % 32 == 0), else NULL */
} loom_linear_multi_desc;

/* Fragment-major layout of an [m, k] bf16 matrix (m <= 64, k % 32 == 0), the
 * operand order of v_mfma_f32_16x16x32_bf16: the 16-byte piece at index
 * (j*(k/32) + s)*64 + l (j < ceil(m/16), s < k/32, l < 64) holds row
 * 16*j + l%16, columns 32*s + 8*(l/16) .. +7; rows >= m are never read.  A
 * decode projection reads its activations from such a copy as whole 1 KB
 * runs per load instruction instead of 16 rows x 64 B (measured about 2 us
 * faster per launch for the 32 x 768 decode activations).  The fused bf16
 * launch of loom_linear_multi reads x_frag / x2_frag instead of x / x2 when
 * they are set (they must hold the same values); loom_linear_ln can write one
 * (out_frag). */

/* Several decode projections in one launch (no counterpart in the reference;
 * the engine's restatement of Model.step, loomformer.py:3951-4091, uses it to
 * merge adjacent nn.Linear calls):
 *   seg s: out_s = (x w_s^T + x2 w2_s^T) [* (1 + gate_alpha * gate_p)] + bias
 * Concatenation along k sums two products in one accumulator (o-projection
 * plus depth read-out before LayerNorm); segments share x (e.g. the depth
 * history projection and W_real of the same hidden state).  bf16 with m <= 64
 * runs as one fused MFMA launch; other dtypes run one product per piece.
 * only_if (may be NULL) lets a captured step skip a product it needs only on
 * some steps: the fused launch reads the flags on the device and does nothing
 * when none is set (the other paths compute the product anyway). */
int loom_linear_multi(int dtype, const loom_linear_multi_desc* desc, void* stream);

/* sizeof(loom_linear_multi_desc), so an FFI binding can check its layout. */
int64_t loom_linear_multi_desc_bytes(void);

/* out = LayerNorm(x w^T + x2 w2^T + bias) * gamma + beta for a one-segment
 * descriptor (no gate; N <= 2048): the sublayer tails
 * ln_attn(skip + attn_out) and ln_ffn(skip + ffn_out) of Model.step
 * (loomformer.py:4000, :4045) with both products in one accumulator.  No
 * counterpart in the reference as one call.  bf16 with m <= 64 splits K over
 * blocks, writing fp32 partial sums to the workspace (at least
 * loom_linear_ln_workspace_bytes(m, n), 16-byte aligned), and the LayerNorm
 * kernel adds them up; other cases write x w^T + x2 w2^T + bias to seg[0].out
 * (dense [m, n]) and normalise that.  out_frag (optional, the bf16 split-K form
 * with n % 32 == 0 only): the result also in fragment-major order. */
int loom_linear_ln(int dtype, const loom_linear_multi_desc* desc, const float* gamma,
                   const float* beta, float eps, void* out, int64_t ldo, float* workspace,
                   int64_t workspace_bytes, void* out_frag, void* stream);
int64_t loom_linear_ln_workspace_bytes(int64_t M, int64_t N);

/* One decode token (T = 1) of the Paraplex FFN core and the Tria depth op. */
typedef struct {
    /* beta space, as loom_beta_forward */
    const void* u;
    const void* q_h;
    const void* k_ctx_h;
    const void* c_h;
    const void* d_h;
    const void* w_compact;
    int64_t M, N, H, imag_in, hidden_per_q_head, head_dim, n_q_heads;
    int32_t open_sectors;
    /* Paraplex pointwise, as loom_paraplex_forward with T = 1 */
    const void* p_real;        /* R [M, H] */
    const void* gate_src;      /* [M, H] amplitude source, or NULL for p_real (paraplex_gate_proj
                                  off, loomformer.py:2849) */
    const float* imag_bias;    /* [H] */
    void* trace;               /* [M, H]: previous phase in, this token's phase out */
    const float* trace_w;      /* [H] */
    float powlu_m;
    void* act;                 /* [M, H] out */
    void* s;                   /* [M, H] out; optional on the fused path */
    void* beta;                /* [M, H] scratch; optional on the fused path */
    /* Tria depth op on (p_real, s, act), as loom_tria_depth_forward with T = 1 */
    const void* carry_prev;
    const void* seed;
    const uint8_t* seed_valid;
    const void* gate_w;
    void* carry_out;
    void* p_out;
    float alpha;
    int32_t axis;
    void* act_frag;            /* optional fragment-major copy of act (fused path, H % 32 == 0) */
    const void* u_frag;        /* optional fragment-major copy of u (head sectors, head_dim and N
                                  multiples of 32): the fused path reads the u sector from it */
    /* optional: d_h is computed by this call, not read: D = DepthAttn over
       history slots 0..depth_S-1 (DepthAttn.forward, loomformer.py:3404-3429;
       as loom_depth_attn_forward, or _rms with depth_rms) is written to d_h.
       bf16 head sectors with M <= 32 and head_dim 64/96/128 read it inside the
       launch (each column block recomputes its head's rows, the first block of
       each head writes them); other cases run the depth launch first. */
    const void* depth_q;       /* [n_q_heads, head_dim] learned queries of the slot, or NULL */
    const void* depth_k;       /* history keys (b, slot, head) at b*depth_sbt + slot*depth_ss + head*head_dim */
    const void* depth_v;
    int64_t depth_sbt, depth_ss;
    int32_t depth_S;
    int32_t depth_rms;         /* nonzero: fixed-RMS q/k/v with the targets below */
    float depth_qt, depth_kt, depth_vt;
    /* optional (plain read, depth_S >= 2, the in-launch form): the read over
       slots 0..depth_S-2 already done, as normalised fp32 rows depth_part_d
       [M, n_q_heads, head_dim] (8-byte aligned) and their log-sum-exp
       depth_part_lse [M, n_q_heads] (natural units), e.g. from
       loom_gqa_decode_step_depth2; the launch then reads slot depth_S-1 only
       and combines the two parts in one softmax.  NULL: every slot is read. */
    const float* depth_part_d;
    const float* depth_part_lse;
} loom_ffn_decode_desc;

/* beta = beta_space(u, q, kctx, c, d); (act, s, trace) = paraplex(R, beta);
 * (carry_out, p_out) = tria_depth(R, s, act) for one decode token: the
 * sequence loom_beta_forward -> loom_paraplex_forward -> loom_tria_depth_forward
 * of Model.step's FFN and depth step (loomformer.py:2818-2893, :4012-4040).
 * No counterpart in the reference as one call.  bf16 with M <= 64 runs as one
 * launch whose epilogue evaluates the pointwise chain and the Tria op on the
 * product in registers (beta and s stay on chip; R, s, act enter the Tria op
 * rounded to bf16 as the unfused sequence stores them); other cases run the
 * three entry points in turn and need the beta and s buffers. */
int loom_ffn_decode(int dtype, const loom_ffn_decode_desc* desc, void* stream);

/* sizeof(loom_ffn_decode_desc), so an FFI binding can check its layout. */
int64_t loom_ffn_decode_desc_bytes(void);

/* ---------------------------------------------------------------------------
 * Depth attention
 * ------------------------------------------------------------------------ */

/* Softmax read over the depth axis with one learned query per q-head.
 * Replaces depth_attn_forward_cuda (kernels/depth_attn/depth_attn_launcher.cu:63,
 * outputs d and weights) and depth_attn_stacked_forward_cuda (:143, outputs d
 * and lse).
 *   q: [QH,HD] dtype.  hist_k/hist_v: element (bt, s, qh, d) at
 *   bt*stride_bt + s*stride_s + qh*HD + d, dtype (a strided history view
 *   such as hist[:, :, :S] of a [B,T,S_max,QH,HD] buffer needs no copy).
 *   d_out: [BT,QH,HD] dtype.  w_out: [BT,QH,S] dtype or NULL.
 *   lse_out: [BT,QH] float or NULL.  Scores are fp32, scale 1/sqrt(HD). */
int loom_depth_attn_forward(int dtype, const void* q, const void* hist_k, const void* hist_v,
                            int64_t stride_bt, int64_t stride_s, void* d_out, void* w_out,
                            float* lse_out, int64_t BT, int64_t S, int64_t QH, int64_t HD,
                            void* stream);

/* Two DepthAttn reads over the same history slots 0..S-1 in one pass over
 * them: q1's read d_out [BT,QH,HD] dtype as loom_depth_attn_forward gives it,
 * and q2's read as normalised fp32 rows part_d [BT,QH,HD] with their
 * log-sum-exp part_lse [BT,QH] (natural units) -- the part of the next
 * sublayer's read over slots 0..S (DepthAttn.forward with that sublayer's
 * query, loomformer.py:3404-3429) that these slots contribute.  head_dim
 * 32/64/96/128, 8-byte aligned rows, even strides.  No counterpart in the
 * reference (it reads every slot again for every sublayer). */
int loom_depth_attn_pair(int dtype, const void* q1, const void* q2, const void* hist_k,
                         const void* hist_v, int64_t stride_bt, int64_t stride_s, void* d_out,
                         float* part_d, float* part_lse, int64_t BT, int64_t S, int64_t QH,
                         int64_t HD, void* stream);

/* The read of query q over slots 0..S-1 (S >= 2) from the read over slots
 * 0..S-2 given as part_d / part_lse (as loom_depth_attn_pair writes them) and
 * slot S-1's key and value rows: one softmax over the two parts, written to
 * d_out [BT,QH,HD] dtype.  Same layouts and limits as loom_depth_attn_pair. */
int loom_depth_attn_fold(int dtype, const void* q, const void* hist_k, const void* hist_v,
                         int64_t stride_bt, int64_t stride_s, int64_t S, const float* part_d,
                         const float* part_lse, void* d_out, int64_t BT, int64_t QH, int64_t HD,
                         void* stream);

/* loom_depth_attn_forward for DepthAttn under depth_attn_qkv_rms
 * (loomformer.py:3397-3407): the query, key and value rows are read as
 * fixed-RMS vectors x * t / sqrt(mean(x^2) + 1e-6) with targets q_target
 * (fanin_std(HD) in the reference), k_target (FANIN_GAIN) and v_target
 * (FANIN_GAIN * DEEPNORM_BETA); the history itself is stored as projected.
 * Same layout and outputs as loom_depth_attn_forward; targets must be > 0.
 * No counterpart in the reference's kernels (its module rescales q, k, v
 * with torch ops before calling depth_attn_forward_cuda). */
int loom_depth_attn_forward_rms(int dtype, const void* q, const void* hist_k, const void* hist_v,
                                int64_t stride_bt, int64_t stride_s, void* d_out, void* w_out,
                                float* lse_out, int64_t BT, int64_t S, int64_t QH, int64_t HD,
                                float q_target, float k_target, float v_target, void* stream);

/* ---------------------------------------------------------------------------
 * Tria (all math fp32; carry tensors [n,3,3] row-major per element)
 * ------------------------------------------------------------------------ */

/* Depth step family.  Per element e=(b,t,h) of n = B*T*H:
 *   M = T(r,i,o; alpha, axis)                          (carrier.cuh:33)
 *   pre = M @ seed[b,h]  if seed && t == 0 && seed_valid[b]
 *         M @ carry_prev[e] if carry_prev
 *         M             otherwise
 *   carry_out[e] = pre / rms(pre);  scale_out[e] = rms(pre);
 *   p_out[e] = sum_k w[k] * carry_out[e][k]           (gate variants)
 * Replaces tria_init_forward, tria_init_gate_forward, tria_init_seed_forward,
 * tria_init_seed_gate_forward, tria_step_forward, tria_step_gate_forward
 * (kernels/tria/bindings.cpp:84-93).
 *   r,i,o: [B,T,H] dtype; carry_prev: [B,T,H,3,3] dtype or NULL;
 *   seed: [B,H,3,3] dtype or NULL; seed_valid: [B] bool (needed with seed);
 *   w: [9] dtype or NULL; carry_out: dtype or NULL; p_out: [B,T,H] dtype (needed
 *   with w); scale_out: [B,T,H] float or NULL.  seed and carry_prev are
 *   mutually exclusive. */
int loom_tria_depth_forward(int dtype, const void* r, const void* i, const void* o,
                            const void* carry_prev, const void* seed, const uint8_t* seed_valid,
                            const void* w, void* carry_out, void* p_out, float* scale_out,
                            int64_t B, int64_t T, int64_t H, float alpha, int axis, void* stream);

/* (act, next_trace) = paraplex(R, beta) and (carry_out, p_out) =
 * tria_depth(R, I, act) in one pass over a [B, T, H] sequence: the sequence
 * form of loom_paraplex_forward (no reset, no anchor snapshot) followed by
 * loom_tria_depth_forward, with the phase I never stored.  Restates
 * ParaplexFFN's pointwise core (loomformer.py:2856-2885) and the block's
 * _tria_depth_op (:3588-3617) as the chunked forward runs them (:3788-3883);
 * no counterpart in the reference as one call.  The Tria op reads I and act
 * rounded to dtype, as the separate ops see them, so the outputs equal theirs.
 *   p_real, gate_src (== p_real when paraplex_gate_proj is off), beta_linear:
 *   [B,T,H] dtype; bias, trace_w: [H] float; trace: [B,H] dtype (the base phase
 *   of the token before t = 0); act: [B,T,H] out; next_trace: [B,H] out (the
 *   base phase of t = T-1; it must not be the trace buffer when T > 1, which
 *   is rejected); carry_prev / seed / seed_valid / w / carry_out / p_out as
 *   loom_tria_depth_forward (carry_out required, no scale_out). */
int loom_paraplex_tria_forward(int dtype, const void* p_real, const void* gate_src,
                               const void* beta_linear, const float* bias, const void* trace,
                               const float* trace_w, float m, const void* carry_prev,
                               const void* seed, const uint8_t* seed_valid, const void* w,
                               void* act, void* next_trace, void* carry_out, void* p_out,
                               int64_t B, int64_t T, int64_t H, float alpha, int axis,
                               void* stream);

/* The last block of a chunk: (act, next_trace) and the Tria step of
 * loom_paraplex_tria_forward with carried records (no gate), and the chunk's
 * temporal carry endpoint of the resulting carries, in one pass that never
 * stores the carries.  The endpoint is the one
 * loom_temporal_carry_endpoint_forward computes from those carries as
 * stored (rounded to dtype), bit for bit.  Restates the block sequence of
 * loomformer.py:2856-2885, :3588-3617 and the chunk endpoint of :3834-3850;
 * no counterpart in the reference as one call.
 *   p_real, gate_src, beta_linear, bias, trace, trace_w, carry_prev, act,
 *   next_trace: as loom_paraplex_tria_forward (carry_prev required);
 *   reset: [B,T] bool, initial: [B,H,3,3] dtype or NULL, initial_valid: [B]
 *   bool or NULL, endpoint: [B,H,3,3] dtype out (may be initial),
 *   endpoint_f32: [B,H,3,3] float out or NULL: as
 *   loom_temporal_carry_endpoint_forward.  H must be even and the element
 *   operands aligned to two elements (bias and trace_w to 8 bytes); B < 65536. */
int loom_paraplex_tria_endpoint_forward(int dtype, const void* p_real, const void* gate_src,
                                        const void* beta_linear, const float* bias,
                                        const void* trace, const float* trace_w, float m,
                                        const void* carry_prev, const uint8_t* reset,
                                        const void* initial, const uint8_t* initial_valid,
                                        void* act, void* next_trace, void* endpoint,
                                        float* endpoint_f32, int64_t B, int64_t T, int64_t H,
                                        float alpha, int axis, void* stream);

/* p[e] = sum_k w[k] * carry[e][k].  Replaces gate_slot_mix_forward
 * (kernels/tria/bindings.cpp:97). carry: [n,9] dtype, w: [9] dtype, p: [n] dtype. */
int loom_gate_slot_mix_forward(int dtype, const void* carry, const void* w, void* p, int64_t n,
                               void* stream);

/* Softmax over H of <score_w, vec C_h> per row, pooled 9-slot mean and lse.
 * Replaces slot_attention_pool_forward (bindings.cpp:99).
 *   carry: [rows,H,9] dtype; score_w: [9] dtype; pooled: [rows,9] dtype;
 *   lse: [rows] dtype (may be NULL). */
int loom_slot_attention_pool_forward(int dtype, const void* carry, const void* score_w,
                                     void* pooled, void* lse, int64_t rows, int64_t H,
                                     void* stream);

/* Temporal carry over T per (b,h) stream: acc_t = N(D_t @ acc_{t-1}), restart
 * acc = N(D_t) on reset[b,t] or when no valid state is held.
 * Full form replaces temporal_carry_forward (bindings.cpp:101): doc [B,T,H,9]
 * float and scale [B,T,H] float (either may be NULL).
 * Endpoint form replaces temporal_carry_endpoint_forward (bindings.cpp:103):
 * initial [B,H,9] dtype or NULL, initial_valid [B] bool or NULL (all valid),
 * endpoint [B,H,9] dtype, endpoint_f32 [B,H,9] float (either may be NULL).
 *   depth: [B,T,H,9] dtype; reset: [B,T] bool. */
int loom_temporal_carry_forward(int dtype, const void* depth, const uint8_t* reset,
                                float* doc, float* scale, int64_t B, int64_t T, int64_t H,
                                void* stream);
int loom_temporal_carry_endpoint_forward(int dtype, const void* depth, const uint8_t* reset,
                                         const void* initial, const uint8_t* initial_valid,
                                         void* endpoint, float* endpoint_f32, int64_t B,
                                         int64_t T, int64_t H, void* stream);

/* PolARM on [n,3,3] matrices, applied where mask[n / per_mask] is set (mask
 * NULL = everywhere): G = M^T M, s = max(mean(diag G), eps),
 * M <- M (I - beta/2 (G/s - I)).  In place allowed (in == out).
 * Replaces tria.polarm (tria.py:128-166), which has no kernel in the reference. */
int loom_polarm_forward(int dtype, const void* in, void* out, const uint8_t* mask,
                        int64_t n, int64_t per_mask, float beta, float eps, void* stream);

/* Tria path of the chunked sequence forward (Model._forward_chunked,
 * loomformer.py:3788-3883) on the fixed fire grid every W tokens (no <CARRY>
 * id; loom_tria_chunked_forward_fires below takes explicit fires), in two
 * launches: every token's L-layer depth composition (axis l % 3, C_1 = N(T_1),
 * C_l = N(T_l C_{l-1})) folded into per-chunk temporal products, then the scan
 * over chunk boundaries (seeded chunk starts, temporal restarts at document
 * resets, PolARM at valid fires).  Replaces the per-chunk sequence of
 * tria_init_seed / tria_step / temporal_carry_endpoint / polarm calls the
 * reference issues (tria.py:814-910, :1089-1141, :128-166); the gated-slot
 * outputs p of the middle layers are not produced (they feed the hidden
 * stream, not the Tria carry).
 *   r, i, o: L stacked [B,T,H] dtype slices, layer l at offset l*layer_stride;
 *   reset: [B,T] bool (document starts; NULL = none after t = 0);
 *   keys: [B, ceil(T/W)-1, H, 3, 3] float, the state after each boundary
 *   (chunk ends except the last, t = T-1 never fires); may be NULL when T <= W;
 *   depth_out: [B,T,H,3,3] dtype final-layer carry per token, or NULL;
 *   ws: loom_tria_chunked_workspace_bytes(B,T,H,W) bytes, no initial contents;
 *   eps: PolARM's floor for mean(diag M^T M) (1e-6 in the reference). */
int64_t loom_tria_chunked_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t W);
int loom_tria_chunked_forward(int dtype, const void* r, const void* i, const void* o,
                              int64_t layer_stride, int64_t L, const uint8_t* reset,
                              float* keys, void* depth_out, void* ws, int64_t ws_bytes,
                              int64_t B, int64_t T, int64_t H, int64_t W, float alpha,
                              float polarm_beta, float eps, void* stream);

/* The same with explicit <CARRY> fires (Model._forward_chunked with a carry
 * token id, loomformer.py:3797-3815, :3852-3861): boundaries are the grid
 * positions plus every position where any row fires explicitly, so chunks are
 * ragged and T-1 can be a boundary; a row's fire at boundary t is
 * (grid(t) & ~reset[t+1]) | explicit_fire[t], and every boundary emits a key
 * for every row with that fire as its validity.
 *   explicit_fire: [B,T] uint8 on the device (NULL = none);
 *   bounds: HOST array of the n_bounds boundary positions, strictly increasing
 *   in [0, T), holding every grid position ((t+1) % W == 0, t < T-1): the
 *   reference's boundary_positions, (grid | explicit_fire.any(0)).nonzero(),
 *   which it too builds on the host (:3814);
 *   keys: [B, n_bounds, H, 3, 3] float; key_valid: [B, n_bounds] uint8 or NULL;
 *   ws: loom_tria_chunked_fires_workspace_bytes(B,T,H,bounds,n_bounds) bytes.
 * The chunk ends are uploaded from the host array and the stream synchronised
 * before the launches (not capturable in a graph). */
int64_t loom_tria_chunked_fires_workspace_bytes(int64_t B, int64_t T, int64_t H,
                                                const int64_t* bounds, int64_t n_bounds);
int loom_tria_chunked_forward_fires(int dtype, const void* r, const void* i, const void* o,
                                    int64_t layer_stride, int64_t L, const uint8_t* reset,
                                    const uint8_t* explicit_fire, const int64_t* bounds,
                                    int64_t n_bounds, float* keys, uint8_t* key_valid,
                                    void* depth_out, void* ws, int64_t ws_bytes, int64_t B,
                                    int64_t T, int64_t H, int64_t W, float alpha,
                                    float polarm_beta, float eps, void* stream);

/* Causal GQA attention of a chunk of T prompt tokens at positions
 * start .. start+T-1, for prefilling the decode state chunk by chunk (the
 * reference runs its stack chunk by chunk in Model._forward_chunked,
 * loomformer.py:3788-3883, with GroupedQueryCausalSelfAttention's readouts
 * C = A.V and Kctx = A.K_roped, :3215-3332).  Ropes q and k of every token
 * (tables as in loom_rope_append), writes the roped q to q_out [B,T,QH,HD],
 * appends (k_roped, v) at rows start.. of the caches (strides as in
 * loom_gqa_decode_step; cache_len = their capacity in positions), then
 * attends token t to cache rows 0..start+t.
 *   qkv: rows (b,t) of [q | k | v] ((QH + 2 KVH) HD) at qkv_ld elements apart,
 *   or NULL: then q_out already holds the chunk's roped q and the caches its
 *   rows (loom_prefill_qkv wrote them), and only the attention runs;
 *   c_out, kctx_out: rows (b,t) of QH*HD at out_ld elements apart.
 * No counterpart in the reference (its chunked forward uses SDPA per chunk). */
int loom_gqa_prefill(int dtype, const void* qkv, int64_t qkv_ld, void* k_cache, void* v_cache,
                     int64_t cache_stride_b, int64_t cache_stride_t, int64_t cache_stride_h,
                     const float* cos_table, const float* sin_table, void* q_out, void* c_out,
                     void* kctx_out, int64_t out_ld, int64_t B, int64_t T, int64_t start,
                     int64_t cache_len, int64_t QH, int64_t KVH, int64_t HD, void* stream);

/* Shared-tile mode of the many-row products (loom_linear, loom_linear_multi,
 * loom_linear_ln, loom_beta_forward, loom_prefill_qkv): on = 1 picks tiles of
 * 128 x 192 (four waves, two blocks per CU) wherever they fit, for products
 * that run beside another stream's kernels (the chunked prefill); on = 0, the
 * default, picks the tiles that are fastest alone.  Results agree with the
 * default mode's to the rounding of the output type (the k order inside an
 * MFMA, and loom_linear_ln's split-K count, may differ).  Process-wide;
 * returns the previous mode.
 * No counterpart in the reference (a scheduling choice of this library). */
int loom_gemm_shared_tiles(int on);

/* The chunked prefill's projections of one hidden state x [B*T, K] (row
 * stride ldx) for the next block: qkv = x w_qkv^T (the block's
 * GroupedQueryCausalSelfAttention qkv Linear, loomformer.py:3262), then
 * loom_gqa_prefill's RoPE + cache append of the chunk (q_out, caches, tables
 * and strides as there), and, with w_hist set, the depth history slot's
 * projection hist_out = x w_hist^T (DepthAttn.project, loomformer.py:3397;
 * n_hist columns at hist_ld elements apart).  Weights are [rows, K] dense.
 * Follow it with loom_gqa_prefill(qkv = NULL).  bf16 with head_dim 96 and at
 * least 256 rows runs as one launch that never stores qkv; other shapes use
 * qkv_scratch ([B*T, (QH + 2 KVH) HD]) and a separate RoPE + append launch.
 * No counterpart in the reference. */
int loom_prefill_qkv(int dtype, const void* x, int64_t ldx, const void* w_qkv, const void* w_hist,
                     void* hist_out, int64_t hist_ld, int64_t n_hist, void* qkv_scratch, void* q_out,
                     void* k_cache, void* v_cache, int64_t cache_stride_b, int64_t cache_stride_t,
                     int64_t cache_stride_h, const float* cos_table, const float* sin_table,
                     int64_t B, int64_t T, int64_t start, int64_t cache_len, int64_t K, int64_t QH,
                     int64_t KVH, int64_t HD, void* stream);

/* Sparse final cross-attention: per row (b,t) a masked softmax over K keys
 * (scale * q.k), out = sum_j w_j v_j, an all-masked row gives exact zeros and
 * lse = -inf.  Replaces final_ca_sparse_forward (bindings.cpp:107).
 *   q: [B,T,D]; k,v: [B,K,D]; allowed: [B,T,K] bool; out: [B,T,D] (dtype);
 *   lse: [B,T] float or NULL.  K <= 1024. */
int loom_final_ca_sparse_forward(int dtype, const void* q, const void* k, const void* v,
                                 const uint8_t* allowed, void* out, float* lse, int64_t B,
                                 int64_t T, int64_t K, int64_t D, float scale, void* stream);

/* final_ca_sparse_forward with explicit layout, for decode caches: k/v row j
 * of batch b at b*kv_stride_b + j*D, allowed row r (= b*T + t) at
 * r*allowed_stride; with residual != NULL, out = residual + gamma * attention
 * (TriaFinalCrossAttention.step, tria.py:1560-1595, h + gamma*out).  With
 * k_dev != NULL the key count is min(*k_dev, K), read on the device (K is then
 * the capacity and may be 0 keys at run time: out = residual). */
int loom_final_ca_sparse_strided(int dtype, const void* q, const void* k, const void* v,
                                 int64_t kv_stride_b, const uint8_t* allowed,
                                 int64_t allowed_stride, const void* residual, float gamma,
                                 void* out, float* lse, int64_t B, int64_t T, int64_t K,
                                 const int64_t* k_dev, int64_t D, float scale, void* stream);

/* ---------------------------------------------------------------------------
 * Decode step (Model.step, loomformer.py:3951-4091)
 * ------------------------------------------------------------------------ */

/* RoPE of the new token and KV-cache append.  Replaces the q/k rotation and
 * cache write of GroupedQueryCausalSelfAttention.step (loomformer.py:3304-3315,
 * YaRNRotaryEmbedding.forward :2983-2985).
 *   qkv: [B, (QH + 2*KVH)*HD] dtype (output of the qkv projection);
 *   q_out: [B,QH,HD] dtype (rotated q); cache element (b, t, kvh, d) at
 *   b*cache_stride_b + t*cache_stride_t + kvh*cache_stride_h + d (a
 *   [B,T,KVH,HD] cache has cache_stride_h = HD, a head-major [B,KVH,T,HD] one
 *   cache_stride_t = HD); position `pos` is written
 *   (or *pos_dev, read on the device, when pos_dev != NULL).
 *   cos_table/sin_table: [>pos, HD] float, already multiplied by the YaRN
 *   attention factor (the reference's cos_cached/sin_cached). */
int loom_rope_append(int dtype, const void* qkv, void* q_out, void* k_cache, void* v_cache,
                     const float* cos_table, const float* sin_table, int64_t B, int64_t pos,
                     const int64_t* pos_dev, int64_t QH, int64_t KVH, int64_t HD,
                     int64_t cache_stride_b, int64_t cache_stride_t, int64_t cache_stride_h,
                     void* stream);

/* Bytes of workspace loom_gqa_decode_attention / loom_gqa_decode_step need for
 * len <= max_len: the per-chunk partial records [B, KVH, nchunks, 2G + 2G*HD]
 * fp32 (G = QH/KVH) that the attention launch writes and the merge launch after
 * it reads; nchunks = min(ceil(1.5 * CUs / (B*KVH)), ceil(max_len/128)) on the
 * current device.  Scratch: no initial contents are needed. */
int64_t loom_gqa_workspace_bytes(int64_t B, int64_t max_len, int64_t QH, int64_t KVH, int64_t HD);

/* Causal GQA attention of one query position over cache positions [0, len):
 * A = softmax(q k^T / sqrt(HD)) in fp32, c_out = A V, kctx_out = A K (the
 * roped keys).  Replaces the score/softmax/context part of
 * GroupedQueryCausalSelfAttention.step (loomformer.py:3316-3329) without
 * materialising the GQA repeat: q-head h reads kv head h / (QH/KVH).
 *   q: [B,QH,HD]; caches as in loom_rope_append; c_out, kctx_out: [B,QH,HD]
 *   (dtype); workspace: see loom_gqa_workspace_bytes.  With pos_dev != NULL
 *   the length is *pos_dev + 1 (read on the device) and `len` is the capacity
 *   the launch covers.  Calls that share a workspace must not overlap. */
int loom_gqa_decode_attention(int dtype, const void* q, const void* k_cache, const void* v_cache,
                              int64_t cache_stride_b, int64_t cache_stride_t,
                              int64_t cache_stride_h, void* c_out, void* kctx_out, float* workspace, int64_t workspace_bytes,
                              int64_t B, int64_t len, const int64_t* pos_dev, int64_t QH,
                              int64_t KVH, int64_t HD, void* stream);

/* The whole attention part of GroupedQueryCausalSelfAttention.step
 * (loomformer.py:3300-3329) in one launch, for position pos = len - 1 (or
 * *pos_dev): rope q and this token's k from the projection row qkv
 * [B, (QH + 2 KVH) HD] (= [q | k | v], YaRN tables as in loom_rope_append),
 * append (k_roped, v) at row pos of the caches, and attend over positions
 * 0..pos as loom_gqa_decode_attention does.  q_out (optional, [B,QH,HD])
 * receives the roped q, which the Paraplex FFN reads.  c_out / kctx_out rows are
 * out_stride_b elements apart (>= QH*HD), so they can land inside a wider
 * row.  Equivalent to loom_rope_append followed by loom_gqa_decode_attention. */
int loom_gqa_decode_step(int dtype, const void* qkv, void* k_cache, void* v_cache,
                         int64_t cache_stride_b, int64_t cache_stride_t, int64_t cache_stride_h,
                         const float* cos_table, const float* sin_table, void* q_out, void* c_out,
                         void* kctx_out,
                         int64_t out_stride_b,
                         float* workspace, int64_t workspace_bytes, int64_t B, int64_t len,
                         const int64_t* pos_dev, int64_t QH, int64_t KVH, int64_t HD,
                         void* stream);

/* loom_gqa_decode_step plus the decode step's DepthAttn read that follows it
 * in Model.step (loomformer.py:3999, DepthAttn.forward :3404-3429, decode
 * T = 1): depth_out [B,QH,HD] = softmax_s(depth_q . hist_k[b,s] / sqrt(HD))
 * weighted hist_v rows, over S history slots at (hist_stride_bt,
 * hist_stride_s) as in loom_depth_attn_forward.  The two reads are
 * independent; the bf16 MFMA form computes the depth rows in extra blocks of
 * the attention launch, other forms run loom_depth_attn_forward after it.
 * No counterpart in the reference (one launch for two of its calls). */
int loom_gqa_decode_step_depth(int dtype, const void* qkv, void* k_cache, void* v_cache,
                               int64_t cache_stride_b, int64_t cache_stride_t,
                               int64_t cache_stride_h, const float* cos_table,
                               const float* sin_table, void* q_out, void* c_out, void* kctx_out,
                               int64_t out_stride_b, float* workspace, int64_t workspace_bytes,
                               int64_t B, int64_t len, const int64_t* pos_dev, int64_t QH,
                               int64_t KVH, int64_t HD, const void* depth_q, const void* hist_k,
                               const void* hist_v, int64_t hist_stride_bt, int64_t hist_stride_s,
                               int64_t S, void* depth_out, void* stream);

/* loom_gqa_decode_step_depth with a second depth query over the same history
 * slots 0..S-1 (one load of each slot row for both): depth_q's read is written
 * to depth_out as there, depth_q2's as the normalised fp32 rows part_d
 * [B, QH, HD] and their log-sum-exp part_lse [B, QH] (natural units) -- the
 * part of the next sublayer's read (DepthAttn.forward with that sublayer's
 * query over slots 0..S, loomformer.py:3404-3429, :4004-4006) that these slots
 * contribute, which loom_ffn_decode folds with slot S.  bf16 only, head_dim
 * 32/64/96/128, QH/KVH in {1, 2, 4, 8}, depth rows 8-byte aligned (other
 * cases are rejected).  No counterpart in the reference as one call. */
int loom_gqa_decode_step_depth2(int dtype, const void* qkv, void* k_cache, void* v_cache,
                                int64_t cache_stride_b, int64_t cache_stride_t,
                                int64_t cache_stride_h, const float* cos_table,
                                const float* sin_table, void* q_out, void* c_out, void* kctx_out,
                                int64_t out_stride_b, float* workspace, int64_t workspace_bytes,
                                int64_t B, int64_t len, const int64_t* pos_dev, int64_t QH,
                                int64_t KVH, int64_t HD, const void* depth_q, const void* depth_q2,
                                const void* hist_k, const void* hist_v, int64_t hist_stride_bt,
                                int64_t hist_stride_s, int64_t S, void* depth_out, float* part_d,
                                float* part_lse, void* stream);

/* Size of the static per-device scratch of loom_gqa_decode_step_noalloc. */
#define LOOM_GQA_NOALLOC_SCRATCH_BYTES (4 << 20)

/* loom_gqa_decode_step without a workspace argument: the partial records live
 * in a static device array of LOOM_GQA_NOALLOC_SCRATCH_BYTES per GPU (held
 * until the process ends), so the call allocates nothing (no hipMalloc, no
 * library allocation).  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, serving
 * loops that forbid it).  Shapes whose records exceed the scratch
 * (loom_gqa_workspace_bytes(B, len, QH, KVH, HD) > LOOM_GQA_NOALLOC_SCRATCH_BYTES)
 * are rejected with LOOM_ERR_INVALID.  Calls on one GPU share the array, so
 * calls that overlap on one GPU (concurrent streams or threads) race. */
int loom_gqa_decode_step_noalloc(int dtype, const void* qkv, void* k_cache, void* v_cache,
                                 int64_t cache_stride_b, int64_t cache_stride_t,
                                 int64_t cache_stride_h, const float* cos_table,
                                 const float* sin_table, void* q_out, void* c_out, void* kctx_out,
                                 int64_t out_stride_b, int64_t B, int64_t len,
                                 const int64_t* pos_dev, int64_t QH, int64_t KVH, int64_t HD,
                                 void* stream);

/* out = LayerNorm(a + b) (b may be NULL) over rows of N <= 2048, fp32 gamma and
 * beta, biased variance.  Replaces ln_attn/ln_ffn(skip + branch)
 * (loomformer.py:4000, :4045). */
int loom_add_layernorm(int dtype, const void* a, const void* b, const float* gamma,
                       const float* beta, void* out, int64_t rows, int64_t N, float eps,
                       void* stream);

/* RMSNorm of final_norm before the head (RMSNorm.forward, loomformer.py:3460-3464):
 * out = round(round(x / sqrt(mean(x^2) + eps)) * weight) per row of N <= 2048,
 * statistics in fp32, rounding to dtype as the reference's .to(dtype) and
 * product in the model dtype.  x, weight, out: dtype. */
int loom_rms_norm(int dtype, const void* x, const void* weight, void* out, int64_t rows, int64_t N,
                  float eps, void* stream);

/* Decode-time temporal Tria update of one token (loomformer.py:4056-4085):
 *   out[b] = depth[b]                      if prev == NULL or reset_now[b]
 *            N(depth[b] @ prev[b])          otherwise
 *   then, where fire[b] (fire may be NULL), PolARM(out[b], polarm_beta, eps).
 *   depth, prev, out: [B,H,3,3] dtype; reset_now, fire: [B] bool. */
int loom_tria_decode_temporal(int dtype, const void* depth, const void* prev,
                              const uint8_t* reset_now, const uint8_t* fire, void* out,
                              int64_t B, int64_t H, float polarm_beta, float eps, void* stream);

/* The per-token Tria tail of a decode step: the loom_tria_decode_temporal
 * update of every head, stored in doc (doc may equal prev: each head's
 * previous state is read before it is written), then the readout of the
 * stored state, TriaAggregator.forward (tria.py:1436-1441): pooled = slot
 * attention pool over H with score_w (tria.py:1351-1389), z = pooled @
 * proj_w^T + proj_b (proj_w [32,9]), a_out[b] = z @ up_w^T + up_b (up_w [N,32],
 * 16-byte aligned).  pooled and z are rounded to dtype between the steps as the
 * separate ops store them.  proj_b, up_b: fp32 or NULL.  H <= 32768.
 * With fire != NULL and no row firing, only doc is written (the readout
 * feeds only the keys staged at a fire, tria.py:1576-1582); a_out is left as
 * it is.
 * workspace: fp32 scratch of loom_decode_tria_readout_workspace_bytes(B, H)
 * bytes (per-block pool records); two launches on stream.  Replaces
 * loom_tria_decode_temporal + loom_slot_attention_pool_forward + two
 * loom_linear calls in Model.step (loomformer.py:4053-4085); no reference
 * counterpart of its own. */
int64_t loom_decode_tria_readout_workspace_bytes(int64_t B, int64_t H);
int loom_decode_tria_readout(int dtype, const void* depth, const void* prev,
                             const uint8_t* reset_now, const uint8_t* fire, void* doc,
                             const void* score_w, const void* proj_w, const float* proj_b,
                             const void* up_w, const float* up_b, void* a_out, float* workspace,
                             int64_t workspace_bytes, int64_t B, int64_t H, int64_t N,
                             float polarm_beta, float eps, void* stream);

/* Start of a decode step with device-resident state (pos = *pos_dev), so a
 * whole step is a fixed launch sequence that a HIP graph can replay.  Token
 * ids: ids[b] = prompt[b, pos] (row stride prompt_ld) while pos < prompt_len
 * (prompt may be NULL), otherwise ids is left as written by the caller (the
 * previous argmax); tokens[b, pos] = ids[b] when tokens != NULL (row stride
 * tokens_ld).
 * fire[b] = hard fire for the next token ((pos+1) % window == 0 and
 * pos+1 < seq_len, loomformer.py:4069-4073) or ids[b] == carry_id (carry_id < 0
 * disables); reset_now[b] = pending[b] (loomformer.py:3985-3990, 4058). */
int loom_decode_prologue(int64_t* ids, const int64_t* prompt, int64_t prompt_len,
                         int64_t prompt_ld, int64_t* tokens, int64_t tokens_ld,
                         const int64_t* pos_dev, const uint8_t* pending, uint8_t* fire,
                         uint8_t* reset_now, int64_t carry_id, int64_t window, int64_t seq_len,
                         int64_t B, void* stream);

/* loom_decode_prologue followed by the step's embedding lookup,
 * h[b] = emb[ids[b]] (emb [V,N], h [B,N] dtype, both 16-byte aligned; ids
 * outside [0, V) read row 0 or V-1: callers validate prompt ids, argmax ids are
 * in range), one launch (nn.Embedding in Model.step, loomformer.py:3971).  No
 * reference counterpart of its own. */
int loom_decode_prologue_embed(int dtype, int64_t* ids, const int64_t* prompt, int64_t prompt_len,
                               int64_t prompt_ld, int64_t* tokens, int64_t tokens_ld,
                               const int64_t* pos_dev, const uint8_t* pending, uint8_t* fire,
                               uint8_t* reset_now, int64_t carry_id, int64_t window,
                               int64_t seq_len, const void* emb, void* h, int64_t N, int64_t V,
                               int64_t B, void* stream);

/* One decode step's prologue in one launch, per batch row b: the token id is
 * prompt[b, pos] while pos < prompt_len (prompt may be NULL), otherwise
 * argmax_v logits[b, v] (first index on ties, as loom_argmax_rows; infer's
 * greedy pick, loomformer.py:5306) or, with logits NULL, ids[b] as written by
 * the caller; ids[b], tokens[b, pos], fire[b] and reset_now[b] as
 * loom_decode_prologue; then row id of `table` [V, row_len] is copied to
 * dst0[b * ld0 + 0 .. n0) and dst1[b * ld1 + 0 .. n1) (table row = [n0 | n1],
 * n0 + n1 == row_len; n1 may be 0 with dst1 NULL).  The engine's table holds,
 * per vocabulary id, the first depth-history slot DepthAttn.project(emb[id])
 * and layer 0's qkv projection of emb[id] (Model.step, loomformer.py:3971-3973,
 * :3300): the projections are linear in the gathered row, so gathering their
 * rows equals projecting the gathered embedding.  No reference counterpart as
 * one call.  logits: [B, V] dtype with V % 8 == 0, V <= 16384, 16-byte aligned. */
int loom_decode_prologue_gather(int dtype, const void* logits, int64_t* ids, const int64_t* prompt,
                                int64_t prompt_len, int64_t prompt_ld, int64_t* tokens,
                                int64_t tokens_ld, const int64_t* pos_dev, const uint8_t* pending,
                                uint8_t* fire, uint8_t* reset_now, int64_t carry_id, int64_t window,
                                int64_t seq_len, const void* table, int64_t row_len, int64_t V,
                                void* dst0, int64_t ld0, int64_t n0, void* dst1, int64_t ld1,
                                int64_t n1, int64_t B, void* stream);

/* Greedy pick ids[r] = argmax_v logits[r, v] (first index on ties, as
 * torch.argmax), the `argmax(logits)` of infer (loomformer.py:5306).
 * logits: [rows, V] dtype; ids: [rows] int64. */
int loom_argmax_rows(int dtype, const void* logits, int64_t rows, int64_t V, int64_t* ids,
                     void* stream);

/* End of a decode step: if any fire[b], the staged final-CA key/value rows
 * stage_k/stage_v [B,N] (w_qk(a_t), w_v(a_t)) are stored at slot *ca_len of
 * ca_k/ca_v [B,max_keys,N], ca_valid[b, slot] = fire[b], *ca_len += 1
 * (TriaFinalCrossAttention.step, tria.py:1576-1582); then pending = fire and
 * *pos_dev += 1. */
int loom_decode_epilogue(int dtype, const void* stage_k, const void* stage_v, void* ca_k,
                         void* ca_v, uint8_t* ca_valid, int64_t* ca_len, const uint8_t* fire,
                         uint8_t* pending, int64_t* pos_dev, int64_t B, int64_t N,
                         int64_t max_keys, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOOM_HIP_H */
