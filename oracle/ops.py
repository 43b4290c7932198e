"""fp32 CPU restatement of the reference's per-op maths (test infrastructure).

Every function works on CPU tensors and computes in float32 (inputs in a
narrower dtype are upcast first).  Citations are ``file:line`` in the
reference checkout.
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

HALF_PI = math.pi / 2.0


def _f(x: torch.Tensor) -> torch.Tensor:
    return x.float() if x.dtype != torch.float32 else x


# --------------------------------------------------------------------------
# Paraplex pointwise chain
# --------------------------------------------------------------------------

def phase_sin(beta: torch.Tensor) -> torch.Tensor:
    """I_base = sin(pi/2 * beta / sqrt(1 + beta^2)).

    loomformer.py:2013-2021 (_PhaseSinFloor.forward); the secant variant's
    forward (:2032-2042) is the same function.
    """
    b = _f(beta)
    return torch.sin(HALF_PI * b * torch.rsqrt(1.0 + b * b))


def sin_space_combine(s_base: torch.Tensor, trace_term: torch.Tensor) -> torch.Tensor:
    """I = z / sqrt(1 + z^2), z = s_base + trace_term (loomformer.py:2621-2623)."""
    z = s_base + trace_term
    return z * torch.rsqrt(1.0 + z * z)


def prev_token_trace(s_base: torch.Tensor, initial_trace: Optional[torch.Tensor],
                     reset_mask: Optional[torch.Tensor]) -> torch.Tensor:
    """Previous-token phase of the same neuron (loomformer.py:2626-2638).

    Row t takes s_base[t-1]; row 0 takes ``initial_trace`` (zeros if None);
    rows where ``reset_mask`` is set are zero.
    """
    B, T, H = s_base.shape
    out = torch.zeros_like(s_base)
    if initial_trace is not None:
        out[:, 0] = _f(initial_trace)
    if T > 1:
        out[:, 1:] = s_base[:, :-1]
    if reset_mask is not None:
        out = out.masked_fill(reset_mask.bool().unsqueeze(-1), 0.0)
    return out


def powlu_gate(x2: torch.Tensor, m: float) -> torch.Tensor:
    """G(A) = A^(m / (sqrt(A) + 1)) * sigmoid(A) (loomformer.py:3441-3444)."""
    return x2.pow(m / (torch.sqrt(x2) + 1.0)) * torch.sigmoid(x2)


def pvpowlu(x1: torch.Tensor, x2: torch.Tensor, m: float = 3.0) -> torch.Tensor:
    """x1 * G(x2): the CPU branch of pvpowlu_act (loomformer.py:2201-2209)."""
    return _f(x1) * powlu_gate(_f(x2), m)


def paraplex_pointwise(p_real: torch.Tensor, gate_src: torch.Tensor, beta_linear: torch.Tensor,
                       bias: torch.Tensor, trace: Optional[torch.Tensor], trace_w: torch.Tensor,
                       reset: Optional[torch.Tensor], m: float
                       ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The Paraplex pointwise chain -> (act=O, s=I, next_trace).

    Unfused composition of ParaplexFFN.forward (loomformer.py:2856-2885):
    A = softplus(gate_src); beta = beta_linear + w1_imag_bias (:2862);
    I_base = phase_sin(beta) (:2873); trace_mat = prev_token_trace (:2874-2875);
    I = sin_space_combine(I_base, trace_mat * w_trace) (:2876);
    P = R + A*I (:2877); O = P * G(A) (:2882); next_trace = I_base[:, -1] (:2880).
    The fused kernel it replaces is paraplex_kernel.cuh:111-145.
    """
    r = _f(p_real)
    amp = F.softplus(_f(gate_src))
    beta = _f(beta_linear) + _f(bias).view(1, 1, -1)
    s_base = phase_sin(beta)
    tr = prev_token_trace(s_base, trace, reset)
    s = sin_space_combine(s_base, tr * _f(trace_w).view(1, 1, -1))
    p = torch.addcmul(r, amp, s)
    act = pvpowlu(p, amp, m)
    return act, s, s_base[:, -1, :].clone()


# --------------------------------------------------------------------------
# W_imag compact layout and beta space
# --------------------------------------------------------------------------

def w1_imag_live_flat_indices(N: int, QH: int, HD: int, H: int, sectors: str = "head") -> torch.Tensor:
    """Flat indices of the live W_imag entries in the dense [H, 5N] matrix.

    loomformer.py:871-900.  Q-head g owns hidden rows [g*Hq, (g+1)*Hq); its
    compact columns, in order, are [Q_g | Kctx_g | C_g | U | D_g] in head mode
    and [Q_g | Kctx | C | U | D] in open mode, taken from the dense column
    blocks [Q | Kctx | C | U | D] (each N wide).
    """
    Hq = H // QH
    rows = []
    for g in range(QH):
        c0 = g * HD
        own = lambda blk: list(range(blk * N + c0, blk * N + c0 + HD))
        full = lambda blk: list(range(blk * N, (blk + 1) * N))
        if sectors == "head":
            cols = own(0) + own(1) + own(2) + full(3) + own(4)
        else:
            cols = own(0) + full(1) + full(2) + full(3) + full(4)
        cols_t = torch.tensor(cols, dtype=torch.long)
        for rrow in range(g * Hq, (g + 1) * Hq):
            rows.append(rrow * (5 * N) + cols_t)
    return torch.cat(rows)


def imag_in(N: int, HD: int, sectors: str = "head") -> int:
    """IMAG_IN (loomformer.py:1091)."""
    return N + 4 * HD if sectors == "head" else 4 * N + HD


def dense_imag_weight(w_compact: torch.Tensor, N: int, QH: int, HD: int,
                      sectors: str = "head") -> torch.Tensor:
    """Scatter the compact [H, IMAG_IN] weight into dense [H, 5N] (loomformer.py:2727-2733)."""
    H = w_compact.shape[0]
    idx = w1_imag_live_flat_indices(N, QH, HD, H, sectors)
    flat = torch.zeros(H * 5 * N, dtype=torch.float32)
    flat = flat.scatter(0, idx, _f(w_compact).reshape(-1))
    return flat.view(H, 5 * N)


def beta_space_dense(u, q_h, k_ctx_h, c_h, d_h, w_compact, QH: int, HD: int,
                     sectors: str = "head") -> torch.Tensor:
    """The reference CPU path: one dense GEMM over cat(Q,Kctx,C,U,D) (loomformer.py:2771-2777)."""
    B, T, N = u.shape
    r_all = torch.cat([_f(q_h).reshape(B, T, N), _f(k_ctx_h).reshape(B, T, N),
                       _f(c_h).reshape(B, T, N), _f(u), _f(d_h).reshape(B, T, N)], dim=-1)
    return F.linear(r_all, dense_imag_weight(w_compact, N, QH, HD, sectors))


def beta_space_grouped(u, q_h, k_ctx_h, c_h, d_h, w_compact, QH: int, HD: int,
                       sectors: str = "head") -> torch.Tensor:
    """Per-q-head grouped form of the same product (beta_space_launcher.cu:225-264,
    pack order beta_space_kernel.cuh:87-135): group g multiplies its packed
    activation row [Q_g|Kctx_g|C_g|U|D_g] by W_compact[g*Hq:(g+1)*Hq]^T."""
    B, T, N = u.shape
    H = w_compact.shape[0]
    Hq = H // QH
    outs = []
    for g in range(QH):
        sl = slice(g * HD, (g + 1) * HD)
        if sectors == "head":
            pack = torch.cat([_f(q_h)[:, :, g], _f(k_ctx_h)[:, :, g], _f(c_h)[:, :, g],
                              _f(u), _f(d_h)[:, :, g]], dim=-1)
        else:
            pack = torch.cat([_f(q_h)[:, :, g], _f(k_ctx_h).reshape(B, T, N),
                              _f(c_h).reshape(B, T, N), _f(u), _f(d_h).reshape(B, T, N)], dim=-1)
        del sl
        outs.append(F.linear(pack, _f(w_compact)[g * Hq:(g + 1) * Hq]))
    return torch.cat(outs, dim=-1)


# --------------------------------------------------------------------------
# Depth attention
# --------------------------------------------------------------------------

def depth_attn_online(q_row: torch.Tensor, hist_k: torch.Tensor, hist_v: torch.Tensor
                      ) -> torch.Tensor:
    """Online softmax over the depth axis (loomformer.py:2212-2238).

    q_row [QH,HD]; hist_k/hist_v [B,T,S,QH,HD] -> d [B,T,QH,HD] (fp32).
    """
    HD = q_row.shape[-1]
    q = _f(q_row).view(1, 1, *q_row.shape)
    k = _f(hist_k)
    v = _f(hist_v)
    sqrt_d = math.sqrt(HD)
    m = l = d = None
    for s in range(k.shape[2]):
        sc = (q * k[:, :, s]).sum(-1) / sqrt_d
        if m is None:
            m = sc
            l = torch.exp(sc - m)
            d = l.unsqueeze(-1) * v[:, :, s]
        else:
            m_new = torch.maximum(m, sc)
            e_old = torch.exp(m - m_new)
            e_new = torch.exp(sc - m_new)
            l = l * e_old + e_new
            d = d * e_old.unsqueeze(-1) + e_new.unsqueeze(-1) * v[:, :, s]
            m = m_new
    return d / l.unsqueeze(-1)


def depth_attn_softmax(q_row: torch.Tensor, hist_k: torch.Tensor, hist_v: torch.Tensor
                       ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Plain-softmax form (loomformer.py:2241-2248 and the stacked fallback
    :2268-2274) returning (d, weights [B,T,QH,S], lse [B,T,QH])."""
    HD = q_row.shape[-1]
    q = _f(q_row).view(1, 1, 1, *q_row.shape)
    k = _f(hist_k)
    v = _f(hist_v)
    scores = (q * k).sum(-1) / math.sqrt(HD)          # [B,T,S,QH]
    scores = scores.permute(0, 1, 3, 2)                # [B,T,QH,S]
    mx = scores.amax(-1, keepdim=True)
    p = torch.exp(scores - mx)
    l = p.sum(-1, keepdim=True)
    w = p / l
    d = torch.einsum("bths,btshd->bthd", w, v)
    lse = (mx + torch.log(l)).squeeze(-1)
    return d, w, lse


# --------------------------------------------------------------------------
# Tria
# --------------------------------------------------------------------------

def build_tria(r: torch.Tensor, i: torch.Tensor, o: torch.Tensor, alpha: float,
               axis: int, eps: float = 1e-6) -> torch.Tensor:
    """Local carrier T(r,i,o) -> [...,3,3] (tria.py:35-69; carrier.cuh:33-54).

    x=(ri,ro,io); (a,b,c) = alpha*tanh(x/sqrt(mean(x^2)+eps));
    T = (I + K(a,b,c)) @ R_axis with the closed forms per axis.
    """
    r, i, o = _f(r), _f(i), _f(o)
    x = torch.stack((r * i, r * o, i * o), dim=-1)
    rms = torch.sqrt(x.square().mean(dim=-1, keepdim=True) + eps)
    t = torch.tanh(x / rms) * float(alpha)
    a, b, c = t[..., 0], t[..., 1], t[..., 2]
    one = torch.ones_like(a)
    if axis == 0:
        rows = ((-c, -one, b), (one, -c, -a), (a, b, one))
    elif axis == 1:
        rows = ((one, b, c), (c, -a, -one), (-b, one, -a))
    elif axis == 2:
        rows = ((-b, -c, one), (a, one, c), (-one, a, -b))
    else:
        raise ValueError(f"axis must be 0, 1 or 2, got {axis}")
    return torch.stack([torch.stack(rw, dim=-1) for rw in rows], dim=-2)


def local_normalize(m: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """M / sqrt(mean_9(M^2) + eps) (tria.py:77-82; carrier.cuh:112-117)."""
    w = _f(m)
    return w / torch.sqrt(w.square().mean(dim=(-1, -2), keepdim=True) + eps)


def tria_slots(carry: torch.Tensor) -> torch.Tensor:
    """[...,3,3] -> [...,9] row-major (tria.py:1251-1254)."""
    return carry.reshape(*carry.shape[:-2], 9)


def gate_slot_mix(carry: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """p = sum_k w_k vec(C)_k (tria.py:1282-1283)."""
    return (tria_slots(_f(carry)) * _f(w)).sum(-1)


def tria_init(r, i, o, alpha, axis) -> torch.Tensor:
    """C_1 = N(T_1) (tria.py:814-832 PyTorch branch)."""
    return local_normalize(build_tria(r, i, o, alpha, axis))


def tria_step(r, i, o, carry_prev, alpha, axis) -> torch.Tensor:
    """C_l = N(T_l @ C_{l-1}) (tria.py:890-910 -> carry_step_pytorch :90-93)."""
    return local_normalize(torch.matmul(build_tria(r, i, o, alpha, axis), _f(carry_prev)))


def tria_init_seed(r, i, o, seed, seed_valid, alpha, axis) -> torch.Tensor:
    """Seeded first layer (tria.py:835-844): at t==0 and valid[b],
    C = N(T @ seed[b]); elsewhere C = N(T)."""
    local = build_tria(r, i, o, alpha, axis)
    first = torch.matmul(local[:, 0], _f(seed))
    first = torch.where(seed_valid.bool()[:, None, None, None], first, local[:, 0])
    pre = torch.cat((first[:, None], local[:, 1:]), dim=1)
    return local_normalize(pre)


def tria_init_and_gate(r, i, o, w, alpha, axis):
    """tria.py:913-944 PyTorch branch -> (carry, p)."""
    c = tria_init(r, i, o, alpha, axis)
    return c, gate_slot_mix(c, w)


def tria_step_and_gate(r, i, o, carry_prev, w, alpha, axis):
    """tria.py:947-978 PyTorch branch -> (carry, p)."""
    c = tria_step(r, i, o, carry_prev, alpha, axis)
    return c, gate_slot_mix(c, w)


def tria_init_seed_and_gate(r, i, o, seed, seed_valid, w, alpha, axis):
    """tria.py:867-887 PyTorch branch -> (carry, p)."""
    c = tria_init_seed(r, i, o, seed, seed_valid, alpha, axis)
    return c, gate_slot_mix(c, w)


def temporal_carry(depth_carry: torch.Tensor, reset_mask: torch.Tensor,
                   eps: float = 1e-6) -> torch.Tensor:
    """Sequential segmented temporal carry, all T rows (tria.py:1015-1041)."""
    d = _f(depth_carry)
    reset = reset_mask.bool()
    state = None
    outs = []
    for t in range(d.shape[1]):
        local = d[:, t]
        if t == 0:
            pre = local
        else:
            pre = torch.where(reset[:, t, None, None, None], local, torch.matmul(local, state))
        state = local_normalize(pre, eps)
        outs.append(state)
    return torch.stack(outs, dim=1)


def temporal_carry_endpoint(depth_carry: torch.Tensor, reset_mask: torch.Tensor,
                            initial_state: Optional[torch.Tensor] = None,
                            initial_valid: Optional[torch.Tensor] = None,
                            eps: float = 1e-6) -> torch.Tensor:
    """Final state of the temporal recurrence (tria.py:1089-1123).

    Restart acc = N(D_t) on reset[b,t] or when no valid state is held yet;
    otherwise acc = N(D_t @ acc).
    """
    d = _f(depth_carry)
    B, T = d.shape[:2]
    reset = reset_mask.bool()
    if initial_state is None:
        state = d[:, 0]
        valid = torch.zeros(B, dtype=torch.bool)
    else:
        state = _f(initial_state)
        valid = (torch.ones(B, dtype=torch.bool) if initial_valid is None
                 else initial_valid.bool())
    for t in range(T):
        local = d[:, t]
        use_local = reset[:, t] | ~valid
        state = local_normalize(torch.where(use_local[:, None, None, None], local,
                                            torch.matmul(local, state)), eps)
        valid = torch.ones_like(valid)
    return state


def polarm(matrix: torch.Tensor, beta: float = 0.1, eps: float = 1e-6) -> torch.Tensor:
    """PolARM correction (tria.py:128-139): G = M^T M; s = mean(diag G)
    clamped to >= eps; M <- M @ (I - beta/2 * (G/s - I))."""
    w = _f(matrix)
    gram = w.transpose(-1, -2) @ w
    s = gram.diagonal(dim1=-2, dim2=-1).mean(-1).clamp_min(eps)[..., None, None]
    eye = torch.eye(3, dtype=w.dtype)
    return w @ (eye - 0.5 * beta * (gram / s - eye))


def tria_chunked(r: torch.Tensor, i: torch.Tensor, o: torch.Tensor, alpha: float, window: int,
                 polarm_beta: float = 0.1, reset: Optional[torch.Tensor] = None,
                 explicit_fire: Optional[torch.Tensor] = None, return_valid: bool = False):
    """Tria part of Model._forward_chunked (loomformer.py:3788-3883), chunk by
    chunk as the reference runs it.  Boundaries are the hard-fire grid
    positions ((t+1) % W == 0, never T-1) plus every position where any row
    has an explicit <CARRY> fire (:3797-3815); a row's fire at a boundary is
    hard_fire & ~next_is_reset | explicit (:3808-3810).  Layer l of the chunk
    uses axis l % 3 (oracle.model's block loop, loomformer.py:3588-3617);
    layer 0 of chunk c >= 1 is seeded with the temporal state where
    seed_valid = fire[s-1] & ~reset[s] (:3826-3828); the endpoint restarts at
    local resets and at a valid seed (:3834-3850); at a boundary the state
    becomes polarm(state) where the fire is valid and is appended as a key for
    every row (:3852-3861).  r, i, o: [L,B,T,H]; reset: [B,T] bool document
    starts (None = position-0 only, :3534-3542); explicit_fire: [B,T] bool
    (None = no <CARRY> id).  Returns (keys [B,K,H,3,3], depth [B,T,H,3,3]),
    plus the key validity [B,K] with return_valid."""
    L, B, T, H = r.shape
    W = int(window)
    doc_reset = torch.zeros(B, T, dtype=torch.bool) if reset is None else reset.bool().clone()
    doc_reset[:, 0] = True
    explicit = (torch.zeros(B, T, dtype=torch.bool) if explicit_fire is None
                else explicit_fire.bool())
    grid = ((torch.arange(T) + 1) % W) == 0
    grid[-1] = False
    next_is_reset = torch.zeros(B, T, dtype=torch.bool)
    next_is_reset[:, :-1] = doc_reset[:, 1:]
    fire = (grid[None, :] & ~next_is_reset) | explicit
    bounds = (grid | explicit.any(dim=0)).nonzero().flatten().tolist()
    bset = set(bounds)
    stops = bounds + ([T - 1] if not bounds or bounds[-1] != T - 1 else [])
    state = None
    keys, depth, valids = [], [], []
    s = 0
    for bp in stops:
        e = min(bp + 1, T)
        seed = seed_valid = None
        if state is not None:
            seed_valid = fire[:, s - 1] & ~doc_reset[:, s]
            seed = state
        carry = None
        for l in range(L):
            ax = l % 3
            rl, il, ol = r[l, :, s:e], i[l, :, s:e], o[l, :, s:e]
            if l == 0:
                carry = (tria_init_seed(rl, il, ol, seed, seed_valid, alpha, ax) if seed is not None
                         else tria_init(rl, il, ol, alpha, ax))
            else:
                carry = tria_step(rl, il, ol, carry, alpha, ax)
        local_reset = doc_reset[:, s:e].clone()
        if seed_valid is not None:
            local_reset[:, 0] |= seed_valid
        if e != T or (e - 1) in bset:
            state = temporal_carry_endpoint(carry, local_reset, initial_state=state)
        depth.append(carry)
        if (e - 1) in bset:
            valid = fire[:, e - 1]
            state = torch.where(valid[:, None, None, None], polarm(state, polarm_beta), state)
            keys.append(state)
            valids.append(valid)
        s = e
    keys_t = torch.stack(keys, dim=1) if keys else torch.zeros(B, 0, H, 3, 3)
    if return_valid:
        valid_t = torch.stack(valids, dim=1) if valids else torch.zeros(B, 0, dtype=torch.bool)
        return keys_t, torch.cat(depth, dim=1), valid_t
    return keys_t, torch.cat(depth, dim=1)


def tria_readout(carry: torch.Tensor, score_w: torch.Tensor, proj_w: torch.Tensor,
                 proj_b: torch.Tensor, up_w: torch.Tensor, up_b: torch.Tensor) -> torch.Tensor:
    """TriaAggregator.forward (tria.py:1436-1441): up(proj(pool(carry)))."""
    pooled, _ = slot_attention_pool(carry, score_w)
    return F.linear(F.linear(pooled, _f(proj_w), _f(proj_b)), _f(up_w), _f(up_b))


def make_score_w(key_proj_w: torch.Tensor, query: torch.Tensor,
                 logit_scale: torch.Tensor) -> torch.Tensor:
    """score_w = normalize(key_proj^T query) * logit_scale (tria.py:1346-1349)."""
    raw = torch.mv(_f(key_proj_w).t(), _f(query))
    return F.normalize(raw, dim=0, eps=1e-6) * _f(logit_scale)


def slot_attention_pool(carry: torch.Tensor, score_w: torch.Tensor
                        ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Softmax over H of <score_w, vec C_h>, pooled 9-slot mean and lse
    (tria.py:1380-1383; slot_attention_pool_kernel.cuh:13-58)."""
    slots = tria_slots(_f(carry))
    scores = (slots * _f(score_w)).sum(-1)
    lse = torch.logsumexp(scores, dim=-1)
    wts = torch.softmax(scores, dim=-1)
    pooled = (wts.unsqueeze(-1) * slots).sum(dim=-2)
    return pooled, lse


def final_ca_sparse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    allowed: torch.Tensor, scale: float) -> torch.Tensor:
    """Masked softmax cross-attention; rows with no allowed key give exact zero
    (tria.py:1444-1455)."""
    q, k, v = _f(q), _f(k), _f(v)
    allowed = allowed.bool()
    scores = torch.bmm(q, k.transpose(1, 2).contiguous()) * float(scale)
    row_any = allowed.any(dim=-1, keepdim=True)
    safe = allowed | ~row_any
    w = torch.softmax(scores.masked_fill(~safe, float("-inf")), dim=-1)
    return torch.bmm(w, v) * row_any.to(q.dtype)


def final_ca_sparse_lse(q, k, v, allowed, scale) -> torch.Tensor:
    """The kernel's second output: per-row log-sum-exp over allowed keys,
    -inf when none is allowed (final_ca_sparse_kernel.cuh:56-75)."""
    q, k = _f(q), _f(k)
    scores = torch.bmm(q, k.transpose(1, 2).contiguous()) * float(scale)
    scores = scores.masked_fill(~allowed.bool(), float("-inf"))
    return torch.logsumexp(scores, dim=-1)


# --------------------------------------------------------------------------
# YaRN rotary embedding
# --------------------------------------------------------------------------

def yarn_inv_freq(head_dim: int, theta: float, factor: float, original_len: int,
                  beta_fast: float, beta_slow: float,
                  attention_factor: Optional[float] = None) -> Tuple[torch.Tensor, float]:
    """YaRN frequencies and attention factor (loomformer.py:2899-2962)."""
    dim = head_dim
    pos_freqs = theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim)
    extra = 1.0 / pos_freqs
    inter = 1.0 / (factor * pos_freqs)

    def corr_dim(nrot):
        return (dim * math.log(original_len / (nrot * 2.0 * math.pi))) / (2.0 * math.log(theta))

    low = max(math.floor(corr_dim(beta_fast)), 0)
    high = min(math.ceil(corr_dim(beta_slow)), dim - 1)
    if low == high:
        high += 0.001
    ramp = torch.clamp((torch.arange(dim // 2, dtype=torch.float32) - low) / (high - low), 0.0, 1.0)
    mask = 1.0 - ramp
    inv_freq = inter * (1.0 - mask) + extra * mask
    if attention_factor is None:
        attention_factor = 1.0 if factor <= 1.0 else 0.1 * math.log(factor) + 1.0
    return inv_freq, float(attention_factor)


def yarn_cos_sin(inv_freq: torch.Tensor, attention_factor: float, seq_len: int
                 ) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos/sin cache [seq_len, HD], scaled by the attention factor (loomformer.py:2964-2971)."""
    t = torch.arange(seq_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().mul(attention_factor), emb.sin().mul(attention_factor)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """(x1, x2) -> (-x2, x1) over the last dim (loomformer.py:2922-2925)."""
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x*cos + rotate_half(x)*sin (loomformer.py:2983-2985)."""
    return x * cos + rotate_half(x) * sin
