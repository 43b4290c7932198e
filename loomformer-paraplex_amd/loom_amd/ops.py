"""Torch-level mirror of the reference's CUDA extension functions.

Each function keeps the reference's name, positional arguments, return arity
and error behaviour (``RuntimeError`` with the reference's message where it
checks), and runs the gfx950 kernel of libloom_hip.so through the C ABI.
Inputs are made contiguous and outputs allocated here, as the reference
launchers do; every launch goes on the current HIP stream.
"""
from __future__ import annotations

import ctypes

import math
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib
from ._lib import call, dtype_code, ptr, stream_of

_FLOATS = (torch.float32, torch.bfloat16, torch.float16)


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _cuda(*ts, name: str) -> None:
    _check(all(t.is_cuda for t in ts), f"{name}: all inputs must be CUDA tensors")
    dev = ts[0].device
    _check(all(t.device == dev for t in ts), f"{name}: all inputs must be on the same CUDA device")


def _same_dtype(*ts, name: str) -> None:
    _check(all(t.dtype == ts[0].dtype for t in ts), f"{name}: all inputs must have the same dtype")
    _check(ts[0].dtype in _FLOATS, f"{name}: unsupported dtype {ts[0].dtype}")


def _c(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if t is None else t.contiguous()


# ---------------------------------------------------------------- loomformer_paraplex

def paraplex_forward(p_real, gate_src, beta_linear, bias, trace, trace_w, reset, anchor,
                     mode: int, update_anchor: bool, decay: float, m: float) -> List[torch.Tensor]:
    """kernels/paraplex/paraplex_launcher.cu:49 (checks :16-47)."""
    _check(all(t.is_cuda for t in (p_real, gate_src, beta_linear, bias, trace, trace_w, anchor)),
           "paraplex: CUDA tensors required")
    dev = p_real.device
    _check(all(t.device == dev for t in (gate_src, beta_linear, bias, trace, trace_w, anchor)),
           "paraplex: device mismatch")
    _check(p_real.dim() == 3 and beta_linear.shape == p_real.shape and gate_src.shape == p_real.shape,
           "p/gate_src/beta must be [B,T,H]")
    _check(gate_src.dtype == p_real.dtype,
           "paraplex: gate_src dtype must match p_real (cast before calling, same as beta_linear)")
    _check(beta_linear.dtype == p_real.dtype and trace.dtype == p_real.dtype,
           "p/beta/trace dtype mismatch")
    _check(trace.dim() == 2 and trace.shape[0] == p_real.shape[0] and trace.shape[1] == p_real.shape[2],
           "trace must be [B,H]")
    _check(bias.dtype == torch.float32 and trace_w.dtype == torch.float32 and anchor.dtype == torch.float32,
           "bias/trace_w/anchor must be float32")
    _check(bias.numel() == p_real.shape[2] and trace_w.numel() == p_real.shape[2] and anchor.numel() == 1,
           "parameter shape mismatch")
    _check(reset.numel() == 0 or (reset.is_cuda and reset.dtype == torch.bool and reset.dim() == 2
                                  and reset.shape[0] == p_real.shape[0] and reset.shape[1] == p_real.shape[1]),
           "reset must be empty or bool [B,T]")
    _check(reset.numel() == 0 or reset.device == dev, "reset device mismatch")
    _check(p_real.numel() > 0, "paraplex: empty tensors are unsupported")
    _check(p_real.dtype in _FLOATS, f"paraplex: unsupported dtype {p_real.dtype}")
    if update_anchor:
        raise RuntimeError("paraplex: the secant-anchor EMA update is training-only and not "
                           "supported by the inference library (update_anchor must be False)")
    B, T, H = p_real.shape
    pc = p_real.contiguous()
    gc = pc if gate_src is p_real else gate_src.contiguous()
    bc = beta_linear.contiguous()
    act = torch.empty_like(pc)
    s = torch.empty_like(pc)
    nxt = torch.empty(B, H, dtype=pc.dtype, device=dev)
    snap = torch.empty(anchor.shape, dtype=torch.float32, device=dev)
    rc = reset.contiguous() if reset.numel() else None
    # contiguous copies are bound to names so they outlive the asynchronous launch
    bias_c, trace_c, tw_c, anchor_c = (t.contiguous() for t in (bias, trace, trace_w, anchor))
    call("loom_paraplex_forward", dtype_code(pc), ptr(pc), ptr(gc), ptr(bc), ptr(bias_c),
         ptr(trace_c), ptr(tw_c), ptr(rc), ptr(anchor_c),
         ptr(act), ptr(s), ptr(nxt), ptr(snap), B, T, H, float(m), stream_of(pc))
    return [act, s, nxt, snap]


def paraplex_backward(*args):
    """kernels/paraplex/paraplex_launcher.cu:95 -- training only, not part of this library."""
    raise RuntimeError("paraplex_backward: training-only entry point is not provided on gfx950")


# ---------------------------------------------------------------- loomformer_beta_space

def beta_forward_cuda(u, q_h, k_ctx_h, c_h, d_h, w1_imag_compact, hidden_per_q_head: int,
                      head_dim: int, n_q_heads: int, open_sectors: bool) -> List[torch.Tensor]:
    """kernels/beta_space/beta_space_launcher.cu:225.

    Returns [out[B,T,H], r_pack, w_contig].  The packed activation copy is never
    materialised by the gfx950 kernel (the sectors are gathered into the GEMM
    tile), so ``r_pack`` is an empty tensor; the reference's callers discard it
    (loomformer.py:2497, :2545).
    """
    ts = (u, q_h, k_ctx_h, c_h, d_h, w1_imag_compact)
    for nm, t in zip(("u", "q_h", "k_ctx_h", "c_h", "d_h", "w1_imag_compact"), ts):
        _check(t.is_cuda, f"{nm} must be a CUDA tensor")
        _check(t.dtype in (torch.float32, torch.bfloat16), f"{nm} must be float32 or bfloat16")
        _check(t.dtype == u.dtype, f"{nm} dtype mismatch")
        _check(t.device == u.device, f"{nm} device mismatch")
    _check(u.dim() == 3, "u must be [B,T,N]")
    B, T, N = u.shape
    H, K = w1_imag_compact.shape
    for nm, t in (("q_h", q_h), ("k_ctx_h", k_ctx_h), ("c_h", c_h), ("d_h", d_h)):
        _check(t.dim() == 4 and tuple(t.shape) == (B, T, n_q_heads, head_dim), f"{nm} must be [B,T,QH,HD]")
    _check(N % 4 == 0 and head_dim % 4 == 0 and K % 4 == 0,
           "maskpack path requires N, head_dim, IMAG_IN divisible by 4")
    out = torch.empty(B, T, H, dtype=u.dtype, device=u.device)
    wc = w1_imag_compact.contiguous()
    uc, qc, kc, cc, dc = (t.contiguous() for t in (u, q_h, k_ctx_h, c_h, d_h))
    call("loom_beta_forward", dtype_code(uc), ptr(uc), ptr(qc), ptr(kc), ptr(cc), ptr(dc), ptr(wc),
         ptr(out), None, B * T, N, H, K, int(hidden_per_q_head), int(head_dim), int(n_q_heads),
         1 if open_sectors else 0, stream_of(uc))
    return [out, torch.empty(0, dtype=u.dtype, device=u.device), wc]


def _unsupported(name):
    def f(*args, **kw):
        raise RuntimeError(f"{name}: training-only entry point is not provided on gfx950")
    f.__name__ = name
    return f


beta_backward_cuda = _unsupported("beta_backward_cuda")
beta_backward_cuda_recompute = _unsupported("beta_backward_cuda_recompute")


# ---------------------------------------------------------------- phase_sin / pvpowlu

def phase_sin_forward_cuda(beta: torch.Tensor) -> torch.Tensor:
    """kernels/phase_sin/phase_sin_launcher.cu:11."""
    _check(beta.is_cuda, "phase_sin_forward_cuda: beta must be a CUDA tensor")
    _check(beta.dtype in _FLOATS, "phase_sin_forward_cuda: unsupported dtype")
    bc = beta.contiguous()
    out = torch.empty_like(bc)
    call("loom_phase_sin_forward", dtype_code(bc), ptr(bc), ptr(out), bc.numel(), stream_of(bc))
    return out


phase_sin_backward_cuda = _unsupported("phase_sin_backward_cuda")
phase_sin_secant_backward_cuda = _unsupported("phase_sin_secant_backward_cuda")


def pvpowlu_forward_cuda(x1: torch.Tensor, x2: torch.Tensor, m: float) -> torch.Tensor:
    """kernels/pvpowlu/pvpowlu_launcher.cu:11."""
    _check(x1.is_cuda and x2.is_cuda, "pvpowlu_forward_cuda: inputs must be CUDA tensors")
    _check(x1.shape == x2.shape, "pvpowlu_forward_cuda: shape mismatch")
    _check(x1.dtype == x2.dtype and x1.dtype in _FLOATS, "pvpowlu_forward_cuda: dtype mismatch")
    a, b = x1.contiguous(), x2.contiguous()
    out = torch.empty_like(a)
    call("loom_pvpowlu_forward", dtype_code(a), ptr(a), ptr(b), ptr(out), a.numel(), float(m),
         stream_of(a))
    return out


pvpowlu_backward_cuda = _unsupported("pvpowlu_backward_cuda")


# ---------------------------------------------------------------- depth attention

def _depth_hist_strides(h: torch.Tensor) -> Tuple[int, int]:
    """(stride_bt, stride_s) if h [B,T,S,QH,HD] can be read in place, else None."""
    B, T, S, QH, HD = h.shape
    st = h.stride()
    if st[4] != 1 or st[3] != HD:
        return None
    if T == 1:
        return st[0], st[2]          # bt == b
    if B > 1 and st[0] != T * st[1]:
        return None
    return st[1], st[2]


def depth_attn_read(q: torch.Tensor, hist_k: torch.Tensor, hist_v: torch.Tensor,
                    want_weights: bool, want_lse: bool):
    """Shared body of the depth-attention forwards.  Strided views of a
    [B,T,S_max,QH,HD] history (e.g. hist[:, :, :s+1] in Model.step) are read in
    place instead of being copied."""
    _check(q.is_cuda and hist_k.is_cuda and hist_v.is_cuda, "depth_attn_forward_cuda: all inputs must be CUDA tensors")
    _check(hist_k.dim() == 5, "hist_k must be [B,T,S,QH,HD]")
    _check(hist_v.shape == hist_k.shape, "hist_v shape mismatch")
    _check(q.dim() == 2, "q must be [QH,HD]")
    B, T, S, QH, HD = hist_k.shape
    _check(q.shape[0] == QH and q.shape[1] == HD, "q shape mismatch")
    _check(q.dtype == hist_k.dtype == hist_v.dtype and q.dtype in _FLOATS, "depth_attn: dtype mismatch")
    sk, sv = _depth_hist_strides(hist_k), _depth_hist_strides(hist_v)
    if sk is None or sv is None or sk != sv:
        hist_k, hist_v = hist_k.contiguous(), hist_v.contiguous()
        sk = (S * QH * HD, QH * HD)
    qc = q.contiguous()
    d = torch.empty(B, T, QH, HD, dtype=hist_k.dtype, device=hist_k.device)
    w = torch.empty(B, T, QH, S, dtype=hist_k.dtype, device=hist_k.device) if want_weights else None
    lse = torch.empty(B, T, QH, dtype=torch.float32, device=hist_k.device) if want_lse else None
    call("loom_depth_attn_forward", dtype_code(qc), ptr(qc), ptr(hist_k), ptr(hist_v), sk[0], sk[1],
         ptr(d), ptr(w), ptr(lse), B * T, S, QH, HD, stream_of(qc))
    return d, w, lse


def depth_attn_forward(q, hist_k, hist_v) -> List[torch.Tensor]:
    """kernels/depth_attn/depth_attn_launcher.cu:63 -> [d, w]."""
    d, w, _ = depth_attn_read(q, hist_k, hist_v, True, False)
    return [d, w]


def depth_attn_stacked_forward(q, hist_k, hist_v) -> Tuple[torch.Tensor, torch.Tensor]:
    """kernels/depth_attn/depth_attn_launcher.cu:143 -> (d, lse fp32)."""
    d, _, lse = depth_attn_read(q, hist_k, hist_v, False, True)
    return d, lse


def depth_attn_list_forward(q, hist_k: Sequence[torch.Tensor], hist_v: Sequence[torch.Tensor]):
    """kernels/depth_attn/depth_attn_launcher.cu:271 -> [d, w]."""
    _check(len(hist_k) > 0, "depth_attn_list_forward_cuda: history must be non-empty")
    _check(len(hist_k) == len(hist_v), "depth_attn_list_forward_cuda: K/V history length mismatch")
    return depth_attn_forward(q, torch.stack(list(hist_k), 2), torch.stack(list(hist_v), 2))


depth_attn_backward = _unsupported("depth_attn_backward")
depth_attn_stacked_backward = _unsupported("depth_attn_stacked_backward")
depth_attn_list_backward = _unsupported("depth_attn_list_backward")


# ---------------------------------------------------------------- tria

def _tria_common(name, r, i, o, extra=()):
    _cuda(r, i, o, *extra, name=name)
    _same_dtype(r, i, o, *extra, name=name)
    _check(i.numel() == r.numel() and o.numel() == r.numel(), f"{name}: r, i, o must have the same numel")


def _tria_call(r, i, o, prev, seed, valid, w, want_scale, alpha, axis, want_carry=True):
    _check(r.dim() == 3, "tria: r must be [B,T,H]")
    B, T, H = r.shape
    n = B * T * H
    rc, ic, oc = r.contiguous(), i.contiguous(), o.contiguous()
    carry = torch.empty(B, T, H, 3, 3, dtype=r.dtype, device=r.device) if want_carry else None
    p = torch.empty_like(rc) if w is not None else None
    scale = torch.empty(n, dtype=torch.float32, device=r.device) if want_scale else None
    prev_c, seed_c, valid_c, w_c = _c(prev), _c(seed), _c(valid), _c(w)
    call("loom_tria_depth_forward", dtype_code(rc), ptr(rc), ptr(ic), ptr(oc), ptr(prev_c),
         ptr(seed_c), ptr(valid_c), ptr(w_c), ptr(carry), ptr(p), ptr(scale), B, T, H,
         float(alpha), int(axis), stream_of(rc))
    return carry, p, scale


def tria_init_forward(r, i, o, alpha, axis):
    """kernels/tria/tria_init/tria_init_launcher.cu (bindings.cpp:84) -> [carry, scale]."""
    _tria_common("tria_init_forward_cuda", r, i, o)
    c, _, s = _tria_call(r, i, o, None, None, None, None, True, alpha, axis)
    return [c, s]


def tria_init_gate_forward(r, i, o, w, alpha, axis):
    """bindings.cpp:85 -> [carry, p, scale]."""
    _tria_common("tria_init_gate_forward_cuda", r, i, o, (w,))
    _check(w.numel() == 9, "tria_init_gate_forward_cuda: w must have exactly 9 elements")
    c, p, s = _tria_call(r, i, o, None, None, None, w, True, alpha, axis)
    return [c, p, s]


def _seed_checks(name, r, seed, valid):
    _check(r.dim() == 3, f"{name}: r must be [B,T,H]")
    _check(seed.dim() == 4 and seed.shape[1] == r.shape[2] and seed.shape[2] == 3 and seed.shape[3] == 3,
           f"{name}: seed must be [B,H,3,3]")
    _check(seed.shape[0] == r.shape[0], f"{name}: batch mismatch")
    _check(valid.dim() == 1 and valid.shape[0] == r.shape[0] and valid.dtype == torch.bool,
           f"{name}: valid must be [B] bool")


def tria_init_seed_forward(r, i, o, seed, valid, alpha, axis):
    """tria_init_seed_launcher.cu (bindings.cpp:86) -> [carry, scale]."""
    name = "tria_init_seed_forward_cuda"
    _tria_common(name, r, i, o, (seed,))
    _check(valid.is_cuda, f"{name}: all inputs must be CUDA tensors")
    _seed_checks(name, r, seed, valid)
    c, _, s = _tria_call(r, i, o, None, seed, valid, None, True, alpha, axis)
    return [c, s]


def tria_init_seed_gate_forward(r, i, o, seed, valid, w, alpha, axis):
    """tria_init_seed_launcher.cu:96-120 (bindings.cpp:87) -> [carry, p]."""
    name = "tria_init_seed_gate_forward_cuda"
    _tria_common(name, r, i, o, (seed, w))
    _check(valid.is_cuda, f"{name}: all inputs must be CUDA tensors")
    _seed_checks(name, r, seed, valid)
    _check(w.numel() == 9, f"{name}: w must have 9 elements")
    c, p, _ = _tria_call(r, i, o, None, seed, valid, w, False, alpha, axis)
    return [c, p]


def tria_step_forward(r, i, o, carry_prev, alpha, axis):
    """bindings.cpp:92 -> [carry, scale]."""
    _tria_common("tria_step_forward_cuda", r, i, o, (carry_prev,))
    _check(carry_prev.numel() == r.numel() * 9,
           "tria_step_forward_cuda: carry_prev must have 9 values per r/i/o element")
    c, _, s = _tria_call(r, i, o, carry_prev, None, None, None, True, alpha, axis)
    return [c, s]


def tria_step_gate_forward(r, i, o, carry_prev, w, alpha, axis):
    """tria_step_gate_launcher.cu:14 (bindings.cpp:93) -> [carry, p, scale]."""
    name = "tria_step_gate_forward_cuda"
    _tria_common(name, r, i, o, (carry_prev, w))
    _check(carry_prev.numel() == r.numel() * 9, f"{name}: carry_prev must have 9 values per r/i/o element")
    _check(w.numel() == 9, f"{name}: w must have exactly 9 elements")
    c, p, s = _tria_call(r, i, o, carry_prev, None, None, w, True, alpha, axis)
    return [c, p, s]


def gate_slot_mix_forward(carry, w):
    """gate_slot_mix_launcher.cu:14 (bindings.cpp:97) -> p[...]."""
    name = "gate_slot_mix_forward_cuda"
    _check(carry.is_cuda and w.is_cuda, f"{name}: inputs must be CUDA tensors")
    _check(carry.device == w.device, f"{name}: inputs must be on the same device")
    _check(carry.dtype == w.dtype, f"{name}: dtype mismatch")
    _check(carry.dim() >= 2 and carry.shape[-1] == 3 and carry.shape[-2] == 3, f"{name}: carry must end in [...,3,3]")
    _check(w.numel() == 9, f"{name}: w must have exactly 9 elements")
    cc = carry.contiguous()
    p = torch.empty(cc.shape[:-2], dtype=cc.dtype, device=cc.device)
    wc = w.contiguous()
    call("loom_gate_slot_mix_forward", dtype_code(cc), ptr(cc), ptr(wc), ptr(p),
         cc.numel() // 9, stream_of(cc))
    return p


def slot_attention_pool_forward(carry, score_w):
    """slot_attention_pool_launcher.cu (bindings.cpp:99) -> [pooled[B,T,9], lse[B,T]]."""
    name = "slot_attention_pool_forward_cuda"
    _check(carry.is_cuda and score_w.is_cuda, f"{name}: inputs must be CUDA tensors")
    _check(carry.dtype == score_w.dtype, f"{name}: dtype mismatch")
    _check(carry.dim() == 5 and carry.shape[-1] == 3 and carry.shape[-2] == 3, f"{name}: carry must be [B,T,H,3,3]")
    _check(score_w.numel() == 9, f"{name}: score_w must have exactly 9 elements")
    B, T, H = carry.shape[:3]
    cc = carry.contiguous()
    pooled = torch.empty(B, T, 9, dtype=cc.dtype, device=cc.device)
    lse = torch.empty(B, T, dtype=cc.dtype, device=cc.device)
    sw = score_w.contiguous()
    call("loom_slot_attention_pool_forward", dtype_code(cc), ptr(cc), ptr(sw),
         ptr(pooled), ptr(lse), B * T, H, stream_of(cc))
    return [pooled, lse]


def temporal_carry_forward(depth_carry, reset_mask):
    """temporal_carry_launcher.cu:13 (bindings.cpp:101) -> [doc fp32, scale fp32]."""
    _check(depth_carry.is_cuda and reset_mask.is_cuda, "temporal_carry: CUDA inputs required")
    _check(depth_carry.dim() == 5 and depth_carry.shape[3] == 3 and depth_carry.shape[4] == 3,
           "depth_carry must be [B,T,H,3,3]")
    _check(reset_mask.shape == depth_carry.shape[:2], "reset_mask must be [B,T]")
    _check(reset_mask.dtype == torch.bool, "reset_mask must be bool")
    _check(depth_carry.dtype in _FLOATS, "temporal_carry: unsupported dtype")
    B, T, H = depth_carry.shape[:3]
    dc = depth_carry.contiguous()
    doc = torch.empty(dc.shape, dtype=torch.float32, device=dc.device)
    scale = torch.empty(B, T, H, dtype=torch.float32, device=dc.device)
    rm = reset_mask.contiguous()
    call("loom_temporal_carry_forward", dtype_code(dc), ptr(dc), ptr(rm),
         ptr(doc), ptr(scale), B, T, H, stream_of(dc))
    return [doc, scale]


def temporal_carry_endpoint_forward(depth, reset, initial, initial_valid):
    """temporal_carry_endpoint_launcher.cu:11 (bindings.cpp:103) -> [endpoint, endpoint_fp32]."""
    _check(depth.is_cuda and reset.is_cuda, "temporal_carry_endpoint_forward_cuda: CUDA inputs required")
    _check(depth.dim() == 5 and depth.shape[3] == 3 and depth.shape[4] == 3,
           "temporal_carry_endpoint_forward_cuda: depth must be [B,T,H,3,3]")
    _check(reset.dtype == torch.bool and reset.shape == depth.shape[:2],
           "temporal_carry_endpoint_forward_cuda: reset must be [B,T] bool")
    _check(depth.dtype in _FLOATS, "temporal_carry_endpoint_forward_cuda: unsupported dtype")
    B, T, H = depth.shape[:3]
    has_initial = initial.numel() != 0
    init_c = valid_c = None
    if has_initial:
        _check(initial.is_cuda and initial_valid.is_cuda, "initial state must be CUDA")
        _check(initial.dim() == 4 and initial.shape[0] == B and initial.shape[1] == H
               and initial.shape[2] == 3 and initial.shape[3] == 3, "initial must be [B,H,3,3]")
        _check(initial_valid.dim() == 1 and initial_valid.shape[0] == B and initial_valid.dtype == torch.bool,
               "initial_valid must be [B] bool")
        _check(initial.dtype == depth.dtype, "initial dtype mismatch")
        init_c, valid_c = initial.contiguous(), initial_valid.contiguous()
    dc = depth.contiguous()
    ep = torch.empty(B, H, 3, 3, dtype=dc.dtype, device=dc.device)
    ep32 = torch.empty(B, H, 3, 3, dtype=torch.float32, device=dc.device)
    rs = reset.contiguous()
    call("loom_temporal_carry_endpoint_forward", dtype_code(dc), ptr(dc), ptr(rs),
         ptr(init_c), ptr(valid_c), ptr(ep), ptr(ep32), B, T, H, stream_of(dc))
    return [ep, ep32]


def final_ca_sparse_forward(q, k, v, allowed, scale: float):
    """final_ca_sparse_launcher.cu:30 (bindings.cpp:107) -> [out, lse fp32]."""
    _check(q.is_cuda and k.is_cuda and v.is_cuda and allowed.is_cuda, "final CA: CUDA inputs required")
    _check(q.dim() == 3 and k.dim() == 3 and v.dim() == 3, "final CA: q/k/v must be rank 3")
    _check(q.shape[0] == k.shape[0] and k.shape == v.shape and q.shape[2] == k.shape[2],
           "final CA: shape mismatch")
    _check(q.dtype == k.dtype == v.dtype and q.dtype in _FLOATS, "final CA: dtype mismatch")
    _check(allowed.dtype == torch.bool and allowed.dim() == 3 and allowed.shape[0] == q.shape[0]
           and allowed.shape[1] == q.shape[1] and allowed.shape[2] == k.shape[1],
           "final CA: allowed must be [B,T,K] bool")
    B, T, D = q.shape
    K = k.shape[1]
    _check(0 < K <= 256, "final CA: expected 1..256 sparse keys")
    qc, kc, vc, ac = q.contiguous(), k.contiguous(), v.contiguous(), allowed.contiguous()
    out = torch.empty_like(qc)
    lse = torch.empty(B, T, dtype=torch.float32, device=q.device)
    call("loom_final_ca_sparse_forward", dtype_code(qc), ptr(qc), ptr(kc), ptr(vc),
         ptr(ac), ptr(out), ptr(lse), B, T, K, D, float(scale), stream_of(qc))
    return [out, lse]


def polarm(matrix: torch.Tensor, beta: float = 0.1, eps: float = 1e-6,
           mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """tria.polarm (tria.py:160-166) as one kernel; ``mask`` [B] selects the
    leading-dim rows to correct (others are copied)."""
    _check(matrix.is_cuda and matrix.shape[-2:] == (3, 3), "polarm: CUDA [...,3,3] input required")
    mc = matrix.contiguous()
    out = torch.empty_like(mc)
    n = mc.numel() // 9
    per = n // mc.shape[0] if mask is not None else 1
    mk = _c(mask)
    call("loom_polarm_forward", dtype_code(mc), ptr(mc), ptr(out), ptr(mk), n, per,
         float(beta), float(eps), stream_of(mc))
    return out


def tria_chunked_forward(r: torch.Tensor, i: torch.Tensor, o: torch.Tensor, alpha: float,
                         window: int, polarm_beta: float = 0.1,
                         reset: Optional[torch.Tensor] = None, want_depth: bool = False,
                         eps: float = 1e-6, explicit_fire: Optional[torch.Tensor] = None,
                         return_valid: bool = False):
    """Tria part of Model._forward_chunked (loomformer.py:3788-3883): r, i, o
    are [L,B,T,H] stacks of the per-layer summaries (layer l uses axis l % 3).
    Boundaries are the grid positions (t+1) % window == 0 (t < T-1) and, with
    explicit_fire ([B,T] bool, the <CARRY> positions), every position where any
    row fires (:3797-3815; the list is built on the host, as the reference's
    boundary_positions is).  Returns (keys [B,K,H,3,3] float32, depth
    [B,T,H,3,3] or None) with K = the boundary count: the document keys (state
    after each boundary's PolARM where the row fired) and optionally each
    token's final-layer depth carry; with return_valid also the key validity
    [B,K] bool (the row's fire at the boundary, :3856)."""
    name = "tria_chunked_forward"
    _cuda(r, i, o, name=name)
    _same_dtype(r, i, o, name=name)
    _check(r.dim() == 4 and r.shape == i.shape == o.shape, f"{name}: r, i, o must be [L,B,T,H]")
    L, B, T, H = r.shape
    _check(T >= 1 and window >= 1, f"{name}: need T >= 1 and window >= 1")
    rc, ic, oc = r.contiguous(), i.contiguous(), o.contiguous()
    rs = None
    if reset is not None:
        _check(reset.is_cuda and reset.dtype == torch.bool and reset.shape == (B, T),
               f"{name}: reset must be a CUDA [B,T] bool tensor")
        rs = reset.contiguous()
    depth = torch.empty(B, T, H, 3, 3, dtype=r.dtype, device=r.device) if want_depth else None
    lib = _lib.load()
    if explicit_fire is None:
        K = -(-T // window) - 1
        keys = torch.empty(B, max(K, 0), H, 3, 3, dtype=torch.float32, device=r.device)
        nbytes = lib.loom_tria_chunked_workspace_bytes(B, T, H, window)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=r.device)
        call("loom_tria_chunked_forward", dtype_code(rc), ptr(rc), ptr(ic), ptr(oc), B * T * H, L,
             ptr(rs), ptr(keys) if K > 0 else None, ptr(depth), ptr(ws), nbytes, B, T, H, window,
             float(alpha), float(polarm_beta), float(eps), stream_of(rc))
        if not return_valid:
            return keys, depth
        valid = torch.ones(B, max(K, 0), dtype=torch.bool, device=r.device)
        if K > 0 and reset is not None:
            valid = ~reset[:, window::window][:, :K]
        return keys, depth, valid
    _check(explicit_fire.is_cuda and explicit_fire.dtype == torch.bool and explicit_fire.shape == (B, T),
           f"{name}: explicit_fire must be a CUDA [B,T] bool tensor")
    grid = (torch.arange(T) + 1) % window == 0
    grid[-1] = False
    bounds = (grid | explicit_fire.any(dim=0).cpu()).nonzero().flatten().to(torch.int64).contiguous()
    K = bounds.numel()
    keys = torch.empty(B, K, H, 3, 3, dtype=torch.float32, device=r.device)
    kv = torch.empty(B, K, dtype=torch.uint8, device=r.device)
    ef = explicit_fire.contiguous().view(torch.uint8)
    bptr = ctypes.c_void_p(bounds.data_ptr())
    nbytes = lib.loom_tria_chunked_fires_workspace_bytes(B, T, H, bptr, K)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=r.device)
    call("loom_tria_chunked_forward_fires", dtype_code(rc), ptr(rc), ptr(ic), ptr(oc), B * T * H, L,
         ptr(rs), ptr(ef), bptr, K, ptr(keys) if K > 0 else None, ptr(kv) if K > 0 else None,
         ptr(depth), ptr(ws), nbytes, B, T, H, window, float(alpha), float(polarm_beta), float(eps),
         stream_of(rc))
    if return_valid:
        return keys, depth, kv.bool()
    return keys, depth


def tria_readout(carry: torch.Tensor, score_w: torch.Tensor, proj_w: torch.Tensor,
                 proj_b: torch.Tensor, up_w: torch.Tensor, up_b: torch.Tensor) -> torch.Tensor:
    """TriaAggregator.forward (tria.py:1436-1441): slot-attention pool over H of
    carry [B,K,H,3,3] with score_w [9], then proj (9 -> k) and up (k -> d_model)."""
    pooled, _ = slot_attention_pool_forward(carry, score_w.to(carry.dtype))
    z = linear(pooled, proj_w.to(carry.dtype), proj_b)
    return linear(z, up_w.to(carry.dtype), up_b)


# ---------------------------------------------------------------- projections

def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
           gate_p: Optional[torch.Tensor] = None, gate_alpha: float = 0.0,
           residual: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """F.linear(x, weight, bias) on the gfx950 GEMM, with the optional
    IdentityAnchoredGate epilogue acc*(1 + gate_alpha*gate_p) (tria.py:1297-1299)
    and a residual add.  bias is float32."""
    _check(x.is_cuda and weight.is_cuda, "linear: CUDA tensors required")
    _check(x.dtype == weight.dtype and x.dtype in _FLOATS, "linear: dtype mismatch")
    K = x.shape[-1]
    _check(weight.dim() == 2 and weight.shape[1] == K, "linear: weight must be [N,K]")
    Nout = weight.shape[0]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    M = x2.shape[0]
    wc = weight if weight.stride(-1) == 1 else weight.contiguous()
    if out is None:
        out = torch.empty(*x.shape[:-1], Nout, dtype=x.dtype, device=x.device)
    b = None if bias is None else bias.float().contiguous()
    gp = None if gate_p is None else gate_p.reshape(M, Nout).contiguous()
    rs = None if residual is None else residual.reshape(M, Nout).contiguous()
    call("loom_linear", dtype_code(x2), ptr(x2), x2.stride(0), ptr(wc), wc.stride(0), ptr(b),
         ptr(gp), float(gate_alpha), ptr(rs), ptr(out), Nout, M, Nout, K, stream_of(x2))
    return out
