"""fp32 CPU restatement of the LoomFormer model and its decode ``step``.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* ``Shapes`` restates the shape derivation of ``apply_config``
  (loomformer.py:904-1134) for the keys the inference path reads.
* ``OracleModel`` builds the parameters in the reference's module-construction
  order so that ``torch.manual_seed(k)`` followed by construction yields the
  same tensors as the reference's ``Model(cfg)`` (loomformer.py:3477-3531 and
  the ``__init__``/``reset_parameters`` of every submodule).  Parameter and
  buffer names equal the reference's ``state_dict`` keys.
* ``OracleModel.step`` restates ``Model.step`` (loomformer.py:3951-4091) on the
  CPU branch of every op; ``greedy_decode`` restates ``infer``
  (loomformer.py:5290-5311) for a batch of equal-length prompts.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops

FANIN_GAIN = 0.88  # loomformer.py:805


@dataclass
class Shapes:
    V: int
    N: int
    QH: int
    HD: int
    KVH: int
    G: int
    H: int
    L: int
    seq_len: int
    sectors: str = "head"
    residual_init: str = "beta"
    powlu_m: float = 3.0
    tria_alpha: float = 0.05
    polarm_beta: float = 0.1
    gamma_max: float = 0.25
    raw_gamma_init: float = 0.0
    window: int = 128
    tied: bool = True
    rope_theta: float = 10000.0
    rope_factor: float = 4.0
    rope_original: int = 0
    rope_beta_fast: float = 32.0
    rope_beta_slow: float = 1.0
    rope_attention_factor: Optional[float] = None
    carry_token_id: Optional[int] = None
    # model variants (Config, loomformer.py:272-274, :358, :366)
    gate_proj: bool = False
    qkv_rms: bool = False
    rms_cap: Optional[float] = None
    final_norm: bool = False
    readout: str = "shared"

    @property
    def Hq(self) -> int:
        return self.H // self.QH

    @property
    def KV(self) -> int:
        return self.KVH * self.HD

    @property
    def imag_in(self) -> int:
        return ops.imag_in(self.N, self.HD, self.sectors)

    @property
    def deepnorm_beta(self) -> float:
        return (8.0 * max(1, self.L)) ** -0.25   # loomformer.py:1093-1095

    @staticmethod
    def from_dict(d: dict, **overrides) -> "Shapes":
        """Shape derivation of apply_config (loomformer.py:904-1120)."""
        d = dict(d)
        d.update(overrides)
        QH = int(d.get("n_q_heads", 6))
        model_dim = d.get("model_dim", 12)          # Config defaults (loomformer.py:225-236)
        if d.get("head_dim") is not None:
            HD = int(d["head_dim"])
            N = QH * HD
            if model_dim is not None and int(model_dim) != N:
                raise ValueError("model_dim != n_q_heads*head_dim")
        elif model_dim is None:
            HD = 32
            N = QH * HD
        else:
            N = int(model_dim)
            HD = N // QH
        gs, nkv = d.get("gqa_group_size"), d.get("n_kv_heads", 3)
        if gs is not None and nkv is not None:
            G, KVH = int(gs), int(nkv)
        elif gs is not None:
            G = int(gs)
            KVH = QH // G
        elif nkv is not None:
            KVH = int(nkv)
            G = QH // KVH
        else:
            G = 4 if QH % 4 == 0 else (2 if QH % 2 == 0 else 1)
            KVH = QH // G
        if d.get("hidden") is None:
            mult = 4.0 if d.get("hidden_mult") is None else float(d["hidden_mult"])
            raw = max(QH, int(round(N * mult)))
            H = ((raw + QH - 1) // QH) * QH
        else:
            H = int(d["hidden"])
        seq_len = int(d.get("seq_len", 128))
        ro = d.get("rope_original_seq_len")
        return Shapes(
            V=int(d.get("vocab", 256)), N=N, QH=QH, HD=HD, KVH=KVH, G=G, H=H,
            L=int(d.get("layers", 3)), seq_len=seq_len,
            sectors=str(d.get("phase_sectors", "head")).lower(),
            residual_init=str(d.get("residual_init", "beta")).lower(),
            powlu_m=float(d.get("powlu_m", 3.0) or 3.0),
            tria_alpha=float(d.get("tria_carrier_alpha", 0.05)),
            polarm_beta=float(d.get("tria_polarm_beta", 0.1)),
            gamma_max=float(d.get("tria_gamma_max", 0.25)),
            raw_gamma_init=float(d.get("tria_raw_gamma_init", 0.0)),
            window=int(d.get("tria_temporal_window") or seq_len),
            tied=bool(d.get("tied_embeddings", True)),
            rope_theta=float(d.get("rope_theta", 10000.0) or 10000.0),
            rope_factor=float(d.get("rope_factor", 4.0) or 4.0),
            rope_original=seq_len if ro is None else int(ro),
            rope_beta_fast=float(d.get("rope_beta_fast", 32.0) or 32.0),
            rope_beta_slow=float(d.get("rope_beta_slow", 1.0) or 1.0),
            rope_attention_factor=(None if d.get("rope_attention_factor") is None
                                   else float(d["rope_attention_factor"])),
            carry_token_id=(None if d.get("carry_token_id") is None else int(d["carry_token_id"])),
            gate_proj=bool(d.get("paraplex_gate_proj", False)),
            qkv_rms=bool(d.get("depth_attn_qkv_rms", False)),
            rms_cap=(None if d.get("residual_branch_rms_cap") is None
                     else float(d["residual_branch_rms_cap"])),
            final_norm=bool(d.get("final_norm", False)),
            readout=str(d.get("depth_attn_readout", "shared") or "shared").lower(),
        )

    @staticmethod
    def from_yaml(path: str, **overrides) -> "Shapes":
        import yaml
        with open(path, encoding="utf-8") as f:
            d = yaml.safe_load(f) or {}
        return Shapes.from_dict(d, **overrides)


def fanin_std(fan_in: int, gain: float = FANIN_GAIN) -> float:
    """loomformer.py:829-832."""
    return gain / math.sqrt(float(fan_in))


def fixed_rms(x: torch.Tensor, target: float = 1.0, eps: float = 1e-6) -> torch.Tensor:
    """Each last-dim vector scaled by target / sqrt(mean(x^2) + eps), the scale
    rounded to x's dtype (loomformer.py:840-844)."""
    work = x.float() if x.dtype in (torch.float16, torch.bfloat16) else x
    scale = torch.rsqrt(work.square().mean(dim=-1, keepdim=True) + eps) * float(target)
    return x * scale.to(dtype=x.dtype)


def capped_rms(x: torch.Tensor, maximum: float = 1.0, eps: float = 1e-6) -> torch.Tensor:
    """RMS scaling down to `maximum`, never up (loomformer.py:847-852)."""
    work = x.float() if x.dtype in (torch.float16, torch.bfloat16) else x
    rms = torch.sqrt(work.square().mean(dim=-1, keepdim=True) + eps)
    scale = (float(maximum) / rms).clamp(max=1.0)
    return x * scale.to(dtype=x.dtype)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm.forward (loomformer.py:3460-3464): fp32 statistics, the
    normalised row rounded to x's dtype, then the learned scale."""
    xf = x.float()
    rms = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (xf * rms).to(x.dtype) * weight


# --------------------------------------------------------------------------
# Modules (construction order == the reference's; names == its state_dict keys)
# --------------------------------------------------------------------------

class _Attn(nn.Module):
    """GroupedQueryCausalSelfAttention parameters (loomformer.py:3215-3230)."""

    def __init__(self, S: Shapes) -> None:
        super().__init__()
        self.qkv_weight = nn.Parameter(torch.empty(S.N + 2 * S.KV, S.N))
        self.o = nn.Linear(S.N, S.N, bias=False)
        rstd = fanin_std(S.N) * (S.deepnorm_beta if S.residual_init == "beta" else 1.0)
        nn.init.normal_(self.qkv_weight[:S.N], mean=0.0, std=fanin_std(S.N))
        nn.init.normal_(self.qkv_weight[S.N:S.N + S.KV], mean=0.0, std=fanin_std(S.N))
        nn.init.normal_(self.qkv_weight[S.N + S.KV:], mean=0.0, std=rstd)
        nn.init.normal_(self.o.weight, mean=0.0, std=rstd)


class _GateSelector(nn.Module):
    def __init__(self) -> None:   # tria.py:1257-1261
        super().__init__()
        self.logits = nn.Parameter(torch.zeros(9))


class _IdentityGate(nn.Module):
    def __init__(self, alpha_max: float = 0.25) -> None:   # tria.py:1287-1292
        super().__init__()
        self.alpha_max = alpha_max
        self.raw_alpha = nn.Parameter(torch.zeros(()))


class _FFN(nn.Module):
    """ParaplexFFN parameters (loomformer.py:2667-2716) with tria carry on."""

    def __init__(self, S: Shapes) -> None:
        super().__init__()
        self.w1_real = nn.Linear(S.N, S.H)
        self.w1_imag = nn.Parameter(torch.empty(S.H, S.imag_in))
        self.w1_imag_trace = nn.Parameter(torch.zeros(S.H))
        self.w1_imag_bias = nn.Parameter(torch.zeros(S.H))
        self.w2 = nn.Linear(S.H, S.N)
        self.register_buffer("beta_anchor", torch.tensor(1.0), persistent=True)
        self.gate_selector = _GateSelector()
        self.identity_gate = _IdentityGate()
        # the independent amplitude source of paraplex_gate_proj (loomformer.py:2704-2707)
        self.gate_proj = nn.Linear(S.N, S.H) if S.gate_proj else None
        rstd = fanin_std(S.H) * (S.deepnorm_beta if S.residual_init == "beta" else 1.0)
        nn.init.normal_(self.w1_real.weight, mean=0.0, std=fanin_std(S.N))
        nn.init.zeros_(self.w1_real.bias)
        nn.init.normal_(self.w1_imag, mean=0.0, std=fanin_std(S.imag_in))
        nn.init.normal_(self.w2.weight, mean=0.0, std=rstd)
        nn.init.zeros_(self.w2.bias)
        if self.gate_proj is not None:                      # loomformer.py:2717-2718
            nn.init.normal_(self.gate_proj.weight, mean=0.0, std=fanin_std(S.N))
            nn.init.zeros_(self.gate_proj.bias)


class _Block(nn.Module):
    def __init__(self, S: Shapes) -> None:   # loomformer.py:3467-3473
        super().__init__()
        self.ln_attn = nn.LayerNorm(S.N)
        self.attn = _Attn(S)
        self.ln_ffn = nn.LayerNorm(S.N)
        self.ffn = _FFN(S)


class _DepthAttn(nn.Module):
    """DepthAttn parameters (loomformer.py:3367-3389): one shared readout w_o,
    or with depth_attn_readout = per-sublayer one [N, N] readout per sublayer
    in w_o_weight [2L, N, N]."""

    def __init__(self, S: Shapes) -> None:
        super().__init__()
        self.kv_weight = nn.Parameter(torch.empty(2 * S.N, S.N))
        if S.readout == "per-sublayer":
            self.w_o_weight = nn.Parameter(torch.empty(2 * S.L, S.N, S.N))
            self.w_o = None
        else:
            self.w_o_weight = None
            self.w_o = nn.Linear(S.N, S.N, bias=False)
        self.q_params = nn.Parameter(torch.empty(2 * S.L, S.QH, S.HD))
        rstd = fanin_std(S.N) * (S.deepnorm_beta if S.residual_init == "beta" else 1.0)
        nn.init.normal_(self.kv_weight[:S.N], mean=0.0, std=fanin_std(S.N))
        nn.init.normal_(self.kv_weight[S.N:], mean=0.0, std=rstd)
        nn.init.normal_(self.w_o_weight if self.w_o is None else self.w_o.weight, mean=0.0, std=rstd)
        nn.init.normal_(self.q_params, mean=0.0, std=fanin_std(S.HD))


class _RMSNormParams(nn.Module):
    def __init__(self, dim: int) -> None:   # RMSNorm.__init__ (loomformer.py:3452-3458)
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))


class _Reader(nn.Module):
    def __init__(self, k: int = 32) -> None:   # tria.py:1302-1338
        super().__init__()
        self.k = k
        self.proj = nn.Linear(9, k)
        self.key_proj = nn.Linear(9, k, bias=False)
        with torch.no_grad():
            self.key_proj.weight.normal_(mean=0.0, std=1.5)


class _Pool(nn.Module):
    def __init__(self, k: int) -> None:   # tria.py:1405-1416
        super().__init__()
        self.query = nn.Parameter(torch.zeros(k))
        self.logit_scale_raw = nn.Parameter(torch.tensor(math.log(math.expm1(1.0))))


class _Agg(nn.Module):
    def __init__(self, reader: _Reader, N: int) -> None:   # tria.py:1429-1434
        super().__init__()
        self.reader = reader
        self.pool = _Pool(reader.k)
        self.up = nn.Linear(reader.k, N)


class _FinalCA(nn.Module):
    def __init__(self, N: int, gamma_max: float, raw_gamma_init: float) -> None:  # tria.py:1501-1508
        super().__init__()
        self.w_qk = nn.Linear(N, N, bias=False)
        self.w_v = nn.Linear(N, N, bias=False)
        self.gamma_max = float(gamma_max)
        self.raw_gamma = nn.Parameter(torch.tensor(float(raw_gamma_init)))
        self.scale = N ** -0.5


@dataclass
class LayerCache:
    k: Optional[torch.Tensor] = None
    v: Optional[torch.Tensor] = None
    phase_trace: Optional[torch.Tensor] = None
    cache_len: int = 0


@dataclass
class CACache:
    k: Optional[torch.Tensor] = None
    v: Optional[torch.Tensor] = None
    valid: Optional[torch.Tensor] = None
    cache_len: int = 0


@dataclass
class TemporalState:
    carry: Optional[torch.Tensor] = None
    pending: Optional[torch.Tensor] = None


@dataclass
class StepState:
    caches: List[LayerCache] = field(default_factory=list)
    ca: CACache = field(default_factory=CACache)
    temporal: TemporalState = field(default_factory=TemporalState)


class OracleModel(nn.Module):
    """Model (loomformer.py:3477-3531) with tria carry + temporal enabled."""

    def __init__(self, S: Shapes) -> None:
        super().__init__()
        self.S = S
        self.emb = nn.Embedding(S.V, S.N)
        self.blocks = nn.ModuleList([_Block(S) for _ in range(S.L)])
        self.depth_attn = _DepthAttn(S)
        self.head = nn.Linear(S.N, S.V, bias=False)
        if S.tied:
            self.head.weight = self.emb.weight
        # final_norm: one RMSNorm before the head (loomformer.py:3490)
        self.ln_final = _RMSNormParams(S.N) if S.final_norm else None
        reader = _Reader(k=32)
        self.tria_agg = _Agg(reader, S.N)
        self.tria_final_ca = _FinalCA(S.N, S.gamma_max, S.raw_gamma_init)
        nn.init.normal_(self.emb.weight, mean=0.0, std=fanin_std(S.N))
        # Model.step never applies residual_branch_rms_cap: only _block_core, the
        # sequence forward, caps its branches (loomformer.py:3568-3570, :3627-3629;
        # step's sublayer tails are :3998-4000, :4045).  Setting this to a cap
        # applies it in step too; tests use that to show the fixtures tell the
        # two apart.
        self.step_branch_cap: Optional[float] = None
        inv_freq, att = ops.yarn_inv_freq(S.HD, S.rope_theta, S.rope_factor, S.rope_original,
                                          S.rope_beta_fast, S.rope_beta_slow,
                                          S.rope_attention_factor)
        self._cos, self._sin = ops.yarn_cos_sin(inv_freq, att, S.seq_len)

    # ---- sub-ops -----------------------------------------------------------

    def kv_project(self, h: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """DepthAttn.project (loomformer.py:3391-3402)."""
        S = self.S
        B, T, _ = h.shape
        kv = F.linear(h, self.depth_attn.kv_weight)
        k, v = torch.split(kv, (S.N, S.N), dim=-1)
        k, v = k.reshape(B, T, S.QH, S.HD), v.reshape(B, T, S.QH, S.HD)
        if S.qkv_rms:                                  # loomformer.py:3397-3401
            k = fixed_rms(k, FANIN_GAIN)
            v = fixed_rms(v, FANIN_GAIN * S.deepnorm_beta)
        return k, v

    def depth_read(self, sub_idx: int, hist_k, hist_v) -> Tuple[torch.Tensor, torch.Tensor]:
        """DepthAttn.forward, tensor-history branch (loomformer.py:3404-3429)."""
        S = self.S
        q_row = self.depth_attn.q_params[sub_idx]
        if S.qkv_rms:                                  # loomformer.py:3406-3407
            q_row = fixed_rms(q_row, fanin_std(S.HD))
        d = ops.depth_attn_online(q_row, hist_k, hist_v)
        B, T = hist_k.shape[:2]
        d_flat = d.reshape(B, T, S.N)
        if self.depth_attn.w_o is None:                # per-sublayer readout (:3424-3428)
            return F.linear(d_flat, self.depth_attn.w_o_weight[sub_idx]), d
        return self.depth_attn.w_o(d_flat), d

    def attn_step(self, blk: _Block, z: torch.Tensor, pos: int, cache: LayerCache):
        """GroupedQueryCausalSelfAttention.step (loomformer.py:3300-3332)."""
        S = self.S
        if cache.cache_len >= S.seq_len:
            raise ValueError(f"generation exceeded seq_len={S.seq_len}; no wraparound support")
        B = z.shape[0]
        qkv = F.linear(z, blk.attn.qkv_weight)
        q_p, k_p, v_p = torch.split(qkv, (S.N, S.KV, S.KV), dim=-1)
        q = q_p.view(B, 1, S.QH, S.HD)
        k_rep = k_p.view(B, 1, S.KVH, S.HD).repeat_interleave(S.G, dim=2)
        cos = self._cos[pos].view(1, 1, 1, S.HD)
        sin = self._sin[pos].view(1, 1, 1, S.HD)
        q = ops.apply_rope(q, cos, sin)
        k_rep = ops.apply_rope(k_rep, cos, sin)
        k_new = k_rep.view(B, 1, S.KVH, S.G, S.HD)[:, :, :, 0, :]
        v_new = v_p.view(B, 1, S.KVH, S.HD)
        if cache.k is None:
            cache.k = z.new_zeros(B, S.seq_len, S.KVH, S.HD)
            cache.v = z.new_zeros(B, S.seq_len, S.KVH, S.HD)
        cache.k[:, cache.cache_len] = k_new[:, 0]
        cache.v[:, cache.cache_len] = v_new[:, 0]
        n = cache.cache_len + 1
        kg = cache.k[:, :n].repeat_interleave(S.G, dim=2).transpose(1, 2)   # [B,QH,n,HD]
        vg = cache.v[:, :n].repeat_interleave(S.G, dim=2).transpose(1, 2)
        qg = q.transpose(1, 2)                                               # [B,QH,1,HD]
        scores = torch.matmul(qg, kg.transpose(-1, -2).contiguous()) / math.sqrt(S.HD)
        a = torch.softmax(scores.float(), dim=-1)
        c = torch.matmul(a, vg).transpose(1, 2).contiguous()                 # [B,1,QH,HD]
        kctx = torch.matmul(a, kg).transpose(1, 2).contiguous()
        out = blk.attn.o(c.reshape(B, 1, S.N))
        return out, q, kctx, c

    def ffn(self, blk: _Block, u, q_h, k_ctx_h, c_h, d_h, phase_trace, p_in):
        """ParaplexFFN.forward, unfused CPU branch (loomformer.py:2818-2893)."""
        S = self.S
        f = blk.ffn
        wx = F.linear(u, f.w1_real.weight)
        if p_in is None:
            p_real = wx + f.w1_real.bias                         # tria.py:1294-1296
        else:
            alpha = f.identity_gate.alpha_max * torch.tanh(f.identity_gate.raw_alpha)
            p_real = wx * (1.0 + alpha * p_in) + f.w1_real.bias  # tria.py:1297-1299
        key = (id(f.w1_imag), f.w1_imag._version)
        if getattr(f, "_dense_key", None) != key:       # scatter once per weight version
            f._dense_w = ops.dense_imag_weight(f.w1_imag, S.N, S.QH, S.HD, S.sectors)
            f._dense_key = key
        B = u.shape[0]
        r_all = torch.cat([q_h.reshape(B, -1, S.N), k_ctx_h.reshape(B, -1, S.N),
                           c_h.reshape(B, -1, S.N), u, d_h.reshape(B, -1, S.N)], dim=-1)
        beta_lin = F.linear(r_all, f._dense_w)                   # loomformer.py:2771-2777
        # amplitude source: p_real itself, or gate_proj(u) (loomformer.py:2849)
        gate_src = p_real if f.gate_proj is None else f.gate_proj(u)
        act, s, next_trace = ops.paraplex_pointwise(
            p_real, gate_src, beta_lin, f.w1_imag_bias, phase_trace, f.w1_imag_trace, None, S.powlu_m)
        return f.w2(act), next_trace, (p_real, s, act)

    def tria_agg_fn(self, carry: torch.Tensor) -> torch.Tensor:
        """TriaAggregator.forward (tria.py:1436-1441)."""
        rd = self.tria_agg.reader
        score_w = ops.make_score_w(rd.key_proj.weight, self.tria_agg.pool.query,
                                   F.softplus(self.tria_agg.pool.logit_scale_raw))
        pooled, _ = ops.slot_attention_pool(carry, score_w)
        return self.tria_agg.up(rd.proj(pooled))

    def final_ca_step(self, a_t, b_t, cache: CACache, fire: torch.Tensor):
        """TriaFinalCrossAttention.step (tria.py:1560-1595)."""
        S = self.S
        ca = self.tria_final_ca
        B, _, D = a_t.shape
        if cache.k is None:
            cache.k = a_t.new_zeros(B, S.seq_len, D)
            cache.v = a_t.new_zeros(B, S.seq_len, D)
            cache.valid = torch.zeros(B, S.seq_len, dtype=torch.bool)
        if bool(fire.any()):
            cache.k[:, cache.cache_len] = ca.w_qk(a_t)[:, 0]
            cache.v[:, cache.cache_len] = ca.w_v(a_t)[:, 0]
            cache.valid[:, cache.cache_len] = fire
            cache.cache_len += 1
        if cache.cache_len == 0:
            return b_t
        n = cache.cache_len
        q = ca.w_qk(b_t)
        out = ops.final_ca_sparse(q, cache.k[:, :n], cache.v[:, :n], cache.valid[:, None, :n], ca.scale)
        gamma = ca.gamma_max * torch.tanh(ca.raw_gamma)
        return b_t + gamma * out

    # ---- Model.step --------------------------------------------------------

    @torch.no_grad()
    def step(self, idx_t: torch.Tensor, pos: int, state: Optional[StepState]):
        """One decode token for a batch (loomformer.py:3951-4091)."""
        S = self.S
        is_bos = pos == 0
        if state is None or is_bos:
            state = StepState(caches=[LayerCache() for _ in range(S.L)])
        B = idx_t.shape[0]
        h = self.emb(idx_t).view(B, 1, S.N)
        n_hist = 2 * S.L
        k0, v0 = self.kv_project(h)
        hist_k = h.new_zeros(B, 1, n_hist, S.QH, S.HD)
        hist_v = h.new_zeros(B, 1, n_hist, S.QH, S.HD)
        hist_k[:, :, 0] = k0
        hist_v[:, :, 0] = v0
        sub = 0
        carry = None
        p = None
        ts = state.temporal
        pending = torch.zeros(B, dtype=torch.bool) if ts.pending is None else ts.pending
        seed_valid = pending & (not is_bos)
        seed = ts.carry
        for bi, blk in enumerate(self.blocks):
            cache = state.caches[bi]
            last = bi == S.L - 1
            attn_out, q_h, kctx_h, c_h = self.attn_step(blk, h, pos, cache)
            skip, _ = self.depth_read(sub, hist_k[:, :, :sub + 1], hist_v[:, :, :sub + 1])
            if self.step_branch_cap is not None:
                skip = capped_rms(skip, self.step_branch_cap)
                attn_out = capped_rms(attn_out, self.step_branch_cap)
            h = F.layer_norm(skip + attn_out, (S.N,), blk.ln_attn.weight, blk.ln_attn.bias, 1e-5)
            k_i, v_i = self.kv_project(h)
            sub += 1
            hist_k[:, :, sub] = k_i
            hist_v[:, :, sub] = v_i
            skip, d_h = self.depth_read(sub, hist_k[:, :, :sub + 1], hist_v[:, :, :sub + 1])
            ffn_out, next_trace, (r, i, o) = self.ffn(blk, h, q_h, kctx_h, c_h, d_h,
                                                      cache.phase_trace, p)
            w = torch.softmax(blk.ffn.gate_selector.logits, dim=0)
            carry, p = tria_layer_op(bi, last, r, i, o, carry, seed, seed_valid, w, S.tria_alpha)
            if self.step_branch_cap is not None:
                skip = capped_rms(skip, self.step_branch_cap)
                ffn_out = capped_rms(ffn_out, self.step_branch_cap)
            h = F.layer_norm(skip + ffn_out, (S.N,), blk.ln_ffn.weight, blk.ln_ffn.bias, 1e-5)
            if not last:
                k_i, v_i = self.kv_project(h)
                sub += 1
                hist_k[:, :, sub] = k_i
                hist_v[:, :, sub] = v_i
            cache.phase_trace = next_trace
            cache.cache_len += 1
        if S.carry_token_id is not None:
            explicit = idx_t.view(-1).eq(int(S.carry_token_id))
        else:
            explicit = torch.zeros(B, dtype=torch.bool)
        doc, fire = tria_temporal_token(carry[:, 0], ts, pending, pos, explicit, S.seq_len,
                                        S.window, S.polarm_beta)
        a_t = self.tria_agg_fn(doc.unsqueeze(1))
        h = self.final_ca_step(a_t, h, state.ca, fire)
        state.temporal = TemporalState(carry=doc, pending=fire)
        return self.head_in(h[:, -1, :]), state

    def head_in(self, x: torch.Tensor) -> torch.Tensor:
        """Model._head_in (loomformer.py:3527-3529): the optional final RMSNorm, then the head."""
        if self.ln_final is not None:
            x = rms_norm(x, self.ln_final.weight)
        return self.head(x)


def tria_layer_op(bi: int, last: bool, r, i, o, carry, seed, seed_valid, w, alpha: float):
    """The Tria depth op of block bi in Model.step (loomformer.py:4012-4040,
    same choice as _block_core :3588-3617): axis bi % 3; the first block is
    seeded when a seed is held, the last block is ungated.  Returns (carry, p)."""
    axis = bi % 3
    if bi == 0 and seed is not None:
        if last:
            return ops.tria_init_seed(r, i, o, seed, seed_valid, alpha, axis), None
        return ops.tria_init_seed_and_gate(r, i, o, seed, seed_valid, w, alpha, axis)
    if last:
        return (ops.tria_init(r, i, o, alpha, axis) if carry is None
                else ops.tria_step(r, i, o, carry, alpha, axis)), None
    return (ops.tria_init_and_gate(r, i, o, w, alpha, axis) if carry is None
            else ops.tria_step_and_gate(r, i, o, carry, w, alpha, axis))


def tria_temporal_token(depth_t, ts: TemporalState, pending, pos: int, explicit,
                        seq_len: int, window: int, polarm_beta: float):
    """Temporal recurrence, fire and PolARM of one decode token
    (loomformer.py:4056-4078): restart from the token's depth carry after a
    fire or at position 0, else N(D_t @ state); hard fire when
    (pos + 1) % window == 0 and pos + 1 < seq_len, or on an explicit <CARRY>
    token; PolARM where fired.  Returns (doc [B,H,3,3], fire [B])."""
    reset_now = pending | (pos == 0)
    if ts.carry is None:
        doc = depth_t
    else:
        cont = ops.local_normalize(torch.matmul(depth_t, ts.carry))
        doc = torch.where(reset_now[:, None, None, None], depth_t, cont)
    hard_fire = (pos + 1 < seq_len) and ((pos + 1) % window == 0)
    fire = explicit | hard_fire
    if hard_fire or bool(explicit.any()):
        doc = torch.where(fire[:, None, None, None], ops.polarm(doc, polarm_beta), doc)
    return doc, fire


@torch.no_grad()
def greedy_decode(model: OracleModel, prompt: torch.Tensor, n_new: int):
    """infer() for a batch of equal-length prompts (loomformer.py:5290-5311).

    Returns (generated ids [B, n_new], logits of every step [B, P+n_new, V]).
    """
    B, P = prompt.shape
    state = None
    all_logits = []
    logits = None
    for pos in range(P):
        logits, state = model.step(prompt[:, pos], pos, state)
        all_logits.append(logits)
    out = []
    for i in range(n_new):
        nxt = torch.argmax(logits, dim=-1)
        out.append(nxt)
        logits, state = model.step(nxt, P + i, state)
        all_logits.append(logits)
    return torch.stack(out, dim=1), torch.stack(all_logits, dim=1)
