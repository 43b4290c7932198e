"""Seeded random initialisation with the reference's RNG stream, and rotary tables.

``init_state_dict(cfg, seed)`` returns CPU fp32 tensors keyed like the
reference's ``Model(cfg).state_dict()`` and equal to it bit for bit after
``torch.manual_seed(seed)``: every draw happens in the reference's
module-construction order (Model.__init__, loomformer.py:3477-3531; the
nn.Linear/nn.Embedding default draws happen before each module's own
reset_parameters overrides them, e.g. ParaplexFFN.__init__ :2667-2716).
"""
from __future__ import annotations

import math
from collections import OrderedDict
from typing import Dict, Tuple

import torch
import torch.nn as nn

from .config import ModelConfig

FANIN_GAIN = 0.88


def _fanin(n: int) -> float:
    return FANIN_GAIN / math.sqrt(float(n))


def _linear(out_f: int, in_f: int, bias: bool = True):
    """Draw exactly what nn.Linear's constructor draws (kaiming-uniform weight, uniform bias)."""
    m = nn.Linear(in_f, out_f, bias=bias)
    return m.weight.data, (m.bias.data if bias else None)


@torch.no_grad()
def init_state_dict(cfg: ModelConfig, seed: int) -> Dict[str, torch.Tensor]:
    torch.manual_seed(seed)
    N, H, L, KV = cfg.N, cfg.H, cfg.L, cfg.KV
    rbeta = cfg.deepnorm_beta if cfg.residual_init == "beta" else 1.0
    sd: Dict[str, torch.Tensor] = OrderedDict()
    emb = nn.Embedding(cfg.V, N).weight.data                 # N(0,1) draw, re-drawn below
    for bi in range(L):
        p = f"blocks.{bi}."
        sd[p + "ln_attn.weight"], sd[p + "ln_attn.bias"] = torch.ones(N), torch.zeros(N)
        qkv = torch.empty(N + 2 * KV, N)
        o_w, _ = _linear(N, N, bias=False)
        nn.init.normal_(qkv[:N], 0.0, _fanin(N))
        nn.init.normal_(qkv[N:N + KV], 0.0, _fanin(N))
        nn.init.normal_(qkv[N + KV:], 0.0, _fanin(N) * rbeta)
        nn.init.normal_(o_w, 0.0, _fanin(N) * rbeta)
        sd[p + "attn.qkv_weight"], sd[p + "attn.o.weight"] = qkv, o_w
        sd[p + "ln_ffn.weight"], sd[p + "ln_ffn.bias"] = torch.ones(N), torch.zeros(N)
        w1r, b1r = _linear(H, N)
        w1i = torch.empty(H, cfg.imag_in)
        w2, b2 = _linear(N, H)
        if cfg.gate_proj:                                # ParaplexFFN.gate_proj (:2704-2707)
            gpw, gpb = _linear(H, N)
        nn.init.normal_(w1r, 0.0, _fanin(N))
        b1r.zero_()
        nn.init.normal_(w1i, 0.0, _fanin(cfg.imag_in))
        nn.init.normal_(w2, 0.0, _fanin(H) * rbeta)
        b2.zero_()
        sd[p + "ffn.w1_real.weight"], sd[p + "ffn.w1_real.bias"] = w1r, b1r
        sd[p + "ffn.w1_imag"] = w1i
        sd[p + "ffn.w1_imag_trace"], sd[p + "ffn.w1_imag_bias"] = torch.zeros(H), torch.zeros(H)
        sd[p + "ffn.w2.weight"], sd[p + "ffn.w2.bias"] = w2, b2
        sd[p + "ffn.beta_anchor"] = torch.tensor(1.0)
        sd[p + "ffn.gate_selector.logits"] = torch.zeros(9)
        sd[p + "ffn.identity_gate.raw_alpha"] = torch.zeros(())
        if cfg.gate_proj:                                # init_linear_fanin (:2717-2718)
            nn.init.normal_(gpw, 0.0, _fanin(N))
            gpb.zero_()
            sd[p + "ffn.gate_proj.weight"], sd[p + "ffn.gate_proj.bias"] = gpw, gpb
    kvw = torch.empty(2 * N, N)
    if cfg.depth_readout == "per-sublayer":              # DepthAttn.__init__ (:3373-3378)
        wo = torch.empty(2 * L, N, N)
    else:
        wo, _ = _linear(N, N, bias=False)
    qp = torch.empty(2 * L, cfg.QH, cfg.HD)
    nn.init.normal_(kvw[:N], 0.0, _fanin(N))
    nn.init.normal_(kvw[N:], 0.0, _fanin(N) * rbeta)
    nn.init.normal_(wo, 0.0, _fanin(N) * rbeta)
    nn.init.normal_(qp, 0.0, _fanin(cfg.HD))
    sd["depth_attn.kv_weight"] = kvw
    sd["depth_attn.w_o_weight" if cfg.depth_readout == "per-sublayer" else "depth_attn.w_o.weight"] = wo
    sd["depth_attn.q_params"] = qp
    head, _ = _linear(cfg.V, N, bias=False)
    proj_w, proj_b = _linear(32, 9)
    key_w, _ = _linear(32, 9, bias=False)
    key_w.normal_(mean=0.0, std=1.5)
    up_w, up_b = _linear(N, 32)
    wqk, _ = _linear(N, N, bias=False)
    wv, _ = _linear(N, N, bias=False)
    nn.init.normal_(emb, 0.0, _fanin(N))
    sd["emb.weight"] = emb
    sd["head.weight"] = emb if cfg.tied else head
    if cfg.final_norm:                                   # Model.ln_final (:3490)
        sd["ln_final.weight"] = torch.ones(N)
    sd["tria_agg.reader.proj.weight"], sd["tria_agg.reader.proj.bias"] = proj_w, proj_b
    sd["tria_agg.reader.key_proj.weight"] = key_w
    sd["tria_agg.pool.query"] = torch.zeros(32)
    sd["tria_agg.pool.logit_scale_raw"] = torch.tensor(math.log(math.expm1(1.0)))
    sd["tria_agg.up.weight"], sd["tria_agg.up.bias"] = up_w, up_b
    sd["tria_final_ca.w_qk.weight"], sd["tria_final_ca.w_v.weight"] = wqk, wv
    sd["tria_final_ca.raw_gamma"] = torch.tensor(float(cfg.raw_gamma_init))
    return sd


def state_keys(cfg: ModelConfig):
    """The state_dict keys of the reference's Model for `cfg` (what
    init_state_dict returns and a checkpoint of that config holds)."""
    keys = ["emb.weight"]
    for bi in range(cfg.L):
        p = f"blocks.{bi}."
        keys += [p + k for k in (
            "ln_attn.weight", "ln_attn.bias", "attn.qkv_weight", "attn.o.weight", "ln_ffn.weight",
            "ln_ffn.bias", "ffn.w1_real.weight", "ffn.w1_real.bias", "ffn.w1_imag",
            "ffn.w1_imag_trace", "ffn.w1_imag_bias", "ffn.w2.weight", "ffn.w2.bias",
            "ffn.beta_anchor", "ffn.gate_selector.logits", "ffn.identity_gate.raw_alpha")]
        if cfg.gate_proj:
            keys += [p + "ffn.gate_proj.weight", p + "ffn.gate_proj.bias"]
    keys += ["depth_attn.kv_weight", "depth_attn.q_params",
             "depth_attn.w_o_weight" if cfg.depth_readout == "per-sublayer" else "depth_attn.w_o.weight",
             "head.weight"]
    if cfg.final_norm:
        keys.append("ln_final.weight")
    keys += ["tria_agg.reader.proj.weight", "tria_agg.reader.proj.bias",
             "tria_agg.reader.key_proj.weight", "tria_agg.pool.query", "tria_agg.pool.logit_scale_raw",
             "tria_agg.up.weight", "tria_agg.up.bias", "tria_final_ca.w_qk.weight",
             "tria_final_ca.w_v.weight", "tria_final_ca.raw_gamma"]
    return keys


def rope_tables(cfg: ModelConfig, length: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """YaRN cos/sin caches [length, HD] fp32, scaled by the attention factor
    (loomformer.py:2899-2971), computed on the CPU in the reference's op order."""
    dim = cfg.HD
    pos_freqs = cfg.rope_theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim)
    extra = 1.0 / pos_freqs
    inter = 1.0 / (cfg.rope_factor * pos_freqs)

    def corr(nrot):
        return (dim * math.log(cfg.rope_original / (nrot * 2.0 * math.pi))) / (2.0 * math.log(cfg.rope_theta))

    low = max(math.floor(corr(cfg.rope_beta_fast)), 0)
    high = min(math.ceil(corr(cfg.rope_beta_slow)), dim - 1)
    if low == high:
        high += 0.001
    ramp = torch.clamp((torch.arange(dim // 2, dtype=torch.float32) - low) / (high - low), 0.0, 1.0)
    mask = 1.0 - ramp
    inv_freq = inter * (1.0 - mask) + extra * mask
    att = cfg.rope_attention_factor
    if att is None:
        att = 1.0 if cfg.rope_factor <= 1.0 else 0.1 * math.log(cfg.rope_factor) + 1.0
    t = torch.arange(length, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().mul(att), emb.sin().mul(att)
