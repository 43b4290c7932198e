"""Model shape for the decode engine.

``ModelConfig.from_dict`` applies the shape derivation of the reference's
``apply_config`` (loomformer.py:904-1120) to a config mapping with the
reference's YAML keys; ``NANO`` and ``NANO_CHK`` carry the model keys of
cfg/nano.yaml and cfg/nano_chk.yaml.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, replace
from typing import Optional

# model keys of cfg/nano.yaml (the CPU-reference config)
NANO = dict(
    vocab=8192, seq_len=1024, model_dim=768, n_q_heads=8, head_dim=96, n_kv_heads=None,
    gqa_group_size=4, hidden=None, hidden_mult=4.0, layers=10, phase_sectors="head",
    residual_init="beta", activation="pvpowlu", powlu_m=3.0, tied_embeddings=False,
    rope_theta=10000.0, rope_original_seq_len=1024, rope_factor=4.0, rope_beta_fast=32.0,
    rope_beta_slow=1.0, rope_attention_factor=None, tria_carry_enabled=True,
    tria_temporal_enabled=True, tria_temporal_window=128, tria_carrier_alpha=0.025,
    tria_gamma_max=0.8, tria_raw_gamma_init=0.25,
)
# cfg/nano_chk.yaml: the 113M-checkpoint shape (vocab 4096, alpha 0.0375)
NANO_CHK = dict(NANO, vocab=4096, tria_carrier_alpha=0.0375)


@dataclass(frozen=True)
class ModelConfig:
    V: int
    N: int
    QH: int
    HD: int
    KVH: int
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
    # model variants a checkpoint can carry (Config, loomformer.py:272-274, :358, :366)
    gate_proj: bool = False              # paraplex_gate_proj: amp = softplus(gate_proj(u))
    depth_qkv_rms: bool = False          # depth_attn_qkv_rms: fixed-RMS depth q/k/v
    residual_rms_cap: Optional[float] = None   # residual_branch_rms_cap
    final_norm: bool = False             # RMSNorm before the head
    depth_readout: str = "shared"        # depth_attn_readout: shared | per-sublayer

    @property
    def G(self) -> int:
        return self.QH // self.KVH

    @property
    def KV(self) -> int:
        return self.KVH * self.HD

    @property
    def Hq(self) -> int:
        return self.H // self.QH

    @property
    def imag_in(self) -> int:
        return self.N + 4 * self.HD if self.sectors == "head" else 4 * self.N + self.HD

    @property
    def fanin_gain(self) -> float:
        return 0.88                      # FANIN_GAIN (loomformer.py:808)

    @property
    def deepnorm_beta(self) -> float:
        return (8.0 * max(1, self.L)) ** -0.25

    def with_seq_len(self, seq_len: int) -> "ModelConfig":
        """Override seq_len (the decode length limit); numerics are unchanged
        except the hard-fire cut-off at pos + 1 == seq_len."""
        return replace(self, seq_len=int(seq_len))

    @staticmethod
    def from_dict(d: dict) -> "ModelConfig":
        QH = int(d.get("n_q_heads", 6))
        model_dim = d.get("model_dim", 12)
        if d.get("head_dim") is not None:
            HD = int(d["head_dim"])
            N = QH * HD
            if model_dim is not None and int(model_dim) != N:
                raise ValueError(f"inconsistent shape: model_dim={model_dim} but n_q_heads*head_dim={N}")
        elif model_dim is None:
            HD, N = 32, QH * 32
        else:
            N = int(model_dim)
            if N % QH:
                raise ValueError("model_dim must be divisible by n_q_heads, or set head_dim")
            HD = N // QH
        gs, nkv = d.get("gqa_group_size"), d.get("n_kv_heads", 3)
        if gs is not None and nkv is not None:
            KVH = int(nkv)
            if KVH * int(gs) != QH:
                raise ValueError("inconsistent GQA")
        elif gs is not None:
            if QH % int(gs):
                raise ValueError("gqa_group_size must divide n_q_heads")
            KVH = QH // int(gs)
        elif nkv is not None:
            KVH = int(nkv)
        else:
            KVH = QH // (4 if QH % 4 == 0 else (2 if QH % 2 == 0 else 1))
        if d.get("hidden") is None:
            mult = 4.0 if d.get("hidden_mult") is None else float(d["hidden_mult"])
            raw = max(QH, int(round(N * mult)))
            H = ((raw + QH - 1) // QH) * QH
        else:
            H = int(d["hidden"])
        if H % QH:
            raise ValueError("hidden must be divisible by n_q_heads")
        seq_len = int(d.get("seq_len", 128))
        ro = d.get("rope_original_seq_len")
        alpha = float(d.get("tria_carrier_alpha", 0.05))
        if not math.isfinite(alpha) or alpha <= 0:
            raise ValueError(f"tria_carrier_alpha must be finite and > 0, got {alpha}")
        beta = float(d.get("tria_polarm_beta", 0.1))
        if not math.isfinite(beta) or not 0.0 <= beta < 1.0:
            raise ValueError(f"tria_polarm_beta must be finite and in [0, 1), got {beta}")
        if not (d.get("tria_carry_enabled", False) and d.get("tria_temporal_enabled", True)):
            raise ValueError("the decode engine implements the tria-carry + temporal model")
        act = str(d.get("activation", "gelu")).lower()
        if act != "pvpowlu":
            raise ValueError(f"the fused Paraplex path needs activation=pvpowlu, got {act}")
        # the variant flags, validated as apply_config does (loomformer.py:1034-1044)
        readout = str(d.get("depth_attn_readout", "shared") or "shared").lower()
        if readout not in ("shared", "per-sublayer"):
            raise ValueError(f"depth_attn_readout must be 'shared' or 'per-sublayer', got {readout!r}")
        cap = d.get("residual_branch_rms_cap")
        if cap is not None:
            cap = float(cap)
            if not math.isfinite(cap) or cap <= 0:
                raise ValueError("residual_branch_rms_cap must be positive or null")
        variants = dict(gate_proj=bool(d.get("paraplex_gate_proj", False)),
                        depth_qkv_rms=bool(d.get("depth_attn_qkv_rms", False)),
                        residual_rms_cap=cap, final_norm=bool(d.get("final_norm", False)),
                        depth_readout=readout)
        return ModelConfig(
            V=int(d.get("vocab", 256)), N=N, QH=QH, HD=HD, KVH=KVH, H=H, L=int(d.get("layers", 3)),
            seq_len=seq_len, sectors=str(d.get("phase_sectors", "head")).lower(),
            residual_init=str(d.get("residual_init", "beta")).lower(),
            powlu_m=float(d.get("powlu_m", 3.0) or 3.0), tria_alpha=alpha, polarm_beta=beta,
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
            **variants,
        )
