#!/usr/bin/env python3
"""Write the golden fixtures under tests/golden/ by running the REFERENCE.

Run only in the build container, where the reference checkout exists:

    python tests/golden/make_golden.py --ref /root/reference

The reference is imported read-only (no bytecode is written into it) on the
CPU with every CUDA path disabled, so each value below comes from the
reference's own PyTorch code.  The files written are data only (inputs and
expected outputs); nothing of the reference's source is stored.

Fixtures:
  init_sha256.json   per-tensor sha256 of Model(cfg).state_dict() for
                     nano.yaml seed 0, nano_chk.yaml seed 2, the tiny config
                     and the tiny config with every variant flag
  tiny_decode.npz    tiny config: perturbed weights, prompts, per-step logits and
                     greedy ids of Model.step (with and without a <CARRY> id)
  variants_decode.npz  the same for the tiny config with every model variant
                     flag set (gate_proj, qkv_rms, branch cap, final_norm,
                     per-sublayer depth readout)
  nano_cpu_ref.npz   nano.yaml seed 0, B=1, 128-token prompt + 64 greedy ids,
                     per-step top-5 logits
  ops.npz            per-op input/output vectors at small shapes
  chunked_keys.npz   Model._forward_chunked's Tria inputs (per-layer r, i, o),
                     document keys and fire mask on the tiny config with
                     explicit <CARRY> fires and mid-row document starts
  configs.json       the model-shape keys of cfg/nano.yaml and cfg/nano_chk.yaml
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

TINY = dict(
    vocab=97, seq_len=64, n_q_heads=4, head_dim=8, model_dim=None, n_kv_heads=None,
    gqa_group_size=2, hidden=None, hidden_mult=4.0, layers=4, phase_sectors="head",
    residual_init="beta", activation="pvpowlu", powlu_m=3.0, phase_grad_mode="floor",
    tied_embeddings=False, rope_original_seq_len=16, rope_factor=4.0,
    tria_carry_enabled=True, tria_temporal_enabled=True, tria_temporal_auto=False,
    tria_temporal_window=8, tria_carrier_alpha=0.05, tria_polarm_beta=0.1,
    tria_gamma_max=0.8, tria_raw_gamma_init=0.25, use_cuda_tria=False,
    use_cuda_beta_space=False, use_cuda_phase_sin=False, use_cuda_pvpowlu=False,
    use_cuda_depth_attn=False, amp_dtype="fp32", device="cpu",
)

# the tiny config with every math-changing model variant a checkpoint can carry
# (Config, loomformer.py:272-274, :358, :366); the branch cap is small enough
# to bind wherever it is applied
VARIANTS = dict(paraplex_gate_proj=True, depth_attn_qkv_rms=True, residual_branch_rms_cap=0.05,
                final_norm=True, depth_attn_readout="per-sublayer")

NO_CUDA = dict(use_cuda_tria=False, use_cuda_beta_space=False, use_cuda_phase_sin=False,
               use_cuda_pvpowlu=False, use_cuda_depth_attn=False, device="cpu", amp_dtype="fp32")


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().contiguous().cpu().numpy().tobytes()).hexdigest()


def load_ref(ref: str):
    sys.dont_write_bytecode = True
    sys.path.insert(0, ref)
    import loomformer as lf   # noqa: E402
    import tria as tr         # noqa: E402
    return lf, tr


def make_cfg(lf, yaml_path=None, **over):
    if yaml_path is not None:
        import yaml
        with open(yaml_path, encoding="utf-8") as f:
            d = yaml.safe_load(f) or {}
    else:
        d = {}
    d.update(over)
    cfg = lf.Config.from_dict(d)
    lf.apply_config(cfg)
    return cfg


def state_sha(model) -> dict:
    return {k: {"shape": list(v.shape), "sha256": sha(v)} for k, v in model.state_dict().items()}


PERTURB = ("identity_gate.raw_alpha", "w1_imag_trace", "w1_imag_bias", "w1_real.bias",
           "w2.bias", "gate_selector.logits", "pool.query", "ln_attn.weight", "ln_attn.bias",
           "ln_ffn.weight", "ln_ffn.bias", "up.bias", "proj.bias", "raw_gamma",
           "gate_proj.bias", "ln_final.weight")


def perturb(model, seed: int) -> None:
    """Give the zero/one-initialised parameters random values so inert paths run."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if any(name.endswith(s) for s in PERTURB):
                p.add_(torch.randn(p.shape, generator=g) * 0.5)


def run_decode(lf, model, prompt: torch.Tensor, n_new: int):
    B, P = prompt.shape
    states = None
    logits_all = []
    logits = None
    for pos in range(P):
        logits, states = model.step(prompt[:, pos], pos, states)
        logits_all.append(logits)
    out = []
    for i in range(n_new):
        nxt = torch.argmax(logits, dim=-1)
        out.append(nxt)
        logits, states = model.step(nxt, P + i, states)
        logits_all.append(logits)
    return torch.stack(out, 1), torch.stack(logits_all, 1)


def golden_init(lf, ref: str) -> dict:
    out = {}
    cfg = make_cfg(lf, os.path.join(ref, "cfg/nano.yaml"), **NO_CUDA)
    torch.manual_seed(0)
    out["nano_seed0"] = state_sha(lf.Model(cfg))
    cfg = make_cfg(lf, os.path.join(ref, "cfg/nano_chk.yaml"), **NO_CUDA)
    torch.manual_seed(2)
    out["nano_chk_seed2"] = state_sha(lf.Model(cfg))
    cfg = make_cfg(lf, None, **TINY)
    torch.manual_seed(0)
    out["tiny_seed0"] = state_sha(lf.Model(cfg))
    cfg = make_cfg(lf, None, **dict(TINY, **VARIANTS))
    torch.manual_seed(0)
    out["tiny_variants_seed0"] = state_sha(lf.Model(cfg))
    make_cfg(lf, None, **TINY)
    return out


def golden_variants(lf) -> dict:
    """Model.step of the tiny config with every variant flag set, perturbed
    weights, with and without <CARRY> ids."""
    cfg = make_cfg(lf, None, **dict(TINY, **VARIANTS))
    torch.manual_seed(0)
    model = lf.Model(cfg).eval()
    perturb(model, 321)
    arrays = {f"w::{k}": v.detach().numpy() for k, v in model.state_dict().items()}
    g = torch.Generator().manual_seed(17)
    prompt = torch.randint(0, TINY["vocab"], (3, 20), generator=g)
    lf.CARRY_TOKEN_ID = None
    ids, logits = run_decode(lf, model, prompt, 12)
    arrays["prompt"], arrays["greedy"], arrays["logits"] = prompt.numpy(), ids.numpy(), logits.numpy()
    prompt2 = prompt.clone()
    prompt2[0, 6] = 5
    prompt2[1, 2] = 5
    prompt2[2, 11] = 5
    lf.CARRY_TOKEN_ID = 5
    ids2, logits2 = run_decode(lf, model, prompt2, 12)
    lf.CARRY_TOKEN_ID = None
    arrays["prompt_carry"], arrays["greedy_carry"] = prompt2.numpy(), ids2.numpy()
    arrays["logits_carry"] = logits2.numpy()
    make_cfg(lf, None, **TINY)
    return arrays


def golden_tiny_decode(lf) -> dict:
    cfg = make_cfg(lf, None, **TINY)
    torch.manual_seed(0)
    model = lf.Model(cfg).eval()
    perturb(model, 123)
    arrays = {f"w::{k}": v.detach().numpy() for k, v in model.state_dict().items()}
    g = torch.Generator().manual_seed(7)
    prompt = torch.randint(0, TINY["vocab"], (3, 20), generator=g)
    lf.CARRY_TOKEN_ID = None
    ids, logits = run_decode(lf, model, prompt, 12)
    arrays["prompt"] = prompt.numpy()
    arrays["greedy"] = ids.numpy()
    arrays["logits"] = logits.numpy()
    # Explicit <CARRY> fires, different per batch row (exercises per-row seeds).
    prompt2 = prompt.clone()
    prompt2[0, 3] = 5
    prompt2[1, 10] = 5
    prompt2[2, 4] = 5
    prompt2[2, 5] = 5
    lf.CARRY_TOKEN_ID = 5
    ids2, logits2 = run_decode(lf, model, prompt2, 12)
    lf.CARRY_TOKEN_ID = None
    arrays["prompt_carry"] = prompt2.numpy()
    arrays["greedy_carry"] = ids2.numpy()
    arrays["logits_carry"] = logits2.numpy()
    return arrays


def golden_chunked(lf, tr) -> dict:
    """Model._forward_chunked (loomformer.py:3788-3883) on the tiny config with
    explicit <CARRY> fires: the per-layer r, i, o the Tria ops consumed
    (captured at tria.record_depth_replay, which _block_core calls with each
    layer's summaries, :3586), the document keys, the fire mask and the
    document resets.  Rows differ: a fire at T-1 (the tail chunk becomes a
    boundary), a document restart after a grid position (its hard fire is
    invalid), consecutive fires, a fire on a grid position and a restart right
    after an explicit fire (valid fire, no seed)."""
    cfg = make_cfg(lf, None, **TINY)
    torch.manual_seed(0)
    model = lf.Model(cfg).eval()
    perturb(model, 123)
    B, T, carry = 3, 30, 5
    g = torch.Generator().manual_seed(21)
    idx = torch.randint(0, TINY["vocab"] - 1, (B, T), generator=g)
    idx[idx >= carry] += 1                       # no accidental <CARRY>
    for b, t in ((0, 3), (0, 29), (1, 10), (2, 4), (2, 5), (2, 15)):
        idx[b, t] = carry
    pos = torch.arange(T).repeat(B, 1)
    pos[1, 16:] = torch.arange(T - 16)           # row 1: a document starts at 16
    pos[2, 6:] = torch.arange(T - 6)             # row 2: a document starts at 6
    rec = []
    orig = tr.record_depth_replay
    tr.record_depth_replay = lambda r, i, o, axis: rec.append((r.detach().clone(), i.detach().clone(),
                                                              o.detach().clone(), axis))
    lf.CARRY_TOKEN_ID = carry
    model.capture_tria_depth_carry = True
    try:
        with torch.no_grad():
            model(idx, position_ids=pos)
    finally:
        tr.record_depth_replay = orig
        lf.CARRY_TOKEN_ID = None
    L = len(model.blocks)
    assert len(rec) % L == 0
    per_layer = [[rec[c * L + l] for c in range(len(rec) // L)] for l in range(L)]
    for l in range(L):
        assert all(x[3] == l % 3 for x in per_layer[l])
    stack = lambda k: torch.stack([torch.cat([x[k] for x in per_layer[l]], dim=1) for l in range(L)])
    return {"r": stack(0).numpy(), "i": stack(1).numpy(), "o": stack(2).numpy(),
            "idx": idx.numpy(), "position_ids": pos.numpy(), "reset": pos.eq(0).numpy(),
            "explicit_fire": idx.eq(carry).numpy(), "fire_mask": model.last_tria_fire_mask.numpy(),
            "keys": model.last_tria_document_carry.numpy(),
            "window": np.array(TINY["tria_temporal_window"]), "alpha": np.array(TINY["tria_carrier_alpha"]),
            "polarm_beta": np.array(TINY["tria_polarm_beta"])}


def golden_nano_cpu(lf, ref: str) -> dict:
    cfg = make_cfg(lf, os.path.join(ref, "cfg/nano.yaml"), **NO_CUDA)
    torch.manual_seed(0)
    model = lf.Model(cfg).eval()
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, int(cfg.vocab), (1, 128), generator=g)
    ids, logits = run_decode(lf, model, prompt, 64)
    top = torch.topk(logits, 5, dim=-1)
    return {"prompt": prompt.numpy(), "greedy": ids.numpy(),
            "top5_values": top.values.numpy(), "top5_indices": top.indices.numpy()}


def golden_ops(lf, tr) -> dict:
    cfg = make_cfg(lf, None, **TINY)
    g = torch.Generator().manual_seed(11)
    rn = lambda *s, scale=1.0: torch.randn(*s, generator=g) * scale
    A = {}
    N, QH, HD, H = lf.N, lf.N_Q_HEADS, lf.HEAD_DIM, lf.HIDDEN
    B, T = 2, 5
    # compact W_imag indices
    A["imag_idx_head"] = lf.make_w1_imag_live_flat_indices().numpy()
    lf.PHASE_SECTORS = "open"
    lf.IMAG_IN = 4 * N + HD
    A["imag_idx_open"] = lf.make_w1_imag_live_flat_indices().numpy()
    lf.PHASE_SECTORS = "head"
    lf.IMAG_IN = N + 4 * HD
    # ParaplexFFN (perturbed params), with and without trace/reset/p_in
    torch.manual_seed(3)
    ffn = lf.ParaplexFFN().eval()
    perturb(ffn, 5)
    with torch.no_grad():
        ffn.w1_imag_trace.copy_(rn(H, scale=0.5))
    for k, v in ffn.state_dict().items():
        A[f"ffn.w::{k}"] = v.numpy()
    u, q, kc, c, d = rn(B, T, N), rn(B, T, QH, HD), rn(B, T, QH, HD), rn(B, T, QH, HD), rn(B, T, QH, HD)
    trace, p_in = rn(B, H, scale=0.7), rn(B, T, H)
    reset = torch.zeros(B, T, dtype=torch.bool)
    reset[0, 2] = True
    reset[1, 0] = True
    for nm, t in (("u", u), ("q", q), ("kctx", kc), ("c", c), ("d", d), ("trace", trace),
                  ("p_in", p_in), ("reset", reset)):
        A[f"ffn.{nm}"] = t.numpy()
    with torch.no_grad():
        out, tr_out, (R, I, O) = ffn(u, q, kc, c, d, phase_trace=trace, phase_reset_mask=reset,
                                     return_tria=True, p_in=p_in)
        A["ffn.out_full"], A["ffn.trace_full"] = out.numpy(), tr_out.numpy()
        A["ffn.R_full"], A["ffn.I_full"], A["ffn.O_full"] = R.numpy(), I.numpy(), O.numpy()
        out, tr_out, (R, I, O) = ffn(u, q, kc, c, d, return_tria=True)
        A["ffn.out_plain"], A["ffn.trace_plain"] = out.numpy(), tr_out.numpy()
        A["ffn.R_plain"], A["ffn.I_plain"], A["ffn.O_plain"] = R.numpy(), I.numpy(), O.numpy()
        A["ffn.beta_dense"] = ffn._beta_space(u, q, kc, c, d).numpy()
    # elementwise ops
    beta = torch.cat([rn(200, scale=3.0), torch.tensor([0.0, 1e-3, -1e-3, 50.0, -50.0, 1e4, -1e4])])
    A["phase.beta"] = beta.numpy()
    A["phase.out"] = lf._PhaseSinFloor.apply(beta, 0.05).numpy()
    x1, x2 = rn(300), torch.nn.functional.softplus(rn(300, scale=4.0))
    A["pvpowlu.x1"], A["pvpowlu.x2"] = x1.numpy(), x2.numpy()
    A["pvpowlu.out"] = lf.pvpowlu_act(x1, x2, 3.0).numpy()
    # depth attention (tensor + list history)
    torch.manual_seed(4)
    da = lf.DepthAttn().eval()
    for k, v in da.state_dict().items():
        A[f"da.w::{k}"] = v.numpy()
    S = 5
    hk, hv = rn(B, T, S, QH, HD), rn(B, T, S, QH, HD)
    A["da.hist_k"], A["da.hist_v"] = hk.numpy(), hv.numpy()
    with torch.no_grad():
        skip, dd = da(3, hk, hv)
        A["da.skip_tensor"], A["da.d_tensor"] = skip.numpy(), dd.numpy()
        skip, dd = da(4, [hk[:, :, j] for j in range(S)], [hv[:, :, j] for j in range(S)])
        A["da.skip_list"], A["da.d_list"] = skip.numpy(), dd.numpy()
        h_in = rn(B, T, N)
        kk, vv = da.project(h_in)
        A["da.h_in"], A["da.proj_k"], A["da.proj_v"] = h_in.numpy(), kk.numpy(), vv.numpy()
    # tria family
    Bt, Tt, Ht = 3, 4, 6
    r, i_, o = rn(Bt, Tt, Ht, scale=2.0), rn(Bt, Tt, Ht), rn(Bt, Tt, Ht, scale=0.5)
    prev = tr._local_normalize(rn(Bt, Tt, Ht, 3, 3))
    seed = tr._local_normalize(rn(Bt, Ht, 3, 3))
    valid = torch.tensor([True, False, True])
    w = torch.softmax(rn(9), dim=0)
    alpha = 0.0375
    for nm, t in (("r", r), ("i", i_), ("o", o), ("prev", prev), ("seed", seed),
                  ("valid", valid), ("w", w)):
        A[f"tria.{nm}"] = t.numpy()
    for axis in range(3):
        A[f"tria.build_{axis}"] = tr.build_tria_pytorch(r, i_, o, alpha, axis).numpy()
        A[f"tria.init_{axis}"] = tr.tria_init(r, i_, o, axis=axis, alpha=alpha).numpy()
        A[f"tria.step_{axis}"] = tr.tria_step(r, i_, o, prev, axis=axis, alpha=alpha).numpy()
        A[f"tria.seed_{axis}"] = tr.tria_init_seed(r, i_, o, seed, valid, axis=axis, alpha=alpha).numpy()
        cc, pp = tr.tria_init_and_gate(r, i_, o, w, axis=axis, alpha=alpha)
        A[f"tria.init_gate_{axis}.carry"], A[f"tria.init_gate_{axis}.p"] = cc.numpy(), pp.numpy()
        cc, pp = tr.tria_step_and_gate(r, i_, o, prev, w, axis=axis, alpha=alpha)
        A[f"tria.step_gate_{axis}.carry"], A[f"tria.step_gate_{axis}.p"] = cc.numpy(), pp.numpy()
        cc, pp = tr.tria_init_seed_and_gate(r, i_, o, seed, valid, w, axis=axis, alpha=alpha)
        A[f"tria.seed_gate_{axis}.carry"], A[f"tria.seed_gate_{axis}.p"] = cc.numpy(), pp.numpy()
    # temporal carry
    Tc = 9
    depth = tr._local_normalize(rn(Bt, Tc, Ht, 3, 3))
    rmask = torch.zeros(Bt, Tc, dtype=torch.bool)
    rmask[0, 4] = True
    rmask[2, 0] = True
    rmask[2, 7] = True
    init_state = tr._local_normalize(rn(Bt, Ht, 3, 3))
    A["tc.depth"], A["tc.reset"], A["tc.init"] = depth.numpy(), rmask.numpy(), init_state.numpy()
    A["tc.full_ref"] = tr.temporal_carry_reference(depth, rmask).numpy()
    A["tc.full_scan"] = tr.temporal_carry_pytorch(depth, rmask).numpy()
    A["tc.end_noinit"] = tr.temporal_carry_endpoint_reference(depth, rmask).numpy()
    A["tc.end_init"] = tr.temporal_carry_endpoint_reference(depth, rmask, initial_state=init_state).numpy()
    A["tc.end_init_valid"] = tr.temporal_carry_endpoint_reference(
        depth, rmask, initial_state=init_state, initial_valid=valid).numpy()
    # PolARM
    M = rn(4, Ht, 3, 3)
    A["polarm.in"] = M.numpy()
    A["polarm.out"] = tr.polarm(M, beta=0.1).numpy()
    A["polarm.out_b03"] = tr.polarm(M, beta=0.3).numpy()
    # readout: aggregator with a non-zero query
    torch.manual_seed(6)
    reader = tr.SharedTriaReader(k=32)
    agg = tr.TriaAggregator(reader, N).eval()
    with torch.no_grad():
        agg.pool.query.copy_(rn(32))
    for k, v in agg.state_dict().items():
        A[f"agg.w::{k}"] = v.numpy()
    carry_in = tr._local_normalize(rn(Bt, 2, Ht, 3, 3))
    A["agg.carry"] = carry_in.numpy()
    with torch.no_grad():
        A["agg.out"] = agg(carry_in).numpy()
        sw = reader.make_score_w(agg.pool.query, agg.pool.logit_scale())
        A["agg.score_w"] = sw.numpy()
    # final CA sparse + step
    Kk, D = 6, N
    qq, kk, vv = rn(Bt, Tt, D), rn(Bt, Kk, D), rn(Bt, Kk, D)
    allowed = torch.rand(Bt, Tt, Kk, generator=g) > 0.5
    allowed[1, 2] = False
    A["fca.q"], A["fca.k"], A["fca.v"], A["fca.allowed"] = qq.numpy(), kk.numpy(), vv.numpy(), allowed.numpy()
    A["fca.out"] = tr.final_ca_sparse_reference(qq, kk, vv, allowed, D ** -0.5).numpy()
    torch.manual_seed(8)
    fca = tr.TriaFinalCrossAttention(N, gamma_max=0.8, raw_gamma_init=0.25).eval()
    for k, v in fca.state_dict().items():
        A[f"fcastep.w::{k}"] = v.numpy()
    cache = tr.TriaCACache()
    seq_a, seq_b = rn(6, Bt, 1, N), rn(6, Bt, 1, N)
    fires = torch.tensor([[0, 0, 0], [1, 0, 1], [0, 0, 0], [0, 1, 1], [1, 1, 1], [0, 0, 0]], dtype=torch.bool)
    outs = []
    with torch.no_grad():
        for t in range(6):
            o_t, cache = fca.step(seq_a[t], seq_b[t], cache, t, 16, carry_key_mask=fires[t][:, None])
            outs.append(o_t)
    A["fcastep.a"], A["fcastep.b"], A["fcastep.fire"] = seq_a.numpy(), seq_b.numpy(), fires.numpy()
    A["fcastep.out"] = torch.stack(outs).numpy()
    # YaRN rope (nano shapes) + attention step
    A["rope.cos"] = lf.YaRNRotaryEmbedding().cos_cached.numpy()
    A["rope.sin"] = lf.YaRNRotaryEmbedding().sin_cached.numpy()
    torch.manual_seed(9)
    attn = lf.GroupedQueryCausalSelfAttention().eval()
    for k, v in attn.state_dict().items():
        A[f"attn.w::{k}"] = v.numpy()
    zs = rn(6, B, 1, N)
    A["attn.z"] = zs.numpy()
    kc_ = vc_ = None
    with torch.no_grad():
        res = {"out": [], "q": [], "kctx": [], "c": []}
        for pos in range(6):
            o_, q_, kx_, c_, kc_, vc_ = attn.step(zs[pos], pos, kc_, vc_, pos)
            for nm, t in (("out", o_), ("q", q_), ("kctx", kx_), ("c", c_)):
                res[nm].append(t)
    for nm, lst in res.items():
        A[f"attn.{nm}"] = torch.stack(lst).numpy()
    return A


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--only", default="")
    args = ap.parse_args()
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    lf, tr = load_ref(args.ref)
    only = set(x for x in args.only.split(",") if x)
    if not only or "cfg" in only:
        import yaml
        keep = ("vocab", "seq_len", "n_q_heads", "head_dim", "model_dim", "n_kv_heads",
                "gqa_group_size", "hidden", "hidden_mult", "layers", "phase_sectors",
                "residual_init", "activation", "powlu_m", "tied_embeddings", "rope_theta",
                "rope_original_seq_len", "rope_factor", "rope_beta_fast", "rope_beta_slow",
                "rope_attention_factor", "tria_carry_enabled", "tria_temporal_enabled",
                "tria_temporal_window", "tria_carrier_alpha", "tria_polarm_beta",
                "tria_gamma_max", "tria_raw_gamma_init")
        cfgs = {}
        for name in ("nano", "nano_chk"):
            with open(os.path.join(args.ref, "cfg", name + ".yaml"), encoding="utf-8") as f:
                d = yaml.safe_load(f)
            cfgs[name] = {k: d[k] for k in keep if k in d}
        cfgs["tiny"] = {k: v for k, v in TINY.items() if k in keep}
        cfgs["tiny_variants"] = dict(cfgs["tiny"], **VARIANTS)
        with open(os.path.join(HERE, "configs.json"), "w") as f:
            json.dump(cfgs, f, indent=1, sort_keys=True)
        print("wrote configs.json")
    if not only or "init" in only:
        with open(os.path.join(HERE, "init_sha256.json"), "w") as f:
            json.dump(golden_init(lf, args.ref), f, indent=0, sort_keys=True)
        print("wrote init_sha256.json")
    if not only or "tiny" in only:
        np.savez_compressed(os.path.join(HERE, "tiny_decode.npz"), **golden_tiny_decode(lf))
        print("wrote tiny_decode.npz")
    if not only or "variants" in only:
        np.savez_compressed(os.path.join(HERE, "variants_decode.npz"), **golden_variants(lf))
        print("wrote variants_decode.npz")
    if not only or "ops" in only:
        np.savez_compressed(os.path.join(HERE, "ops.npz"), **golden_ops(lf, tr))
        print("wrote ops.npz")
    if not only or "chunked" in only:
        np.savez_compressed(os.path.join(HERE, "chunked_keys.npz"), **golden_chunked(lf, tr))
        print("wrote chunked_keys.npz")
    if not only or "nano" in only:
        np.savez_compressed(os.path.join(HERE, "nano_cpu_ref.npz"), **golden_nano_cpu(lf, args.ref))
        print("wrote nano_cpu_ref.npz")


if __name__ == "__main__":
    main()
