"""Trained-checkpoint formats (CPU): training checkpoints and loom.aio v1
packages load into the engine's ModelConfig + canonical state dict, legacy
key layouts and config fields migrate as the reference migrates them
(canonicalize_model_state_dict, loomformer.py:4363-4408;
Config.from_checkpoint_dict, :432-450), and malformed files are refused with
the reference's messages.  The packages are built here with torch.save of
plain tensors and bytes, the layout loompack.build_package writes
(loompack.py:198-284)."""
import json
import os

import numpy as np
import pytest
import torch

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _tiny():
    with open(os.path.join(GOLD, "configs.json")) as f:
        cfg = json.load(f)["tiny"]
    z = np.load(os.path.join(GOLD, "tiny_decode.npz"))
    state = {k[3:]: torch.from_numpy(z[k]) for k in z.files if k.startswith("w::")}
    return cfg, state


def _legacy(state, layers):
    """The older key layout canonicalize_model_state_dict accepts."""
    s = dict(state)
    for l in range(layers):
        p = f"blocks.{l}.attn."
        qkv = s.pop(p + "qkv_weight")
        N = s["emb.weight"].shape[1]
        kv = (qkv.shape[0] - N) // 2
        s[p + "q.weight"], s[p + "k.weight"], s[p + "v.weight"] = qkv.split([N, kv, kv], 0)
    kvw = s.pop("depth_attn.kv_weight")
    s["depth_attn.w_k.weight"], s["depth_attn.w_v.weight"] = kvw.chunk(2, 0)
    s["_tria_reader.proj.weight"] = s.pop("tria_agg.reader.proj.weight")
    return s


def _tokenizer_json(vocab):
    from tokenizers import Tokenizer, models
    words = {f"w{i}": i for i in range(vocab - 1)}
    tok = Tokenizer(models.WordLevel(vocab=words, unk_token="w0"))
    tok.add_special_tokens(["<CARRY>"])
    return tok.to_str().encode("utf-8")


def test_training_checkpoint_with_legacy_layout(tmp_path):
    from loom_amd.checkpoint import load_checkpoint
    from loom_amd.config import ModelConfig
    cfg, state = _tiny()
    raw = dict(cfg)
    raw["tria_temporal_deadline"] = raw.pop("tria_temporal_window")
    path = tmp_path / "ckpt.pt"
    torch.save({"model": _legacy(state, cfg["layers"]), "cfg": raw, "step": 10}, path)
    got = load_checkpoint(str(path))
    assert got.cfg == ModelConfig.from_dict(cfg)
    assert set(got.state) == set(state)
    for k, v in state.items():
        assert torch.equal(got.state[k], v), k


def test_aio_package(tmp_path):
    from loom_amd.checkpoint import load_aio
    cfg, state = _tiny()
    tok = _tokenizer_json(cfg["vocab"])
    pkg = {"format": "loom.aio", "version": 1,
           "manifest": {"quantization": {"target_dtype": "bf16"}},
           "checkpoint": {"model_kind": "loomformer", "ffn_type": "paraplex", "cfg": cfg,
                          "ablation": False, "model": {k: v.to(torch.bfloat16) for k, v in state.items()}},
           "tokenizer_json": tok, "chat_template_jinja": b"{{ messages }}"}
    path = tmp_path / "m.aio"
    torch.save(pkg, path)
    got = load_aio(str(path))
    assert got.carry_token_id == cfg["vocab"] - 1
    assert got.cfg.V == cfg["vocab"] and got.archive_dtype == "bf16"
    assert got.chat_template == "{{ messages }}"
    assert torch.equal(got.state["blocks.0.attn.qkv_weight"], state["blocks.0.attn.qkv_weight"].to(torch.bfloat16))


@pytest.mark.parametrize("mutate,msg", [
    (lambda p: p.update(format="other"), "not a loom.aio archive"),
    (lambda p: p.update(version=2), "unsupported AIO version"),
    (lambda p: p.pop("tokenizer_json"), "no tokenizer JSON"),
    (lambda p: p["checkpoint"].update(ffn_type="gelu"), "not a Paraplex model"),
    (lambda p: p["checkpoint"].update(ablation=True), "ablation"),
    (lambda p: p["checkpoint"]["cfg"].update(tria_temporal_deadline=9), "conflicting tria_temporal_window"),
    (lambda p: p["checkpoint"]["cfg"].update(baseline_hidden=64), "removed GeluFFN"),
    (lambda p: p["checkpoint"]["model"].pop("blocks.1.attn.k.weight"), "incomplete QKV"),
    (lambda p: p["checkpoint"]["model"].update({"blocks.0.attn.qkv_weight": torch.zeros(1)}),
     "packed QKV .* disagrees"),
])
def test_aio_rejects(tmp_path, mutate, msg):
    from loom_amd.checkpoint import load_aio
    cfg, state = _tiny()
    legacy = _legacy(state, cfg["layers"])
    pkg = {"format": "loom.aio", "version": 1, "manifest": {},
           "checkpoint": {"model_kind": "loomformer", "ffn_type": "paraplex", "cfg": dict(cfg),
                          "model": legacy},
           "tokenizer_json": _tokenizer_json(cfg["vocab"]), "chat_template_jinja": b"t"}
    mutate(pkg)
    path = tmp_path / "bad.aio"
    torch.save(pkg, path)
    with pytest.raises(ValueError, match=msg):
        load_aio(str(path))


def test_aio_suffix_required(tmp_path):
    from loom_amd.checkpoint import load_aio
    with pytest.raises(ValueError, match="not a .aio package"):
        load_aio(str(tmp_path / "x.pt"))


@pytest.mark.parametrize("flag,value,field,want", [
    ("paraplex_gate_proj", True, "gate_proj", True), ("depth_attn_qkv_rms", True, "depth_qkv_rms", True),
    ("residual_branch_rms_cap", 2.0, "residual_rms_cap", 2.0), ("final_norm", True, "final_norm", True),
    ("depth_attn_readout", "Per-Sublayer", "depth_readout", "per-sublayer")])
def test_config_carries_variant_flags(flag, value, field, want):
    """The math-changing model flags (loomformer.py:272-274, :358, :366) reach
    the engine's config instead of being dropped."""
    from loom_amd.config import ModelConfig
    cfg, _ = _tiny()
    assert getattr(ModelConfig.from_dict(dict(cfg, **{flag: value})), field) == want


@pytest.mark.parametrize("flag,value", [("paraplex_gate_proj", True), ("final_norm", True),
                                        ("depth_attn_readout", "per-sublayer")])
def test_checkpoint_refuses_weights_that_do_not_match_its_variant_flags(tmp_path, flag, value):
    """A config that sets a variant whose weights the state dict lacks (or the
    other way round) is refused like the reference's strict load, not decoded
    as a different model."""
    from loom_amd.checkpoint import load_checkpoint
    cfg, state = _tiny()
    path = tmp_path / "ck.pt"
    torch.save({"cfg": dict(cfg, **{flag: value}), "model": state}, path)
    with pytest.raises(ValueError, match="does not match its config"):
        load_checkpoint(str(path))
    # and the variant's own checkpoint loads
    z = np.load(os.path.join(GOLD, "variants_decode.npz"))
    with open(os.path.join(GOLD, "configs.json")) as f:
        vcfg = json.load(f)["tiny_variants"]
    vstate = {k[3:]: torch.from_numpy(z[k]) for k in z.files if k.startswith("w::")}
    torch.save({"cfg": vcfg, "model": vstate}, path)
    loaded = load_checkpoint(str(path))
    assert loaded.cfg.gate_proj and loaded.cfg.final_norm
    assert loaded.cfg.depth_readout == "per-sublayer"


def test_config_validates_variant_values_like_apply_config():
    from loom_amd.config import ModelConfig
    cfg, _ = _tiny()
    with pytest.raises(ValueError, match="shared' or 'per-sublayer"):
        ModelConfig.from_dict(dict(cfg, depth_attn_readout="per-head"))
    with pytest.raises(ValueError, match="positive or null"):
        ModelConfig.from_dict(dict(cfg, residual_branch_rms_cap=0.0))
    # defaults spelled out are accepted
    ModelConfig.from_dict(dict(cfg, paraplex_gate_proj=False, depth_attn_qkv_rms=False,
                               residual_branch_rms_cap=None, final_norm=False,
                               depth_attn_readout="shared"))
