"""Trained-checkpoint formats for the decode engine.

Two containers reach the reference's inference code:
  * a training checkpoint: a ``torch.save`` mapping with ``model`` (the
    state dict) and ``cfg`` (the config mapping), read by loompack's
    ``_load_checkpoint`` (loompack.py:171-179);
  * a ``loom.aio`` v1 package (loompack.py:198-284, read by
    ``loomchat.load_aio``, loomchat.py:278-316): the same ``checkpoint``
    mapping plus the tokenizer JSON and the chat template.
Both are read with ``torch.load(weights_only=True)``, which executes nothing
from the file.  The state dict is canonicalised as
``canonicalize_model_state_dict`` does (loomformer.py:4363-4408) and the
config migrated as ``Config.from_checkpoint_dict`` does (loomformer.py:432-450).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, Mapping, Optional

import torch

from .config import ModelConfig
from .weights import state_keys

AIO_FORMAT = "loom.aio"
AIO_VERSION = 1

# legacy reader aliases -> canonical keys (loomformer.py:4365-4369)
_READER_ALIASES = (
    ("_tria_reader.proj.weight", "tria_agg.reader.proj.weight"),
    ("_tria_reader.proj.bias", "tria_agg.reader.proj.bias"),
    ("_tria_reader.key_proj.weight", "tria_agg.reader.key_proj.weight"),
)


def _merge_group(state: Dict[str, Any], parts, packed: str, what: str) -> None:
    """Concatenate a legacy split projection along dim 0 into its packed key,
    refusing an incomplete group or a packed value that disagrees."""
    values = [state.get(k) for k in parts]
    if all(v is None for v in values):
        return
    if any(v is None for v in values):
        raise ValueError(f"incomplete {what} checkpoint group")
    merged = torch.cat(values, dim=0)
    current = state.get(packed)
    if current is not None and not torch.equal(current, merged):
        raise ValueError(f"packed {what} disagrees with legacy weights")
    state[packed] = merged
    for k in parts:
        state.pop(k)


def canonicalize_state_dict(state: Mapping[str, Any], layers: int) -> Dict[str, Any]:
    """The reference's canonical key set from older layouts
    (canonicalize_model_state_dict, loomformer.py:4363-4408):
    ``_tria_reader.*`` aliases become ``tria_agg.reader.*``; per-layer
    ``attn.q/k/v.weight`` become ``attn.qkv_weight``; ``depth_attn.w_k/w_v``
    become ``depth_attn.kv_weight``."""
    out = dict(state)
    for legacy, canonical in _READER_ALIASES:
        value = out.pop(legacy, None)
        if value is None:
            continue
        current = out.get(canonical)
        if current is not None and not torch.equal(value, current):
            raise ValueError(f"checkpoint reader aliases disagree: {legacy!r} != {canonical!r}")
        if current is None:
            out[canonical] = value
    for layer in range(layers):
        p = f"blocks.{layer}.attn."
        _merge_group(out, [p + "q.weight", p + "k.weight", p + "v.weight"], p + "qkv_weight",
                     f"QKV (layer {layer})")
    _merge_group(out, ["depth_attn.w_k.weight", "depth_attn.w_v.weight"], "depth_attn.kv_weight",
                 "depth K/V")
    return out


def migrate_config(d: Mapping[str, Any]) -> Dict[str, Any]:
    """Config.from_checkpoint_dict's migration (loomformer.py:432-450): the
    legacy ``tria_temporal_deadline`` names the window; the removed GeluFFN
    baseline fields are refused."""
    values = dict(d)
    legacy = values.pop("tria_temporal_deadline", None)
    current = values.get("tria_temporal_window")
    if legacy is not None and current is not None and int(legacy) != int(current):
        raise ValueError("checkpoint has conflicting tria_temporal_window/tria_temporal_deadline "
                         f"values: {current!r} vs {legacy!r}")
    if current is None and legacy is not None:
        values["tria_temporal_window"] = int(legacy)
    if values.pop("baseline_hidden", None) is not None:
        raise ValueError("checkpoint requests removed GeluFFN baseline_hidden")
    if bool(values.pop("train_baseline", False)):
        raise ValueError("checkpoint requests removed GeluFFN baseline training")
    return values


@dataclass
class LoadedModel:
    cfg: ModelConfig
    state: Dict[str, torch.Tensor]
    raw_cfg: Dict[str, Any]
    tokenizer_json: Optional[bytes] = None
    chat_template: Optional[str] = None
    manifest: Dict[str, Any] = field(default_factory=dict)
    archive_dtype: str = "fp32"
    carry_token_id: Optional[int] = None

    def decoder(self, batch: int, dtype: torch.dtype = torch.bfloat16, device="cuda",
                max_len: Optional[int] = None):
        """A LoomDecoder over these weights (the <CARRY> id of the package's
        tokenizer, if any, fires explicitly as loomchat sets it, loomchat.py:301)."""
        from .engine import LoomDecoder
        return LoomDecoder(self.cfg, self.state, batch, dtype=dtype, device=device,
                           max_len=max_len, carry_token_id=self.carry_token_id)


def _from_checkpoint(ck: Mapping[str, Any], vocab: Optional[int] = None) -> LoadedModel:
    if ck.get("model_kind", "loomformer") != "loomformer":
        raise ValueError("checkpoint is not a LoomFormer model")
    if ck.get("ffn_type", "paraplex") != "paraplex":
        raise ValueError("checkpoint is not a Paraplex model")
    if bool(ck.get("ablation", False)):
        raise ValueError("ablation checkpoints (plain FFN, no Paraplex phase path or Tria carry) "
                         "are not served by this engine")
    raw = migrate_config(ck["cfg"])
    if vocab is not None:
        raw["vocab"] = int(vocab)
    cfg = ModelConfig.from_dict(raw)
    state = canonicalize_state_dict(ck["model"], cfg.L)
    state = {k: v for k, v in state.items() if torch.is_tensor(v)}
    if cfg.tied and "head.weight" not in state and "emb.weight" in state:
        state["head.weight"] = state["emb.weight"]
    # the strict load of load_model_blob_into (loomformer.py:4424): the keys must
    # be exactly the config's model (a variant flag without its weights, or
    # weights of a variant the config does not set, is refused)
    want = set(state_keys(cfg))
    missing, unexpected = sorted(want - set(state)), sorted(set(state) - want)
    if missing or unexpected:
        raise ValueError(f"checkpoint state_dict does not match its config: missing keys "
                         f"{missing[:8]}, unexpected keys {unexpected[:8]}")
    emb = state.get("emb.weight")
    if emb is None or emb.shape != (cfg.V, cfg.N):
        raise ValueError(f"emb.weight {None if emb is None else tuple(emb.shape)} does not match "
                         f"vocab {cfg.V} x model_dim {cfg.N}")
    return LoadedModel(cfg=cfg, state=state, raw_cfg=raw)


def load_checkpoint(path: str) -> LoadedModel:
    """A training checkpoint (loompack.py:171-179): ``{'model': ..., 'cfg': ...}``."""
    blob = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(blob, Mapping):
        raise TypeError("checkpoint must be a mapping")
    if not isinstance(blob.get("model"), Mapping):
        raise ValueError("checkpoint must contain a model state dict under key 'model'")
    if not isinstance(blob.get("cfg"), Mapping):
        raise ValueError("checkpoint must contain configuration under key 'cfg'")
    return _from_checkpoint(blob)


def _tokenizer_facts(tokenizer_json: bytes):
    """(vocabulary size, id of <CARRY> or None) of a tokenizers JSON: loomchat
    sets cfg.vocab and CARRY_TOKEN_ID from the package's tokenizer
    (loomchat.py:297-301).  (None, None) if the library is not importable."""
    try:
        from tokenizers import Tokenizer
    except ImportError:
        return None, None
    tok = Tokenizer.from_str(bytes(tokenizer_json).decode("utf-8"))
    return tok.get_vocab_size(), tok.token_to_id("<CARRY>")


def load_aio(path: str) -> LoadedModel:
    """A ``loom.aio`` v1 package (loomchat.load_aio, loomchat.py:278-316)."""
    if not str(path).lower().endswith(".aio"):
        raise ValueError(f"{path}: not a .aio package (expected the .aio extension)")
    package = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(package, Mapping) or package.get("format") != AIO_FORMAT:
        raise ValueError(f"not a {AIO_FORMAT} archive")
    if int(package.get("version", -1)) != AIO_VERSION:
        raise ValueError(f"unsupported AIO version {package.get('version')!r}")
    ck = package.get("checkpoint")
    tok = package.get("tokenizer_json")
    tmpl = package.get("chat_template_jinja")
    if not isinstance(ck, Mapping):
        raise ValueError("AIO archive has no checkpoint")
    if not isinstance(tok, (bytes, bytearray)):
        raise ValueError("AIO archive has no tokenizer JSON")
    if not isinstance(tmpl, (bytes, bytearray)):
        raise ValueError("AIO archive has no chat template")
    vocab, carry_id = _tokenizer_facts(tok)
    loaded = _from_checkpoint(ck, vocab=vocab)
    loaded.carry_token_id = carry_id
    loaded.tokenizer_json = bytes(tok)
    loaded.chat_template = bytes(tmpl).decode("utf-8")
    loaded.manifest = dict(package.get("manifest", {}))
    target = str(loaded.manifest.get("quantization", {}).get("target_dtype", "none"))
    loaded.archive_dtype = target if target in ("bf16", "fp16", "fp32") else "fp32"
    return loaded
