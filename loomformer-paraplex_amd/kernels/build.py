"""``build_or_load`` for the gfx950 library (replaces kernels/build.py:262-344).

Same signature as the reference.  ``sources``, ``extra_cflags``,
``extra_cuda_cflags`` and ``ptx_kernels`` name the reference's CUDA files and
nvcc flags; they are accepted and ignored, because the HIP library is built
ahead of time (``python loomformer-paraplex_amd/build_lib.py``).  The module
returned for each extension name exposes the functions the reference's pybind
module exposes; forward entry points run the gfx950 kernels, backward/replay
entry points (training) raise ``RuntimeError``.

Like the reference, the call fails closed: a missing library or an unknown
extension name raises, and the reference's callers then fall back to their
PyTorch paths exactly as they do when nvcc is unavailable.
"""
from __future__ import annotations

import threading
import types
from typing import Dict, List, Optional, Sequence

_STATE_LOCK = threading.Lock()
_MODULES: Dict[str, types.ModuleType] = {}

# extension name -> exported function names (reference pybind/TORCH_LIBRARY)
EXPORTS = {
    "loomformer_paraplex": ("paraplex_forward", "paraplex_backward"),
    "loomformer_beta_space": ("beta_forward_cuda", "beta_backward_cuda",
                              "beta_backward_cuda_recompute"),
    "loomformer_phase_sin": ("phase_sin_forward_cuda", "phase_sin_backward_cuda",
                             "phase_sin_secant_backward_cuda"),
    "loomformer_pvpowlu": ("pvpowlu_forward_cuda", "pvpowlu_backward_cuda"),
    "loomformer_depth_attn_online": ("depth_attn_forward", "depth_attn_backward",
                                     "depth_attn_stacked_forward", "depth_attn_stacked_backward",
                                     "depth_attn_list_forward", "depth_attn_list_backward"),
    "loomformer_tria_carry": (
        "tria_init_forward", "tria_init_gate_forward", "tria_init_seed_forward",
        "tria_init_seed_gate_forward", "tria_step_forward", "tria_step_gate_forward",
        "gate_slot_mix_forward", "slot_attention_pool_forward", "temporal_carry_forward",
        "temporal_carry_endpoint_forward", "final_ca_sparse_forward",
        # training-only entry points of bindings.cpp:88-110
        "tria_init_backward", "tria_init_gate_backward", "tria_init_seed_backward",
        "tria_init_seed_gate_backward", "tria_step_backward", "tria_step_gate_backward",
        "tria_step_reverse_backward", "tria_step_gate_reverse_backward",
        "gate_slot_mix_backward", "slot_attention_pool_backward", "temporal_carry_backward",
        "temporal_carry_endpoint_backward", "depth_replay_backward",
        "depth_replay_gate_backward", "final_ca_sparse_backward"),
}


def _make_module(ext_name: str) -> types.ModuleType:
    from loom_amd import _lib, ops  # imported lazily: loading needs the built library

    _lib.load()   # raise now (not at first call) if the library is missing
    mod = types.ModuleType(ext_name, f"gfx950 implementation of the reference's {ext_name}")
    for fn in EXPORTS[ext_name]:
        impl = getattr(ops, fn, None)
        if impl is None:
            impl = ops._unsupported(fn)
        setattr(mod, fn, impl)
    mod.__file__ = _lib.LIB_PATH
    return mod


def build_or_load(
    ext_name: str,
    sources: Sequence[str] = (),
    extra_cflags: Optional[List[str]] = None,
    extra_cuda_cflags: Optional[List[str]] = None,
    ptx_kernels: Optional[Dict[str, str]] = None,
):
    """Return the gfx950 module for ``ext_name`` (cached), or raise."""
    del sources, extra_cflags, extra_cuda_cflags, ptx_kernels
    if ext_name not in EXPORTS:
        raise RuntimeError(f"kernels.build_or_load: unknown extension {ext_name!r}")
    with _STATE_LOCK:
        mod = _MODULES.get(ext_name)
        if mod is None:
            mod = _make_module(ext_name)
            _MODULES[ext_name] = mod
        return mod
