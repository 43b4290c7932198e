"""ctypes binding of libloom_hip.so (declared in include/loom_hip.h).

The library is built in-tree by ``build_lib.py``; there is no fallback: if it
is missing or fails to load, every op raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from ctypes import c_float, c_int, c_int64, c_void_p

import torch

# descriptor layouts and signatures below are those of loom_abi_version() == ABI_VERSION
ABI_VERSION = 10
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libloom_hip.so")

_P = c_void_p


class LinearSegment(ctypes.Structure):
    """loom_linear_segment (include/loom_hip.h)."""
    _fields_ = [("w", c_void_p), ("ldw", c_int64), ("w2", c_void_p), ("ldw2", c_int64),
                ("out", c_void_p), ("ldc", c_int64), ("bias", c_void_p), ("gate_p", c_void_p),
                ("gate_ld", c_int64), ("gate_alpha", c_float), ("n", c_int64)]


class LinearMultiDesc(ctypes.Structure):
    """loom_linear_multi_desc (include/loom_hip.h)."""
    _fields_ = [("x", c_void_p), ("ldx", c_int64), ("k", c_int64), ("x2", c_void_p),
                ("ldx2", c_int64), ("k2", c_int64), ("m", c_int64), ("nseg", ctypes.c_int32),
                ("seg", LinearSegment * 4), ("only_if", c_void_p), ("only_if_n", c_int64),
                ("x_frag", c_void_p), ("x2_frag", c_void_p)]

# name -> argument types (all return c_int status)
SIGNATURES = {
    "loom_paraplex_forward": [c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                              c_int64, c_int64, c_int64, c_float, _P],
    "loom_phase_sin_forward": [c_int, _P, _P, c_int64, _P],
    "loom_pvpowlu_forward": [c_int, _P, _P, _P, c_int64, c_float, _P],
    "loom_beta_forward": [c_int, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64,
                          c_int64, c_int64, c_int64, c_int64, c_int, _P],
    "loom_linear_multi": [c_int, _P, _P],
    "loom_ffn_decode": [c_int, _P, _P],
    "loom_linear_ln": [c_int, _P, _P, _P, c_float, _P, c_int64, _P, c_int64, _P, _P],
    "loom_linear": [c_int, _P, c_int64, _P, c_int64, _P, _P, c_float, _P, _P, c_int64,
                    c_int64, c_int64, c_int64, _P],
    "loom_depth_attn_forward": [c_int, _P, _P, _P, c_int64, c_int64, _P, _P, _P, c_int64,
                                c_int64, c_int64, c_int64, _P],
    "loom_tria_depth_forward": [c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64,
                                c_int64, c_int64, c_float, c_int, _P],
    "loom_paraplex_tria_forward": [c_int, _P, _P, _P, _P, _P, _P, c_float, _P, _P, _P, _P, _P, _P,
                                   _P, _P, c_int64, c_int64, c_int64, c_float, c_int, _P],
    "loom_paraplex_tria_endpoint_forward": [c_int, _P, _P, _P, _P, _P, _P, c_float, _P, _P, _P, _P,
                                            _P, _P, _P, _P, c_int64, c_int64, c_int64, c_float,
                                            c_int, _P],
    "loom_gate_slot_mix_forward": [c_int, _P, _P, _P, c_int64, _P],
    "loom_slot_attention_pool_forward": [c_int, _P, _P, _P, _P, c_int64, c_int64, _P],
    "loom_temporal_carry_forward": [c_int, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P],
    "loom_temporal_carry_endpoint_forward": [c_int, _P, _P, _P, _P, _P, _P, c_int64, c_int64,
                                             c_int64, _P],
    "loom_polarm_forward": [c_int, _P, _P, _P, c_int64, c_int64, c_float, c_float, _P],
    "loom_tria_chunked_forward": [c_int, _P, _P, _P, c_int64, c_int64, _P, _P, _P, _P, c_int64,
                                  c_int64, c_int64, c_int64, c_int64, c_float, c_float, c_float,
                                  _P],
    "loom_tria_chunked_forward_fires": [c_int, _P, _P, _P, c_int64, c_int64, _P, _P, _P, c_int64,
                                        _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64,
                                        c_float, c_float, c_float, _P],
    "loom_final_ca_sparse_forward": [c_int, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64,
                                     c_int64, c_float, _P],
    "loom_final_ca_sparse_strided": [c_int, _P, _P, _P, c_int64, _P, c_int64, _P, c_float, _P,
                                     _P, c_int64, c_int64, c_int64, _P, c_int64, c_float, _P],
    "loom_rope_append": [c_int, _P, _P, _P, _P, _P, _P, c_int64, c_int64, _P, c_int64, c_int64,
                         c_int64, c_int64, c_int64, c_int64, _P],
    "loom_gqa_decode_attention": [c_int, _P, _P, _P, c_int64, c_int64, c_int64, _P, _P, _P,
                                  c_int64, c_int64, c_int64, _P, c_int64, c_int64, c_int64, _P],
    "loom_gqa_decode_step": [c_int, _P, _P, _P, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P,
                             c_int64, _P, c_int64, c_int64, c_int64, _P, c_int64, c_int64, c_int64,
                             _P],
    "loom_depth_attn_pair": [c_int, _P, _P, _P, _P, c_int64, c_int64, _P, _P, _P, c_int64,
                             c_int64, c_int64, c_int64, _P],
    "loom_depth_attn_fold": [c_int, _P, _P, _P, c_int64, c_int64, c_int64, _P, _P, _P, c_int64,
                             c_int64, c_int64, _P],
    "loom_depth_attn_forward_rms": [c_int, _P, _P, _P, c_int64, c_int64, _P, _P, _P, c_int64,
                                    c_int64, c_int64, c_int64, c_float, c_float, c_float, _P],
    "loom_rms_norm": [c_int, _P, _P, _P, c_int64, c_int64, c_float, _P],
    "loom_gqa_decode_step_noalloc": [c_int, _P, _P, _P, c_int64, c_int64, c_int64, _P, _P, _P, _P,
                                     _P, c_int64, c_int64, c_int64, _P, c_int64, c_int64, c_int64,
                                     _P],
    "loom_prefill_qkv": [c_int, _P, c_int64, _P, _P, _P, c_int64, c_int64, _P, _P, _P, _P, c_int64,
                         c_int64, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64,
                         c_int64, c_int64, c_int64, _P],
    "loom_gqa_prefill": [c_int, _P, c_int64, _P, _P, c_int64, c_int64, c_int64, _P, _P, _P, _P,
                         _P, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
                         c_int64, _P],
    "loom_gqa_decode_step_depth": [c_int, _P, _P, _P, c_int64, c_int64, c_int64, _P, _P, _P, _P,
                                   _P, c_int64, _P, c_int64, c_int64, c_int64, _P, c_int64,
                                   c_int64, c_int64, _P, _P, _P, c_int64, c_int64, c_int64, _P,
                                   _P],
    "loom_gqa_decode_step_depth2": [c_int, _P, _P, _P, c_int64, c_int64, c_int64, _P, _P, _P, _P,
                                    _P, c_int64, _P, c_int64, c_int64, c_int64, _P, c_int64,
                                    c_int64, c_int64, _P, _P, _P, _P, c_int64, c_int64, c_int64,
                                    _P, _P, _P, _P],
    "loom_decode_prologue": [_P, _P, c_int64, c_int64, _P, c_int64, _P, _P, _P, _P, c_int64,
                             c_int64, c_int64, c_int64, _P],
    "loom_decode_prologue_embed": [c_int, _P, _P, c_int64, c_int64, _P, c_int64, _P, _P, _P, _P,
                                   c_int64, c_int64, c_int64, _P, _P, c_int64, c_int64, c_int64, _P],
    "loom_decode_prologue_gather": [c_int, _P, _P, _P, c_int64, c_int64, _P, c_int64, _P, _P, _P,
                                    _P, c_int64, c_int64, c_int64, _P, c_int64, c_int64, _P,
                                    c_int64, c_int64, _P, c_int64, c_int64, c_int64, _P],
    "loom_decode_epilogue": [c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64,
                             _P],
    "loom_argmax_rows": [c_int, _P, c_int64, c_int64, _P, _P],
    "loom_add_layernorm": [c_int, _P, _P, _P, _P, _P, c_int64, c_int64, c_float, _P],
    "loom_tria_decode_temporal": [c_int, _P, _P, _P, _P, _P, c_int64, c_int64, c_float, c_float,
                                  _P],
    "loom_decode_tria_readout": [c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64,
                                 c_int64, c_int64, c_int64, c_float, c_float, _P],
}
# entry points that return a value instead of a status
QUERIES = {"loom_gqa_workspace_bytes": ([c_int64] * 5, c_int64),
           "loom_gemm_shared_tiles": ([c_int], c_int),
           "loom_linear_multi_desc_bytes": ([], c_int64),
           "loom_decode_tria_readout_workspace_bytes": ([c_int64, c_int64], c_int64),
           "loom_ffn_decode_desc_bytes": ([], c_int64),
           "loom_linear_ln_workspace_bytes": ([c_int64, c_int64], c_int64),
           "loom_tria_chunked_workspace_bytes": ([c_int64] * 4, c_int64),
           "loom_tria_chunked_fires_workspace_bytes": ([c_int64, c_int64, c_int64, _P, c_int64],
                                                       c_int64)}

_lib = None
_lock = threading.Lock()

DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library once and set every declared signature."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"libloom_hip.so not found at {path}; build it with "
                "`python loomformer-paraplex_amd/build_lib.py` (or __graft_entry__.build())")
        lib = ctypes.CDLL(path)
        lib.loom_last_error.restype = ctypes.c_char_p
        lib.loom_last_error.argtypes = []
        lib.loom_abi_version.restype = c_int
        if lib.loom_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"{path} implements C ABI version {lib.loom_abi_version()}, this binding "
                f"declares version {ABI_VERSION}; rebuild the library")
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = c_int
        for name, (argtypes, restype) in QUERIES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = lib
        return lib


def call(name: str, *args) -> None:
    """Call an entry point; raise RuntimeError(loom_last_error()) on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.loom_last_error().decode("utf-8", "replace")
        raise RuntimeError(msg or f"{name} failed with status {rc}")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODE[t.dtype]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {t.dtype}; expected float32, bfloat16 or float16")


class FfnDecodeDesc(ctypes.Structure):
    """loom_ffn_decode_desc (include/loom_hip.h)."""
    _fields_ = [("u", c_void_p), ("q_h", c_void_p), ("k_ctx_h", c_void_p), ("c_h", c_void_p),
                ("d_h", c_void_p), ("w_compact", c_void_p),
                ("M", c_int64), ("N", c_int64), ("H", c_int64), ("imag_in", c_int64),
                ("hidden_per_q_head", c_int64), ("head_dim", c_int64), ("n_q_heads", c_int64),
                ("open_sectors", ctypes.c_int32),
                ("p_real", c_void_p), ("gate_src", c_void_p), ("imag_bias", c_void_p),
                ("trace", c_void_p),
                ("trace_w", c_void_p), ("powlu_m", c_float),
                ("act", c_void_p), ("s", c_void_p), ("beta", c_void_p),
                ("carry_prev", c_void_p), ("seed", c_void_p), ("seed_valid", c_void_p),
                ("gate_w", c_void_p), ("carry_out", c_void_p), ("p_out", c_void_p),
                ("alpha", c_float), ("axis", ctypes.c_int32), ("act_frag", c_void_p),
                ("u_frag", c_void_p), ("depth_q", c_void_p), ("depth_k", c_void_p),
                ("depth_v", c_void_p), ("depth_sbt", c_int64), ("depth_ss", c_int64),
                ("depth_S", ctypes.c_int32), ("depth_rms", ctypes.c_int32), ("depth_qt", c_float),
                ("depth_kt", c_float), ("depth_vt", c_float), ("depth_part_d", c_void_p),
                ("depth_part_lse", c_void_p)]


def linear_multi_desc(x, segments, x2=None, m=None, only_if=None, x_frag=None, x2_frag=None):
    """Build a LinearMultiDesc.  x, x2: [m, k] tensors (row-strided views are
    fine); segments: dicts with w, out and optional w2, bias, gate_p,
    gate_alpha (tensors keep their own row strides); only_if: optional uint8
    device flags (the fused launch skips the product when none is set);
    x_frag / x2_frag: optional fragment-major copies of x / x2."""
    d = LinearMultiDesc()
    if x_frag is not None:
        d.x_frag = x_frag.data_ptr()
    if x2_frag is not None:
        d.x2_frag = x2_frag.data_ptr()
    d.x, d.ldx, d.k = x.data_ptr(), x.stride(0), x.shape[1]
    if x2 is not None:
        d.x2, d.ldx2, d.k2 = x2.data_ptr(), x2.stride(0), x2.shape[1]
    d.m = x.shape[0] if m is None else m
    if not 1 <= len(segments) <= 4:
        raise ValueError("linear_multi takes 1 to 4 segments")
    d.nseg = len(segments)
    if only_if is not None:
        d.only_if, d.only_if_n = only_if.data_ptr(), only_if.numel()
    for i, sg in enumerate(segments):
        e = d.seg[i]
        w, out = sg["w"], sg["out"]
        e.w, e.ldw, e.out, e.ldc, e.n = w.data_ptr(), w.stride(0), out.data_ptr(), out.stride(0), w.shape[0]
        if sg.get("w2") is not None:
            e.w2, e.ldw2 = sg["w2"].data_ptr(), sg["w2"].stride(0)
        if sg.get("bias") is not None:
            e.bias = sg["bias"].data_ptr()
        if sg.get("gate_p") is not None:
            e.gate_p, e.gate_ld = sg["gate_p"].data_ptr(), sg["gate_p"].stride(0)
            e.gate_alpha = float(sg.get("gate_alpha", 0.0))
    return d


def ffn_decode_desc(**kw):
    """Build an FfnDecodeDesc from keyword fields; tensors give their device
    pointers, None gives NULL."""
    d = FfnDecodeDesc()
    for k, v in kw.items():
        if isinstance(v, torch.Tensor):
            v = v.data_ptr()
        setattr(d, k, v)
    return d


def frag_major(x: torch.Tensor) -> torch.Tensor:
    """The fragment-major copy of an [m, k] matrix (m <= 64, k % 32 == 0) as
    loom_linear_multi_desc.x_frag expects it (rows padded to a multiple of 16
    with zeros), built with torch ops (tests and one-off callers)."""
    m, k = x.shape
    mp = -(-m // 16) * 16
    xp = torch.zeros(mp, k, dtype=x.dtype, device=x.device)
    xp[:m] = x
    # [j, r, s, q, e] -> [j, s, q, r, e]: piece (j, s, l = r + 16 q) holds row 16j + r, cols 32s + 8q ..
    return xp.view(mp // 16, 16, k // 32, 4, 8).permute(0, 2, 3, 1, 4).contiguous().view(-1)


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return c_void_p(torch.cuda.current_stream(t.device).cuda_stream)
