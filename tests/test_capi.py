"""CPU checks of the C-ABI boundary: the library loads, exports every symbol the
header declares, and the Python mirror/drop-in reject bad input like the
reference does (no GPU compute here)."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "loom_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(loom_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from loom_amd import _lib
    lib = _lib.load()
    syms = declared_symbols()
    assert "loom_paraplex_forward" in syms and len(syms) >= 15
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    assert lib.loom_abi_version() == 10
    # every declared compute entry point has a ctypes signature
    compute = [s for s in syms if s not in ("loom_last_error", "loom_abi_version")]
    bound = set(_lib.SIGNATURES) | set(_lib.QUERIES)
    assert set(compute) == bound, set(compute) ^ bound
    # chunk records [B, KVH, chunks, record] fp32; chunks = min(~1.5 blocks per CU over
    # the B*KVH rows, ceil(max_len / 128)) = min(96, 3) with no device (256 CUs assumed)
    assert lib.loom_gqa_workspace_bytes(2, 300, 8, 2, 96) == 2 * 2 * 3 * (8 + 2 * 4 * 96) * 4
    # the ctypes mirror of the descriptor struct has the C layout
    assert lib.loom_linear_multi_desc_bytes() == ctypes.sizeof(_lib.LinearMultiDesc)
    assert lib.loom_ffn_decode_desc_bytes() == ctypes.sizeof(_lib.FfnDecodeDesc)


def test_error_channel_reports_argument_errors():
    from loom_amd import _lib
    with pytest.raises(RuntimeError, match="axis must be 0"):
        # argument validation happens before any device work
        _lib.call("loom_tria_depth_forward", 0, ctypes.c_void_p(16), ctypes.c_void_p(16),
                  ctypes.c_void_p(16), None, None, None, None, None, None, None, 1, 1, 1,
                  0.05, 7, None)
    with pytest.raises(RuntimeError, match="K=0"):
        _lib.call("loom_final_ca_sparse_forward", 0, *([ctypes.c_void_p(16)] * 5), None,
                  1, 1, 0, 8, 1.0, None)
    p = ctypes.c_void_p(16)
    with pytest.raises(RuntimeError, match="paraplex_tria_endpoint: bad shape"):
        # H odd: the column pairs need H even
        _lib.call("loom_paraplex_tria_endpoint_forward", 1, p, p, p, p, p, p, 3.0, p, p, None,
                  None, p, p, p, None, 1, 1, 3, 0.0375, 0, None)


def test_drop_in_modules_expose_reference_names():
    from kernels.build import EXPORTS, build_or_load
    for ext, names in EXPORTS.items():
        mod = build_or_load(ext, ["ignored.cu"], ptx_kernels={"x": "y"})
        for n in names:
            assert callable(getattr(mod, n)), (ext, n)
    with pytest.raises(RuntimeError, match="unknown extension"):
        build_or_load("loomformer_chunk_attn", [])


def test_mirror_rejects_cpu_tensors_like_the_reference():
    from loom_amd import ops
    x = torch.zeros(2, 3, 8)
    with pytest.raises(RuntimeError, match="CUDA tensors required"):
        ops.paraplex_forward(x, x, x, torch.zeros(8), torch.zeros(2, 8), torch.zeros(8),
                             torch.empty(0, dtype=torch.bool), torch.ones(()), 0, False, 0.99, 3.0)
    with pytest.raises(RuntimeError, match="must be CUDA"):
        ops.tria_step_forward(x, x, x, torch.zeros(2, 3, 8, 3, 3), 0.05, 0)
    with pytest.raises(RuntimeError, match="training-only"):
        ops.paraplex_backward()


def test_tria_chunked_fires_rejects_bad_boundary_lists():
    """The boundary list is validated on the host before any device work."""
    from loom_amd import _lib
    lib = _lib.load()
    arr = lambda *v: (ctypes.c_int64 * len(v))(*v)
    # T=30, W=8: grid positions 7, 15, 23 must be present
    assert lib.loom_tria_chunked_fires_workspace_bytes(3, 30, 128, arr(7, 15, 23), 3) > 0
    args = lambda b, n: (0, ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 3 * 30 * 4, 4,
                         None, None, b, n, ctypes.c_void_p(16), None, None, ctypes.c_void_p(16),
                         1 << 30, 3, 30, 4, 8, 0.05, 0.1, 1e-6, None)
    with pytest.raises(RuntimeError, match="lacks 1 of the 3 grid positions"):
        _lib.call("loom_tria_chunked_forward_fires", *args(arr(3, 7, 23), 3))
    with pytest.raises(RuntimeError, match="must increase"):
        _lib.call("loom_tria_chunked_forward_fires", *args(arr(7, 7, 15, 23), 4))
    with pytest.raises(RuntimeError, match="outside"):
        _lib.call("loom_tria_chunked_forward_fires", *args(arr(7, 15, 23, 30), 4))


def test_noalloc_rejects_records_beyond_the_scratch():
    """The static-scratch decode step refuses shapes whose chunk records exceed
    its array before any device call (null tensors: nothing is dereferenced)."""
    from loom_amd import _lib
    lib = _lib.load()
    B, QH, KVH, HD, length = 4096, 8, 1, 128, 4096
    need = lib.loom_gqa_workspace_bytes(B, length, QH, KVH, HD)
    assert need > 4 << 20
    with pytest.raises(RuntimeError, match="static scratch"):
        _lib.call("loom_gqa_decode_step_noalloc", 1, None, None, None, KVH * length * HD, HD,
                  length * HD, None, None, None, None, None, QH * HD, B, length, None, QH, KVH,
                  HD, None)


def test_gemm_shared_tiles_is_a_process_switch():
    """loom_gemm_shared_tiles sets the tile mode and returns the previous one
    (host-side state: no device needed)."""
    from loom_amd import _lib
    lib = _lib.load()
    prev = lib.loom_gemm_shared_tiles(1)
    try:
        assert lib.loom_gemm_shared_tiles(1) == 1
        assert lib.loom_gemm_shared_tiles(0) == 1
        assert lib.loom_gemm_shared_tiles(7) == 0      # any nonzero value turns it on
        assert lib.loom_gemm_shared_tiles(0) == 1
    finally:
        lib.loom_gemm_shared_tiles(prev)
