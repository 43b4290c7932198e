"""GPU parity of the chunked Tria path (loom_tria_chunked_forward and the
readout) against the CPU oracle's chunk-by-chunk restatement of
Model._forward_chunked (oracle.ops.tria_chunked, itself pinned against the
decode step's Tria bookkeeping in test_oracle_props.py).

The kernel composes each chunk's tokens into one product and applies the seed
at the scan (N is a positive rescale, so the two orders agree up to the eps
inside N and fp32 rounding); fp32 tolerance rtol 1e-3 as the north star
states, bf16 inputs are rounded first and the oracle sees the same values.
"""
import pytest
import torch

from oracle import ops as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from loom_amd import _lib
    _lib.load()


def _inputs(seed, L, B, T, H, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(L, B, T, H, generator=g).to(dtype) for _ in range(3)]


@pytest.mark.parametrize("L,B,T,H,W,alpha", [
    (24, 2, 256, 300, 64, 0.025),    # TR layer count, H not a multiple of the block
    (5, 2, 200, 40, 64, 0.3),        # ragged last chunk
    (3, 3, 33, 7, 1, 0.2),           # every token a chunk
    (4, 1, 50, 9, 64, 0.2),          # one chunk: no keys
    (1, 2, 40, 17, 8, 0.5),          # single layer (init only)
])
def test_tria_chunked_matches_oracle(L, B, T, H, W, alpha):
    from loom_amd import ops
    r, i, o = _inputs(100 + L + T, L, B, T, H)
    keys, depth = ops.tria_chunked_forward(r.to(DEV), i.to(DEV), o.to(DEV), alpha, W, 0.1,
                                           want_depth=True)
    w_keys, w_depth = ref.tria_chunked(r, i, o, alpha, W, 0.1)
    assert keys.shape == w_keys.shape
    torch.testing.assert_close(keys.cpu(), w_keys, rtol=1e-3, atol=1e-4)
    torch.testing.assert_close(depth.cpu(), w_depth, rtol=1e-3, atol=1e-4)


def test_tria_chunked_resets():
    """Document starts inside a chunk, at a chunk start (suppresses the fire
    before it and the seed) and on the last token."""
    from loom_amd import ops
    L, B, T, H, W = 6, 3, 96, 70, 16
    r, i, o = _inputs(7, L, B, T, H)
    reset = torch.zeros(B, T, dtype=torch.bool)
    reset[0, 0] = True
    reset[0, 21] = True
    reset[1, 32] = True
    reset[1, 33] = True
    reset[2, 95] = True
    keys, depth = ops.tria_chunked_forward(r.to(DEV), i.to(DEV), o.to(DEV), 0.2, W, 0.1,
                                           reset=reset.to(DEV), want_depth=True)
    w_keys, w_depth = ref.tria_chunked(r, i, o, 0.2, W, 0.1, reset)
    torch.testing.assert_close(keys.cpu(), w_keys, rtol=1e-3, atol=1e-4)
    torch.testing.assert_close(depth.cpu(), w_depth, rtol=1e-3, atol=1e-4)


def test_tria_chunked_bf16_inputs():
    from loom_amd import ops
    L, B, T, H, W = 8, 2, 130, 64, 32
    r, i, o = _inputs(9, L, B, T, H, torch.bfloat16)
    keys, depth = ops.tria_chunked_forward(r.to(DEV), i.to(DEV), o.to(DEV), 0.1, W, 0.1,
                                           want_depth=True)
    w_keys, w_depth = ref.tria_chunked(r.float(), i.float(), o.float(), 0.1, W, 0.1)
    torch.testing.assert_close(keys.cpu(), w_keys, rtol=1e-3, atol=1e-4)
    torch.testing.assert_close(depth.float().cpu(), w_depth, rtol=2e-2, atol=1e-2)


def test_tria_chunked_strided_layers_and_repeat():
    """Layers at a stride larger than one slice; a second call with the same
    workspace contents left over gives the same keys."""
    from loom_amd import _lib, ops
    from loom_amd._lib import call, dtype_code, ptr, stream_of
    L, B, T, H, W = 6, 2, 64, 33, 16
    r, i, o = _inputs(11, L, B, T, H)
    pad = 5
    big = [torch.zeros(L, B * T * H + pad) for _ in range(3)]
    for dst, src in zip(big, (r, i, o)):
        dst[:, :B * T * H] = src.reshape(L, -1)
    rd, idv, od = (x.to(DEV) for x in big)
    K = T // W - 1
    nbytes = _lib.load().loom_tria_chunked_workspace_bytes(B, T, H, W)
    ws = torch.full((nbytes,), 0x7F, dtype=torch.uint8, device=DEV)
    w_keys, _ = ref.tria_chunked(r, i, o, 0.2, W, 0.1)
    for _ in range(2):
        keys = torch.empty(B, K, H, 3, 3, device=DEV)
        call("loom_tria_chunked_forward", dtype_code(rd), ptr(rd), ptr(idv), ptr(od),
             B * T * H + pad, L, None, ptr(keys), None, ptr(ws), nbytes, B, T, H, W, 0.2, 0.1,
             1e-6, stream_of(rd))
        torch.testing.assert_close(keys.cpu(), w_keys, rtol=1e-3, atol=1e-4)


def test_tria_chunked_explicit_fires_match_reference_keys():
    """loom_tria_chunked_forward_fires on the fixture Model._forward_chunked
    wrote with <CARRY> fires: keys and validity against the reference's own,
    the depth output against the oracle."""
    import numpy as np
    import os
    from loom_amd import ops
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "chunked_keys.npz"))
    t = lambda k: torch.from_numpy(z[k])
    r, i, o = t("r"), t("i"), t("o")
    alpha, W, beta = float(z["alpha"]), int(z["window"]), float(z["polarm_beta"])
    keys, depth, valid = ops.tria_chunked_forward(
        r.to(DEV), i.to(DEV), o.to(DEV), alpha, W, beta, reset=t("reset").to(DEV), want_depth=True,
        explicit_fire=t("explicit_fire").to(DEV), return_valid=True)
    torch.testing.assert_close(keys.cpu(), t("keys"), rtol=1e-3, atol=1e-4)
    bounds = [3, 4, 5, 7, 10, 15, 23, 29]
    assert torch.equal(valid.cpu(), t("fire_mask")[:, bounds])
    _, w_depth = ref.tria_chunked(r, i, o, alpha, W, beta, t("reset"), t("explicit_fire"))
    torch.testing.assert_close(depth.cpu(), w_depth, rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("L,B,T,H,W,density,dtype", [
    (5, 4, 70, 40, 16, 0.05, torch.float32),    # sparse ragged fires, L not a multiple of 3
    (6, 3, 33, 300, 8, 0.5, torch.float32),     # dense fires: many one-token chunks
    (10, 2, 130, 64, 32, 0.03, torch.bfloat16),
])
def test_tria_chunked_explicit_fires_match_oracle(L, B, T, H, W, density, dtype):
    from loom_amd import ops
    r, i, o = _inputs(31 + T, L, B, T, H, dtype)
    g = torch.Generator().manual_seed(5 + T)
    fire = torch.rand(B, T, generator=g) < density
    fire[0, T - 1] = True                       # the tail chunk becomes a boundary
    fire[B - 1, W - 1] = True                   # an explicit fire on a grid position
    reset = torch.rand(B, T, generator=g) < 0.03
    reset[:, 0] = True
    reset[1, W] = True                          # a document start after a grid boundary
    keys, depth, valid = ops.tria_chunked_forward(
        r.to(DEV), i.to(DEV), o.to(DEV), 0.2, W, 0.1, reset=reset.to(DEV), want_depth=True,
        explicit_fire=fire.to(DEV), return_valid=True)
    w_keys, w_depth, w_valid = ref.tria_chunked(r.float(), i.float(), o.float(), 0.2, W, 0.1, reset,
                                                fire, return_valid=True)
    assert keys.shape == w_keys.shape
    assert torch.equal(valid.cpu(), w_valid)
    torch.testing.assert_close(keys.cpu(), w_keys, rtol=1e-3, atol=1e-4)
    tol = dict(rtol=1e-3, atol=1e-4) if dtype == torch.float32 else dict(rtol=2e-2, atol=1e-2)
    torch.testing.assert_close(depth.float().cpu(), w_depth, **tol)


def test_tria_chunked_fires_without_explicit_equals_grid_entry():
    """An explicit-fire mask with no fires gives the grid entry's keys."""
    from loom_amd import ops
    L, B, T, H, W = 4, 2, 64, 33, 16
    r, i, o = (x.to(DEV) for x in _inputs(13, L, B, T, H))
    k1, _ = ops.tria_chunked_forward(r, i, o, 0.2, W, 0.1)
    k2, _ = ops.tria_chunked_forward(r, i, o, 0.2, W, 0.1,
                                     explicit_fire=torch.zeros(B, T, dtype=torch.bool, device=DEV))
    assert torch.equal(k1, k2)


def test_tria_readout_matches_oracle():
    from loom_amd import ops
    g = torch.Generator().manual_seed(12)
    B, K, H, N = 2, 5, 300, 96
    carry = ref.local_normalize(torch.randn(B, K, H, 3, 3, generator=g))
    key_w = torch.randn(32, 9, generator=g) * 1.5
    query = torch.randn(32, generator=g)
    score_w = ref.make_score_w(key_w, query, torch.tensor(1.3))
    pw, pb = torch.randn(32, 9, generator=g) / 3, torch.randn(32, generator=g) / 3
    uw, ub = torch.randn(N, 32, generator=g) / 6, torch.randn(N, generator=g) / 6
    z = ops.tria_readout(carry.to(DEV), score_w.to(DEV), pw.to(DEV), pb.to(DEV), uw.to(DEV),
                         ub.to(DEV))
    want = ref.tria_readout(carry, score_w, pw, pb, uw, ub)
    torch.testing.assert_close(z.cpu(), want, rtol=1e-3, atol=1e-4)
