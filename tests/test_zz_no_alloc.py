"""loom_gqa_decode_step_noalloc (static per-device scratch, no allocation)
against loom_gqa_decode_step with a caller workspace: two calls in a row, the
second on a smaller input, with bit-identical outputs and cache rows (both
entry points run the same kernels)."""
import pytest
import torch

from oracle import ops as ref

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _tables(HD, n):
    inv, af = ref.yarn_inv_freq(HD, 10000.0, 4.0, 256, 32.0, 1.0)
    return ref.yarn_cos_sin(inv, af, n)


def _case(lib, dtype, B, QH, KVH, HD, length, seed):
    """Run both entry points on copies of the same inputs; return both result sets."""
    from loom_amd import _lib
    P = _lib.ptr
    cap = length + 3
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(B, (QH + 2 * KVH) * HD, generator=g).to(DEV, dtype)
    kc0 = torch.randn(B, KVH, cap, HD, generator=g).to(DEV, dtype)      # head-major cache
    vc0 = torch.randn(B, KVH, cap, HD, generator=g).to(DEV, dtype)
    cos, sin = (t.to(DEV) for t in _tables(HD, cap))
    code = _lib.dtype_code(qkv)
    st = _lib.stream_of(qkv)
    sb, stt, sh = KVH * cap * HD, HD, cap * HD
    res = []
    for noalloc in (False, True):
        kc, vc = kc0.clone(), vc0.clone()
        q = torch.full((B, QH, HD), float("nan"), device=DEV, dtype=dtype)
        c = torch.full_like(q, float("nan"))
        kx = torch.full_like(q, float("nan"))
        if noalloc:
            _lib.call("loom_gqa_decode_step_noalloc", code, P(qkv), P(kc), P(vc), sb, stt, sh,
                      P(cos), P(sin), P(q), P(c), P(kx), QH * HD, B, length, None, QH, KVH, HD, st)
        else:
            nb = lib.loom_gqa_workspace_bytes(B, length, QH, KVH, HD)
            ws = torch.full((nb // 4 + 64,), float("nan"), device=DEV)
            _lib.call("loom_gqa_decode_step", code, P(qkv), P(kc), P(vc), sb, stt, sh, P(cos),
                      P(sin), P(q), P(c), P(kx), QH * HD, P(ws), nb, B, length, None, QH, KVH, HD,
                      st)
        torch.cuda.synchronize()
        res.append((q, c, kx, kc, vc))
    return res


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_step_equals_workspace_step_twice(dtype):
    from loom_amd import _lib
    lib = _lib.load()
    # the second call is smaller (fewer rows, shorter context, fewer chunk
    # records), so stale records of the first call sit in the scratch
    for (B, QH, KVH, HD, length, seed) in ((32, 8, 2, 96, 2100, 1), (3, 8, 2, 96, 300, 2)):
        print(f"noalloc case dtype={dtype} B={B} len={length}", flush=True)
        want, got = _case(lib, dtype, B, QH, KVH, HD, length, seed)
        for name, a, b in zip(("q", "c", "kctx", "k_cache", "v_cache"), want, got):
            assert torch.equal(a, b), (name, B, length)
        assert not torch.isnan(got[1].float()).any()
