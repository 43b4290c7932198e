"""GPU parity of the decode-step kernels against fp32 references (oracle ops
or plain torch on the CPU)."""
import contextlib
import ctypes
import math

import pytest
import torch

from oracle import ops as ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float32: dict(rtol=1e-3, atol=1e-4), torch.bfloat16: dict(rtol=2e-2, atol=1e-2)}
DTYPES = [torch.float32, torch.bfloat16]


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def L():
    from loom_amd import _lib
    return _lib


def P(t):
    return L().ptr(t)


def S(t):
    return L().stream_of(t)


def code(t):
    return L().dtype_code(t)


def host(t):
    return t.detach().float().cpu()


def check(got, want, dtype):
    torch.testing.assert_close(host(got), want.float(), **TOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,N", [(32, 768), (3, 32), (5, 20), (1, 2048)])
def test_rms_norm(dtype, rows, N):
    """final_norm's RMSNorm (loomformer.py:3460-3464) against the oracle's
    restatement, with the weight in the model dtype."""
    from oracle.model import rms_norm
    g = torch.Generator().manual_seed(rows * 7 + N)
    x = (torch.randn(rows, N, generator=g) * 3).to(DEV, dtype)
    w = (torch.randn(N, generator=g) * 0.5 + 1).to(DEV, dtype)
    out = torch.empty_like(x)
    L().call("loom_rms_norm", code(x), P(x), P(w), P(out), rows, N, 1e-6, S(x))
    want = rms_norm(x.cpu(), w.cpu()).float()     # in the model dtype, as the reference rounds
    check(out, want, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,N", [(32, 768), (3, 32), (5, 20), (1, 2048)])
def test_add_layernorm(dtype, rows, N):
    g = torch.Generator().manual_seed(rows + N)
    a = torch.randn(rows, N, generator=g).to(DEV, dtype)
    b = torch.randn(rows, N, generator=g).to(DEV, dtype)
    w = torch.randn(N, generator=g).to(DEV)
    bb = torch.randn(N, generator=g).to(DEV)
    out = torch.empty_like(a)
    L().call("loom_add_layernorm", code(a), P(a), P(b), P(w), P(bb), P(out), rows, N, 1e-5, S(a))
    want = torch.nn.functional.layer_norm(host(a) + host(b), (N,), host(w), host(bb), 1e-5)
    check(out, want, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_append(dtype):
    B, QH, KVH, HD, max_len, pos = 3, 8, 2, 96, 40, 17
    g = torch.Generator().manual_seed(1)
    qkv = torch.randn(B, (QH + 2 * KVH) * HD, generator=g).to(DEV, dtype)
    inv, att = ref.yarn_inv_freq(HD, 10000.0, 4.0, 16, 32.0, 1.0)
    cos, sin = ref.yarn_cos_sin(inv, att, max_len)
    kc = torch.zeros(B, max_len, KVH, HD, device=DEV, dtype=dtype)
    vc = torch.zeros_like(kc)
    q = torch.empty(B, QH, HD, device=DEV, dtype=dtype)
    cos_d, sin_d = cos.to(DEV), sin.to(DEV)       # keep the device copies alive across the call
    L().call("loom_rope_append", code(qkv), P(qkv), P(q), P(kc), P(vc), P(cos_d), P(sin_d),
             B, pos, None, QH, KVH, HD, max_len * KVH * HD, KVH * HD, HD, S(qkv))
    x = host(qkv)
    c, s = cos[pos].view(1, 1, HD), sin[pos].view(1, 1, HD)
    check(q, ref.apply_rope(x[:, :QH * HD].view(B, QH, HD), c, s), dtype)
    check(kc[:, pos], ref.apply_rope(x[:, QH * HD:(QH + KVH) * HD].view(B, KVH, HD), c, s), dtype)
    check(vc[:, pos], x[:, (QH + KVH) * HD:].view(B, KVH, HD), dtype)
    assert float(host(kc[:, pos + 1]).abs().max()) == 0.0
    # the position can come from device memory instead (graph replay)
    pos_d = torch.tensor([pos + 1], dtype=torch.int64, device=DEV)
    L().call("loom_rope_append", code(qkv), P(qkv), P(q), P(kc), P(vc), P(cos_d), P(sin_d),
             B, 0, P(pos_d), QH, KVH, HD, max_len * KVH * HD, KVH * HD, HD, S(qkv))
    c1, s1 = cos[pos + 1].view(1, 1, HD), sin[pos + 1].view(1, 1, HD)
    check(kc[:, pos + 1], ref.apply_rope(x[:, QH * HD:(QH + KVH) * HD].view(B, KVH, HD), c1, s1), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,QH,KVH,HD,length", [(4, 8, 2, 96, 1), (2, 8, 2, 96, 255), (2, 8, 2, 96, 256),
                                                 (2, 8, 2, 96, 257), (3, 8, 2, 96, 1000),
                                                 (3, 4, 2, 8, 37), (2, 4, 1, 64, 300),
                                                 (32, 8, 2, 96, 2100)])
def test_gqa_decode_attention(dtype, B, QH, KVH, HD, length):
    from loom_amd import _lib
    max_len = length + 5
    g = torch.Generator().manual_seed(length + HD)
    q = torch.randn(B, QH, HD, generator=g).to(DEV, dtype)
    kc = torch.randn(B, max_len, KVH, HD, generator=g).to(DEV, dtype)
    vc = torch.randn(B, max_len, KVH, HD, generator=g).to(DEV, dtype)
    c = torch.empty(B, QH, HD, device=DEV, dtype=dtype)
    kx = torch.empty_like(c)
    nb = _lib.load().loom_gqa_workspace_bytes(B, max_len, QH, KVH, HD)
    ws = torch.full((nb // 4 + 1,), float("nan"), device=DEV)   # chunk records: scratch, no initial contents
    _lib.call("loom_gqa_decode_attention", code(q), P(q), P(kc), P(vc), max_len * KVH * HD, KVH * HD,
              HD, P(c), P(kx), P(ws), nb, B, length, None, QH, KVH, HD, S(q))
    G = QH // KVH
    K = host(kc)[:, :length].repeat_interleave(G, dim=2).transpose(1, 2)   # [B,QH,len,HD]
    V = host(vc)[:, :length].repeat_interleave(G, dim=2).transpose(1, 2)
    a = torch.softmax((host(q).unsqueeze(2) @ K.transpose(-1, -2)) / math.sqrt(HD), dim=-1)
    check(c, (a @ V).squeeze(2), dtype)
    check(kx, (a @ K).squeeze(2), dtype)
    # device-resident length (pos + 1) with the launch covering the whole capacity
    c.zero_()
    kx.zero_()
    pos_d = torch.tensor([length - 1], dtype=torch.int64, device=DEV)
    _lib.call("loom_gqa_decode_attention", code(q), P(q), P(kc), P(vc), max_len * KVH * HD, KVH * HD,
              HD, P(c), P(kx), P(ws), nb, B, max_len, P(pos_d), QH, KVH, HD, S(q))
    check(c, (a @ V).squeeze(2), dtype)
    check(kx, (a @ K).squeeze(2), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,QH,KVH,HD,start,Tc", [(2, 8, 2, 96, 0, 128), (3, 8, 2, 96, 300, 70),
                                                  (2, 4, 1, 64, 64, 33), (2, 8, 1, 128, 5, 40),
                                                  (2, 4, 2, 32, 17, 100), (1, 8, 4, 96, 1000, 16),
                                                  (2, 4, 2, 8, 9, 20)])
def test_gqa_prefill_matches_causal_attention(dtype, B, QH, KVH, HD, start, Tc):
    """loom_gqa_prefill: RoPE + cache append of a chunk of Tc tokens at
    positions start.., then token t attends to cache rows 0..start+t (the
    earlier chunks' rows already in the cache); both readouts against a torch
    fp32 causal attention over the same (rounded) rows.  head_dim 8 takes the
    element-per-thread RoPE/append kernel, the others the 16-byte one."""
    from loom_amd import _lib
    g = torch.Generator().manual_seed(B + QH + HD + start + Tc)
    max_len = start + Tc + 3
    cos, sin = _rope_tables(HD, max_len)
    cos_d, sin_d = cos.to(DEV), sin.to(DEV)
    kc = torch.zeros(B, max_len, KVH, HD, device=DEV, dtype=dtype)
    vc = torch.zeros_like(kc)
    kc[:, :start] = torch.randn(B, start, KVH, HD, generator=g).to(DEV, dtype)
    vc[:, :start] = torch.randn(B, start, KVH, HD, generator=g).to(DEV, dtype)
    W = (QH + 2 * KVH) * HD
    qkv = torch.randn(B, Tc, W, generator=g).to(DEV, dtype)
    q = torch.empty(B, Tc, QH, HD, device=DEV, dtype=dtype)
    c = torch.empty(B, Tc, QH * HD, device=DEV, dtype=dtype)
    kx = torch.empty_like(c)
    _lib.call("loom_gqa_prefill", code(qkv), P(qkv), W, P(kc), P(vc), max_len * KVH * HD, KVH * HD, HD,
              P(cos_d), P(sin_d), P(q), P(c), P(kx), QH * HD, B, Tc, start, max_len, QH, KVH, HD, S(qkv))
    x = host(qkv)
    cs, sn = cos[start:start + Tc].view(1, Tc, 1, HD), sin[start:start + Tc].view(1, Tc, 1, HD)
    wq = ref.apply_rope(x[..., :QH * HD].reshape(B, Tc, QH, HD), cs, sn)
    wk = ref.apply_rope(x[..., QH * HD:(QH + KVH) * HD].reshape(B, Tc, KVH, HD), cs, sn)
    check(q, wq, dtype)
    check(kc[:, start:start + Tc], wk, dtype)
    # attention over the cache as stored (rounded to dtype), rows 0..start+t
    Kall = host(kc)[:, :start + Tc].repeat_interleave(QH // KVH, dim=2).transpose(1, 2)   # [B,QH,L,HD]
    Vall = host(vc)[:, :start + Tc].repeat_interleave(QH // KVH, dim=2).transpose(1, 2)
    qq = host(q).transpose(1, 2)                                                         # [B,QH,Tc,HD]
    sc = (qq @ Kall.transpose(-1, -2)) / math.sqrt(HD)
    mask = torch.arange(start + Tc)[None, :] <= (start + torch.arange(Tc))[:, None]
    a = torch.softmax(sc.masked_fill(~mask, float("-inf")), dim=-1)
    check(c, (a @ Vall).transpose(1, 2).reshape(B, Tc, QH * HD), dtype)
    check(kx, (a @ Kall).transpose(1, 2).reshape(B, Tc, QH * HD), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,Tc,start,HD,hist,shared", [(32, 128, 37, 96, True, False),
                                                       (16, 17, 500, 96, False, False),
                                                       (2, 20, 3, 96, True, False), (4, 70, 9, 64, True, False),
                                                       (32, 128, 37, 96, True, True),
                                                       (16, 17, 500, 96, False, True)])
def test_prefill_qkv_matches_products_and_rope(dtype, B, Tc, start, HD, hist, shared):
    """loom_prefill_qkv = the qkv product, loom_gqa_prefill's RoPE + cache append
    and the history projection, to the bit (bf16, head_dim 96, >= 256 rows: one
    launch with the RoPE in the product's epilogue; the rest: the separate
    products and RoPE launch), and against torch: the product rounded to the
    dtype, then the oracle's RoPE.  `shared`: in shared-tile mode (128 x 192
    tiles), as the chunked prefill runs it."""
    with shared_tiles(shared):
        _prefill_qkv_case(dtype, B, Tc, start, HD, hist)


def _prefill_qkv_case(dtype, B, Tc, start, HD, hist):
    from loom_amd import _lib
    QH, KVH, N = 8, 2, 768
    W = (QH + 2 * KVH) * HD
    M = B * Tc
    g = torch.Generator().manual_seed(B * Tc + start + HD)
    max_len = start + Tc + 2
    cos, sin = _rope_tables(HD, max_len)
    cos_d, sin_d = cos.to(DEV), sin.to(DEV)
    x = torch.randn(M, N, generator=g).to(DEV, dtype)
    wq = (torch.randn(W, N, generator=g) * N ** -0.5).to(DEV, dtype)
    wh = (torch.randn(2 * N, N, generator=g) * N ** -0.5).to(DEV, dtype)
    cs = (max_len * KVH * HD, HD, max_len * HD)          # head-major cache [B, KVH, max_len, HD]
    outs = []
    for fused in (True, False):
        kc = torch.zeros(B, KVH, max_len, HD, device=DEV, dtype=dtype)
        vc = torch.zeros_like(kc)
        q = torch.zeros(M, QH * HD, device=DEV, dtype=dtype)
        hs = torch.zeros(M, 3, 2 * N, device=DEV, dtype=dtype)   # history slot 1 of [M, 3, 2N]
        qkv = torch.zeros(M, W, device=DEV, dtype=dtype)
        if fused:
            _lib.call("loom_prefill_qkv", code(x), P(x), N, P(wq), P(wh) if hist else None,
                      P(hs[:, 1]) if hist else None, 3 * 2 * N, 2 * N, P(qkv), P(q), P(kc), P(vc), *cs,
                      P(cos_d), P(sin_d), B, Tc, start, max_len, N, QH, KVH, HD, S(x))
        else:
            _lib.call("loom_linear", code(x), P(x), N, P(wq), N, None, None, 0.0, None, P(qkv), W, M,
                      W, N, S(x))
            if hist:
                _lib.call("loom_linear", code(x), P(x), N, P(wh), N, None, None, 0.0, None, P(hs[:, 1]),
                          3 * 2 * N, M, 2 * N, N, S(x))
            c = torch.empty(M, QH * HD, device=DEV, dtype=dtype)
            kx = torch.empty_like(c)
            _lib.call("loom_gqa_prefill", code(x), P(qkv), W, P(kc), P(vc), *cs, P(cos_d), P(sin_d),
                      P(q), P(c), P(kx), QH * HD, B, Tc, start, max_len, QH, KVH, HD, S(x))
        torch.cuda.synchronize()
        outs.append((q, kc, vc, hs))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    q, kc, vc, hs = outs[0]
    y = (host(x) @ host(wq).t()).to(dtype).float().view(B, Tc, QH + 2 * KVH, HD)
    csn, snn = cos[start:start + Tc].view(1, Tc, 1, HD), sin[start:start + Tc].view(1, Tc, 1, HD)
    check(q.view(B, Tc, QH, HD), ref.apply_rope(y[:, :, :QH], csn, snn), dtype)
    check(kc[:, :, start:start + Tc].transpose(1, 2), ref.apply_rope(y[:, :, QH:QH + KVH], csn, snn), dtype)
    check(vc[:, :, start:start + Tc].transpose(1, 2), y[:, :, QH + KVH:], dtype)
    if hist:
        check(hs[:, 1], host(x) @ host(wh).t(), dtype)
    assert not kc[:, :, :start].any() and not kc[:, :, start + Tc:].any()


@contextlib.contextmanager
def shared_tiles(on):
    """The library's shared-tile mode set for the block, restored after."""
    lib = L().load()
    prev = lib.loom_gemm_shared_tiles(1 if on else 0)
    try:
        yield
    finally:
        lib.loom_gemm_shared_tiles(prev)


@pytest.mark.parametrize("M,N,K", [(4096, 3072, 768), (4000, 1152, 768), (300, 768, 1536),
                                   (4096, 768, 3072), (4096, 1536, 768)])
def test_shared_tiles_equal_default_tiles(M, N, K):
    """Shared-tile mode (128 x 192 tiles of four waves, two blocks per CU)
    against the default tiles: loom_linear with bias, gate and residual and
    loom_linear_ln (whose split-K count may differ) against torch in both
    modes, the W_imag gather product of both modes against each other."""
    from loom_amd import _lib, ops
    dt = torch.bfloat16
    g = torch.Generator().manual_seed(M + N + K)
    r = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(DEV, dt)
    x, w = r(M, K), r(N, K, sc=K ** -0.5)
    bias = torch.randn(N, generator=g).to(DEV)
    p, res = r(M, N), r(M, N)
    QH, HD, Hq = 8, 96, 384
    u = r(1, M, QH * HD)
    q, kc, c, d = (r(1, M, QH, HD) for _ in range(4))
    w_imag = r(QH * Hq, ref.imag_in(QH * HD, HD, "head"), sc=0.03)
    gam = (torch.rand(N, generator=g) + 0.5).to(DEV)
    bet = torch.randn(N, generator=g).to(DEV)
    nb = L().load().loom_linear_ln_workspace_bytes(M, N)
    ws = torch.empty(nb // 4, device=DEV)
    outs = []
    for on in (False, True):
        with shared_tiles(on):
            y = ops.linear(x, w, bias, gate_p=p, gate_alpha=0.2, residual=res)
            beta = ops.beta_forward_cuda(u, q, kc, c, d, w_imag, Hq, HD, QH, False)[0]
            ln = None
            if N <= 2048:                   # loom_linear_ln's row length limit
                ln = torch.zeros(M, N, device=DEV, dtype=dt)
                yy = torch.zeros(M, N, device=DEV, dtype=dt)
                desc = _lib.linear_multi_desc(x, [dict(w=w, out=yy, bias=bias)])
                _lib.call("loom_linear_ln", code(x), ctypes.byref(desc), P(gam), P(bet), 1e-5, P(ln), N,
                          P(ws), nb, None, S(x))
            torch.cuda.synchronize()
        outs.append((y, beta, ln))
    # 64-k full-line stages and 32-k stages give an MFMA's lanes different k,
    # so the two modes agree to bf16 rounding (to the bit where both pick
    # 32-k stages, as at 4096 x 3072 x 768)
    want_y = (host(x) @ host(w).T) * (1.0 + 0.2 * host(p)) + host(bias) + host(res)
    for o in outs:
        check(o[0], want_y, dt)
    check(outs[1][1], host(outs[0][1]), dt)
    if N <= 2048:
        want = torch.nn.functional.layer_norm(host(x) @ host(w).T + host(bias), (N,), host(gam), host(bet),
                                              1e-5)
        for o in outs:
            check(o[2], want, dt)


def _rope_tables(HD, n):
    inv, af = ref.yarn_inv_freq(HD, 10000.0, 4.0, 256, 32.0, 1.0)
    return ref.yarn_cos_sin(inv, af, n)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,QH,KVH,HD,length,S_,L2", [
    (32, 8, 2, 96, 700, 3, 20), (2, 8, 2, 96, 1, 1, 20), (3, 4, 2, 64, 300, 7, 8),
    (2, 8, 1, 128, 260, 12, 12), (2, 4, 2, 8, 40, 2, 4)])
def test_gqa_decode_step_depth(dtype, B, QH, KVH, HD, length, S_, L2):
    """The attention step with the depth read in the same launch gives exactly
    what the two separate entry points give (bf16 with head_dim 32-128 takes the
    fused grid, the rest runs the depth kernel after), and the depth rows match
    the oracle's softmax over the history slots."""
    from loom_amd import _lib
    max_len = length + 5
    pos = length - 1
    g = torch.Generator().manual_seed(length + 31 * S_ + HD)
    qkv = torch.randn(B, (QH + 2 * KVH) * HD, generator=g).to(DEV, dtype)
    kc0 = torch.randn(B, KVH, max_len, HD, generator=g).to(DEV, dtype)
    vc0 = torch.randn(B, KVH, max_len, HD, generator=g).to(DEV, dtype)
    hist = torch.randn(B, L2, 2 * QH * HD, generator=g).to(DEV, dtype)   # slot s = [k | v]
    dq = (torch.randn(QH, HD, generator=g) * 0.3).to(DEV, dtype)
    cos, sin = _rope_tables(HD, max_len)
    cos_d, sin_d = cos.to(DEV), sin.to(DEV)
    strides = (KVH * max_len * HD, HD, max_len * HD)
    nb = _lib.load().loom_gqa_workspace_bytes(B, max_len, QH, KVH, HD)
    pos_d = torch.tensor([pos], dtype=torch.int64, device=DEV)
    N = QH * HD
    outs = []
    for fused in (False, True):
        kc, vc = kc0.clone(), vc0.clone()
        ws = torch.zeros(nb // 4 + 1, device=DEV)
        c = torch.zeros(B, N, device=DEV, dtype=dtype)
        kx = torch.zeros_like(c)
        qo = torch.zeros_like(c)
        d = torch.zeros_like(c)
        args = (P(qkv), P(kc), P(vc), *strides, P(cos_d), P(sin_d), P(qo), P(c), P(kx), N, P(ws),
                nb, B, max_len, P(pos_d), QH, KVH, HD)
        if fused:
            _lib.call("loom_gqa_decode_step_depth", code(qkv), *args, P(dq), P(hist),
                      P(hist[:, :, N:]), L2 * 2 * N, 2 * N, S_, P(d), S(qkv))
        else:
            _lib.call("loom_gqa_decode_step", code(qkv), *args, S(qkv))
            _lib.call("loom_depth_attn_forward", code(qkv), P(dq), P(hist), P(hist[:, :, N:]),
                      L2 * 2 * N, 2 * N, P(d), None, None, B, S_, QH, HD, S(qkv))
        outs.append([host(t) for t in (c, kx, qo, d, kc, vc)])
    for x, y in zip(*outs):
        assert torch.equal(x, y)
    hk = host(hist)[:, :S_, :N].view(B, S_, QH, HD)
    hv = host(hist)[:, :S_, N:].view(B, S_, QH, HD)
    w = torch.softmax((hk * host(dq)).sum(-1) / math.sqrt(HD), dim=1)      # [B, S, QH]
    check(outs[1][3].view(B, QH, HD), (w.unsqueeze(-1) * hv).sum(1), dtype)
    # a second query over the same slots (loom_gqa_decode_step_depth2): the
    # other outputs as before, its read as fp32 rows and log-sum-exp
    dq2 = (torch.randn(QH, HD, generator=g) * 0.3).to(DEV, dtype)
    kc, vc = kc0.clone(), vc0.clone()
    ws = torch.zeros(nb // 4 + 1, device=DEV)
    c, kx, qo, d = (torch.zeros(B, N, device=DEV, dtype=dtype) for _ in range(4))
    pd = torch.full((B, QH, HD), float("nan"), device=DEV)
    pl = torch.full((B, QH), float("nan"), device=DEV)
    args = (P(qkv), P(kc), P(vc), *strides, P(cos_d), P(sin_d), P(qo), P(c), P(kx), N, P(ws),
            nb, B, max_len, P(pos_d), QH, KVH, HD, P(dq), P(dq2), P(hist), P(hist[:, :, N:]),
            L2 * 2 * N, 2 * N, S_, P(d), P(pd), P(pl), S(qkv))
    if dtype != torch.bfloat16 or HD not in (32, 64, 96, 128):
        with pytest.raises(RuntimeError, match="bf16 MFMA form"):
            _lib.call("loom_gqa_decode_step_depth2", code(qkv), *args)
        return
    _lib.call("loom_gqa_decode_step_depth2", code(qkv), *args)
    for x, y in zip([host(t) for t in (c, kx, qo, kc, vc)], [outs[1][i] for i in (0, 1, 2, 4, 5)]):
        assert torch.equal(x, y)
    torch.testing.assert_close(host(d), outs[1][3], rtol=1e-2, atol=1e-2)
    sc2 = (hk * host(dq2)).sum(-1) / math.sqrt(HD)                          # [B, S, QH]
    w2 = torch.softmax(sc2, dim=1)
    torch.testing.assert_close(pd.cpu(), (w2.unsqueeze(-1) * hv).sum(1), rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(pl.cpu(), torch.logsumexp(sc2, dim=1), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_major", [False, True])
@pytest.mark.parametrize("B,QH,KVH,HD,length", [
    (2, 8, 2, 96, 1), (3, 8, 2, 96, 255), (2, 8, 2, 96, 257), (32, 8, 2, 96, 700),
    (2, 4, 4, 64, 300), (2, 8, 1, 64, 513), (1, 4, 2, 8, 90), (2, 8, 2, 32, 256)])
def test_gqa_decode_step(dtype, head_major, B, QH, KVH, HD, length):
    """RoPE + cache append + attention + merge in one launch, against the
    oracle's RoPE and a plain softmax over the appended cache."""
    from loom_amd import _lib
    max_len = length + 7
    pos = length - 1
    g = torch.Generator().manual_seed(length * 7 + HD + QH)
    qkv = torch.randn(B, (QH + 2 * KVH) * HD, generator=g).to(DEV, dtype)
    kc = torch.randn(B, max_len, KVH, HD, generator=g).to(DEV, dtype)
    vc = torch.randn(B, max_len, KVH, HD, generator=g).to(DEV, dtype)
    kc0, vc0 = host(kc), host(vc)
    cos, sin = _rope_tables(HD, max_len)
    cos_d, sin_d = cos.to(DEV), sin.to(DEV)
    out_sb = 2 * QH * HD                            # outputs written with a row stride
    cbuf = torch.zeros(B, out_sb, device=DEV, dtype=dtype)
    kbuf = torch.zeros(B, out_sb, device=DEV, dtype=dtype)
    nb = _lib.load().loom_gqa_workspace_bytes(B, max_len, QH, KVH, HD)
    ws = torch.zeros(nb // 4 + 1, device=DEV)
    pos_d = torch.tensor([pos], dtype=torch.int64, device=DEV)
    qout = torch.zeros(B, QH, HD, device=DEV, dtype=dtype)
    # oracle: rope q and this token's k, append, attend over positions 0..pos
    x = host(qkv)
    qr = ref.apply_rope(x[:, :QH * HD].view(B, QH, HD), cos[pos], sin[pos])
    kr = ref.apply_rope(x[:, QH * HD:(QH + KVH) * HD].view(B, KVH, HD), cos[pos], sin[pos])
    vn = x[:, (QH + KVH) * HD:].view(B, KVH, HD)
    kr = kr.to(dtype).float()                       # the cache stores T
    Kc, Vc = kc0.clone(), vc0.clone()
    Kc[:, pos], Vc[:, pos] = kr, vn
    G = QH // KVH
    K = Kc[:, :length].repeat_interleave(G, dim=2).transpose(1, 2)
    V = Vc[:, :length].repeat_interleave(G, dim=2).transpose(1, 2)
    a = torch.softmax((qr.unsqueeze(2) @ K.transpose(-1, -2)) / math.sqrt(HD), dim=-1)
    # cache layouts: [B, T, KVH, HD] (stride_h = HD) or head-major [B, KVH, T, HD]
    if head_major:
        kc = kc.transpose(1, 2).contiguous()
        vc = vc.transpose(1, 2).contiguous()
        strides = (KVH * max_len * HD, HD, max_len * HD)
        view = lambda t: host(t).transpose(1, 2)   # back to [B, T, KVH, HD]
    else:
        strides = (max_len * KVH * HD, KVH * HD, HD)
        view = host
    for call in range(2):                           # host length, then device position
        cbuf.zero_()
        kbuf.zero_()
        src_k, src_v = (kc0, vc0) if not head_major else (kc0.transpose(1, 2), vc0.transpose(1, 2))
        kc.copy_(src_k.to(dtype))
        vc.copy_(src_v.to(dtype))
        _lib.call("loom_gqa_decode_step", code(qkv), P(qkv), P(kc), P(vc), *strides,
                  P(cos_d), P(sin_d), P(qout), P(cbuf), P(kbuf), out_sb, P(ws), nb, B,
                  length if call == 0 else max_len, None if call == 0 else P(pos_d), QH, KVH, HD,
                  S(qkv))
        check(cbuf[:, :QH * HD].view(B, QH, HD), (a @ V).squeeze(2), dtype)
        check(kbuf[:, :QH * HD].view(B, QH, HD), (a @ K).squeeze(2), dtype)
        check(qout, qr, dtype)
        assert bool((cbuf[:, QH * HD:] == 0).all()) and bool((kbuf[:, QH * HD:] == 0).all())
        torch.testing.assert_close(view(kc)[:, pos], kr, **TOL[dtype])
        torch.testing.assert_close(view(vc)[:, pos], vn.to(dtype).float(), rtol=0, atol=0)
        rest = [t for t in range(max_len) if t != pos]
        assert torch.equal(view(kc)[:, rest], kc0[:, rest])
        assert torch.equal(view(vc)[:, rest], vc0[:, rest])


@pytest.mark.parametrize("dtype", DTYPES)
def test_decode_temporal(dtype):
    B, H = 4, 300
    g = torch.Generator().manual_seed(3)
    depth = ref.local_normalize(torch.randn(B, H, 3, 3, generator=g)).to(DEV, dtype)
    prev = ref.local_normalize(torch.randn(B, H, 3, 3, generator=g)).to(DEV, dtype)
    reset = torch.tensor([1, 0, 0, 1], dtype=torch.uint8)
    fire = torch.tensor([0, 1, 0, 1], dtype=torch.uint8)
    out = torch.empty_like(depth)
    reset_d, fire_d = reset.to(DEV), fire.to(DEV)
    L().call("loom_tria_decode_temporal", code(depth), P(depth), P(prev), P(reset_d),
             P(fire_d), P(out), B, H, 0.1, 1e-6, S(depth))
    D, Pv = host(depth), host(prev)
    doc = torch.where(reset.bool()[:, None, None, None], D, ref.local_normalize(D @ Pv))
    doc = torch.where(fire.bool()[:, None, None, None], ref.polarm(doc, 0.1), doc)
    check(out, doc, dtype)
    # first token: no previous state, no fire -> the depth carry itself
    L().call("loom_tria_decode_temporal", code(depth), P(depth), None, None, None, P(out), B, H,
             0.1, 1e-6, S(depth))
    check(out, D, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_final_ca_strided_with_residual(dtype):
    B, Kmax, K, D = 3, 9, 4, 96
    g = torch.Generator().manual_seed(4)
    q = torch.randn(B, 1, D, generator=g).to(DEV, dtype)
    kb = torch.randn(B, Kmax, D, generator=g).to(DEV, dtype)
    vb = torch.randn(B, Kmax, D, generator=g).to(DEV, dtype)
    valid = torch.zeros(B, Kmax, dtype=torch.uint8)
    valid[0, :3] = 1
    valid[2, 1] = 1                           # row 1: no key -> output == residual
    res = torch.randn(B, 1, D, generator=g).to(DEV, dtype)
    out = torch.empty_like(res)
    valid_d = valid.to(DEV)
    L().call("loom_final_ca_sparse_strided", code(q), P(q), P(kb), P(vb), Kmax * D, P(valid_d),
             Kmax, P(res), 0.7, P(out), None, B, 1, K, None, D, D ** -0.5, S(q))
    att = ref.final_ca_sparse(host(q), host(kb)[:, :K], host(vb)[:, :K], valid[:, None, :K].bool(), D ** -0.5)
    check(out, host(res) + 0.7 * att, dtype)
    # key count from the device: K keys, and 0 keys (exact identity)
    for kd in (K, 0):
        k_d = torch.tensor([kd], dtype=torch.int64, device=DEV)
        L().call("loom_final_ca_sparse_strided", code(q), P(q), P(kb), P(vb), Kmax * D, P(valid_d),
                 Kmax, P(res), 0.7, P(out), None, B, 1, Kmax, P(k_d), D, D ** -0.5, S(q))
        if kd == 0:
            assert torch.equal(out.cpu(), res.cpu())
        else:
            check(out, host(res) + 0.7 * att, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("V", [4096, 1000, 12000, 4097, 20000])
def test_argmax_rows_first_index_on_ties(dtype, V):
    # 4096 / 1000 / 12000: vector form (1, 1 and 8 vectors per thread); 4097, 20000: scalar form
    g = torch.Generator().manual_seed(5)
    x = torch.randn(33, V, generator=g)
    x[3, 100] = x[3, V - 96] = 50.0         # tie: first index wins
    x[7, :] = 1.0                           # all equal -> 0
    x[9, V - 1] = 60.0                      # maximum at the last index
    xd = x.to(DEV, dtype)
    ids = torch.empty(33, dtype=torch.int64, device=DEV)
    L().call("loom_argmax_rows", code(xd), P(xd), 33, V, P(ids), S(xd))
    assert torch.equal(ids.cpu(), torch.argmax(host(xd), dim=-1))
    assert int(ids[3]) == 100 and int(ids[7]) == 0 and int(ids[9]) == V - 1


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("H,N", [(300, 96), (3072, 768), (1100, 40), (5000, 200)])
def test_decode_tria_readout(dtype, H, N):
    # temporal step + PolARM + slot pool + proj + up in one launch, against the
    # oracle ops with the intermediates rounded to dtype as the unfused ops store them
    B = 4
    g = torch.Generator().manual_seed(H + N)
    depth = ref.local_normalize(torch.randn(B, H, 3, 3, generator=g)).to(DEV, dtype)
    prev = ref.local_normalize(torch.randn(B, H, 3, 3, generator=g)).to(DEV, dtype)
    key_w, query = torch.randn(32, 9, generator=g) * 1.5, torch.randn(32, generator=g)
    sw = (torch.nn.functional.normalize(key_w.t() @ query, dim=0) * 2.0).to(DEV, dtype)
    pw = (torch.randn(32, 9, generator=g) / 3).to(DEV, dtype)
    pb = torch.randn(32, generator=g).to(DEV)
    uw = (torch.randn(N, 32, generator=g) / 6).to(DEV, dtype)
    ub = torch.randn(N, generator=g).to(DEV)
    reset = torch.tensor([1, 0, 0, 1], dtype=torch.uint8)
    fire = torch.tensor([0, 1, 0, 1], dtype=torch.uint8)
    reset_d, fire_d = reset.to(DEV), fire.to(DEV)
    rnd = lambda t: t.to(dtype).float()

    def want(D, Pv):
        doc = D if Pv is None else torch.where(reset.bool()[:, None, None, None], D,
                                                ref.local_normalize(D @ Pv))
        doc = torch.where(fire.bool()[:, None, None, None], ref.polarm(doc, 0.1), doc)
        doc = rnd(doc)
        pooled = rnd(ref.slot_attention_pool(doc, host(sw))[0])
        z = rnd(pooled @ host(pw).t() + host(pb))
        return doc, z @ host(uw).t() + host(ub)

    doc = prev.clone()                      # in place: prev and doc are one buffer
    a = torch.empty(B, N, device=DEV, dtype=dtype)
    nb = L().load().loom_decode_tria_readout_workspace_bytes(B, H)
    ws = torch.full((nb // 4,), float("nan"), device=DEV)   # scratch: no zeroing needed
    wd, wa = want(host(depth), host(prev))
    L().call("loom_decode_tria_readout", code(depth), P(depth), P(doc), P(reset_d), P(fire_d),
             P(doc), P(sw), P(pw), P(pb), P(uw), P(ub), P(a), P(ws), nb, B, H, N, 0.1, 1e-6,
             S(depth))
    check(doc, wd, dtype)
    check(a, wa, dtype)
    # no row fires: the state is updated, the readout (keys for a fire) is not
    calm = torch.zeros(B, dtype=torch.uint8, device=DEV)
    doc = prev.clone()
    a.fill_(3.0)
    L().call("loom_decode_tria_readout", code(depth), P(depth), P(doc), P(reset_d), P(calm),
             P(doc), P(sw), P(pw), P(pb), P(uw), P(ub), P(a), P(ws), nb, B, H, N, 0.1, 1e-6,
             S(depth))
    D, Pv = host(depth), host(prev)
    check(doc, rnd(torch.where(reset.bool()[:, None, None, None], D, ref.local_normalize(D @ Pv))), dtype)
    assert bool((a == 3.0).all())
    # first token: no previous state (no reset flags needed)
    wd, wa = want(host(depth), None)
    L().call("loom_decode_tria_readout", code(depth), P(depth), None, None, P(fire_d), P(doc),
             P(sw), P(pw), P(pb), P(uw), P(ub), P(a), P(ws), nb, B, H, N, 0.1, 1e-6, S(depth))
    check(doc, wd, dtype)
    check(a, wa, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M", [1, 3, 32, 64])
def test_linear_multi(dtype, M):
    """Fused decode projections: output segments sharing x (own weights,
    strided outputs, bias, gate) and concatenation along k, against fp32
    products of the same (dtype-rounded) operands."""
    from loom_amd import _lib
    g = torch.Generator().manual_seed(M)
    K, K2 = 768, 256
    r = lambda *s: (torch.randn(*s, generator=g) * 0.5).to(DEV, dtype)
    xw = r(M, K + 8)
    x = xw[:, :K]                                   # row stride K + 8
    w0, w1, w2 = r(64, K), r(96, K), r(40, K)
    b1 = torch.randn(96, generator=g).to(DEV)
    gate = r(M, 96)
    wide = torch.zeros(M, 200, device=DEV, dtype=dtype)
    out0 = wide[:, 16:80]                           # strided output view
    out1 = torch.zeros(M, 96, device=DEV, dtype=dtype)
    out2 = torch.zeros(M, 40, device=DEV, dtype=dtype)
    d = _lib.linear_multi_desc(x, [dict(w=w0, out=out0),
                                   dict(w=w1, out=out1, bias=b1, gate_p=gate, gate_alpha=0.3),
                                   dict(w=w2, out=out2)])
    _lib.call("loom_linear_multi", code(x), ctypes.byref(d), S(x))
    X = host(x)
    check(out0, X @ host(w0).T, dtype)
    check(out1, (X @ host(w1).T) * (1 + 0.3 * host(gate)) + host(b1), dtype)
    check(out2, X @ host(w2).T, dtype)
    assert bool((wide[:, :16] == 0).all()) and bool((wide[:, 80:] == 0).all())
    # concatenation along k: out = x w^T + x2 w2^T + b
    x2 = r(M, K2)
    wa, wb = r(768, K), r(768, K2)
    bb = torch.randn(768, generator=g).to(DEV)
    out = torch.zeros(M, 768, device=DEV, dtype=dtype)
    d = _lib.linear_multi_desc(x, [dict(w=wa, w2=wb, out=out, bias=bb)], x2=x2)
    _lib.call("loom_linear_multi", code(x), ctypes.byref(d), S(x))
    check(out, X @ host(wa).T + host(x2) @ host(wb).T + host(bb), dtype)
    # a long second input (120 k-steps: the widest block shape)
    x3 = r(M, 3072)
    wc = r(768, 3072) * 0.25
    d = _lib.linear_multi_desc(x, [dict(w=wa, w2=wc, out=out, bias=bb)], x2=x3)
    _lib.call("loom_linear_multi", code(x), ctypes.byref(d), S(x))
    check(out, X @ host(wa).T + host(x3) @ host(wc).T + host(bb), dtype)
    # device flags: with none set the bf16 fused launch leaves the outputs as
    # they are; with one set it computes them
    flags = torch.zeros(5, dtype=torch.uint8, device=DEV)
    out3 = torch.full((M, 96), 7.0, device=DEV, dtype=dtype)
    d = _lib.linear_multi_desc(x, [dict(w=w1, out=out3, bias=b1)], only_if=flags)
    _lib.call("loom_linear_multi", code(x), ctypes.byref(d), S(x))
    if dtype == torch.bfloat16:
        assert bool((out3 == 7.0).all())
    flags[3] = 1
    _lib.call("loom_linear_multi", code(x), ctypes.byref(d), S(x))
    check(out3, X @ host(w1).T + host(b1), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M,n0,n1,shared,gate", [(4096, 1152, 1536, False, False),
                                                 (1000, 768, 640, False, False),
                                                 (300, 1000, 64, False, False), (4096, 1152, 1536, True, False),
                                                 (4096, 3072, 1536, True, True), (1000, 768, 640, False, True)])
def test_linear_multi_two_segments_many_rows(dtype, M, n0, n1, shared, gate):
    """Two projections of one activation with many rows: bf16 runs them as one
    launch of DMA-staged tiles when the first segment ends on a tile boundary
    (the second product's own weight, strided output and bias; `gate`: the
    first product with the anchored gate, as W_real beside the history slot);
    to the bit the two separate products, and against the fp32 products
    (`shared`: in shared-tile mode)."""
    with shared_tiles(shared):
        _two_segment_case(dtype, M, n0, n1, gate)


def _two_segment_case(dtype, M, n0, n1, gate=False):
    from loom_amd import _lib
    g = torch.Generator().manual_seed(M + n0 + n1)
    K = 768
    r = lambda *s: (torch.randn(*s, generator=g) * 0.5).to(DEV, dtype)
    x = r(M, K)
    w0, w1 = r(n0, K) * 0.1, r(n1, K) * 0.1
    b1 = torch.randn(n1, generator=g).to(DEV)
    p0 = r(M, n0)
    outs = []
    for fused in (True, False):
        o0 = torch.zeros(M, n0, device=DEV, dtype=dtype)
        wide = torch.zeros(M, n1 + 40, device=DEV, dtype=dtype)
        o1 = wide[:, 8:8 + n1]
        seg0 = dict(w=w0, out=o0, gate_p=p0, gate_alpha=0.3) if gate else dict(w=w0, out=o0)
        segs = [seg0, dict(w=w1, out=o1, bias=b1)]
        calls = [segs] if fused else [[sg] for sg in segs]
        for sg in calls:
            d = _lib.linear_multi_desc(x, sg)
            _lib.call("loom_linear_multi", code(x), ctypes.byref(d), S(x))
        torch.cuda.synchronize()
        outs.append((o0, wide))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    o0, wide = outs[0]
    check(o0, (host(x) @ host(w0).T) * ((1.0 + 0.3 * host(p0)) if gate else 1.0), dtype)
    check(wide[:, 8:8 + n1], host(x) @ host(w1).T + host(b1), dtype)
    assert not wide[:, :8].any() and not wide[:, 8 + n1:].any()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("mode,gate,axis,gsrc", [(1, True, 0, False), (1, True, 1, False),
                                                 (1, False, 2, False), (0, True, 2, False),
                                                 (2, True, 1, False), (2, False, 0, False),
                                                 (1, True, 1, True), (2, False, 2, True)])
def test_ffn_decode(dtype, mode, gate, axis, gsrc):
    """One decode token of beta space -> Paraplex chain -> Tria depth op (one
    launch in bf16) against the oracle: beta_space_grouped, paraplex_pointwise
    and tria_*_and_gate on the same (dtype-rounded) inputs; with gsrc the
    amplitude comes from a separate gate source (paraplex_gate_proj)."""
    from loom_amd import _lib
    g = torch.Generator().manual_seed(10 * mode + axis + (5 if gate else 0) + (50 if gsrc else 0))
    M, QH, HD, H = 32, 8, 96, 3072
    N = QH * HD
    K = N + 4 * HD
    r = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(DEV, dtype)
    u = r(M, N)
    q, kc, c, d = (r(M, QH, HD) for _ in range(4))
    w = r(H, K, sc=K ** -0.5)
    R = r(M, H, sc=2.0)
    G = r(M, H, sc=2.0) if gsrc else None
    ib = (torch.randn(H, generator=g) * 0.3).to(DEV)
    tw = (torch.rand(H, generator=g) - 0.5).to(DEV)
    trace0 = r(M, H, sc=0.5)
    trace = trace0.clone()
    prev = ref.local_normalize(torch.randn(M, H, 3, 3, generator=g)).to(DEV, dtype)
    valid = (torch.arange(M) % 3 != 1).to(torch.uint8).to(DEV)
    gw = torch.softmax(torch.randn(9, generator=g), 0).to(DEV, dtype)
    act, s, beta = (torch.empty(M, H, device=DEV, dtype=dtype) for _ in range(3))
    carry = torch.empty(M, H, 3, 3, device=DEV, dtype=dtype)
    p = torch.empty(M, H, device=DEV, dtype=dtype)
    # the fragment-major copy of act (bf16 fused path)
    act_frag = torch.empty(M * H, device=DEV, dtype=dtype) if dtype == torch.bfloat16 else None
    # and the u sector read from a fragment-major copy of u
    u_frag = _lib.frag_major(u) if act_frag is not None and mode != 0 else None
    desc = _lib.ffn_decode_desc(
        u=u, q_h=q, k_ctx_h=kc, c_h=c, d_h=d, w_compact=w, M=M, N=N, H=H, imag_in=K,
        hidden_per_q_head=H // QH, head_dim=HD, n_q_heads=QH, open_sectors=0,
        p_real=R, gate_src=G, imag_bias=ib, trace=trace, trace_w=tw, powlu_m=3.0, act=act, s=s,
        beta=beta, carry_prev=prev if mode == 1 else None, seed=prev if mode == 2 else None,
        seed_valid=valid if mode == 2 else None, gate_w=gw if gate else None, carry_out=carry,
        p_out=p if gate else None, alpha=0.0375, axis=axis, act_frag=act_frag,
        u_frag=u_frag)
    _lib.call("loom_ffn_decode", code(u), ctypes.byref(desc), S(u))
    if act_frag is not None:
        assert torch.equal(act_frag, _lib.frag_major(act))
    # oracle, fp32 on the host
    be = ref.beta_space_grouped(host(u)[:, None], host(q)[:, None], host(kc)[:, None],
                                host(c)[:, None], host(d)[:, None], host(w), QH, HD, "head")
    wa, ws_, wt = ref.paraplex_pointwise(host(R)[:, None], host(G if gsrc else R)[:, None], be,
                                         host(ib), host(trace0), host(tw), None, 3.0)
    check(act, wa[:, 0], dtype)
    check(s, ws_[:, 0], dtype)
    check(trace, wt, dtype)
    ri = [host(R)[:, None], ws_.to(dtype).float(), wa.to(dtype).float()]   # Tria sees stored R, I, O
    wgt = host(gw) if gate else torch.zeros(9)
    if mode == 1:
        wc, wp = ref.tria_step_and_gate(*ri, host(prev)[:, None], wgt, 0.0375, axis)
    elif mode == 2:
        wc, wp = ref.tria_init_seed_and_gate(*ri, host(prev), host(valid).bool(), wgt, 0.0375, axis)
    else:
        wc, wp = ref.tria_init_and_gate(*ri, wgt, 0.0375, axis)
    check(carry, wc[:, 0], dtype)
    if gate:
        check(p, wp[:, 0], dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M,rms,slots,QH,HD,part", [
    (32, False, 4, 8, 96, False), (32, True, 11, 8, 96, False), (9, False, 20, 8, 96, False),
    (40, False, 7, 8, 96, False),
    # W_imag input 512 wide: 4-wave blocks, so 20 or 32 rows of 16 lanes take two rounds
    (20, False, 5, 4, 64, False), (20, True, 7, 4, 64, False), (32, False, 13, 4, 64, False),
    (32, True, 9, 4, 64, False),
    # the read over slots 0..S-2 given (normalised fp32 rows + log-sum-exp): the
    # launch folds in slot S-1 only (the fixed-RMS read ignores the part)
    (32, False, 20, 8, 96, True), (32, False, 2, 8, 96, True), (20, False, 5, 4, 64, True),
    (32, True, 11, 8, 96, True), (40, False, 7, 8, 96, True)])
def test_ffn_decode_with_depth_read(dtype, M, rms, slots, QH, HD, part):
    """ffn_decode computing its own d_h: the depth read of history slot S-1
    (DepthAttn over slots 0..S-1, fixed-RMS q/k/v with rms) inside the launch
    (bf16, M <= 32) or as a launch before it (fp32, M > 32).  d_h against the
    oracle's depth read, the FFN outputs against the oracle fed with that d_h."""
    from loom_amd import _lib
    from oracle.model import fixed_rms
    g = torch.Generator().manual_seed(M * 7 + slots + (3 if rms else 0) + HD)
    H, L2 = 3072, 20
    N = QH * HD
    K = N + 4 * HD
    r = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(DEV, dtype)
    u = r(M, N)
    q, kc, c = (r(M, QH, HD) for _ in range(3))
    d = torch.full((M, QH, HD), float("nan"), device=DEV, dtype=dtype)   # written by the call
    hist = r(M, L2, 2 * N, sc=2.0)
    dq = r(QH, HD, sc=0.5)
    w = r(H, K, sc=K ** -0.5)
    R = r(M, H, sc=2.0)
    ib = (torch.randn(H, generator=g) * 0.3).to(DEV)
    tw = (torch.rand(H, generator=g) - 0.5).to(DEV)
    trace0 = r(M, H, sc=0.5)
    trace = trace0.clone()
    prev = ref.local_normalize(torch.randn(M, H, 3, 3, generator=g)).to(DEV, dtype)
    gw = torch.softmax(torch.randn(9, generator=g), 0).to(DEV, dtype)
    act, s, beta = (torch.empty(M, H, device=DEV, dtype=dtype) for _ in range(3))
    carry = torch.empty(M, H, 3, 3, device=DEV, dtype=dtype)
    p = torch.empty(M, H, device=DEV, dtype=dtype)
    tg = (0.88 / HD ** 0.5, 0.88, 0.88 * 0.4)
    pd = pl = None
    if part:
        # the oracle's read over slots 0..S-2 with this query, as fp32 rows + log-sum-exp
        hk0 = host(hist)[:, :slots - 1, :N].reshape(M, slots - 1, QH, HD)
        hv0 = host(hist)[:, :slots - 1, N:].reshape(M, slots - 1, QH, HD)
        sc0 = (hk0 * host(dq)).sum(-1) / math.sqrt(HD)
        pd = (torch.softmax(sc0, dim=1).unsqueeze(-1) * hv0).sum(1).to(DEV)
        pl = torch.logsumexp(sc0, dim=1).to(DEV)
    desc = _lib.ffn_decode_desc(
        u=u, q_h=q, k_ctx_h=kc, c_h=c, d_h=d, w_compact=w, M=M, N=N, H=H, imag_in=K,
        hidden_per_q_head=H // QH, head_dim=HD, n_q_heads=QH, open_sectors=0,
        p_real=R, gate_src=None, imag_bias=ib, trace=trace, trace_w=tw, powlu_m=3.0, act=act, s=s,
        beta=beta, carry_prev=prev, seed=None, seed_valid=None, gate_w=gw, carry_out=carry, p_out=p,
        alpha=0.0375, axis=1, depth_q=dq, depth_k=hist, depth_v=hist[:, :, N:],
        depth_sbt=L2 * 2 * N, depth_ss=2 * N, depth_S=slots, depth_rms=1 if rms else 0,
        depth_part_d=pd, depth_part_lse=pl,
        **(dict(zip(("depth_qt", "depth_kt", "depth_vt"), tg)) if rms else {}))
    _lib.call("loom_ffn_decode", code(u), ctypes.byref(desc), S(u))
    # fixed_rms on the stored dtype, as the reference applies it
    hk = hist.cpu()[:, :slots, :N].reshape(M, slots, QH, HD)
    hv = hist.cpu()[:, :slots, N:].reshape(M, slots, QH, HD)
    qd = dq.cpu()
    if rms:
        qd, hk, hv = fixed_rms(qd, tg[0]), fixed_rms(hk, tg[1]), fixed_rms(hv, tg[2])
    qd, hk, hv = qd.float(), hk.float(), hv.float()
    want_d, _, _ = ref.depth_attn_softmax(qd, hk[:, None], hv[:, None])
    check(d, want_d[:, 0], dtype)
    be = ref.beta_space_grouped(host(u)[:, None], host(q)[:, None], host(kc)[:, None],
                                host(c)[:, None], host(d)[:, None], host(w), QH, HD, "head")
    wa, ws_, wt = ref.paraplex_pointwise(host(R)[:, None], host(R)[:, None], be, host(ib),
                                         host(trace0), host(tw), None, 3.0)
    check(act, wa[:, 0], dtype)
    check(trace, wt, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M,K2,N", [(1, 768, 768), (4, 3072, 768), (32, 768, 768), (32, 3072, 768),
                                    (64, 3072, 768), (7, 0, 768), (4096, 768, 768), (4096, 3072, 768),
                                    (300, 768, 768), (512, 0, 768), (520, 768, 200)])
def test_linear_ln(dtype, M, K2, N):
    """LayerNorm(x w^T + x2 w2^T + b): split-K partial sums reduced inside the
    LayerNorm kernel (bf16: the skinny form up to 64 rows, the 256 x 128 MFMA
    tiles over both inputs from 256 rows on, edge rows and columns included) or
    product + LayerNorm (fp32), against torch."""
    from loom_amd import _lib
    g = torch.Generator().manual_seed(M + K2 + N)
    K = 768
    r = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(DEV, dtype)
    x = r(M, K)
    w = r(N, K, sc=K ** -0.5)
    x2 = r(M, K2) if K2 else None
    w2 = r(N, K2, sc=K2 ** -0.5) if K2 else None
    b = torch.randn(N, generator=g).to(DEV)
    gam = (torch.rand(N, generator=g) + 0.5).to(DEV)
    bet = torch.randn(N, generator=g).to(DEV)
    y = torch.zeros(M, N, device=DEV, dtype=dtype)
    out = torch.zeros(M, N, device=DEV, dtype=dtype)
    nb = _lib.load().loom_linear_ln_workspace_bytes(M, N)
    ws = torch.empty(nb // 4, device=DEV)
    d = _lib.linear_multi_desc(x, [dict(w=w, w2=w2, out=y, bias=b)], x2=x2)
    _lib.call("loom_linear_ln", code(x), ctypes.byref(d), P(gam), P(bet), 1e-5, P(out), N, P(ws),
              nb, None, S(x))
    pre = host(x) @ host(w).T + host(b)
    if K2:
        pre = pre + host(x2) @ host(w2).T
    want = torch.nn.functional.layer_norm(pre, (N,), host(gam), host(bet), 1e-5)
    check(out, want, dtype)


@pytest.mark.parametrize("M,K2", [(4, 3072), (32, 768), (32, 3072), (20, 0), (64, 768)])
def test_fragment_major_activations(M, K2):
    """loom_linear_ln's out_frag is the fragment-major copy of its output, and
    loom_linear_ln / loom_linear_multi reading x_frag / x2_frag give the same
    bits as reading x / x2 (bf16 fused launch)."""
    from loom_amd import _lib
    g = torch.Generator().manual_seed(3 + M + K2)
    N, K, bf = 768, 768, torch.bfloat16
    r = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(DEV, bf)
    x, w = r(M, K), r(N, K, sc=K ** -0.5)
    x2 = r(M, K2) if K2 else None
    w2 = r(N, K2, sc=K2 ** -0.5) if K2 else None
    b = torch.randn(N, generator=g).to(DEV)
    gam = (torch.rand(N, generator=g) + 0.5).to(DEV)
    bet = torch.randn(N, generator=g).to(DEV)
    nb = _lib.load().loom_linear_ln_workspace_bytes(M, N)
    ws = torch.empty(nb // 4, device=DEV)
    wq = r(1152, N, sc=N ** -0.5)
    outs = []
    for frag in (False, True):
        y = torch.zeros(M, N, device=DEV, dtype=bf)
        out = torch.zeros(M, N, device=DEV, dtype=bf)
        of = torch.full((-(-M // 16) * 16 * N,), float("nan"), device=DEV, dtype=bf)
        d = _lib.linear_multi_desc(x, [dict(w=w, w2=w2, out=y, bias=b)], x2=x2,
                                   x_frag=_lib.frag_major(x) if frag else None,
                                   x2_frag=_lib.frag_major(x2) if frag and K2 else None)
        _lib.call("loom_linear_ln", code(x), ctypes.byref(d), P(gam), P(bet), 1e-5, P(out), N,
                  P(ws), nb, P(of), S(x))
        torch.cuda.synchronize()
        got = of.view(-1)[:_lib.frag_major(out).numel()]
        want = _lib.frag_major(out)
        rows = torch.arange(want.numel(), device=DEV) // 8 % 64 % 16 + \
            16 * (torch.arange(want.numel(), device=DEV) // 8 // 64 // (N // 32))
        assert torch.equal(got[rows < M], want[rows < M])
        outs.append(out)
        # a projection of the normalised rows through the copy
        q = torch.zeros(M, 1152, device=DEV, dtype=bf)
        dq = _lib.linear_multi_desc(out, [dict(w=wq, out=q)], x_frag=of if frag else None)
        _lib.call("loom_linear_multi", code(x), ctypes.byref(dq), S(x))
        outs.append(q)
    assert torch.equal(outs[0], outs[2])
    torch.cuda.synchronize()
    assert torch.equal(outs[1], outs[3])


@pytest.mark.parametrize("dtype", DTYPES)
def test_decode_prologue_embed(dtype):
    # ids from the prompt while pos < prompt_len, else the caller's ids; fire on a
    # hard boundary or the carry id; reset_now = pending; h = emb[ids]
    B, V, N, W = 5, 50, 40, 4
    g = torch.Generator().manual_seed(9)
    emb = torch.randn(V, N, generator=g).to(DEV, dtype)
    prompt = torch.randint(0, V, (B, 6), generator=g)
    prompt[2, 3] = 7                          # carry id at pos 3 in row 2
    prompt_d = prompt.to(DEV)
    pending = torch.tensor([1, 0, 1, 0, 0], dtype=torch.uint8, device=DEV)
    for pos, from_prompt in ((3, True), (7, False)):
        ids = torch.randint(0, V, (B,), generator=g).to(DEV)
        ids0 = ids.clone()
        tokens = torch.zeros(B, 10, dtype=torch.int64, device=DEV)
        fire = torch.empty(B, dtype=torch.uint8, device=DEV)
        reset = torch.empty(B, dtype=torch.uint8, device=DEV)
        h = torch.empty(B, N, device=DEV, dtype=dtype)
        pos_d = torch.tensor([pos], dtype=torch.int64, device=DEV)
        L().call("loom_decode_prologue_embed", code(h), P(ids), P(prompt_d), 6, 6, P(tokens), 10,
                 P(pos_d), P(pending), P(fire), P(reset), 7, W, 100, P(emb), P(h), N, V, B, S(h))
        want_ids = prompt[:, pos] if from_prompt else ids0.cpu()
        assert torch.equal(ids.cpu(), want_ids)
        assert torch.equal(tokens[:, pos].cpu(), want_ids)
        hard = (pos + 1) % W == 0
        assert torch.equal(fire.cpu().bool(), torch.tensor(hard) | (want_ids == 7))
        assert torch.equal(reset.cpu(), pending.cpu())
        assert torch.equal(h.cpu(), emb.cpu()[want_ids])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("V", [64, 4096, 5000])
def test_decode_prologue_gather(dtype, V):
    """loom_decode_prologue_gather: the id from the prompt while pos < prompt_len,
    else the greedy pick of the logits (the same ids as loom_argmax_rows, ties
    included) or, without logits, the caller's ids; fire / reset_now as the
    prologue; the id's table row split into the two destinations exactly."""
    B, n1, W = 6, 40, 4
    n0 = 24 if V % 8 == 0 else 20       # 20: the element-wise copy (rows not 16-byte pieces)
    g = torch.Generator().manual_seed(V)
    table = torch.randn(V, n0 + n1, generator=g).to(DEV, dtype)
    logits = torch.randn(B, V, generator=g)
    logits[1, V // 3] = logits[1, V - 2] = 50.0          # a tie: the first index wins
    logits = logits.to(DEV, dtype)
    prompt = torch.randint(0, V, (B, 6), generator=g)
    prompt[2, 3] = 7                                      # the carry id at pos 3 in row 2
    prompt_d = prompt.to(DEV)
    pending = torch.tensor([1, 0, 1, 0, 0, 1], dtype=torch.uint8, device=DEV)
    want_argmax = torch.empty(B, dtype=torch.int64, device=DEV)
    L().call("loom_argmax_rows", code(logits), P(logits), B, V, P(want_argmax), S(logits))
    assert int(want_argmax[1]) == V // 3
    for pos, mode in ((3, "prompt"), (7, "argmax"), (8, "ids")):
        ids = torch.randint(0, V, (B,), generator=g).to(DEV)
        ids0 = ids.clone()
        tokens = torch.zeros(B, 10, dtype=torch.int64, device=DEV)
        fire = torch.empty(B, dtype=torch.uint8, device=DEV)
        reset = torch.empty(B, dtype=torch.uint8, device=DEV)
        d0 = torch.full((B, 2 * n0), float("nan"), device=DEV, dtype=dtype)   # row stride 2*n0
        d1 = torch.full((B, n1), float("nan"), device=DEV, dtype=dtype)
        pos_d = torch.tensor([pos], dtype=torch.int64, device=DEV)
        if V % 8 != 0 and mode == "argmax":
            with pytest.raises(RuntimeError, match="logits need"):
                L().call("loom_decode_prologue_gather", code(table), P(logits), P(ids), P(prompt_d),
                         6, 6, P(tokens), 10, P(pos_d), P(pending), P(fire), P(reset), 7, W, 100,
                         P(table), n0 + n1, V, P(d0), 2 * n0, n0, P(d1), n1, n1, B, S(table))
            continue
        L().call("loom_decode_prologue_gather", code(table), P(logits) if mode == "argmax" else None,
                 P(ids), P(prompt_d) if mode != "ids" else None, 6, 6, P(tokens), 10, P(pos_d),
                 P(pending), P(fire), P(reset), 7, W, 100, P(table), n0 + n1, V, P(d0), 2 * n0,
                 n0, P(d1), n1, n1, B, S(table))
        want = (prompt[:, pos] if mode == "prompt" else want_argmax.cpu() if mode == "argmax"
                else ids0.cpu())
        assert torch.equal(ids.cpu(), want)
        assert torch.equal(tokens[:, pos].cpu(), want)
        hard = (pos + 1) % W == 0
        assert torch.equal(fire.cpu().bool(), torch.tensor(hard) | (want == 7))
        assert torch.equal(reset.cpu(), pending.cpu())
        rows = table.cpu()[want]
        assert torch.equal(d0.cpu()[:, :n0], rows[:, :n0])
        assert torch.isnan(d0.float().cpu()[:, n0:]).all()      # past n0 untouched
        assert torch.equal(d1.cpu(), rows[:, n0:])
