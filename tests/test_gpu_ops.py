"""GPU parity of every gfx950 op against the CPU oracle (and, where the
fixtures hold them, against the reference's own output vectors).

Tolerances (stated by the north star): fp32 rtol 1e-3, bf16 rtol 2e-2; fp16,
which the reference's launchers also dispatch (depth_attn_launcher.cu:87,
tria_step_launcher.cu:40, temporal_carry_launcher.cu:23,
phase_sin_launcher.cu:27, pvpowlu_launcher.cu:23), rtol 5e-3 (11 significant
bits).  The
oracle always runs in fp32 on the CPU, on exactly the inputs the GPU saw
(bf16 inputs are rounded first and upcast), so the bf16 error is the kernel's
output rounding plus fp32-vs-fp32 ordering differences.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import ops as ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float32: dict(rtol=1e-3, atol=1e-4), torch.bfloat16: dict(rtol=2e-2, atol=1e-2),
       torch.float16: dict(rtol=5e-3, atol=2e-3)}
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from loom_amd import _lib
    _lib.load()


def gen(seed):
    return torch.Generator().manual_seed(seed)


def rnd(g, *shape, scale=1.0):
    return torch.randn(*shape, generator=g) * scale


def dev(t, dtype):
    return t.to(DEV, dtype)


def host(t):
    return t.detach().float().cpu()


def check(got, want, dtype, rtol=None, atol=None):
    tol = dict(TOL[dtype])
    if rtol is not None:
        tol["rtol"] = rtol
    if atol is not None:
        tol["atol"] = atol
    torch.testing.assert_close(host(got), want.float(), **tol)


DTYPES = [torch.float32, torch.bfloat16]
# the ops the reference's launchers also dispatch in Half
DTYPES3 = [torch.float32, torch.bfloat16, torch.float16]


# ----------------------------------------------------------------- paraplex

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,T,H,same_gate,with_reset", [
    (2, 5, 24, True, False), (2, 7, 20, False, True), (3, 37, 3072, True, True),
    (1, 1, 3072, True, False), (32, 1, 3072, True, False), (2, 300, 256, False, False),
    # chunks of 16 tokens (the unrolled path for 16-bit rows) with a ragged last
    # chunk, and chunks of 15 tokens
    (8, 1030, 3072, True, True), (4, 2000, 3072, False, False),
    # chunks of 8 tokens (the chunked prefill's [32, 128] tokens, the loop form)
    (32, 128, 3072, True, False),
])
def test_paraplex_forward(dtype, B, T, H, same_gate, with_reset):
    from loom_amd import ops
    g = gen(B * 1000 + T * 10 + H)
    r = dev(rnd(g, B, T, H, scale=2.0), dtype)
    gs = r if same_gate else dev(rnd(g, B, T, H, scale=3.0), dtype)
    beta = dev(rnd(g, B, T, H, scale=2.0), dtype)
    bias = dev(rnd(g, H, scale=0.5), torch.float32)
    trace = dev(rnd(g, B, H, scale=0.5), dtype)
    tw = dev(torch.rand(H, generator=g) - 0.5, torch.float32)
    reset = torch.zeros(B, T, dtype=torch.bool)
    if with_reset:
        reset[0, min(2, T - 1)] = True
        reset[-1, 0] = True
    anchor = torch.ones((), device=DEV)
    act, s, nt, snap = ops.paraplex_forward(r, gs, beta, bias, trace, tw,
                                            dev(reset, torch.bool) if with_reset else torch.empty(0, dtype=torch.bool, device=DEV),
                                            anchor, 1, False, 0.99, 3.0)
    w_act, w_s, w_nt = ref.paraplex_pointwise(host(r), host(gs), host(beta), host(bias), host(trace),
                                              host(tw), reset if with_reset else None, 3.0)
    check(s, w_s, dtype)
    check(act, w_act, dtype)
    check(nt, w_nt, dtype)
    assert float(snap) == 1.0
    # a second call writes the same bits (every stored lane holds its own result)
    act2, s2, nt2, _ = ops.paraplex_forward(r, gs, beta, bias, trace, tw,
                                            dev(reset, torch.bool) if with_reset else torch.empty(0, dtype=torch.bool, device=DEV),
                                            anchor, 1, False, 0.99, 3.0)
    assert torch.equal(act2, act) and torch.equal(s2, s) and torch.equal(nt2, nt)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B,T,H", [(4, 16, 3072), (2, 33, 3072), (8, 1024, 3072), (3, 47, 256),
                                   (32, 128, 3072)])
def test_paraplex_row_end_tokens(dtype, B, T, H):
    """The last token of each row (the final store of the chunk that ends the
    row, followed by the next-trace store) and the next trace, element by
    element against the oracle, over three launches with identical bits."""
    from loom_amd import ops
    g = gen(B * 77 + T * 5 + H)
    r = dev(rnd(g, B, T, H, scale=2.0), dtype)
    beta = dev(rnd(g, B, T, H, scale=2.0), dtype)
    bias = dev(rnd(g, H, scale=0.5), torch.float32)
    trace = dev(rnd(g, B, H, scale=0.5), dtype)
    tw = dev(torch.rand(H, generator=g) - 0.5, torch.float32)
    no_reset = torch.empty(0, dtype=torch.bool, device=DEV)
    anchor = torch.ones((), device=DEV)
    w_act, w_s, w_nt = ref.paraplex_pointwise(host(r), host(r), host(beta), host(bias), host(trace),
                                              host(tw), None, 3.0)
    tol = TOL[dtype] if dtype in TOL else dict(rtol=5e-3, atol=5e-3)
    first = None
    for _ in range(3):
        act, s_, nt, _ = ops.paraplex_forward(r, r, beta, bias, trace, tw, no_reset, anchor, 1,
                                              False, 0.99, 3.0)
        torch.testing.assert_close(host(act[:, -1]), w_act[:, -1], **tol)
        torch.testing.assert_close(host(s_[:, -1]), w_s[:, -1], **tol)
        torch.testing.assert_close(host(nt), w_nt, **tol)
        if first is None:
            first = (act.clone(), s_.clone(), nt.clone())
        else:
            assert torch.equal(first[0], act) and torch.equal(first[1], s_) and torch.equal(first[2], nt)


@pytest.mark.parametrize("B,T,H,same_gate,with_reset", [
    (3, 37, 3072, True, True), (8, 1030, 3072, False, True), (2, 7, 20, True, False),
])
def test_paraplex_forward_f16(B, T, H, same_gate, with_reset):
    """fp16 rows through the same kernels (16-bit rows like bf16, with the exact
    log1p softplus); fp16 keeps 11 significant bits, so the bound is rtol 5e-3."""
    from loom_amd import ops
    dtype = torch.float16
    g = gen(B * 999 + T * 10 + H)
    r = dev(rnd(g, B, T, H, scale=2.0), dtype)
    gs = r if same_gate else dev(rnd(g, B, T, H, scale=3.0), dtype)
    beta = dev(rnd(g, B, T, H, scale=2.0), dtype)
    bias = dev(rnd(g, H, scale=0.5), torch.float32)
    trace = dev(rnd(g, B, H, scale=0.5), dtype)
    tw = dev(torch.rand(H, generator=g) - 0.5, torch.float32)
    reset = torch.zeros(B, T, dtype=torch.bool)
    if with_reset:
        reset[0, min(2, T - 1)] = True
        reset[-1, 0] = True
    rs = dev(reset, torch.bool) if with_reset else torch.empty(0, dtype=torch.bool, device=DEV)
    anchor = torch.ones((), device=DEV)
    act, s, nt, _ = ops.paraplex_forward(r, gs, beta, bias, trace, tw, rs, anchor, 1, False, 0.99, 3.0)
    w_act, w_s, w_nt = ref.paraplex_pointwise(host(r), host(gs), host(beta), host(bias), host(trace),
                                              host(tw), reset if with_reset else None, 3.0)
    for got, want in ((s, w_s), (act, w_act), (nt, w_nt)):
        torch.testing.assert_close(host(got), want.float(), rtol=5e-3, atol=2e-3)


@pytest.mark.parametrize("dtype", DTYPES3)
def test_phase_sin_and_pvpowlu(dtype):
    from loom_amd import ops
    g = gen(5)
    beta = torch.cat([rnd(g, 1000, scale=3.0), torch.tensor([0.0, 1e-4, -1e-4, 80.0, -80.0, 3e4, -3e4, 7.0])])
    b = dev(beta, dtype)
    check(ops.phase_sin_forward_cuda(b), ref.phase_sin(host(b)), dtype)
    x1 = dev(rnd(g, 1003), dtype)
    x2 = dev(torch.nn.functional.softplus(rnd(g, 1003, scale=4.0)), dtype)
    check(ops.pvpowlu_forward_cuda(x1, x2, 3.0), ref.pvpowlu(host(x1), host(x2), 3.0), dtype)
    check(ops.pvpowlu_forward_cuda(x1, x2, 0.0), host(x1) * torch.sigmoid(host(x2)), dtype)


def test_golden_phase_and_pvpowlu_vs_reference():
    from loom_amd import ops
    z = np.load(os.path.join(GOLD, "ops.npz"))
    b = torch.from_numpy(z["phase.beta"]).to(DEV)
    check(ops.phase_sin_forward_cuda(b), torch.from_numpy(z["phase.out"]), torch.float32)
    x1, x2 = torch.from_numpy(z["pvpowlu.x1"]).to(DEV), torch.from_numpy(z["pvpowlu.x2"]).to(DEV)
    check(ops.pvpowlu_forward_cuda(x1, x2, 3.0), torch.from_numpy(z["pvpowlu.out"]), torch.float32)


# ----------------------------------------------------------------- projections

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M,N,K", [(1, 16, 8), (37, 100, 72), (32, 3072, 768), (130, 768, 3072),
                                   (256, 256, 1152), (5, 4096, 768), (3, 768, 3072), (8, 1000, 772),
                                   # the large-M MFMA tiles: 256 x 128 (ragged), 128 x 256
                                   # (N % 256 == 0, ragged rows), 128 x 128 (fewer than
                                   # 256 rows, or K not a multiple of 192) and 256 x 192
                                   # (N % 192 == 0 where it takes fewer rounds, ragged rows)
                                   (8229, 3000, 768), (6000, 1536, 1152), (4100, 770, 3072),
                                   (4096, 1152, 768), (8192, 768, 3072), (4000, 1536, 768),
                                   (200, 384, 1024), (1000, 640, 512), (4096, 3072, 768),
                                   (4000, 3072, 1152)])
def test_linear(dtype, M, N, K):
    from loom_amd import ops
    g = gen(M * 7 + N + K)
    x = dev(rnd(g, M, K), dtype)
    w = dev(rnd(g, N, K, scale=K ** -0.5), dtype)
    bias = dev(rnd(g, N), torch.float32)
    want = host(x) @ host(w).t()
    check(ops.linear(x, w), want, dtype)
    check(ops.linear(x, w, bias), want + host(bias), dtype)
    p = dev(rnd(g, M, N), dtype)
    res = dev(rnd(g, M, N), dtype)
    check(ops.linear(x, w, bias, gate_p=p, gate_alpha=0.2, residual=res),
          want * (1.0 + 0.2 * host(p)) + host(bias) + host(res), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("QH,HD,Hq,M,sectors", [(4, 8, 32, 10, "head"), (8, 96, 384, 40, "head"),
                                                 (8, 96, 384, 300, "head"), (4, 8, 32, 6, "open"),
                                                 (8, 96, 384, 20, "open"), (8, 96, 384, 8200, "head"),
                                                 (8, 96, 384, 600, "open"), (8, 96, 384, 1, "head"),
                                                 (4, 8, 32, 3, "open"), (8, 96, 384, 8192, "head"),
                                                 # 256 x 192 tiles (whole and ragged rows)
                                                 (8, 96, 384, 4096, "head"), (8, 96, 384, 4000, "open")])
def test_beta_forward(dtype, QH, HD, Hq, M, sectors):
    from loom_amd import ops
    N, H = QH * HD, QH * Hq
    K = ref.imag_in(N, HD, sectors)
    g = gen(QH + HD + M)
    B, T = 1, M
    u = dev(rnd(g, B, T, N), dtype)
    q, kc, c, d = (dev(rnd(g, B, T, QH, HD), dtype) for _ in range(4))
    w = dev(rnd(g, H, K, scale=K ** -0.5), dtype)
    out, pack, wc = ops.beta_forward_cuda(u, q, kc, c, d, w, Hq, HD, QH, sectors == "open")
    want = ref.beta_space_dense(host(u), host(q), host(kc), host(c), host(d), host(w), QH, HD, sectors)
    check(out, want, dtype)
    assert pack.numel() == 0 and wc.shape == w.shape


# ----------------------------------------------------------------- depth attention

@pytest.mark.parametrize("dtype", DTYPES3)
@pytest.mark.parametrize("HD", [96, 8, 64])
def test_depth_attn_decode_strided_view(dtype, HD):
    from loom_amd import ops
    g = gen(HD)
    B, S_max, QH = 3, 20, 8
    hk = dev(rnd(g, B, 1, S_max, QH, HD), dtype)
    hv = dev(rnd(g, B, 1, S_max, QH, HD), dtype)
    q = dev(rnd(g, QH, HD, scale=HD ** -0.25), dtype)
    for s in (1, 2, 9, 20):
        d, w = ops.depth_attn_forward(q, hk[:, :, :s], hv[:, :, :s])
        want_d, want_w, _ = ref.depth_attn_softmax(host(q), host(hk)[:, :, :s], host(hv)[:, :, :s])
        check(d, want_d, dtype)
        check(w, want_w, dtype)
    # S=1 returns v_0 exactly (up to the output rounding)
    d, _ = ops.depth_attn_forward(q, hk[:, :, :1], hv[:, :, :1])
    check(d, host(hv)[:, :, 0], dtype)


@pytest.mark.parametrize("dtype", DTYPES3)
@pytest.mark.parametrize("HD,S", [(96, 20), (96, 1), (8, 7), (64, 9)])
def test_depth_attn_fixed_rms(dtype, HD, S):
    """DepthAttn under depth_attn_qkv_rms (loomformer.py:3397-3407): the entry
    point reads q, k, v as fixed-RMS rows; against the oracle's fixed_rms
    applied first, then the plain softmax read (d, weights and lse)."""
    from loom_amd import _lib
    from oracle.model import fixed_rms
    g = gen(HD * 31 + S)
    BT, QH = 37, 8
    hk = dev(rnd(g, BT, S, QH, HD, scale=3.0), dtype)
    hv = dev(rnd(g, BT, S, QH, HD, scale=0.2), dtype)
    q = dev(rnd(g, QH, HD, scale=0.7), dtype)
    qt, kt, vt = 0.88 / HD ** 0.5, 0.88, 0.88 * 0.4
    d = torch.empty(BT, QH, HD, device=DEV, dtype=dtype)
    w = torch.empty(BT, QH, S, device=DEV, dtype=dtype)
    lse = torch.empty(BT, QH, device=DEV)
    _lib.call("loom_depth_attn_forward_rms", _lib.dtype_code(q), _lib.ptr(q), _lib.ptr(hk),
              _lib.ptr(hv), S * QH * HD, QH * HD, _lib.ptr(d), _lib.ptr(w), _lib.ptr(lse), BT, S,
              QH, HD, qt, kt, vt, _lib.stream_of(q))
    # fixed_rms on the stored dtype, as the reference applies it (scale and
    # scaled rows rounded to bf16/fp16)
    qn = fixed_rms(q.cpu(), qt).float()
    kn, vn = fixed_rms(hk.cpu(), kt).float(), fixed_rms(hv.cpu(), vt).float()
    want_d, want_w, want_lse = ref.depth_attn_softmax(qn, kn[None], vn[None])
    check(d, want_d[0], dtype)
    check(w, want_w[0], dtype)
    check(lse, want_lse[0], torch.float32, rtol=1e-3, atol=1e-3)
    with pytest.raises(RuntimeError, match="targets must be positive"):
        _lib.call("loom_depth_attn_forward_rms", _lib.dtype_code(q), _lib.ptr(q), _lib.ptr(hk),
                  _lib.ptr(hv), S * QH * HD, QH * HD, _lib.ptr(d), None, None, BT, S, QH, HD,
                  0.0, kt, vt, _lib.stream_of(q))


@pytest.mark.parametrize("dtype", DTYPES3)
@pytest.mark.parametrize("BT,S", [(50, 24), (7, 33), (1, 1), (4096, 24)])
def test_depth_attn_stacked(dtype, BT, S):
    from loom_amd import ops
    g = gen(BT + S)
    QH, HD = 8, 96
    hk = dev(rnd(g, 1, BT, S, QH, HD), dtype)
    hv = dev(rnd(g, 1, BT, S, QH, HD), dtype)
    q = dev(rnd(g, QH, HD, scale=0.02), dtype)
    d, lse = ops.depth_attn_stacked_forward(q, hk, hv)
    want_d, _, want_lse = ref.depth_attn_softmax(host(q), host(hk), host(hv))
    check(d, want_d, dtype)
    check(lse, want_lse, torch.float32, rtol=1e-4, atol=1e-4)
    # equal keys -> mean of V
    hk_eq = hk[:, :, :1].expand(-1, -1, S, -1, -1).contiguous()
    d, _ = ops.depth_attn_stacked_forward(q, hk_eq, hv)
    check(d, host(hv).mean(2), dtype)


@pytest.mark.parametrize("dtype", DTYPES3)
@pytest.mark.parametrize("BT,S,HD", [(50, 1, 96), (4096, 19, 96), (7, 8, 64), (33, 3, 128), (5, 12, 32)])
def test_depth_attn_pair_and_fold(dtype, BT, S, HD):
    """loom_depth_attn_pair: two queries over slots 0..S-1 in one pass (the
    first as loom_depth_attn_forward, the second as fp32 rows + log-sum-exp);
    loom_depth_attn_fold: the second query's read over slots 0..S from that
    part and slot S, against the oracle's read over all S + 1 slots."""
    from loom_amd import _lib
    g = gen(BT * 7 + S + HD)
    QH, L2 = 8, S + 3
    N = QH * HD
    hist = dev(rnd(g, BT, L2, 2 * N), dtype)          # slot s = [k | v]
    q1, q2 = dev(rnd(g, QH, HD, scale=0.4), dtype), dev(rnd(g, QH, HD, scale=0.4), dtype)
    d1 = torch.empty(BT, QH, HD, device=DEV, dtype=dtype)
    pd = torch.full((BT, QH, HD), float("nan"), device=DEV)
    pl = torch.full((BT, QH), float("nan"), device=DEV)
    st = _lib.stream_of(hist)
    _lib.call("loom_depth_attn_pair", _lib.dtype_code(hist), _lib.ptr(q1), _lib.ptr(q2), _lib.ptr(hist),
              _lib.ptr(hist[:, :, N:]), L2 * 2 * N, 2 * N, _lib.ptr(d1), _lib.ptr(pd), _lib.ptr(pl),
              BT, S, QH, HD, st)
    hk = host(hist)[:, :, :N].reshape(BT, L2, QH, HD)
    hv = host(hist)[:, :, N:].reshape(BT, L2, QH, HD)
    want1, _, _ = ref.depth_attn_softmax(host(q1), hk[:, :S][None], hv[:, :S][None])
    check(d1, want1[0], dtype)
    want2, _, lse2 = ref.depth_attn_softmax(host(q2), hk[:, :S][None], hv[:, :S][None])
    torch.testing.assert_close(pd.cpu(), want2[0], rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(pl.cpu(), lse2[0], rtol=1e-5, atol=1e-5)
    d2 = torch.empty(BT, QH, HD, device=DEV, dtype=dtype)
    _lib.call("loom_depth_attn_fold", _lib.dtype_code(hist), _lib.ptr(q2), _lib.ptr(hist),
              _lib.ptr(hist[:, :, N:]), L2 * 2 * N, 2 * N, S + 1, _lib.ptr(pd), _lib.ptr(pl),
              _lib.ptr(d2), BT, QH, HD, st)
    want3, _, _ = ref.depth_attn_softmax(host(q2), hk[:, :S + 1][None], hv[:, :S + 1][None])
    check(d2, want3[0], dtype)
    with pytest.raises(RuntimeError, match="head_dim must be"):
        _lib.call("loom_depth_attn_fold", _lib.dtype_code(hist), _lib.ptr(q2), _lib.ptr(hist),
                  _lib.ptr(hist[:, :, N:]), L2 * 2 * N, 2 * N, S + 1, _lib.ptr(pd), _lib.ptr(pl),
                  _lib.ptr(d2), BT, QH, 80, st)          # rejected before any launch


def test_golden_depth_attn_vs_reference():
    from loom_amd import ops
    z = np.load(os.path.join(GOLD, "ops.npz"))
    hk, hv = torch.from_numpy(z["da.hist_k"]).to(DEV), torch.from_numpy(z["da.hist_v"]).to(DEV)
    q = torch.from_numpy(z["da.w::q_params"]).to(DEV)
    d, _ = ops.depth_attn_forward(q[3], hk, hv)
    check(d, torch.from_numpy(z["da.d_tensor"]), torch.float32)
    S = hk.shape[2]
    d, _ = ops.depth_attn_list_forward(q[4], [hk[:, :, j] for j in range(S)], [hv[:, :, j] for j in range(S)])
    check(d, torch.from_numpy(z["da.d_list"]), torch.float32)


# ----------------------------------------------------------------- tria

def _tria_inputs(g, B, T, H, dtype):
    r = dev(rnd(g, B, T, H, scale=2.0), dtype)
    i = dev(rnd(g, B, T, H), dtype)
    o = dev(rnd(g, B, T, H, scale=0.5), dtype)
    prev = dev(ref.local_normalize(rnd(g, B, T, H, 3, 3)), dtype)
    seed = dev(ref.local_normalize(rnd(g, B, H, 3, 3)), dtype)
    valid = torch.rand(B, generator=g) > 0.4
    valid[0] = True
    w = dev(torch.softmax(rnd(g, 9), 0), dtype)
    return r, i, o, prev, seed, dev(valid, torch.bool), w


@pytest.mark.parametrize("dtype", DTYPES3)
@pytest.mark.parametrize("axis", [0, 1, 2])
@pytest.mark.parametrize("B,T,H", [(3, 4, 6), (2, 3, 1000), (8, 1, 3072)])
def test_tria_depth_family(dtype, axis, B, T, H):
    from loom_amd import ops
    g = gen(B + T + H + axis)
    r, i, o, prev, seed, valid, w = _tria_inputs(g, B, T, H, dtype)
    a = 0.0375
    R, I, O, P, SD, W = host(r), host(i), host(o), host(prev), host(seed), host(w)
    c, s = ops.tria_init_forward(r, i, o, a, axis)
    check(c, ref.tria_init(R, I, O, a, axis), dtype)
    want_scale = ref.build_tria(R, I, O, a, axis).square().mean(dim=(-1, -2)).add(1e-6).sqrt()
    check(s, want_scale.reshape(-1), torch.float32, rtol=1e-4)
    c, p, _ = ops.tria_init_gate_forward(r, i, o, w, a, axis)
    wc, wp = ref.tria_init_and_gate(R, I, O, W, a, axis)
    check(c, wc, dtype)
    check(p, wp, dtype)
    c, _ = ops.tria_step_forward(r, i, o, prev, a, axis)
    check(c, ref.tria_step(R, I, O, P, a, axis), dtype)
    c, p, _ = ops.tria_step_gate_forward(r, i, o, prev, w, a, axis)
    wc, wp = ref.tria_step_and_gate(R, I, O, P, W, a, axis)
    check(c, wc, dtype)
    check(p, wp, dtype)
    c, _ = ops.tria_init_seed_forward(r, i, o, seed, valid, a, axis)
    check(c, ref.tria_init_seed(R, I, O, SD, valid.cpu(), a, axis), dtype)
    c, p = ops.tria_init_seed_gate_forward(r, i, o, seed, valid, w, a, axis)
    wc, wp = ref.tria_init_seed_and_gate(R, I, O, SD, valid.cpu(), W, a, axis)
    check(c, wc, dtype)
    check(p, wp, dtype)
    # invariant: every carrier has RMS 1 (to eps)
    rms = host(c).square().mean(dim=(-1, -2)).sqrt()
    rms_tol = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 3e-3}[dtype]
    torch.testing.assert_close(rms, torch.ones_like(rms), rtol=rms_tol, atol=0)


@pytest.mark.parametrize("dtype", DTYPES3)
@pytest.mark.parametrize("B,T,H,mode,gate,axis,same", [
    (2, 5, 24, "init", False, 0, True), (2, 5, 24, "step", True, 1, False),
    (3, 4, 6, "seed", True, 2, True), (3, 9, 20, "seed", False, 1, False),
    (1, 1, 3072, "step", False, 2, True), (4, 33, 1000, "init", True, 2, False),
    # odd H: one element per lane (even H moves element pairs as one word)
    (2, 3, 25, "step", True, 1, False), (3, 5, 7, "seed", True, 0, True),
    (2, 4, 9, "init", False, 2, True),
    # the chunked prefill's shape: [32, 128] tokens of 3072
    (32, 128, 3072, "step", True, 1, True), (32, 128, 3072, "init", True, 0, True),
    (32, 128, 3072, "seed", True, 2, True), (32, 128, 3072, "step", False, 0, False),
])
def test_paraplex_tria_fused(dtype, B, T, H, mode, gate, axis, same):
    """loom_paraplex_tria_forward against the two launches it replaces
    (loom_paraplex_forward then loom_tria_depth_forward on the stored I and O):
    the same bits for act, the next trace, the carry and p; and against the
    oracle's composition paraplex_pointwise -> tria_* on I and O rounded to
    dtype (the reference stores both before the Tria op reads them)."""
    from loom_amd import ops
    from loom_amd._lib import call, dtype_code, ptr, stream_of
    g = gen(B * 131 + T * 7 + H + axis)
    r = dev(rnd(g, B, T, H, scale=2.0), dtype)
    gs = r if same else dev(rnd(g, B, T, H, scale=3.0), dtype)
    beta = dev(rnd(g, B, T, H, scale=2.0), dtype)
    bias = dev(rnd(g, H, scale=0.5), torch.float32)
    trace = dev(rnd(g, B, H, scale=0.5), dtype)
    tw = dev(torch.rand(H, generator=g) - 0.5, torch.float32)
    prev = dev(ref.local_normalize(rnd(g, B, T, H, 3, 3)), dtype) if mode == "step" else None
    seed = dev(ref.local_normalize(rnd(g, B, H, 3, 3)), dtype) if mode == "seed" else None
    valid = torch.rand(B, generator=g) > 0.4
    valid[0] = True
    valid = dev(valid, torch.bool) if mode == "seed" else None
    w = dev(torch.softmax(rnd(g, 9), 0), dtype) if gate else None
    a, m = 0.0375, 3.0

    # the two launches
    no_reset = torch.empty(0, dtype=torch.bool, device=DEV)
    act2, s2, nt2, _ = ops.paraplex_forward(r, gs, beta, bias, trace, tw, no_reset,
                                            torch.ones((), device=DEV), 1, False, 0.99, m)
    carry2, p2, _ = ops._tria_call(r, s2, act2, prev, seed, valid, w, False, a, axis)

    for _ in range(2):  # a second call writes the same bits
        act = torch.full_like(r, float("nan"))
        nt = torch.full_like(trace, float("nan"))
        carry = torch.full((B, T, H, 3, 3), float("nan"), dtype=dtype, device=DEV)
        p = torch.full_like(r, float("nan")) if gate else None
        call("loom_paraplex_tria_forward", dtype_code(r), ptr(r), ptr(gs), ptr(beta), ptr(bias),
             ptr(trace), ptr(tw), m, ptr(prev), ptr(seed), ptr(valid), ptr(w), ptr(act), ptr(nt),
             ptr(carry), ptr(p), B, T, H, a, axis, stream_of(r))
        torch.cuda.synchronize()
        assert torch.equal(act, act2)
        assert torch.equal(nt, nt2)
        assert torch.equal(carry, carry2)
        if gate:
            assert torch.equal(p, p2)

    w_act, w_s, w_nt = ref.paraplex_pointwise(host(r), host(gs), host(beta), host(bias), host(trace),
                                              host(tw), None, m)
    check(act, w_act, dtype)
    check(nt, w_nt, dtype)
    R, I, O = host(r), w_s.to(dtype).float(), w_act.to(dtype).float()
    if mode == "init":
        wc = ref.tria_init(R, I, O, a, axis)
    elif mode == "step":
        wc = ref.tria_step(R, I, O, host(prev), a, axis)
    else:
        wc = ref.tria_init_seed(R, I, O, host(seed), valid.cpu(), a, axis)
    # 16-bit types: the carrier of O rounded on the GPU vs O rounded in the
    # oracle (one ulp apart where the fp32 values straddle a rounding boundary)
    tol = {torch.bfloat16: dict(rtol=2e-2, atol=2e-2),
           torch.float16: dict(rtol=5e-3, atol=5e-3)}.get(dtype, {})
    check(carry, wc, dtype, **tol)
    if gate:
        check(p, ref.gate_slot_mix(wc, host(w)), dtype, **tol)


@pytest.mark.parametrize("dtype", DTYPES3)
@pytest.mark.parametrize("B,T,H,axis,same,initial", [
    (2, 5, 24, 0, True, "none"), (3, 1, 6, 1, False, "valid"), (2, 7, 200, 2, True, "some"),
    (1, 33, 130, 1, False, "some"), (2, 4, 128, 0, True, "valid"),
    # the chunked prefill's last block: [32, 128] tokens of 3072
    (32, 128, 3072, 0, True, "some"),
])
def test_paraplex_tria_endpoint_fused(dtype, B, T, H, axis, same, initial):
    """loom_paraplex_tria_endpoint_forward against the two launches it
    replaces (loom_paraplex_tria_forward with carried records, then
    loom_temporal_carry_endpoint_forward on the stored carries): the same bits
    for act, the next trace and the endpoint (both precisions), with resets
    inside the chunk and at its first token, and an initial state valid for
    none, some or all rows."""
    from loom_amd._lib import call, dtype_code, ptr, stream_of
    g = gen(B * 97 + T * 5 + H + axis)
    r = dev(rnd(g, B, T, H, scale=2.0), dtype)
    gs = r if same else dev(rnd(g, B, T, H, scale=3.0), dtype)
    beta = dev(rnd(g, B, T, H, scale=2.0), dtype)
    bias = dev(rnd(g, H, scale=0.5), torch.float32)
    trace = dev(rnd(g, B, H, scale=0.5), dtype)
    tw = dev(torch.rand(H, generator=g) - 0.5, torch.float32)
    prev = dev(ref.local_normalize(rnd(g, B, T, H, 3, 3)), dtype)
    reset = torch.rand(B, T, generator=g) > 0.9
    reset[:, 0] = torch.rand(B, generator=g) > 0.5
    reset = dev(reset, torch.bool)
    init = dev(ref.local_normalize(rnd(g, B, H, 3, 3)), dtype) if initial != "none" else None
    valid = None
    if initial == "some":
        valid = torch.rand(B, generator=g) > 0.5
        valid[0] = True
        valid = dev(valid, torch.bool)
    a, m = 0.0375, 3.0

    # the two launches
    act2 = torch.empty_like(r)
    nt2 = torch.empty_like(trace)
    carry2 = torch.empty(B, T, H, 3, 3, dtype=dtype, device=DEV)
    call("loom_paraplex_tria_forward", dtype_code(r), ptr(r), ptr(gs), ptr(beta), ptr(bias), ptr(trace),
         ptr(tw), m, ptr(prev), None, None, None, ptr(act2), ptr(nt2), ptr(carry2), None, B, T, H, a,
         axis, stream_of(r))
    end2 = torch.empty(B, H, 3, 3, dtype=dtype, device=DEV)
    end2_32 = torch.empty(B, H, 3, 3, dtype=torch.float32, device=DEV)
    call("loom_temporal_carry_endpoint_forward", dtype_code(r), ptr(carry2), ptr(reset), ptr(init),
         ptr(valid), ptr(end2), ptr(end2_32), B, T, H, stream_of(r))

    for _ in range(2):  # a second call writes the same bits
        act = torch.full_like(r, float("nan"))
        nt = torch.full_like(trace, float("nan"))
        end = torch.full((B, H, 3, 3), float("nan"), dtype=dtype, device=DEV)
        end32 = torch.full((B, H, 3, 3), float("nan"), dtype=torch.float32, device=DEV)
        call("loom_paraplex_tria_endpoint_forward", dtype_code(r), ptr(r), ptr(gs), ptr(beta),
             ptr(bias), ptr(trace), ptr(tw), m, ptr(prev), ptr(reset), ptr(init), ptr(valid),
             ptr(act), ptr(nt), ptr(end), ptr(end32), B, T, H, a, axis, stream_of(r))
        torch.cuda.synchronize()
        assert torch.equal(act, act2)
        assert torch.equal(nt, nt2)
        assert torch.equal(end, end2)
        assert torch.equal(end32, end2_32)


def test_paraplex_tria_endpoint_in_place_initial():
    """The endpoint may overwrite the initial state (the chunked prefill's
    use): the same bits as with separate buffers."""
    from loom_amd._lib import call, dtype_code, ptr, stream_of
    B, T, H, dtype = 4, 9, 256, torch.bfloat16
    g = gen(5)
    r = dev(rnd(g, B, T, H, scale=2.0), dtype)
    beta = dev(rnd(g, B, T, H, scale=2.0), dtype)
    bias = dev(rnd(g, H, scale=0.5), torch.float32)
    trace = dev(rnd(g, B, H, scale=0.5), dtype)
    tw = dev(torch.rand(H, generator=g) - 0.5, torch.float32)
    prev = dev(ref.local_normalize(rnd(g, B, T, H, 3, 3)), dtype)
    reset = dev(torch.zeros(B, T, dtype=torch.bool), torch.bool)
    init = dev(ref.local_normalize(rnd(g, B, H, 3, 3)), dtype)
    outs = []
    for in_place in (False, True):
        state = init.clone()
        end = state if in_place else torch.empty_like(init)
        act, nt = torch.empty_like(r), torch.empty_like(trace)
        call("loom_paraplex_tria_endpoint_forward", dtype_code(r), ptr(r), ptr(r), ptr(beta),
             ptr(bias), ptr(trace), ptr(tw), 3.0, ptr(prev), ptr(reset), ptr(state), None,
             ptr(act), ptr(nt), ptr(end), None, B, T, H, 0.0375, 1, stream_of(r))
        torch.cuda.synchronize()
        outs.append(end.clone())
    assert torch.equal(outs[0], outs[1])


def test_paraplex_tria_endpoint_argument_errors():
    from loom_amd._lib import call, ptr
    x = torch.zeros(2, 3, 4, device=DEV)
    t = torch.zeros(2, 4, device=DEV)
    h = torch.zeros(4, device=DEV)
    c = torch.zeros(2, 3, 4, 9, device=DEV)
    rs = torch.zeros(2, 3, dtype=torch.bool, device=DEV)
    e = torch.zeros(2, 4, 9, device=DEV)
    base = [0, ptr(x), ptr(x), ptr(x), ptr(h), ptr(t), ptr(h), 3.0, ptr(c), ptr(rs), None, None,
            ptr(x), ptr(t), ptr(e), None, 2, 3, 4, 0.0375, 0, None]
    # bad axis, no carried records, no reset, odd H, trace aliasing next_trace
    cases = [[(20, 3)], [(8, None)], [(9, None)], [(18, 3)], [(13, ptr(t))]]
    for edits in cases:
        args = list(base)
        for k, v in edits:
            args[k] = v
        with pytest.raises(RuntimeError, match="paraplex_tria_endpoint"):
            call("loom_paraplex_tria_endpoint_forward", *args)
    torch.cuda.synchronize()
    assert torch.count_nonzero(e) == 0  # nothing was launched


def test_paraplex_tria_argument_errors():
    from loom_amd._lib import call, ptr
    x = torch.zeros(2, 3, 4, device=DEV)
    t = torch.zeros(2, 4, device=DEV)
    h = torch.zeros(4, device=DEV)
    c = torch.zeros(2, 3, 4, 9, device=DEV)
    base = [0, ptr(x), ptr(x), ptr(x), ptr(h), ptr(t), ptr(h), 3.0, None, None, None, None,
            ptr(x), ptr(t), ptr(c), None, 2, 3, 4, 0.0375, 0, None]
    cases = {20: [(20, 3)], 8: [(8, ptr(c)), (9, ptr(c)), (10, ptr(x))], 11: [(11, ptr(h))],
             12: [(12, None)]}
    for edits in cases.values():
        args = list(base)
        for k, v in edits:
            args[k] = v
        with pytest.raises(RuntimeError, match="paraplex_tria"):
            call("loom_paraplex_tria_forward", *args)
    torch.cuda.synchronize()
    assert torch.count_nonzero(c) == 0  # nothing was launched


def test_golden_tria_vs_reference():
    from loom_amd import ops
    z = np.load(os.path.join(GOLD, "ops.npz"))
    t = {k: torch.from_numpy(z[f"tria.{k}"]).to(DEV) for k in ("r", "i", "o", "prev", "seed", "valid", "w")}
    a = 0.0375
    f32 = torch.float32
    for axis in range(3):
        G = lambda nm: torch.from_numpy(z[f"tria.{nm}"])
        check(ops.tria_init_forward(t["r"], t["i"], t["o"], a, axis)[0], G(f"init_{axis}"), f32)
        check(ops.tria_step_forward(t["r"], t["i"], t["o"], t["prev"], a, axis)[0], G(f"step_{axis}"), f32)
        check(ops.tria_init_seed_forward(t["r"], t["i"], t["o"], t["seed"], t["valid"], a, axis)[0],
              G(f"seed_{axis}"), f32)
        c, p, _ = ops.tria_step_gate_forward(t["r"], t["i"], t["o"], t["prev"], t["w"], a, axis)
        check(c, G(f"step_gate_{axis}.carry"), f32)
        check(p, G(f"step_gate_{axis}.p"), f32)
        c, p = ops.tria_init_seed_gate_forward(t["r"], t["i"], t["o"], t["seed"], t["valid"], t["w"], a, axis)
        check(c, G(f"seed_gate_{axis}.carry"), f32)
        check(p, G(f"seed_gate_{axis}.p"), f32)
    depth, rs, ini = (torch.from_numpy(z[k]).to(DEV) for k in ("tc.depth", "tc.reset", "tc.init"))
    doc, _ = ops.temporal_carry_forward(depth, rs)
    check(doc, torch.from_numpy(z["tc.full_ref"]), f32)
    e, e32 = ops.temporal_carry_endpoint_forward(depth, rs, torch.empty(0, device=DEV),
                                                 torch.empty(0, dtype=torch.bool, device=DEV))
    check(e, torch.from_numpy(z["tc.end_noinit"]), f32)
    e, _ = ops.temporal_carry_endpoint_forward(depth, rs, ini, t["valid"])
    check(e, torch.from_numpy(z["tc.end_init_valid"]), f32)
    e, _ = ops.temporal_carry_endpoint_forward(depth, rs, ini, torch.ones(3, dtype=torch.bool, device=DEV))
    check(e, torch.from_numpy(z["tc.end_init"]), f32)
    check(ops.polarm(torch.from_numpy(z["polarm.in"]).to(DEV), 0.1), torch.from_numpy(z["polarm.out"]), f32)
    q, k, v, al = (torch.from_numpy(z[f"fca.{n}"]).to(DEV) for n in ("q", "k", "v", "allowed"))
    out, _ = ops.final_ca_sparse_forward(q, k, v, al, q.shape[-1] ** -0.5)
    check(out, torch.from_numpy(z["fca.out"]), f32)
    sw = torch.from_numpy(z["agg.score_w"]).to(DEV)
    carry = torch.from_numpy(z["agg.carry"]).to(DEV)
    pooled, lse = ops.slot_attention_pool_forward(carry, sw)
    want, want_lse = ref.slot_attention_pool(carry.cpu(), sw.cpu())
    check(pooled, want, f32)
    check(lse, want_lse, f32)


@pytest.mark.parametrize("dtype", DTYPES3)
def test_gate_mix_and_slot_pool(dtype):
    from loom_amd import ops
    g = gen(9)
    carry = dev(ref.local_normalize(rnd(g, 2, 3, 3072, 3, 3)), dtype)
    w = dev(torch.softmax(rnd(g, 9), 0), dtype)
    check(ops.gate_slot_mix_forward(carry, w), ref.gate_slot_mix(host(carry), host(w)), dtype)
    sw = dev(rnd(g, 9, scale=3.0), dtype)
    pooled, lse = ops.slot_attention_pool_forward(carry, sw)
    wp, wl = ref.slot_attention_pool(host(carry), host(sw))
    check(pooled, wp, dtype)
    check(lse, wl, dtype)
    # H = 1 -> pooled is the single carrier
    pooled, _ = ops.slot_attention_pool_forward(carry[:, :, :1].contiguous(), sw)
    check(pooled, host(carry)[:, :, 0].reshape(2, 3, 9), dtype)


@pytest.mark.parametrize("dtype", DTYPES3)
@pytest.mark.parametrize("B,T,H", [(3, 9, 6), (2, 64, 1000), (1, 1, 5), (1, 3, 7), (4, 128, 3072)])
def test_temporal_carry(dtype, B, T, H):
    from loom_amd import ops
    g = gen(B * T + H)
    depth = dev(ref.local_normalize(rnd(g, B, T, H, 3, 3)), dtype)
    reset = torch.rand(B, T, generator=g) > 0.85
    rs = dev(reset, torch.bool)
    ini = dev(ref.local_normalize(rnd(g, B, H, 3, 3)), dtype)
    valid = torch.rand(B, generator=g) > 0.5
    D = host(depth)
    doc, scale = ops.temporal_carry_forward(depth, rs)
    full = ref.temporal_carry(D, reset)
    if dtype == torch.float32 and T > 64:
        # 128 chained fp32 products: the rounding of both sides grows along the
        # chain (measured up to 1.7e-4 absolute near zero over 14 M entries)
        torch.testing.assert_close(host(doc), full, rtol=1e-3, atol=5e-4)
    else:
        check(doc, full, torch.float32 if dtype == torch.float32 else dtype)
    e, e32 = ops.temporal_carry_endpoint_forward(depth, rs, torch.empty(0, device=DEV, dtype=dtype),
                                                 torch.empty(0, dtype=torch.bool, device=DEV))
    check(e32, full[:, -1], dtype)           # endpoint == last row of the full recurrence
    e, e32 = ops.temporal_carry_endpoint_forward(depth, rs, ini, dev(valid, torch.bool))
    check(e32, ref.temporal_carry_endpoint(D, reset, host(ini), valid), dtype)


@pytest.mark.parametrize("dtype", DTYPES3)
def test_polarm_and_final_ca(dtype):
    from loom_amd import ops
    g = gen(77)
    M = dev(rnd(g, 4, 50, 3, 3), dtype)
    mask = torch.tensor([True, False, True, False])
    got = ops.polarm(M, 0.1, mask=dev(mask, torch.bool))
    want = torch.where(mask[:, None, None, None], ref.polarm(host(M), 0.1), host(M))
    check(got, want, dtype)
    # fixed point: an orthogonal matrix is unchanged
    Q, _ = torch.linalg.qr(rnd(g, 6, 3, 3))
    check(ops.polarm(dev(Q, torch.float32), 0.3), Q, torch.float32, atol=1e-5)
    B, T, K, D = 3, 5, 40, 768
    q, k, v = dev(rnd(g, B, T, D), dtype), dev(rnd(g, B, K, D), dtype), dev(rnd(g, B, K, D), dtype)
    allowed = torch.rand(B, T, K, generator=g) > 0.6
    allowed[1, 3] = False                     # a row with no key -> exact zeros
    out, lse = ops.final_ca_sparse_forward(q, k, v, dev(allowed, torch.bool), D ** -0.5)
    check(out, ref.final_ca_sparse(host(q), host(k), host(v), allowed, D ** -0.5), dtype)
    assert torch.all(host(out)[1, 3] == 0) and float(lse[1, 3]) == -math.inf
    wl = ref.final_ca_sparse_lse(host(q), host(k), host(v), allowed, D ** -0.5)
    ok = allowed.any(-1)
    check(lse[ok.to(DEV)], wl[ok], torch.float32, rtol=1e-3, atol=1e-3)


# ----------------------------------------------------------------- drop-in

def test_drop_in_build_or_load_runs_on_gpu():
    from kernels.build import build_or_load
    mod = build_or_load("loomformer_tria_carry", ["tria/bindings.cpp"], extra_cuda_cflags=["--use_fast_math"])
    g = gen(3)
    r, i, o, prev, seed, valid, w = _tria_inputs(g, 2, 3, 16, torch.float32)
    c, p, s = mod.tria_step_gate_forward(r, i, o, prev, w, 0.05, 1)
    wc, wp = ref.tria_step_and_gate(host(r), host(i), host(o), host(prev), host(w), 0.05, 1)
    check(c, wc, torch.float32)
    check(p, wp, torch.float32)
    with pytest.raises(RuntimeError, match="axis"):
        mod.tria_step_forward(r, i, o, prev, 0.05, 3)
