"""Oracle pinned by mathematics: closed forms, invariants, library routines
and brute force on tiny inputs (CPU only).

Each check uses a formulation independent of the oracle's own code, chosen so
that a plausible slip in the restatement (a dropped term, a sign, a
transposed operand, a wrong index) fails it.  The reference-generated
fixtures in tests/golden/ pin the same functions from the other side
(test_oracle_golden.py).
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import ops

torch.set_default_dtype(torch.float32)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ------------------------------------------------------------------ Paraplex

def test_phase_sin_is_sin_of_tanh_asinh():
    """beta/sqrt(1+beta^2) == tanh(asinh(beta)); the phase is odd, monotone,
    0 at 0 and tends to +-1."""
    b = torch.linspace(-40, 40, 4001, dtype=torch.float64)
    got = ops.phase_sin(b.float()).double()
    want = torch.sin(math.pi / 2 * torch.tanh(torch.asinh(b)))
    torch.testing.assert_close(got, want, rtol=0, atol=2e-7)
    assert ops.phase_sin(torch.zeros(1)).item() == 0.0
    torch.testing.assert_close(ops.phase_sin(-b.float()), -ops.phase_sin(b.float()), rtol=0, atol=0)
    assert bool((got[1:] >= got[:-1]).all())
    assert abs(ops.phase_sin(torch.tensor([1e6])).item() - 1.0) < 1e-6


def test_sin_space_combine_is_tanh_asinh():
    z = torch.randn(1000, generator=_gen(1), dtype=torch.float64) * 5
    s0, tr = z[:500], z[500:]
    got = ops.sin_space_combine(s0.float(), tr.float()).double()
    zf = (s0.float() + tr.float()).double()          # the sum the fp32 oracle forms
    torch.testing.assert_close(got, torch.tanh(torch.asinh(zf)), rtol=0, atol=2e-7)


def test_prev_token_trace_brute_force():
    g = _gen(2)
    B, T, H = 3, 5, 4
    s = torch.randn(B, T, H, generator=g)
    init = torch.randn(B, H, generator=g)
    reset = torch.rand(B, T, generator=g) < 0.3
    got = ops.prev_token_trace(s, init, reset)
    for b in range(B):
        for t in range(T):
            for h in range(H):
                want = 0.0 if reset[b, t] else (init[b, h] if t == 0 else s[b, t - 1, h])
                assert got[b, t, h].item() == float(want)
    # no initial trace -> zeros at t = 0
    assert bool((ops.prev_token_trace(s, None, None)[:, 0] == 0).all())


def test_pvpowlu_special_cases():
    """G(A) = A^(m/(sqrt A + 1)) * sigmoid(A): m = 0 leaves sigmoid (a
    library routine); at A = 4, m = 3 the exponent is 1 so G = 4 sigmoid(4);
    at A = 1 the power is 1 for every m; A -> 0 gives 0."""
    x1 = torch.randn(200, generator=_gen(3))
    a = torch.rand(200, generator=_gen(4)) * 9 + 0.01
    torch.testing.assert_close(ops.pvpowlu(x1, a, 0.0), x1 * torch.sigmoid(a), rtol=1e-6, atol=0)
    four = torch.full((1,), 4.0)
    torch.testing.assert_close(ops.powlu_gate(four, 3.0), 4 * torch.sigmoid(four), rtol=1e-6, atol=0)
    one = torch.ones(1)
    for m in (0.5, 3.0, 7.0):
        torch.testing.assert_close(ops.powlu_gate(one, m), torch.sigmoid(one), rtol=1e-6, atol=0)
    assert ops.powlu_gate(torch.tensor([1e-30]), 3.0).item() < 1e-20


def _expected_head_columns(N, QH, HD):
    """Compact W_imag column -> dense column, head mode, written out per
    sector: q-head g reads [Q_g | Kctx_g | C_g | U | D_g] from the dense
    blocks [Q | Kctx | C | U | D], each N wide."""
    cols = []
    for g in range(QH):
        row = []
        row += [0 * N + g * HD + d for d in range(HD)]      # Q_g
        row += [1 * N + g * HD + d for d in range(HD)]      # Kctx_g
        row += [2 * N + g * HD + d for d in range(HD)]      # C_g
        row += [3 * N + n for n in range(N)]                # U
        row += [4 * N + g * HD + d for d in range(HD)]      # D_g
        cols.append(row)
    return cols


def test_imag_layout_and_grouped_equals_brute_force():
    """beta for head-mode sectors by explicit sums over the written-out
    sector layout, against both the grouped and the dense-scatter forms."""
    g = _gen(5)
    B, T, QH, HD = 2, 3, 2, 4
    N, H = QH * HD, 16
    Hq = H // QH
    K = ops.imag_in(N, HD, "head")
    assert K == N + 4 * HD
    u = torch.randn(B, T, N, generator=g)
    q, kc, c, d = (torch.randn(B, T, QH, HD, generator=g) for _ in range(4))
    w = torch.randn(H, K, generator=g)
    dense_in = torch.cat([q.reshape(B, T, N), kc.reshape(B, T, N), c.reshape(B, T, N), u,
                          d.reshape(B, T, N)], dim=-1)
    cols = _expected_head_columns(N, QH, HD)
    want = torch.zeros(B, T, H, dtype=torch.float64)
    for h in range(H):
        gq = h // Hq
        for k in range(K):
            want[:, :, h] += w[h, k].double() * dense_in[:, :, cols[gq][k]].double()
    got_g = ops.beta_space_grouped(u, q, kc, c, d, w, QH, HD, "head")
    got_d = ops.beta_space_dense(u, q, kc, c, d, w, QH, HD, "head")
    torch.testing.assert_close(got_g.double(), want, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(got_d.double(), want, rtol=1e-5, atol=1e-5)
    # and the flat-index helper names exactly those dense cells
    flat = ops.w1_imag_live_flat_indices(N, QH, HD, H, "head")
    expect = torch.tensor([h * 5 * N + cols[h // Hq][k] for h in range(H) for k in range(K)])
    assert torch.equal(flat.flatten().sort().values, expect.sort().values)


# ------------------------------------------------------------------ DepthAttn

def test_depth_attention_invariants():
    g = _gen(6)
    B, T, S, QH, HD = 2, 3, 5, 2, 8
    q = torch.randn(QH, HD, generator=g)
    k = torch.randn(B, T, S, QH, HD, generator=g)
    v = torch.randn(B, T, S, QH, HD, generator=g)
    # S = 1: the read is the single value row, exactly
    torch.testing.assert_close(ops.depth_attn_online(q, k[:, :, :1], v[:, :, :1]), v[:, :, 0],
                               rtol=0, atol=0)
    # equal keys: the mean of the values
    keq = k[:, :, :1].expand(-1, -1, S, -1, -1).contiguous()
    torch.testing.assert_close(ops.depth_attn_online(q, keq, v), v.mean(dim=2), rtol=1e-5,
                               atol=1e-6)
    # online form == plain softmax form == library attention; lse == logsumexp
    d_on = ops.depth_attn_online(q, k, v)
    d_sm, w, lse = ops.depth_attn_softmax(q, k, v)
    qq = q.view(1, 1, QH, 1, HD).expand(B, T, QH, 1, HD)
    kk = k.permute(0, 1, 3, 2, 4)
    vv = v.permute(0, 1, 3, 2, 4)
    lib = F.scaled_dot_product_attention(qq.reshape(-1, 1, HD), kk.reshape(-1, S, HD),
                                         vv.reshape(-1, S, HD)).reshape(B, T, QH, HD)
    torch.testing.assert_close(d_on, lib, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(d_sm, lib, rtol=1e-5, atol=1e-6)
    scores = (qq * kk).sum(-1) / math.sqrt(HD)
    torch.testing.assert_close(lse, torch.logsumexp(scores, -1), rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(w.sum(-1), torch.ones(B, T, QH), rtol=1e-6, atol=1e-6)


# ------------------------------------------------------------------ Tria

def _hat(v):
    a, b, c = v.unbind(-1)
    z = torch.zeros_like(a)
    return torch.stack([torch.stack([z, -c, b], -1), torch.stack([c, z, -a], -1),
                        torch.stack([-b, a, z], -1)], -2)


def _rot90(axis):
    """Right-handed rotation by +90 degrees about z (axis 0), x (1), y (2)."""
    c, s = round(math.cos(math.pi / 2)), round(math.sin(math.pi / 2))
    if axis == 0:
        m = [[c, -s, 0], [s, c, 0], [0, 0, 1]]
    elif axis == 1:
        m = [[1, 0, 0], [0, c, -s], [0, s, c]]
    else:
        m = [[c, 0, s], [0, 1, 0], [-s, 0, c]]
    return torch.tensor(m, dtype=torch.float32)


@pytest.mark.parametrize("axis", [0, 1, 2])
def test_carrier_is_cross_matrix_times_rotation(axis):
    """T = (I + hat(v)) @ R_axis(+90 deg), v = alpha * tanh(x / rms(x)),
    x = (ri, ro, io): the structure the reference's comments state
    (tria.py:50-65); det T = 1 + |v|^2 (> 0.9 as the reference self-test
    asserts, tria.py:1640) and T is full rank at zero signal."""
    g = _gen(7 + axis)
    r, i, o = (torch.randn(4, 5, 6, generator=g) * 3 for _ in range(3))
    alpha = 0.0375
    x = torch.stack((r * i, r * o, i * o), -1)
    vvec = alpha * torch.tanh(x / torch.sqrt(x.square().mean(-1, keepdim=True) + 1e-6))
    want = (torch.eye(3) + _hat(vvec)) @ _rot90(axis)
    got = ops.build_tria(r, i, o, alpha, axis)
    torch.testing.assert_close(got, want, rtol=0, atol=1e-7)
    torch.testing.assert_close(torch.linalg.det(got.double()),
                               1 + vvec.double().square().sum(-1), rtol=1e-6, atol=1e-6)
    z = torch.zeros(2, 2, 2)
    assert bool((torch.linalg.matrix_rank(ops.build_tria(z, z, z, alpha, axis)) == 3).all())


def test_tria_chain_rms_and_composition():
    """Every (b,t,h) carry has RMS 1 whatever its input scale (tria.py
    self-test 2-3); a step is the normalised left product (brute force)."""
    g = _gen(11)
    scale = torch.tensor([1.0, 5.0, 20.0])
    r, i, o = (torch.randn(4, 8, 3, generator=g) * scale for _ in range(3))
    c = ops.tria_init(r, i, o, 0.025, 0)
    rms = c.square().mean(dim=(-1, -2)).sqrt()
    torch.testing.assert_close(rms, torch.ones_like(rms), rtol=0, atol=1e-5)
    for layer in range(1, 30):
        r, i, o = (torch.randn(4, 8, 3, generator=g) * 15 for _ in range(3))
        prev = c
        c = ops.tria_step(r, i, o, prev, 0.025, layer % 3)
        T_ = ops.build_tria(r, i, o, 0.025, layer % 3)
        b, t, h = layer % 4, layer % 8, layer % 3
        m = [[sum(T_[b, t, h, rr, kk].item() * prev[b, t, h, kk, cc].item() for kk in range(3))
              for cc in range(3)] for rr in range(3)]
        nrm = math.sqrt(sum(e * e for row in m for e in row) / 9 + 1e-6)
        torch.testing.assert_close(c[b, t, h], torch.tensor(m) / nrm, rtol=1e-5, atol=1e-6)
    rms = c.square().mean(dim=(-1, -2)).sqrt()
    torch.testing.assert_close(rms, torch.ones_like(rms), rtol=0, atol=1e-4)


def test_seeded_init_and_gate():
    g = _gen(12)
    B, T, H = 3, 4, 5
    r, i, o = (torch.randn(B, T, H, generator=g) for _ in range(3))
    seed = ops.local_normalize(torch.randn(B, H, 3, 3, generator=g))
    valid = torch.tensor([True, False, True])
    c = ops.tria_init_seed(r, i, o, seed, valid, 0.025, 1)
    plain = ops.tria_init(r, i, o, 0.025, 1)
    T_ = ops.build_tria(r, i, o, 0.025, 1)
    torch.testing.assert_close(c[1], plain[1], rtol=0, atol=0)          # invalid seed row
    torch.testing.assert_close(c[:, 1:], plain[:, 1:], rtol=0, atol=0)   # t > 0 untouched
    torch.testing.assert_close(c[0, 0], ops.local_normalize(T_[0, 0] @ seed[0]), rtol=1e-6, atol=1e-7)
    # a one-hot gate picks that slot of vec(C) (row-major)
    for k in range(9):
        w = F.one_hot(torch.tensor(k), 9).float()
        _, p = ops.tria_step_and_gate(r, i, o, plain, w, 0.025, 2)
        cc = ops.tria_step(r, i, o, plain, 0.025, 2)
        torch.testing.assert_close(p, cc[..., k // 3, k % 3], rtol=0, atol=0)


def test_temporal_carry_endpoint_is_last_row_and_prepend():
    """endpoint == last row of the sequential carry (with resets); carrying
    an initial state == prepending it as an extra first row (the carry is
    positively homogeneous, so N(D @ (c S)) == N(D @ S))."""
    g = _gen(13)
    B, T, H = 3, 9, 4
    d = torch.randn(B, T, H, 3, 3, generator=g)
    reset = torch.rand(B, T, generator=g) < 0.25
    seq = ops.temporal_carry(d, reset)
    end = ops.temporal_carry_endpoint(d, reset)
    torch.testing.assert_close(end, seq[:, -1], rtol=1e-5, atol=1e-6)
    init = ops.local_normalize(torch.randn(B, H, 3, 3, generator=g))
    valid = torch.tensor([True, False, True])
    got = ops.temporal_carry_endpoint(d, reset, init, valid)
    for b in range(B):
        if valid[b]:
            dd = torch.cat([init[b:b + 1, None], d[b:b + 1]], dim=1)
            rr = torch.cat([torch.zeros(1, 1, dtype=torch.bool), reset[b:b + 1]], dim=1)
        else:
            dd, rr = d[b:b + 1], reset[b:b + 1]
        torch.testing.assert_close(got[b], ops.temporal_carry(dd, rr)[0, -1], rtol=1e-5, atol=1e-5)


def test_polarm_fixed_points_and_contraction():
    """M^T M proportional to I is a fixed point; beta = 0 is the identity;
    a near-orthogonal M moves towards orthogonality."""
    g = _gen(14)
    Q, _ = torch.linalg.qr(torch.randn(6, 3, 3, generator=g, dtype=torch.float64))
    Qf = (Q * 2.5).float()
    torch.testing.assert_close(ops.polarm(Qf, 0.3), Qf, rtol=1e-5, atol=1e-5)
    M = Qf + 0.05 * torch.randn(6, 3, 3, generator=g)
    torch.testing.assert_close(ops.polarm(M, 0.0), M, rtol=0, atol=0)

    def defect(X):
        G = X.transpose(-1, -2) @ X
        s = G.diagonal(dim1=-2, dim2=-1).mean(-1)[..., None, None]
        return (G / s - torch.eye(3)).norm(dim=(-1, -2))

    assert bool((defect(ops.polarm(M, 0.5)) < defect(M)).all())


# ------------------------------------------------------------------ readout

def test_slot_pool_brute_force_and_score_norm():
    g = _gen(15)
    B, T, H = 2, 3, 5
    carry = torch.randn(B, T, H, 3, 3, generator=g)
    sw = torch.randn(9, generator=g)
    pooled, lse = ops.slot_attention_pool(carry, sw)
    for b in range(B):
        for t in range(T):
            sc = [sum(sw[k].item() * carry[b, t, h].flatten()[k].item() for k in range(9))
                  for h in range(H)]
            mx = max(sc)
            ex = [math.exp(x - mx) for x in sc]
            tot = sum(ex)
            assert abs(lse[b, t].item() - (mx + math.log(tot))) < 1e-5
            for k in range(9):
                want = sum(ex[h] / tot * carry[b, t, h].flatten()[k].item() for h in range(H))
                assert abs(pooled[b, t, k].item() - want) < 1e-5
    key = torch.randn(32, 9, generator=g)
    query = torch.randn(32, generator=g)
    scale = torch.tensor(1.7)
    s = ops.make_score_w(key, query, scale)
    assert abs(s.norm().item() - 1.7) < 1e-5
    assert torch.allclose(s / s.norm(), (key.t() @ query) / (key.t() @ query).norm(), atol=1e-6)


def test_final_ca_special_cases_and_library():
    g = _gen(16)
    B, T, K, D = 2, 4, 6, 8
    q, k, v = (torch.randn(B, n, D, generator=g) for n in (T, K, K))
    scale = D ** -0.5
    none = torch.zeros(B, T, K, dtype=torch.bool)
    assert bool((ops.final_ca_sparse(q, k, v, none, scale) == 0).all())
    assert bool(torch.isneginf(ops.final_ca_sparse_lse(q, k, v, none, scale)).all())
    one = torch.zeros(B, T, K, dtype=torch.bool)
    one[:, :, 3] = True
    torch.testing.assert_close(ops.final_ca_sparse(q, k, v, one, scale),
                               v[:, 3:4].expand(B, T, D), rtol=0, atol=1e-6)
    allow = torch.rand(B, T, K, generator=g) < 0.6
    allow[:, :, 0] = True
    lib = F.scaled_dot_product_attention(q, k, v, attn_mask=allow, scale=scale)
    torch.testing.assert_close(ops.final_ca_sparse(q, k, v, allow, scale), lib, rtol=1e-5,
                               atol=1e-6)
    lse = ops.final_ca_sparse_lse(q, k, v, allow, scale)
    for b in range(B):
        for t in range(T):
            xs = [scale * float(q[b, t] @ k[b, j]) for j in range(K) if allow[b, t, j]]
            mx = max(xs)
            assert abs(lse[b, t].item() - (mx + math.log(sum(math.exp(x - mx) for x in xs)))) < 1e-5


# ------------------------------------------------------------------ RoPE

def test_yarn_reduces_to_rope_and_rotation_preserves_pairs():
    """factor 1: plain RoPE frequencies theta^(-2i/d) and attention factor 1;
    the rotation keeps each (x_i, x_{i+d/2}) pair's norm and is the identity
    at position 0."""
    HD, theta = 16, 10000.0
    inv, af = ops.yarn_inv_freq(HD, theta, 1.0, 2048, 32.0, 1.0)
    want = torch.tensor([theta ** (-2 * i / HD) for i in range(HD // 2)], dtype=torch.float32)
    torch.testing.assert_close(inv, want, rtol=1e-6, atol=0)
    assert af == 1.0
    cos, sin = ops.yarn_cos_sin(inv, af, 64)
    x = torch.randn(64, HD, generator=_gen(17))
    y = ops.apply_rope(x, cos, sin)
    h = HD // 2
    torch.testing.assert_close(y[:, :h] ** 2 + y[:, h:] ** 2, x[:, :h] ** 2 + x[:, h:] ** 2,
                               rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(y[0], x[0], rtol=0, atol=0)
    # position p rotates pair i by angle p * inv_freq[i]
    p, i = 37, 3
    ang = p * inv[i].item()
    want_pair = (x[p, i] * math.cos(ang) - x[p, i + h] * math.sin(ang),
                 x[p, i] * math.sin(ang) + x[p, i + h] * math.cos(ang))
    assert abs(y[p, i].item() - want_pair[0].item()) < 1e-4
    assert abs(y[p, i + h].item() - want_pair[1].item()) < 1e-4
    # factor > 1: attention factor 0.1 ln(s) + 1, frequencies between the
    # extrapolated and interpolated ones
    inv4, af4 = ops.yarn_inv_freq(HD, theta, 4.0, 2048, 32.0, 1.0)
    assert abs(af4 - (0.1 * math.log(4.0) + 1.0)) < 1e-7
    assert bool(((inv4 <= want * (1 + 1e-6)) & (inv4 >= want / 4 * (1 - 1e-6))).all())


# ------------------------------------------------------------------ chunked Tria path

def _tria_by_token(r, i, o, alpha, window, beta):
    """Keys of the token-by-token formulation: Model.step's Tria bookkeeping
    (oracle.model.tria_layer_op / tria_temporal_token, pinned by the decode
    fixtures the reference wrote) driven by given per-layer summaries."""
    from oracle.model import TemporalState, tria_layer_op, tria_temporal_token
    L, B, T, H = r.shape
    w = torch.full((9,), 1.0 / 9.0)
    ts = TemporalState()
    keys = []
    for t in range(T):
        pending = torch.zeros(B, dtype=torch.bool) if ts.pending is None else ts.pending
        seed_valid = pending & (t != 0)
        carry = None
        for l in range(L):
            sl = slice(t, t + 1)
            carry, _ = tria_layer_op(l, l == L - 1, r[l, :, sl], i[l, :, sl], o[l, :, sl], carry,
                                     ts.carry, seed_valid, w, alpha)
        doc, fire = tria_temporal_token(carry[:, 0], ts, pending, t,
                                        torch.zeros(B, dtype=torch.bool), T, window, beta)
        if bool(fire.any()):
            keys.append(doc)
        ts = TemporalState(carry=doc, pending=fire)
    return torch.stack(keys, dim=1)


@pytest.mark.parametrize("L,T,W", [(4, 23, 5), (3, 20, 4), (1, 9, 2)])
def test_tria_chunked_matches_token_by_token_step(L, T, W):
    """The chunked forward and the decode step carry the same Tria state
    (_forward_chunked vs step, loomformer.py:3788-3883 / :4012-4078): the
    document keys at every fire agree (up to the eps of the extra N at a
    restart)."""
    g = _gen(51)
    B, H = 2, 6
    r, i, o = (torch.randn(L, B, T, H, generator=g) for _ in range(3))
    keys, depth = ops.tria_chunked(r, i, o, 0.3, W, 0.1)
    assert keys.shape == (B, -(-T // W) - 1, H, 3, 3) and depth.shape == (B, T, H, 3, 3)
    want = _tria_by_token(r, i, o, 0.3, W, 0.1)
    torch.testing.assert_close(keys, want, rtol=1e-5, atol=1e-5)


def test_tria_chunked_rotation_products_at_alpha_zero():
    """alpha = 0 makes every local operator the signed permutation R_axis
    (axis l % 3), whose products are exact: the first key is the normalised
    product D_{W-1} ... D_0 with D = R_{(L-1)%3} ... R_1 R_0 (layer 0 rightmost),
    and PolARM leaves a scaled orthogonal matrix unchanged."""
    Rz = torch.tensor([[0., -1, 0], [1, 0, 0], [0, 0, 1]])
    Rx = torch.tensor([[1., 0, 0], [0, 0, -1], [0, 1, 0]])
    Ry = torch.tensor([[0., 0, 1], [0, 1, 0], [-1, 0, 0]])
    axes = [Rz, Rx, Ry]
    L, B, T, H, W = 4, 1, 7, 3, 2
    g = _gen(52)
    r, i, o = (torch.randn(L, B, T, H, generator=g) for _ in range(3))
    keys, _ = ops.tria_chunked(r, i, o, 0.0, W, 0.1)
    assert keys.shape[1] == 3
    D, D_rev = torch.eye(3), torch.eye(3)
    for l in range(L):
        D = axes[l % 3] @ D
        D_rev = D_rev @ axes[l % 3]
    P = torch.linalg.matrix_power(D, W)
    # the layer order and the chunk chaining are visible in these products
    assert not torch.allclose(P, torch.linalg.matrix_power(D_rev, W))
    assert not torch.allclose(P @ P, torch.eye(3))
    for c in range(3):
        Pc = torch.linalg.matrix_power(P, c + 1)   # chunk c continues from key c-1
        torch.testing.assert_close(keys[0, c], (Pc / Pc.square().mean().sqrt()).expand(H, 3, 3),
                                   rtol=0, atol=1e-5)


def test_tria_chunked_reset_cuts_history_and_fire():
    """A document start inside a chunk makes its key independent of every
    earlier token; a document start at a chunk's first token suppresses the
    previous boundary's fire (hard_fire & ~next_is_reset, :3808-3810), so that
    key is the uncorrected state, which PolARM maps to the fired key."""
    g = _gen(53)
    L, B, T, H, W = 3, 2, 16, 5, 4
    r, i, o = (torch.randn(L, B, T, H, generator=g) for _ in range(3))
    reset = torch.zeros(B, T, dtype=torch.bool)
    reset[0, 9] = True                # inside chunk 2 of batch 0
    keys, _ = ops.tria_chunked(r, i, o, 0.3, W, 0.1, reset)
    r2 = r.clone()
    r2[:, 0, :9] += 1.0               # tokens before the reset
    keys2, _ = ops.tria_chunked(r2, i, o, 0.3, W, 0.1, reset)
    torch.testing.assert_close(keys2[0, 2:], keys[0, 2:], rtol=0, atol=0)
    assert not torch.allclose(keys2[0, 1], keys[0, 1])
    reset_b = torch.zeros(B, T, dtype=torch.bool)
    reset_b[1, 8] = True              # start of chunk 2 of batch 1
    keys_b, _ = ops.tria_chunked(r, i, o, 0.3, W, 0.1, reset_b)
    keys_n, _ = ops.tria_chunked(r, i, o, 0.3, W, 0.1)
    torch.testing.assert_close(ops.polarm(keys_b[1, 1], 0.1), keys_n[1, 1], rtol=1e-6, atol=1e-6)
    assert not torch.allclose(keys_b[1, 1], keys_n[1, 1], atol=1e-4)
