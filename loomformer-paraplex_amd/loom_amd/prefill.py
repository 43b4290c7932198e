"""Chunked prefill of the decode state.

The reference runs a prompt through ``Model._forward_chunked``
(loomformer.py:3788-3883): the whole block stack for one temporal chunk of
tokens at a time, the temporal Tria carry from boundary to boundary, PolARM
and a document key at every fire, and the final cross-attention over the keys
of earlier fires.  ``prefill`` does the same on the gfx950 kernels and leaves
the engine exactly where token-by-token ``Model.step`` (:3951-4091) would be
after the last prompt token: KV caches, per-layer phase traces, the Tria
document state and pending fire, the final-CA key cache, the position and the
last token's logits.  Decoding then continues with the captured step.

Chunk boundaries are the step's fire positions: (t + 1) % W == 0 while
t + 1 < seq_len, plus every position where some row holds the <CARRY> id;
the fire of row b at a boundary t is hard(t) or prompt[b, t] == <CARRY>
(loomformer.py:4067-4078).  A chunk's first token is seeded from the state
after the previous boundary in the rows where that boundary fired
(tria_init_seed, tria.py:835-844), and the temporal carry restarts there
(:3834-3850).
"""
from __future__ import annotations

from typing import List

import torch

from . import _lib

_P = _lib.ptr

# batch rows of a layer's attention on the aux stream (the rest on main, after
# its depth read): at B = 32, 24 rows measured 62.2-62.3 ms against 62.5-62.6
# with all 32 on aux (16 and 20: 62.3-62.4)
PREFILL_AUX_ROWS = 24


def chunk_bounds(prompt_cpu: torch.Tensor, window: int, seq_len: int, carry_id) -> List[int]:
    """Last position of every chunk of a [B, P] prompt (the final one is P-1)."""
    B, P = prompt_cpu.shape
    fires = set(t for t in range(P) if (t + 1) % window == 0 and t + 1 < seq_len)
    if carry_id is not None:
        hit = (prompt_cpu == int(carry_id)).any(dim=0)
        fires |= set(int(t) for t in hit.nonzero().flatten().tolist())
    ends = sorted(fires)
    if not ends or ends[-1] != P - 1:
        ends.append(P - 1)
    return ends


@torch.no_grad()
def prefill(eng, prompt: torch.Tensor) -> None:
    """Run ``prompt`` [B, P] through the chunked forward and set ``eng`` up to
    decode position P (see the module docstring).  The many-row products run
    in the library's shared-tile mode (half-CU blocks), since they run beside
    the other streams' kernels; the previous mode is restored on return."""
    lib = _lib.load()
    prev = lib.loom_gemm_shared_tiles(1)
    try:
        _prefill(eng, prompt)
    finally:
        lib.loom_gemm_shared_tiles(prev)


def _prefill(eng, prompt: torch.Tensor) -> None:
    c = eng.cfg
    B, P = prompt.shape
    if B != eng.B or P < 1:
        raise ValueError("prompt must be [batch, >=1]")
    eng._check_capacity(P - 1)
    eng._check_ids(prompt)
    N, H, L, QH, KVH, HD = c.N, c.H, c.L, c.QH, c.KVH, c.HD
    dev, dt, code = eng.dev, eng.dtype, eng.code
    st = eng._stream()
    call = eng._call
    prompt_d = prompt.to(dev)
    prompt_cpu = prompt.cpu()
    ends = chunk_bounds(prompt_cpu, c.window, c.seq_len, eng.carry_token_id)
    hard = torch.tensor([(t + 1) % c.window == 0 and t + 1 < c.seq_len for t in range(P)])
    fire_all = hard[None, :].expand(B, P).clone()
    if eng.carry_token_id is not None:
        fire_all |= prompt_cpu == int(eng.carry_token_id)
    fire_all_d = fire_all.to(dev)

    eng.reset()
    eng.prompt_buf[:, :P].copy_(prompt_d)
    eng.tokens[:, :P].copy_(prompt_d)
    Tmax = max(e - s + 1 for s, e in zip([0] + [x + 1 for x in ends[:-1]], ends))
    z = lambda *s, dtype=dt: torch.zeros(*s, dtype=dtype, device=dev)
    # the chunk buffers stay on the engine from one prefill to the next (each
    # is written before it is read; first allocated NaN-filled, so that a read
    # before the first write shows in the results): no allocation and no fill
    # launches ahead of the first chunk
    kept = eng._prefill_buffers

    def buf(name, *shape, dtype=dt):
        t = kept.get(name)
        if t is None or t.shape != torch.Size(shape) or t.dtype != dtype:
            t = kept[name] = torch.full(shape, float("nan"), dtype=dtype, device=dev)
        return t
    M = B * Tmax
    h = buf("h", M, N)
    y = buf("y", M, N)
    qkv = buf("qkv", M, N + 2 * c.KV)
    q = buf("q", M, QH, HD)
    cbuf = buf("cbuf", M, N)
    kctx = buf("kctx", M, N)
    d = buf("d", M, N)
    dh = buf("dh", M, N)
    R = buf("R", M, H)
    gbuf = buf("gbuf", M, H) if c.gate_proj else None
    beta = buf("beta", M, H)
    act = buf("act", M, H)
    hist = buf("hist", M, 2 * L, 2 * N)
    h0 = buf("h0", M, N)                 # token embeddings of a chunk
    carry = buf("carry", 2, M, H, 3, 3)
    pbuf = buf("pbuf", 2, M, H)
    traces = buf("traces", 2, L, B, H)   # phase traces in / out of a chunk (swapped per chunk)
    traces[0].zero_()                    # the first chunk starts from a zero trace
    state = buf("state", B, H, 3, 3)
    state32 = buf("state32", B, H, 3, 3, dtype=torch.float32)
    pooled, z32, a_key = buf("pooled", B, 9), buf("z32", B, 32), buf("a_key", B, N)
    stage_k, stage_v = buf("stage_k", B, N), buf("stage_v", B, N)
    cache_sb = KVH * eng.max_len * HD
    cache_st = HD
    cache_sh = eng.max_len * HD

    def lin(x, w, out, rows, nout, k, **kw):
        eng._linear(x, w, out, rows, nout, k, **kw)

    # LayerNorm(x w^T + x2 w2^T + bias) -> h (y: the product, on the unfused path)
    ln_ws = buf("ln_ws", _lib.load().loom_linear_ln_workspace_bytes(M, N) // 4, dtype=torch.float32)

    descs = {}

    def lin_ln(key, x, w, x2, w2, bias, gamma, beta_ln, rows):
        dsc = descs.get((key, rows))
        if dsc is None:
            dsc = descs[(key, rows)] = _lib.linear_multi_desc(
                x[:rows], [dict(w=w, w2=w2, out=y[:rows], bias=bias)], x2=x2[:rows])
        call("loom_linear_ln", code, _lib.ctypes.byref(dsc), _P(gamma), _P(beta_ln), 1e-5, _P(h), N,
             _P(ln_ws), ln_ws.numel() * 4, None, st)

    # the attention sublayer's read of slots 0..2bi also reads them with the FFN
    # sublayer's query (its part, fp32); the FFN read then folds in slot 2bi+1
    pair = eng.pair_reads
    part_d = buf("part_d", M, QH, HD, dtype=torch.float32) if pair else None
    part_lse = buf("part_lse", M, QH, dtype=torch.float32) if pair else None

    def depth(sub, out, rows):
        if not pair:
            eng.depth_read(sub, hist, out, rows)
        elif sub % 2 == 0:
            eng.depth_read_pair(sub, hist, out, part_d, part_lse, rows)
        else:
            eng.depth_read_fold(sub, hist, out, part_d, part_lse, rows)

    spans = list(zip([0] + [x + 1 for x in ends[:-1]], ends))

    gathered = torch.cuda.Event()
    qkv_ready = torch.cuda.Event()      # a layer's q and cache rows written (aux)
    # batch rows whose attention runs on aux right after the qkv product; the
    # rest run on main after its depth read (the two branches then take about
    # as long)
    aux_rows = min(B, PREFILL_AUX_ROWS)

    def next_qkv(x, bi, sub, s_, Tc_):
        """Block bi's qkv of x with RoPE + cache append (loomformer.py:3262, :3300-3320)
        and, unless sub is None, history slot `sub` (DepthAttn.project, :3397): one
        launch where the shapes allow, on the current stream; the attention then runs
        with qkv = NULL."""
        wh = None if sub is None else _P(eng.kvw)
        ho = None if sub is None else _P(hist[:, sub])
        call("loom_prefill_qkv", code, _P(x), N, _P(eng.blocks[bi]["qkv"]), wh, ho, 2 * L * 2 * N,
             2 * N, _P(qkv), _P(q), _P(eng.k_cache[bi]), _P(eng.v_cache[bi]), cache_sb, cache_st,
             cache_sh, _P(eng.cos), _P(eng.sin), B, Tc_, s_, eng.max_len, N, QH, KVH, HD,
             eng._stream())

    def attend(bi, s_, Tc_, b0=0, b1=B):
        """Block bi's attention for batch rows b0..b1-1 (their cache rows and
        chunk rows are contiguous views), on the current stream."""
        r0 = b0 * Tc_
        call("loom_gqa_prefill", code, None, 0, _P(eng.k_cache[bi][b0:]), _P(eng.v_cache[bi][b0:]),
             cache_sb, cache_st, cache_sh, _P(eng.cos), _P(eng.sin), _P(q[r0:]), _P(cbuf[r0:]),
             _P(kctx[r0:]), N, b1 - b0, Tc_, s_, eng.max_len, QH, KVH, HD, eng._stream())

    def chunk_head(ci):
        """Layer 0's attention inputs of chunk ci, which need only the chunk's
        tokens and the layer-0 K/V rows of earlier chunks: embeddings, qkv with
        RoPE + cache append and history slot 0, attention (on the current stream;
        `gathered` is recorded once history slot 0 is written)."""
        s_, e_ = spans[ci]
        rows_ = B * (e_ - s_ + 1)
        torch.index_select(eng.emb, 0, prompt_d[:, s_:e_ + 1].reshape(-1), out=h0[:rows_])
        next_qkv(h0, 0, 0, s_, e_ - s_ + 1)
        gathered.record()
        attend(0, s_, e_ - s_ + 1)

    main = torch.cuda.current_stream(dev)
    aux = eng.aux_stream
    tail = eng.tail_stream        # a chunk's temporal carry and document key
    tail_st = _lib.c_void_p(tail.cuda_stream)

    def fork():                 # aux continues after everything queued on main so far
        aux.wait_stream(main)

    def join():                 # main continues after everything queued on aux so far
        main.wait_stream(aux)

    have_state = False
    tin = 0
    seed_valid = z(B, dtype=torch.uint8)
    ca_len = 0
    # Three streams, default priority: `aux` runs the work of a layer that does
    # not depend on the depth history (qkv -> attention, W_real) while the main
    # stream runs the history projections and depth reads; they meet before
    # every product that needs both.  Layer 0's attention of the next chunk
    # runs on aux while main finishes the chunk (its last Paraplex + Tria and
    # FFN tail), and `tail` takes the chunk's temporal carry and document key
    # beside the next chunk's first sublayer.
    fork()
    with torch.cuda.stream(aux):
        chunk_head(0)
    for ci, (s, e) in enumerate(spans):
        Tc = e - s + 1
        rows = B * Tc
        hv = hist[:rows]
        sub = 0
        # the depth read of history slot 0, on main once the slot is written
        main.wait_event(gathered)
        depth(0, d, rows)
        carry_i, p_i = None, None
        for bi, blk in enumerate(eng.blocks):
            last = bi == L - 1
            # ---- attention over the cache (rows < s) and this chunk (loomformer.py:3215-3332),
            # on aux after this layer's qkv; the depth read 2*bi on main (layer 0's
            # ran ahead on aux)
            if bi > 0:
                with torch.cuda.stream(aux):
                    attend(bi, s, Tc, 0, aux_rows)
                depth(sub, d, rows)
                if aux_rows < B:
                    # the other rows' attention on main after its depth read,
                    # once aux has written this layer's q and cache rows
                    main.wait_event(qkv_ready)
                    attend(bi, s, Tc, aux_rows, B)
            join()
            # ---- LN(o(C) + w_o(depth read 2*bi)) (loomformer.py:3999-4000)
            lin_ln(("attn", bi), cbuf, blk["o"], d, eng.wo_for(sub), None, blk["ln1_w"], blk["ln1_b"],
                   rows)
            # ---- W_real (+ gate with the previous block's p) and history slot 2*bi+1
            # in one launch of two products of h (one launch's fixed cost fewer than
            # W_real on aux beside the history projection: 62.2-62.5 -> 61.6-61.9 ms),
            # then the slot's depth read
            sub += 1
            key = ("kvr", bi, p_i, rows)
            dsc = descs.get(key)
            if dsc is None:
                real = dict(w=blk["w1r"], out=R[:rows], bias=blk["b1r"])
                if p_i is not None:
                    real.update(gate_p=pbuf[p_i][:rows], gate_alpha=blk["alpha"])
                dsc = descs[key] = _lib.linear_multi_desc(h[:rows], [real, dict(w=eng.kvw, out=hv[:, sub])])
            call("loom_linear_multi", code, _lib.ctypes.byref(dsc), st)
            depth(sub, dh, rows)
            # ---- Paraplex FFN (loomformer.py:2818-2893): beta space, fused pointwise
            # chain with the phase trace carried from the previous chunk; the
            # amplitude source is R, or gate_proj(h) under paraplex_gate_proj (:2849)
            call("loom_beta_forward", code, _P(h), _P(q), _P(kctx), _P(cbuf), _P(dh),
                 _P(blk["w1i"]), _P(beta), None, rows, N, H, c.imag_in, c.Hq, HD, QH,
                 1 if c.sectors == "open" else 0, st)
            gsrc = R
            if c.gate_proj:
                gsrc = gbuf
                lin(h, blk["gpw"], gbuf, rows, H, N, bias=blk["gpb"])
            join()
            if last and ci + 1 < len(spans):
                # the next chunk's layer-0 attention inputs, after this layer's
                # beta space has read q, kctx and c
                fork()
                with torch.cuda.stream(aux):
                    chunk_head(ci + 1)
            # ---- with the block's Tria depth op (loomformer.py:3588-3617), axis bi % 3,
            # in the same pass: the phase I never leaves the chip
            out_i = 0 if carry_i != 0 else 1
            gate = not last
            new_p = (0 if p_i != 0 else 1) if gate else None
            seeded = bi == 0 and have_state
            if seeded:
                main.wait_stream(tail)      # the state after the previous chunk
            if last and carry_i is not None and H % 2 == 0:
                # the last block and the chunk's temporal carry endpoint (loomformer.py:
                # 3834-3850) in one pass: the carry restarts at position 0 and at a
                # seeded first token, else continues from the state; the chunk's
                # last carries are never stored
                reset = z(B, Tc, dtype=torch.uint8)
                if s == 0:
                    reset[:, 0] = 1
                else:
                    reset[:, 0] = seed_valid
                call("loom_paraplex_tria_endpoint_forward", code, _P(R), _P(gsrc), _P(beta),
                     _P(blk["ib"]), _P(traces[tin, bi]), _P(blk["tw"]), float(c.powlu_m),
                     _P(carry[carry_i]), _P(reset), _P(state) if have_state else None, None,
                     _P(act), _P(traces[1 - tin, bi]), _P(state), _P(state32), B, Tc, H,
                     float(c.tria_alpha), bi % 3, st)
                endpoint_done = True
            else:
                call("loom_paraplex_tria_forward", code, _P(R), _P(gsrc), _P(beta), _P(blk["ib"]),
                     _P(traces[tin, bi]), _P(blk["tw"]), float(c.powlu_m),
                     None if (carry_i is None or seeded) else _P(carry[carry_i]),
                     _P(state) if seeded else None, _P(seed_valid) if seeded else None,
                     _P(blk["gate_w"]) if gate else None, _P(act), _P(traces[1 - tin, bi]),
                     _P(carry[out_i]), _P(pbuf[new_p]) if gate else None, B, Tc, H,
                     float(c.tria_alpha), bi % 3, st)
                endpoint_done = False
            carry_i, p_i = out_i, new_p
            if last:
                tail.wait_stream(main)      # the chunk's last carries (or its state) are written
            # ---- LN(w_o(d_h) + W2(act) + b2) (loomformer.py:4045)
            lin_ln(("ffn", bi), dh, eng.wo_for(sub), act, blk["w2"], blk["b2"], blk["ln2_w"],
                   blk["ln2_b"], rows)
            if not last:
                # history slot 2*bi+2 (loomformer.py:4050) on main, the next block's
                # qkv with RoPE + cache append on aux (its attention follows there)
                sub += 1
                fork()
                with torch.cuda.stream(aux):
                    next_qkv(h, bi + 1, None, s, Tc)
                    qkv_ready.record()
                lin(h, eng.kvw, hv[:, sub], rows, 2 * N, N, ldc=2 * L * 2 * N)
        # ---- on the third stream, beside the next chunk's first sublayer: the
        # temporal carry over the chunk, restarting at position 0 and at a
        # seeded first token, else continuing from the state (loomformer.py:3834-3850)
        with torch.cuda.stream(tail):
            if not endpoint_done:
                reset = z(B, Tc, dtype=torch.uint8)
                if s == 0:
                    reset[:, 0] = 1
                else:
                    reset[:, 0] = seed_valid
                call("loom_temporal_carry_endpoint_forward", code, _P(carry[carry_i]), _P(reset),
                     _P(state) if have_state else None, None, _P(state), _P(state32), B, Tc, H,
                     tail_st)
            have_state = True
            fire_e = fire_all_d[:, e]
            if bool(fire_all[:, e].any()):
                # PolARM where the row fired, then the document key of this boundary
                fmask = fire_e.to(torch.uint8)
                call("loom_polarm_forward", code, _P(state), _P(state), _P(fmask), B * H, H,
                     float(c.polarm_beta), 1e-6, tail_st)
                call("loom_slot_attention_pool_forward", code, _P(state), _P(eng.score_w),
                     _P(pooled), None, B, H, tail_st)
                lin(pooled, eng.proj_w, z32, B, 32, 9, bias=eng.proj_b)
                lin(z32, eng.up_w, a_key, B, N, 32, bias=eng.up_b)
                lin(a_key, eng.wqk, stage_k, B, N, N)
                lin(a_key, eng.wv, stage_v, B, N, N)
                if ca_len >= eng.max_keys:
                    raise ValueError("final-CA key cache is full")
                eng.ca_k[:, ca_len].copy_(stage_k)
                eng.ca_v[:, ca_len].copy_(stage_v)
                eng.ca_valid[:, ca_len].copy_(fmask)
                ca_len += 1
                seed_valid.copy_(fmask)
            else:
                seed_valid.zero_()
        tin = 1 - tin
    main.wait_stream(tail)
    # ---- final cross-attention and head of the last prompt token (tria.py:1560-1595)
    Tc = ends[-1] - (ends[-2] + 1 if len(ends) > 1 else 0) + 1
    h_last = h[:B * Tc].view(B, Tc, N)[:, Tc - 1].contiguous()
    eng.h.copy_(h_last)
    lin(eng.h, eng.wqk, eng.q_ca, B, N, N)
    eng.ca_len.fill_(ca_len)
    call("loom_final_ca_sparse_strided", code, _P(eng.q_ca), _P(eng.ca_k), _P(eng.ca_v),
         eng.max_keys * N, _P(eng.ca_valid), eng.max_keys, _P(eng.h), float(eng.gamma),
         _P(eng.h2), None, B, 1, eng.max_keys, _P(eng.ca_len), N, float(N ** -0.5), st)
    eng.head_logits(eng.h2, eng.logits, B)
    # ---- the engine's decode state after position P-1
    eng.trace.copy_(traces[tin])
    eng.doc.copy_(state)
    eng.pending.copy_(fire_all_d[:, P - 1].to(torch.uint8))
    eng.pos_dev.fill_(P)
    eng.ids.copy_(prompt_d[:, P - 1])
    eng.pos = P
    eng._prompt_len = P
