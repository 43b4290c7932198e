#!/usr/bin/env python3
"""Benchmark of the LoomFormer fused-kernel inference path on one MI355X.

Headline (``value``): end-to-end greedy decode tokens/s of the 113M-shape
LoomFormer (cfg/nano_chk.yaml shape, seq_len raised to 4096, random-init
weights from seed 2, bf16) at batch 32: a 2048-token prompt of uniform ids is
prefilled by the chunked forward (one chunk of the stack per fire window,
timed separately as ``prefill_tokens_per_s``), then ``--steps`` greedy decode
steps are timed (one step = one token for all 32 sequences) after
``--warmup`` untimed greedy steps.

Microbenchmarks, each timed live with HIP events on
the stream the kernels run on:
  PX  Paraplex FFN, 8192 tokens as [8, 1024], N=768, H=3072, bf16
  DA  DepthAttn, 16384 tokens, 24 earlier-depth states, 8x96, bf16
  TR  Tria, B=8 x T=4096 x H=3072, 24 layers, fp32: the gated depth step
      alone, and the whole chunked path (depth composition, temporal carry
      every 64 tokens with PolARM at fires) plus the readout to d_model=768
``roofline`` reports the fused Paraplex pointwise kernel (the path's fused
HBM-bound kernel): algorithmic bytes (R, beta in; I, O out = 8 B/elem in
bf16) per launch over its mean launch time, against 8 TB/s.

``cpu_baseline`` is the CPU oracle (fp32 PyTorch restatement of the
reference's unfused path) running the e2e decode step on all host cores on a
bounded sample (B=32 from position 2048 on a synthetic state of that size);
``cpu_reference_config`` times BASELINE.json's CPU-reference config (nano.yaml,
B=1, 128 + 64 tokens, fp32) on the host cores and on the fp32 GPU engine;
``cpu_micro`` times the oracle on PX and DA at full size and on a slice of TR
scaled to its full size.  CPU figures are 1 warm-up plus the median of 3.

Prints ONE JSON line.  One GPU only: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "loomformer-paraplex_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode tokens/s (113M shape, bs32) + fused-kernel HBM GB/s as % of peak"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def timed(fn, iters: int, warmup: int = 3) -> float:
    """Mean milliseconds per call of fn over `iters` calls.

    The calls are captured into one HIP graph and the graph replay is bracketed
    by HIP events on the stream it runs on, so host-side op overhead (output
    allocation, the ctypes call) cannot starve the GPU between launches and
    the figure is device time (plus the graph's own node-to-node gaps).
    """
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(iters):
            fn()
    g.replay()                      # first replay uploads the graph
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    g.replay()
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / iters
    del g
    torch.cuda.empty_cache()
    return ms


# ----------------------------------------------------------------------------- e2e

def bench_decode(args):
    import torch
    from loom_amd.config import NANO_CHK, ModelConfig
    from loom_amd.engine import LoomDecoder
    from loom_amd.weights import init_state_dict

    cfg = ModelConfig.from_dict(NANO_CHK).with_seq_len(4096)
    B, P, K, W = args.batch, args.prompt, args.steps, args.warmup
    state = init_state_dict(cfg, 2)
    eng = LoomDecoder(cfg, state, batch=B, dtype=torch.bfloat16, max_len=P + W + K + 1)
    g = torch.Generator().manual_seed(2)
    prompt = torch.randint(0, cfg.V, (B, P), generator=g).to("cuda")
    log(f"chunked prefill of {P} tokens x B={B} (one chunk per {cfg.window}-token fire window)")
    eng.prefill(prompt)                                # warm-up (allocations, code objects)
    torch.cuda.synchronize()
    t_runs = []
    for _ in range(3):                                 # the median of three timed prefills
        t0 = time.perf_counter()
        eng.prefill(prompt)
        torch.cuda.synchronize()
        t_runs.append(time.perf_counter() - t0)
    t_prefill = sorted(t_runs)[1]
    eng.warm_graphs()                                  # capture every graph replay_steps uses
    eng.replay_steps(W)                                # warm-up greedy steps
    torch.cuda.synchronize()
    log(f"prefill {t_prefill * 1e3:.1f} ms ({B * P / t_prefill:.0f} tokens/s); timing {K} greedy steps")
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    s.record()
    eng.replay_steps(K)                                # K greedy decode steps
    e.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = s.elapsed_time(e)
    out = eng.generated()
    return dict(ms_total=ms, ms_per_step=ms / K, tokens_per_s=B * K / (ms / 1e3),
                wall_s=wall, prefill_s=t_prefill, prefill_tokens_per_s=B * P / t_prefill,
                ids_head=out[0, :8].tolist())


# ----------------------------------------------------------------------------- micro

def bench_px(iters):
    import torch
    from loom_amd import ops

    dev, bf = "cuda", torch.bfloat16
    B, T, N, QH, HD, H = 8, 1024, 768, 8, 96, 3072
    M, K_imag = B * T, N + 4 * HD
    torch.manual_seed(1)
    mk = lambda o, i: torch.nn.Linear(i, o, bias=True)  # Kaiming-uniform (nn.Linear default), seed 1
    w_real = mk(H, N).weight.data.to(dev, bf)
    w_imag = torch.nn.init.kaiming_uniform_(torch.empty(H, K_imag), a=math.sqrt(5)).to(dev, bf)
    w2 = mk(N, H).weight.data.to(dev, bf)
    g = torch.Generator(device=dev).manual_seed(1)
    rn = lambda *s: torch.randn(*s, generator=g, device=dev).to(bf)
    u = rn(B, T, N)
    q, kc, c, d = (rn(B, T, QH, HD) for _ in range(4))
    b_real = torch.zeros(H, device=dev)
    b2 = torch.zeros(N, device=dev)
    imag_bias = torch.zeros(H, device=dev)
    trace_w = (torch.rand(H, generator=g, device=dev) - 0.5)
    trace = torch.zeros(B, H, device=dev, dtype=bf)
    anchor = torch.ones((), device=dev)
    empty_reset = torch.empty(0, dtype=torch.bool, device=dev)
    R = ops.linear(u, w_real, b_real)
    beta = ops.beta_forward_cuda(u, q, kc, c, d, w_imag, H // QH, HD, QH, False)[0]
    act = ops.paraplex_forward(R, R, beta, imag_bias, trace, trace_w, empty_reset, anchor, 1, False,
                               0.99, 3.0)[0]
    res = {}
    res["w_real_ms"] = timed(lambda: ops.linear(u, w_real, b_real, out=R), iters)
    res["w_imag_ms"] = timed(lambda: ops.beta_forward_cuda(u, q, kc, c, d, w_imag, H // QH, HD, QH, False), iters)
    # the pointwise chain on one set of R / beta / I / O (201 MB, inside the 256 MB
    # Infinity Cache: the cache-warm figure) and rotating over three sets (604 MB:
    # every launch streams its operands from HBM, the figure the roofline uses)
    res["pointwise_warm_ms"] = timed(lambda: ops.paraplex_forward(R, R, beta, imag_bias, trace, trace_w,
                                                                   empty_reset, anchor, 1, False, 0.99, 3.0), iters)
    from loom_amd import _lib
    sets = [(R, beta)] + [(R.clone(), beta.clone()) for _ in range(2)]
    outs = [(torch.empty_like(R), torch.empty_like(R)) for _ in sets]
    nt = torch.empty(B, H, device=dev, dtype=bf)
    snap = torch.empty((), device=dev)
    rot = [0]

    def pointwise_rotated():
        k = rot[0] % len(sets)
        rot[0] += 1
        (r_, b_), (a_, s_) = sets[k], outs[k]
        _lib.call("loom_paraplex_forward", 1, _lib.ptr(r_), _lib.ptr(r_), _lib.ptr(b_), _lib.ptr(imag_bias),
                  _lib.ptr(trace), _lib.ptr(trace_w), None, _lib.ptr(anchor), _lib.ptr(a_), _lib.ptr(s_),
                  _lib.ptr(nt), _lib.ptr(snap), B, T, H, 3.0, _lib.stream_of(r_))
    res["pointwise_ms"] = timed(pointwise_rotated, max(iters, 3 * 8))
    del sets, outs
    out = torch.empty(B, T, N, device=dev, dtype=bf)
    res["w2_ms"] = timed(lambda: ops.linear(act, w2, b2, out=out), iters)

    def ffn():
        R_ = ops.linear(u, w_real, b_real)
        be = ops.beta_forward_cuda(u, q, kc, c, d, w_imag, H // QH, HD, QH, False)[0]
        a_ = ops.paraplex_forward(R_, R_, be, imag_bias, trace, trace_w, empty_reset, anchor, 1,
                                  False, 0.99, 3.0)[0]
        return ops.linear(a_, w2, b2)
    res["ffn_ms"] = timed(ffn, iters)
    elems = M * H
    res["pointwise_bytes"] = elems * 8            # R, beta in; I, O out (bf16)
    res["pointwise_GBs"] = res["pointwise_bytes"] / (res["pointwise_ms"] * 1e-3) / 1e9
    res["pointwise_warm_GBs"] = res["pointwise_bytes"] / (res["pointwise_warm_ms"] * 1e-3) / 1e9
    fl = {"w_real": 2 * M * N * H, "w_imag": 2 * M * K_imag * H, "w2": 2 * M * H * N}
    for k, v in fl.items():
        res[f"{k}_TFLOPs"] = v / (res[f"{k}_ms"] * 1e-3) / 1e12
    res["gemm_gflop"] = sum(fl.values()) / 1e9
    return res


def bench_da(iters):
    import torch
    from loom_amd import ops

    dev, bf = "cuda", torch.bfloat16
    BT, S, QH, HD = 16384, 24, 8, 96
    g = torch.Generator(device=dev).manual_seed(3)
    K = torch.randn(1, BT, S, QH, HD, generator=g, device=dev).to(bf)
    V = torch.randn(1, BT, S, QH, HD, generator=g, device=dev).to(bf)
    q = (torch.randn(QH, HD, generator=g, device=dev) * 0.02).to(bf)
    ms = timed(lambda: ops.depth_attn_stacked_forward(q, K, V), iters)
    nbytes = 2 * K.numel() * 2 + BT * QH * HD * 2 + BT * QH * 4
    return dict(ms=ms, bytes=nbytes, GBs=nbytes / (ms * 1e-3) / 1e9)


def bench_tr(iters):
    import torch
    from loom_amd import ops

    dev = "cuda"
    B, T, H = 8, 4096, 3072
    g = torch.Generator(device=dev).manual_seed(4)
    r, i, o = (torch.randn(B, T, H, generator=g, device=dev) for _ in range(3))
    prev = torch.randn(B, T, H, 3, 3, generator=g, device=dev)
    prev /= prev.square().mean(dim=(-1, -2), keepdim=True).add(1e-6).sqrt()
    w = torch.full((9,), 1.0 / 9.0, device=dev)
    # the reference API (carry, p and the backward-only scale: 92 B per element)
    ms92 = timed(lambda: ops.tria_step_gate_forward(r, i, o, prev, w, 0.025, 1), iters)
    # the inference form tria_step_and_gate uses (no scale output): 88 B per element
    from loom_amd import _lib
    carry = torch.empty(B, T, H, 3, 3, device=dev)
    p = torch.empty(B, T, H, device=dev)
    P = _lib.ptr
    ms = timed(lambda: _lib.call("loom_tria_depth_forward", 0, P(r), P(i), P(o), P(prev), None, None,
                                 P(w), P(carry), P(p), None, B, T, H, 0.025, 1, _lib.stream_of(r)),
               iters)
    n = B * T * H
    nbytes = n * (12 + 36 + 36 + 4)               # r,i,o; C_prev; C; p (fp32)
    del prev, carry, p
    depth = torch.randn(B, 64, H, 3, 3, generator=g, device=dev)
    reset = torch.zeros(B, 64, dtype=torch.bool, device=dev)
    empty = torch.empty(0, device=dev)
    ms_end = timed(lambda: ops.temporal_carry_endpoint_forward(depth, reset, empty,
                                                               torch.empty(0, dtype=torch.bool, device=dev)), iters)
    end_bytes = depth.numel() * 4 + B * H * 9 * 8
    return dict(step_gate_ms=ms, step_gate_bytes=nbytes, step_gate_GBs=nbytes / (ms * 1e-3) / 1e9,
                step_gate_with_scale_ms=ms92,
                step_gate_with_scale_GBs=n * 92 / (ms92 * 1e-3) / 1e9,
                endpoint_w64_ms=ms_end, endpoint_w64_GBs=end_bytes / (ms_end * 1e-3) / 1e9)


def bench_tr_pipeline(iters):
    """The whole TR microbench path: B=8 x T=4096 tokens, 24 layers, H=3072,
    fp32, fires every 64 tokens (63 boundaries), PolARM beta 0.1, then the
    readout of the 63 document keys to d_model=768."""
    import torch
    from loom_amd import ops

    dev = "cuda"
    L, B, T, H, W, N = 24, 8, 4096, 3072, 64, 768
    g = torch.Generator(device=dev).manual_seed(5)
    r, i, o = (torch.randn(L, B, T, H, generator=g, device=dev) for _ in range(3))
    key_w = torch.randn(32, 9, generator=g, device=dev) * 1.5
    query = torch.randn(32, generator=g, device=dev)
    raw = key_w.t() @ query
    score_w = raw / raw.norm().clamp_min(1e-6)
    pw, pb = torch.randn(32, 9, generator=g, device=dev) / 3, torch.zeros(32, device=dev)
    uw, ub = torch.randn(N, 32, generator=g, device=dev) / 6, torch.zeros(N, device=dev)
    out = {}

    def chunked():
        out["keys"] = ops.tria_chunked_forward(r, i, o, 0.025, W, 0.1)[0]

    ms = timed(chunked, iters)
    keys = out["keys"]
    ms_read = timed(lambda: ops.tria_readout(keys, score_w, pw, pb, uw, ub), iters)
    K = keys.shape[1]
    nbytes = 3 * L * B * T * H * 4 + B * K * H * 36
    del r, i, o
    return dict(ms=ms, bytes=nbytes, GBs=nbytes / (ms * 1e-3) / 1e9, readout_ms=ms_read,
                keys=K)


def bench_gqa(iters):
    """The decode step's attention: B=32, 8 q heads over 2 kv heads of 96, a
    head-major bf16 cache at 2176 positions (the middle of the timed decode),
    RoPE + append + attention in one launch and the chunk merge in a second."""
    import torch
    from loom_amd import _lib

    dev, bf = "cuda", torch.bfloat16
    B, QH, KVH, HD, L, cap = 32, 8, 2, 96, 2176, 2305
    g = torch.Generator(device=dev).manual_seed(6)
    qkv = torch.randn(B, (QH + 2 * KVH) * HD, generator=g, device=dev).to(bf)
    kc = torch.randn(B, KVH, cap, HD, generator=g, device=dev).to(bf)
    vc = torch.randn(B, KVH, cap, HD, generator=g, device=dev).to(bf)
    from loom_amd.weights import rope_tables
    from loom_amd.config import NANO_CHK, ModelConfig
    cos, sin = (t.to(dev) for t in rope_tables(ModelConfig.from_dict(NANO_CHK).with_seq_len(4096), cap))
    out = torch.empty(3, B, QH * HD, device=dev, dtype=bf)
    nb = _lib.load().loom_gqa_workspace_bytes(B, cap, QH, KVH, HD)
    ws = torch.zeros(nb // 4 + 1, device=dev)
    P = _lib.ptr

    def fn():   # on the current stream (the capture stream inside timed())
        _lib.call("loom_gqa_decode_step", 1, P(qkv), P(kc), P(vc), KVH * cap * HD, HD, cap * HD,
                  P(cos), P(sin), P(out[0]), P(out[1]), P(out[2]), QH * HD, P(ws), nb, B, L, None,
                  QH, KVH, HD, _lib.stream_of(qkv))
    ms = timed(fn, iters)
    nbytes = 2 * B * KVH * L * HD * 2
    return dict(ms=ms, bytes=nbytes, GBs=nbytes / (ms * 1e-3) / 1e9)


def bench_decode_gemm(iters):
    """The decode step's largest kernel class, a weight-streaming projection at
    M = 32: history K/V (kv_weight [1536, 768]) and W_real ([3072, 768] + bias)
    of one hidden state in one launch, as the engine issues it.  Weights rotate
    over 24 sets (170 MB) so consecutive launches do not find them in cache."""
    import torch
    from loom_amd import _lib

    dev, bf = "cuda", torch.bfloat16
    B, N, H, NS = 32, 768, 3072, 24
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(B, N, generator=g, device=dev).to(bf)
    kvw = [(torch.randn(2 * N, N, generator=g, device=dev) * 0.03).to(bf) for _ in range(NS)]
    w1r = [(torch.randn(H, N, generator=g, device=dev) * 0.03).to(bf) for _ in range(NS)]
    b1r = torch.zeros(H, device=dev)
    o_kv = torch.empty(B, 2 * N, device=dev, dtype=bf)
    o_r = torch.empty(B, H, device=dev, dtype=bf)
    descs = [_lib.linear_multi_desc(x, [dict(w=kvw[i], out=o_kv), dict(w=w1r[i], out=o_r, bias=b1r)])
             for i in range(NS)]
    it = [0]

    def fn():
        d = descs[it[0] % NS]
        it[0] += 1
        _lib.call("loom_linear_multi", 1, _lib.ctypes.byref(d), _lib.stream_of(x))
    ms = timed(fn, max(iters, NS))
    nbytes = (2 * N + H) * N * 2 + B * N * 2 + B * (2 * N + H) * 2
    return dict(ms=ms, bytes=nbytes, GBs=nbytes / (ms * 1e-3) / 1e9)


def copy_bandwidth():
    import torch
    x = torch.empty(1 << 28, dtype=torch.float32, device="cuda")   # 1 GiB
    y = torch.empty_like(x)
    ms = timed(lambda: y.copy_(x), 10)
    return 2 * x.numel() * 4 / (ms * 1e-3) / 1e9


def measured_traffic():
    """HBM bytes per launch of the fused kernels, from the rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes summarised in profiles/ (FETCH scaled by the copy-kernel
    factor, see the profile texts); empty if the file is absent."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return {k: v["hbm_bytes_per_launch"] for k, v in json.load(f).items()}


# ----------------------------------------------------------------------------- cpu

def _host_cores() -> int:
    return len(os.sched_getaffinity(0))


def _synthetic_state(model, B: int, ctx: int, big):
    """A decode state of the oracle at position `ctx`: KV caches of `ctx`
    positions, phase traces, a Tria document state and ctx // W final-CA keys,
    holding the seeded values of `big` (reused between timed runs; a step only
    appends rows past `ctx`).  The per-step cost of the fp32 step depends on
    the context only through these shapes."""
    import torch
    from oracle.model import CACache, LayerCache, StepState, TemporalState
    S = model.S
    caches = [LayerCache(k=big["k"][l], v=big["v"][l], phase_trace=big["trace"][l].clone(),
                         cache_len=ctx) for l in range(S.L)]
    ca = CACache(k=big["ca_k"], v=big["ca_v"], valid=torch.ones(B, big["ca_k"].shape[1], dtype=torch.bool),
                 cache_len=ctx // S.window)
    temporal = TemporalState(carry=big["doc"].clone(), pending=torch.zeros(B, dtype=torch.bool))
    return StepState(caches=caches, ca=ca, temporal=temporal)


def _synthetic_tensors(S, B: int, cap: int, seed: int):
    """Seeded cache contents for `cap` positions (the timed steps append below cap)."""
    import torch
    from oracle import ops as ref
    g = torch.Generator().manual_seed(seed)
    rn = lambda *shape: torch.randn(*shape, generator=g)
    return {"k": [rn(B, cap, S.KVH, S.HD) for _ in range(S.L)],
            "v": [rn(B, cap, S.KVH, S.HD) for _ in range(S.L)],
            "trace": [rn(B, S.H).tanh() for _ in range(S.L)],
            "ca_k": rn(B, cap // S.window + 2, S.N), "ca_v": rn(B, cap // S.window + 2, S.N),
            "doc": ref.local_normalize(rn(B, S.H, 3, 3))}


def cpu_baseline(args):
    """The e2e workload's decode step on the host cores: the fp32 oracle
    Model.step at B = 32 from position 2048 (the GPU's decode starts there),
    on a synthetic decode state of that size; 1 warm-up step, then the median
    of 3 timed runs of `cpu_steps` greedy steps."""
    import torch
    from oracle.model import OracleModel, Shapes  # the checker, timed as baseline
    from loom_amd.config import NANO_CHK

    cores = _host_cores()
    torch.set_num_threads(cores)
    S = Shapes.from_dict(dict(NANO_CHK, seq_len=4096))
    torch.manual_seed(2)
    model = OracleModel(S).eval()
    B, ctx, K = args.batch, args.prompt, args.cpu_steps
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, S.V, (B,), generator=g)
    times = []
    big = _synthetic_tensors(S, B, ctx + K + 1, 5)
    with torch.no_grad():
        for rep in range(4):                         # run 0 is the warm-up
            state = _synthetic_state(model, B, ctx, big)
            nxt = ids
            t0 = time.perf_counter()
            for i in range(K if rep else 1):
                logits, state = model.step(nxt, ctx + i, state)
                nxt = torch.argmax(logits, dim=-1)
            if rep:
                times.append(time.perf_counter() - t0)
    dt = sorted(times)[1]
    return dict(value=B * K / dt, unit="tokens/s", cores=cores, kind="port", cpu=_cpu_model(),
                sample=f"fp32 oracle Model.step (the reference's unfused path restated), nano_chk shape "
                       f"seed 2, B={B}, {K} greedy steps from position {ctx} on a synthetic decode "
                       f"state of that size; 1 warm-up step, median of 3 runs")


def cpu_reference_config(args):
    """BASELINE.json's CPU-reference config: cfg/nano.yaml weights from seed 0,
    fp32, B = 1, a 128-token prompt (ids from a generator seeded 0), 128
    prefill steps and 64 greedy steps (Model.step each, as infer runs them).
    Timed with the fp32 oracle on the host cores (1 warm-up, median of 3)
    and with the fp32 GPU engine (token-by-token prefill through the
    captured step); the greedy ids of the two are compared."""
    import torch
    from oracle.model import OracleModel, Shapes  # the checker, timed as baseline
    from loom_amd.config import NANO, ModelConfig
    from loom_amd.engine import LoomDecoder
    from loom_amd.weights import init_state_dict

    cores = _host_cores()
    torch.set_num_threads(cores)
    P, K = 128, 64
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, NANO["vocab"], (1, P), generator=g)
    torch.manual_seed(0)
    model = OracleModel(Shapes.from_dict(NANO)).eval()

    def cpu_run():
        state, logits, out = None, None, []
        t0 = time.perf_counter()
        with torch.no_grad():
            for pos in range(P):
                logits, state = model.step(prompt[:, pos], pos, state)
            t1 = time.perf_counter()
            for i in range(K):
                nxt = torch.argmax(logits, dim=-1)
                out.append(nxt)
                logits, state = model.step(nxt, P + i, state)
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1, torch.stack(out, 1)
    runs = [cpu_run() for _ in range(4)][1:]
    pre_s = sorted(r[0] for r in runs)[1]
    dec_s = sorted(r[1] for r in runs)[1]
    ids_cpu = runs[0][2]

    cfg = ModelConfig.from_dict(NANO)
    eng = LoomDecoder(cfg, init_state_dict(cfg, 0), batch=1, dtype=torch.float32, max_len=P + K + 1)
    gpu = []
    for rep in range(4):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.start(prompt)
        eng.replay_steps(P - 1)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        eng.replay_steps(K)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        if rep == 0:
            eng.warm_graphs()
        else:
            gpu.append((t1 - t0, t2 - t1))
    gpre = sorted(x[0] for x in gpu)[1]
    gdec = sorted(x[1] for x in gpu)[1]
    ids_gpu = eng.generated()[:, :K].cpu()
    return {"config": "cfg/nano.yaml seed 0, fp32, B=1, 128-token prompt + 64 greedy tokens",
            "cpu": {"prefill_tokens_per_s": P / pre_s, "decode_tokens_per_s": K / dec_s,
                    "cores": cores, "kind": "port", "cpu": _cpu_model()},
            "gpu_fp32": {"prefill_tokens_per_s": P / gpre, "decode_tokens_per_s": K / gdec,
                         "note": "token-by-token prefill through the captured step, host wall clock"},
            "greedy_ids_equal": bool(torch.equal(ids_cpu, ids_gpu))}


def _cpu_model() -> str:
    """The host CPU's model string (lscpu's, which names the part where
    /proc/cpuinfo may give only the family)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_wall(fn, reps: int = 3) -> float:
    fn()                                                   # warm-up
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def cpu_micro():
    """The microbenchmark configs on the host cores with the CPU oracle (the
    reference's unfused fp32 path restated): PX and DA at full size, TR on a
    slice of the streams (B=1, H=64 of 8 x 3072), scaled to the full size by the
    stream count (the streams are independent).  1 warm-up, median of 3."""
    import torch
    from oracle import ops as ref  # the checker, timed as baseline

    cores = _host_cores()
    torch.set_num_threads(cores)
    out = {"cores": cores, "cpu": _cpu_model(), "kind": "port"}
    with torch.no_grad():
        B, T, N, QH, HD, H = 8, 1024, 768, 8, 96, 3072
        g = torch.Generator().manual_seed(1)
        u = torch.randn(B, T, N, generator=g)
        q, kc, c, d = (torch.randn(B, T, QH, HD, generator=g) for _ in range(4))
        w_real = torch.randn(H, N, generator=g) / math.sqrt(N)
        w_imag = torch.randn(H, N + 4 * HD, generator=g) / math.sqrt(N + 4 * HD)
        w2 = torch.randn(N, H, generator=g) / math.sqrt(H)
        trace_w = torch.rand(H, generator=g) - 0.5
        zH = torch.zeros(H)

        def px():
            R = torch.nn.functional.linear(u, w_real)
            beta = ref.beta_space_grouped(u, q, kc, c, d, w_imag, QH, HD)
            act = ref.paraplex_pointwise(R, R, beta, zH, None, trace_w, None, 3.0)[0]
            return torch.nn.functional.linear(act, w2)
        out["px_ms"] = _median_wall(px) * 1e3
        del u, q, kc, c, d
        BT, S = 16384, 24
        g = torch.Generator().manual_seed(3)
        K = torch.randn(1, BT, S, QH, HD, generator=g).to(torch.bfloat16).float()
        V = torch.randn(1, BT, S, QH, HD, generator=g).to(torch.bfloat16).float()
        qd = torch.randn(QH, HD, generator=g) * 0.02
        out["da_ms"] = _median_wall(lambda: ref.depth_attn_softmax(qd, K, V)) * 1e3
        del K, V
        L, Bs, Ts, Hs, W = 24, 1, 4096, 64, 64
        g = torch.Generator().manual_seed(5)
        r, i, o = (torch.randn(L, Bs, Ts, Hs, generator=g) for _ in range(3))
        slice_s = _median_wall(lambda: ref.tria_chunked(r, i, o, 0.025, W, 0.1))
        scale = (8 * 3072) / (Bs * Hs)
        out["tr_ms"] = slice_s * 1e3 * scale
        out["tr_sample"] = (f"chunked Tria path on B=1 x H=64 streams of T=4096, 24 layers, W=64 "
                            f"({slice_s * 1e3:.0f} ms), scaled x{scale:.0f} to B=8 x H=3072")
    return out


# ----------------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--micro-iters", type=int, default=20)
    ap.add_argument("--no-micro", action="store_true")
    ap.add_argument("--no-e2e", action="store_true",
                    help="microbenchmarks only (for counter passes); value is then null")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-steps", type=int, default=4,
                    help="greedy steps per timed CPU run of the e2e decode sample")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(run with --gpus 1).", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a HIP device")
    from loom_amd import _lib
    _lib.load()

    if args.no_e2e:
        dec = dict(tokens_per_s=None, ms_per_step=None, prefill_tokens_per_s=None)
    else:
        dec = bench_decode(args)
        log(f"decode: {dec['tokens_per_s']:.0f} tok/s, {dec['ms_per_step']:.3f} ms/step")
    kernels = {}
    roofline = None
    if not args.no_micro:
        px = bench_px(args.micro_iters)
        log(f"PX: {json.dumps({k: round(v, 3) for k, v in px.items()})}")
        da = bench_da(args.micro_iters)
        log(f"DA: {json.dumps({k: round(v, 3) for k, v in da.items()})}")
        tr = bench_tr(max(3, args.micro_iters // 4))
        log(f"TR: {json.dumps({k: round(v, 3) for k, v in tr.items()})}")
        trp = bench_tr_pipeline(max(3, args.micro_iters // 4))
        log(f"TR pipeline: {json.dumps({k: round(v, 3) for k, v in trp.items()})}")
        gq = bench_gqa(args.micro_iters)
        log(f"GQA decode: {json.dumps({k: round(v, 3) for k, v in gq.items()})}")
        dg = bench_decode_gemm(args.micro_iters)
        log(f"decode GEMM: {json.dumps({k: round(v, 3) for k, v in dg.items()})}")
        copy_gbs = copy_bandwidth()
        kernels = {
            "paraplex_pointwise": {"ms": px["pointwise_ms"], "GB/s": px["pointwise_GBs"],
                                   "frac": px["pointwise_GBs"] / HBM_PEAK_GBS,
                                   "note": "rotating over 3 operand sets (604 MB, beyond the 256 MB "
                                           "Infinity Cache)",
                                   "cache_warm_ms": px["pointwise_warm_ms"],
                                   "cache_warm_GB/s": px["pointwise_warm_GBs"]},
            "depth_attn": {"ms": da["ms"], "GB/s": da["GBs"], "frac": da["GBs"] / HBM_PEAK_GBS},
            "tria_step_gate": {"ms": tr["step_gate_ms"], "GB/s": tr["step_gate_GBs"],
                               "frac": tr["step_gate_GBs"] / HBM_PEAK_GBS,
                               "basis": "88 B per element (r,i,o; C_prev; C; p), the inference form "
                                        "without the backward-only scale",
                               "with_scale_ms": tr["step_gate_with_scale_ms"],
                               "with_scale_GB/s_92B": tr["step_gate_with_scale_GBs"]},
            "temporal_endpoint_w64": {"ms": tr["endpoint_w64_ms"], "GB/s": tr["endpoint_w64_GBs"]},
            "tria_chunked_tr": {"ms": trp["ms"], "GB/s": trp["GBs"], "frac": trp["GBs"] / HBM_PEAK_GBS,
                                "algorithmic_bytes": trp["bytes"], "readout_ms": trp["readout_ms"]},
            "w_real_gemm": {"ms": px["w_real_ms"], "TFLOP/s": px["w_real_TFLOPs"],
                            "frac": px["w_real_TFLOPs"] / BF16_PEAK_TFLOPS},
            "w_imag_gemm": {"ms": px["w_imag_ms"], "TFLOP/s": px["w_imag_TFLOPs"],
                            "frac": px["w_imag_TFLOPs"] / BF16_PEAK_TFLOPS},
            "w2_gemm": {"ms": px["w2_ms"], "TFLOP/s": px["w2_TFLOPs"],
                        "frac": px["w2_TFLOPs"] / BF16_PEAK_TFLOPS},
            "gqa_decode_ctx2176": {"ms": gq["ms"], "GB/s": gq["GBs"], "frac": gq["GBs"] / HBM_PEAK_GBS,
                                   "algorithmic_bytes": gq["bytes"]},
            "decode_gemm_kv_wreal_m32": {"ms": dg["ms"], "GB/s": dg["GBs"], "frac": dg["GBs"] / HBM_PEAK_GBS,
                                         "algorithmic_bytes": dg["bytes"]},
            "paraplex_ffn_total_ms": px["ffn_ms"],
            "device_copy_GB/s": copy_gbs,
        }
        traffic = measured_traffic()
        for key, name in (("paraplex_chunk_kernel_px", "paraplex_pointwise"),
                          ("depth_attn_kernel_da", "depth_attn"),
                          ("tria_depth_kernel_step_gate_tr", "tria_step_gate")):
            kernels[name]["hbm_traffic_bytes"] = traffic.get(key)
        roofline = {"bound": "hbm", "kernel": "paraplex_chunk_kernel (PX: 8x1024x3072 bf16)",
                    "achieved": px["pointwise_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": px["pointwise_GBs"] / HBM_PEAK_GBS,
                    "traffic": traffic.get("paraplex_chunk_kernel_px"),
                    "traffic_source": "profiles/hbm_traffic.json (rocprofv3 FETCH_SIZE and WRITE_SIZE "
                                      "passes, committed; not measured in this run)",
                    "algorithmic_bytes": px["pointwise_bytes"],
                    "timing": "HIP events over a replayed graph of launches rotating over 3 operand sets",
                    "cache_warm_GB/s": px["pointwise_warm_GBs"]}
    cpu = None
    cpu_mi = None
    cpu_ref = None
    if not args.no_cpu:
        log("CPU baseline (oracle on host cores)")
        cpu = cpu_baseline(args)
        log(f"CPU: {cpu['value']:.2f} tok/s on {cpu['cores']} cores")
        log("CPU-reference config (nano.yaml, B=1, fp32) on host cores and on the GPU engine")
        cpu_ref = cpu_reference_config(args)
        log(f"CPU-reference config: {json.dumps(cpu_ref)}")
        if not args.no_micro:
            log("CPU microbenchmarks (oracle on host cores)")
            cpu_mi = cpu_micro()
            log(f"CPU micro: {json.dumps(cpu_mi)}")
    line = {
        "metric": METRIC, "value": dec["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": dec["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (uniform prompt ids, random-init weights from seed 2)",
        "config": {"workload": f"e2e greedy decode, nano_chk shape (seq_len 4096), batch {args.batch}, "
                               f"{args.prompt}-token prompt prefilled by the chunked forward, "
                               f"{args.warmup} untimed then {args.steps} timed greedy steps",
                   "batch": args.batch, "prompt": args.prompt, "decode_steps": args.steps},
        "roofline": roofline, "cpu_baseline": cpu, "kernels": kernels, "cpu_micro": cpu_mi,
        "cpu_reference_config": cpu_ref,
        "prefill_tokens_per_s": dec["prefill_tokens_per_s"],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
