"""Batched greedy decode of LoomFormer on the gfx950 kernels.

``LoomDecoder.step`` is ``Model.step`` (loomformer.py:3951-4091) for a batch
of sequences that share one position counter, and ``generate`` is ``infer``
(loomformer.py:5290-5311): token-by-token prefill through ``step``, then
greedy argmax.  Every matrix product, attention, LayerNorm, the fused Paraplex
chain, depth attention and all Tria ops run in libloom_hip.so on persistent
buffers; torch provides the device memory, the embedding row gather and the
argmax.  Activations and weight matrices are in ``dtype`` (bf16 or fp32);
biases, LayerNorm parameters and the rotary tables stay fp32.

The per-step state that changes with the position (position, KV length,
final-CA key count, fire / reset / pending flags, the token ids) lives on the
device, so one step is a fixed sequence of launches.  ``generate`` captures
that sequence once in a HIP graph (``torch.cuda.CUDAGraph``) and replays it
for every position after the first: the host issues one graph launch per
token instead of ~300 kernel launches.

Layouts (all device-resident, allocated once):
  k_cache/v_cache [L, B, max_len, KVH, HD]    KV cache (preallocated, no wrap)
  hist            [B, 2L, 2N]                 depth history, row s = [k_s | v_s]
  trace           [L, B, H]                   previous-token phase per layer
  doc             [B, H, 3, 3]                temporal carry (updated in place)
  ca_k/ca_v       [B, max_keys, N], ca_valid [B, max_keys]   final-CA keys
  tokens          [B, max_len]                token fed at each position
"""
from __future__ import annotations

import math
from typing import Dict, Optional

import torch

from . import _lib
from .config import ModelConfig
from .weights import rope_tables

_P = _lib.ptr


class LoomDecoder:
    """Model.step / infer for a batch of sequences on the gfx950 kernels."""

    STEPS_PER_GRAPH = 8      # decode steps chained in one replayed graph
    PROJ_TABLE_MAX_BYTES = 1 << 30   # largest per-vocabulary projection table built

    def __init__(self, cfg: ModelConfig, state: Dict[str, torch.Tensor], batch: int,
                 dtype: torch.dtype = torch.bfloat16, device="cuda", max_len: Optional[int] = None,
                 carry_token_id: Optional[int] = None):
        if dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"dtype must be float32 or bfloat16, got {dtype}")
        self.cfg = cfg
        self.B = int(batch)
        self.dtype = dtype
        self.dev = torch.device(device)
        self.code = _lib.DTYPE_CODE[dtype]
        self.max_len = int(max_len or cfg.seq_len)
        if self.max_len > cfg.seq_len:
            raise ValueError(f"max_len {self.max_len} exceeds seq_len {cfg.seq_len}")
        self.carry_token_id = carry_token_id
        self.lib = _lib.load()
        c = cfg
        dev, dt = self.dev, dtype

        def mat(k):
            return state[k].detach().to(dev, dt).contiguous()

        def f32(k):
            return state[k].detach().to(dev, torch.float32).contiguous()

        self.emb = mat("emb.weight")
        self.head = mat("head.weight")
        self.blocks = []
        for bi in range(c.L):
            p = f"blocks.{bi}."
            raw_alpha = float(state[p + "ffn.identity_gate.raw_alpha"])
            logits = state[p + "ffn.gate_selector.logits"].detach().float()
            self.blocks.append(dict(
                ln1_w=f32(p + "ln_attn.weight"), ln1_b=f32(p + "ln_attn.bias"),
                qkv=mat(p + "attn.qkv_weight"), o=mat(p + "attn.o.weight"),
                ln2_w=f32(p + "ln_ffn.weight"), ln2_b=f32(p + "ln_ffn.bias"),
                w1r=mat(p + "ffn.w1_real.weight"), b1r=f32(p + "ffn.w1_real.bias"),
                w1i=mat(p + "ffn.w1_imag"), ib=f32(p + "ffn.w1_imag_bias"),
                tw=f32(p + "ffn.w1_imag_trace"),
                w2=mat(p + "ffn.w2.weight"), b2=f32(p + "ffn.w2.bias"),
                gate_w=torch.softmax(logits, 0).to(dev, dt),           # GateSelector weights
                alpha=0.25 * math.tanh(raw_alpha),                      # IdentityAnchoredGate
                anchor=torch.ones((), device=dev),
            ))
            if c.gate_proj:                      # independent amplitude source (:2849)
                self.blocks[-1].update(gpw=mat(p + "ffn.gate_proj.weight"),
                                       gpb=f32(p + "ffn.gate_proj.bias"))
        self.kvw = mat("depth_attn.kv_weight")
        # depth readouts: one shared [N, N], or one per sublayer [2L, N, N] (:3424-3428)
        if c.depth_readout == "per-sublayer":
            self.wo_sub = mat("depth_attn.w_o_weight")
        else:
            self.wo = mat("depth_attn.w_o.weight")
        self.qp = mat("depth_attn.q_params")
        # depth_attn_qkv_rms targets of q, k, v (loomformer.py:3397-3407)
        self.depth_rms = ((c.fanin_gain / math.sqrt(c.HD), c.fanin_gain,
                           c.fanin_gain * c.deepnorm_beta) if c.depth_qkv_rms else None)
        self.ln_final = mat("ln_final.weight") if c.final_norm else None
        key_w = state["tria_agg.reader.key_proj.weight"].detach().float()
        query = state["tria_agg.pool.query"].detach().float()
        lsr = state["tria_agg.pool.logit_scale_raw"].detach().float()
        raw = torch.mv(key_w.t(), query)                                 # tria.py:1346-1349
        score_w = torch.nn.functional.normalize(raw, dim=0, eps=1e-6) * torch.nn.functional.softplus(lsr)
        self.score_w = score_w.to(dev, dt)
        self.proj_w, self.proj_b = mat("tria_agg.reader.proj.weight"), f32("tria_agg.reader.proj.bias")
        self.up_w, self.up_b = mat("tria_agg.up.weight"), f32("tria_agg.up.bias")
        self.wqk, self.wv = mat("tria_final_ca.w_qk.weight"), mat("tria_final_ca.w_v.weight")
        # per vocabulary id: [DepthAttn.project(emb[id]) | layer 0's qkv(emb[id])], the
        # step's first depth-history slot and first qkv row (loomformer.py:3971-3973),
        # gathered by the step's prologue instead of projected each step (both
        # projections are linear in the embedding row); built when it is small
        qkv_w = (c.QH + 2 * c.KVH) * c.HD
        self.ptab_row = 2 * c.N + qkv_w
        elt = torch.tensor([], dtype=dt).element_size()
        self.ptab = None
        if c.V * self.ptab_row * elt <= self.PROJ_TABLE_MAX_BYTES and c.V % 8 == 0 and c.V <= 16384:
            self.ptab = torch.empty(c.V, self.ptab_row, dtype=dt, device=dev)
            self._linear(self.emb, self.kvw, self.ptab, c.V, 2 * c.N, c.N, ldc=self.ptab_row)
            self._linear(self.emb, self.blocks[0]["qkv"], self.ptab[:, 2 * c.N:], c.V, qkv_w, c.N,
                         ldc=self.ptab_row)
        self.gamma = c.gamma_max * math.tanh(float(state["tria_final_ca.raw_gamma"]))
        cos, sin = rope_tables(c, self.max_len)
        self.cos, self.sin = cos.to(dev), sin.to(dev)

        B, N, H, L = self.B, c.N, c.H, c.L
        z = lambda *s, dtype=dt: torch.zeros(*s, dtype=dtype, device=dev)
        # head-major caches [L, B, KVH, max_len, HD]: one kv head's rows are contiguous
        self.k_cache = z(L, B, c.KVH, self.max_len, c.HD)
        self.v_cache = z(L, B, c.KVH, self.max_len, c.HD)
        self.hist = z(B, 2 * L, 2 * N)
        self.trace = z(L, B, H)
        self.doc = z(B, H, 3, 3)
        # final-CA key slots: one per hard fire (every `window` tokens); with an
        # explicit <CARRY> id any position may fire
        if carry_token_id is None:
            self.max_keys = max(1, self.max_len // max(1, c.window) + 1)
        else:
            self.max_keys = min(self.max_len, 1024)
        self.ca_k = z(B, self.max_keys, N)
        self.ca_v = z(B, self.max_keys, N)
        self.ca_valid = z(B, self.max_keys, dtype=torch.uint8)
        self.pending = z(B, dtype=torch.uint8)
        self.reset_now = z(B, dtype=torch.uint8)
        self.fire = z(B, dtype=torch.uint8)
        self.pos_dev = z(1, dtype=torch.int64)
        self.ca_len = z(1, dtype=torch.int64)
        self.ids = z(B, dtype=torch.int64)
        self.tokens = z(B, self.max_len, dtype=torch.int64)
        self.prompt_buf = z(B, self.max_len, dtype=torch.int64)
        ws = self.lib.loom_gqa_workspace_bytes(B, self.max_len, c.QH, c.KVH, c.HD)
        self.ws = torch.zeros((ws + 3) // 4, dtype=torch.float32, device=dev)   # GQA chunk records
        self.ws_bytes = ws
        # per-block slot-pool records of the decode Tria readout
        rb = self.lib.loom_decode_tria_readout_workspace_bytes(B, H)
        self.rd_ws = torch.empty((rb + 3) // 4, dtype=torch.float32, device=dev)
        self.rd_ws_bytes = rb
        # activations
        self.h = z(B, N)
        # fragment-major copy of h written by the sublayer LayerNorms (bf16 fused
        # form), read by the projections of h that follow them
        self.h_frag = (z(-(-B // 16) * 16 * N) if dtype == torch.bfloat16 and B <= 64 and N % 32 == 0
                       else None)
        self.h2 = z(B, N)
        self.qkv = z(B, N + 2 * c.KV)
        self.q = z(B, c.QH, c.HD)
        self.c = z(B, c.QH, c.HD)
        self.kctx = z(B, c.QH, c.HD)
        self.d = z(B, c.QH, c.HD)
        self.dh = z(B, c.QH, c.HD)
        # the attention launch's depth slice also reads history slots 0..2bi with the
        # FFN sublayer's query (normalised fp32 rows and log-sum-exp); ffn_decode then
        # folds in slot 2bi+1 alone (bf16 MFMA attention, plain depth read)
        self.depth_pair = (dtype == torch.bfloat16 and self.depth_rms is None
                           and c.HD in (32, 64, 96, 128) and c.QH // c.KVH in (1, 2, 4, 8))
        self.part_d = z(B, c.QH, c.HD, dtype=torch.float32) if self.depth_pair else None
        self.part_lse = z(B, c.QH, dtype=torch.float32) if self.depth_pair else None
        self.attn_out = z(B, N)
        self.skip = z(B, N)
        self.R = z(B, H)
        self.G = z(B, H) if c.gate_proj else None      # gate_proj(u), the amplitude source
        self.beta = z(B, H)
        self.act = z(B, H)
        self.act_frag = (z(-(-B // 16) * 16 * H) if self.h_frag is not None and H % 32 == 0
                         else None)
        self.s = z(B, H)
        self.ffn_out = z(B, N)
        self.y = z(B, N)                # pre-LayerNorm sum of a sublayer (unfused path)
        ln_ws = self.lib.loom_linear_ln_workspace_bytes(B, N)
        self.ln_ws = torch.empty((ln_ws + 3) // 4, dtype=torch.float32, device=dev)
        self.carry = z(2, B, H, 3, 3)
        self.p = z(2, B, H)
        self.a_t = z(B, N)
        self.stage_k = z(B, N)
        self.stage_v = z(B, N)
        self.q_ca = z(B, N)
        self.h3 = z(B, N) if c.final_norm else None     # RMSNorm(h) before the head
        self.logits = z(B, c.V)
        self.snap = torch.empty((), dtype=torch.float32, device=dev)
        self.pos = 0
        self._graphs: Dict[int, torch.cuda.CUDAGraph] = {}
        self._descs: Dict[object, object] = {}
        # the chunked prefill's second and third streams, created once: HIP deals new
        # streams round-robin over a few hardware queues, so a stream made per
        # call would in time share the main stream's queue and serialise
        self.aux_stream = torch.cuda.Stream(device=dev)
        self.tail_stream = torch.cuda.Stream(device=dev)
        # the chunked prefill's chunk buffers, kept from one prompt to the next
        # (≈1 GB at B = 32, 128-token chunks, H = 3072); free_prefill_buffers()
        # drops them
        self._prefill_buffers: Dict[str, torch.Tensor] = {}

    # ------------------------------------------------------------------ helpers

    def _call(self, name, *args):
        rc = getattr(self.lib, name)(*args)
        if rc != 0:
            raise RuntimeError(self.lib.loom_last_error().decode())

    def _stream(self):
        return _lib.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)

    def wo_for(self, sub: int) -> torch.Tensor:
        """The depth readout of sublayer `sub` (DepthAttn.forward, loomformer.py:3424-3428)."""
        return self.wo_sub[sub] if self.cfg.depth_readout == "per-sublayer" else self.wo

    def head_logits(self, x: torch.Tensor, out: torch.Tensor, rows: int) -> None:
        """Model._head_in (loomformer.py:3527-3529): the optional final RMSNorm
        (eps 1e-6), then the head."""
        if self.ln_final is not None:
            self._call("loom_rms_norm", self.code, _P(x), _P(self.ln_final), _P(self.h3), rows,
                       self.cfg.N, 1e-6, self._stream())
            x = self.h3
        self._linear(x, self.head, out, rows, self.cfg.V, self.cfg.N)

    def depth_read(self, sub: int, hist: torch.Tensor, out: torch.Tensor, rows: int) -> None:
        """DepthAttn read over history slots [0, sub] of `hist` [rows, 2L, 2N]
        (loomformer.py:3404-3429, tensor branch), fixed-RMS q/k/v under
        depth_attn_qkv_rms."""
        c, N, L = self.cfg, self.cfg.N, self.cfg.L
        args = [self.code, _P(self.qp[sub]), _P(hist), _P(hist[:, :, N:]), 2 * L * 2 * N, 2 * N,
                _P(out), None, None, rows, sub + 1, c.QH, c.HD]
        if self.depth_rms is None:
            self._call("loom_depth_attn_forward", *args, self._stream())
        else:
            self._call("loom_depth_attn_forward_rms", *args, *self.depth_rms, self._stream())

    @property
    def pair_reads(self) -> bool:
        """The plain depth read at a head size the paired / folded kernels take."""
        return self.depth_rms is None and self.cfg.HD in (32, 64, 96, 128)

    def depth_read_pair(self, sub: int, hist: torch.Tensor, out: torch.Tensor,
                        part_d: torch.Tensor, part_lse: torch.Tensor, rows: int) -> None:
        """DepthAttn reads over history slots [0, sub] for sublayers sub (into out) and
        sub + 1 (its part over these slots: fp32 rows part_d and log-sum-exp
        part_lse), one pass over the slots (loomformer.py:3404-3429)."""
        c, N, L = self.cfg, self.cfg.N, self.cfg.L
        self._call("loom_depth_attn_pair", self.code, _P(self.qp[sub]), _P(self.qp[sub + 1]),
                   _P(hist), _P(hist[:, :, N:]), 2 * L * 2 * N, 2 * N, _P(out), _P(part_d),
                   _P(part_lse), rows, sub + 1, c.QH, c.HD, self._stream())

    def depth_read_fold(self, sub: int, hist: torch.Tensor, out: torch.Tensor,
                        part_d: torch.Tensor, part_lse: torch.Tensor, rows: int) -> None:
        """DepthAttn read of sublayer sub over slots [0, sub] from its part over
        slots [0, sub - 1] (depth_read_pair of sublayer sub - 1) and slot sub."""
        c, N, L = self.cfg, self.cfg.N, self.cfg.L
        self._call("loom_depth_attn_fold", self.code, _P(self.qp[sub]), _P(hist),
                   _P(hist[:, :, N:]), 2 * L * 2 * N, 2 * N, sub + 1, _P(part_d), _P(part_lse),
                   _P(out), rows, c.QH, c.HD, self._stream())

    def _linear(self, x, w, out, M, Nout, K, bias=None, ldx=None, ldc=None, gate_p=None,
                gate_alpha=0.0, residual=None):
        self._call("loom_linear", self.code, _P(x), ldx or K, _P(w), K, _P(bias), _P(gate_p),
                   float(gate_alpha), _P(residual), _P(out), ldc or Nout, M, Nout, K, self._stream())

    def _multi(self, key, x, segments, x2=None, only_if=None, x_frag=None) -> None:
        """loom_linear_multi with a descriptor built once per call site (every
        pointer in it is a persistent engine buffer or weight)."""
        d = self._descs.get(key)
        if d is None:
            d = _lib.linear_multi_desc(x, segments, x2=x2, only_if=only_if, x_frag=x_frag)
            self._descs[key] = d
        self._call("loom_linear_multi", self.code, _lib.ctypes.byref(d), self._stream())

    def _linear_ln(self, key, x, segment, x2, gamma, beta, x2_frag=None) -> None:
        """h = LayerNorm(x w^T + x2 w2^T + bias) through loom_linear_ln (h and
        its fragment-major copy)."""
        d = self._descs.get(key)
        if d is None:
            d = _lib.linear_multi_desc(x, [segment], x2=x2, x2_frag=x2_frag)
            self._descs[key] = d
        self._call("loom_linear_ln", self.code, _lib.ctypes.byref(d), _P(gamma), _P(beta), 1e-5,
                   _P(self.h), self.cfg.N, _P(self.ln_ws), self.ln_ws.numel() * 4, _P(self.h_frag),
                   self._stream())

    def free_prefill_buffers(self) -> None:
        """Release the chunk buffers the chunked prefill keeps between prompts
        (the next prefill allocates them again)."""
        self._prefill_buffers.clear()

    def reset(self) -> None:
        """Forget all sequence state (Model.step at pos 0 starts afresh)."""
        self.pos = 0
        self.trace.zero_()
        self.pending.zero_()
        self.ca_valid.zero_()
        self.ca_len.zero_()
        self.pos_dev.zero_()

    # ------------------------------------------------------------------ the step

    def _launch_step(self, first: bool, prompt_len: int, argmax: bool = False) -> None:
        """Enqueue one Model.step for position *pos_dev (device-resident).  `first`
        selects the position-0 variant (no seed, no previous temporal state);
        `argmax`: the step's token is the greedy pick of the current logits
        (infer's argmax, loomformer.py:5306) once the prompt is consumed, else the
        id the caller wrote into self.ids."""
        c, B, N, H, L = self.cfg, self.B, self.cfg.N, self.cfg.H, self.cfg.L
        st = self._stream()
        carry_id = -1 if self.carry_token_id is None else int(self.carry_token_id)
        hist = self.hist
        if self.ptab is not None:
            # token ids (greedy pick or prompt), fire / reset flags, and the rows of
            # depth history slot 0 (DepthAttn.project(emb[id]), loomformer.py:3973) and
            # layer 0's qkv gathered from the projection table, one launch
            self._call("loom_decode_prologue_gather", self.code,
                       _P(self.logits) if argmax else None, _P(self.ids),
                       _P(self.prompt_buf) if prompt_len > 0 else None, prompt_len, self.max_len,
                       _P(self.tokens), self.max_len, _P(self.pos_dev), _P(self.pending),
                       _P(self.fire), _P(self.reset_now), carry_id, c.window, c.seq_len,
                       _P(self.ptab), self.ptab_row, c.V, _P(hist), hist.stride(0), 2 * N,
                       _P(self.qkv), self.qkv.stride(0), self.ptab_row - 2 * N, B, st)
        else:
            if argmax:
                self._argmax()
            # token ids, fire / reset flags and the embedding row of this step, one launch
            self._call("loom_decode_prologue_embed", self.code, _P(self.ids),
                       _P(self.prompt_buf) if prompt_len > 0 else None, prompt_len, self.max_len,
                       _P(self.tokens), self.max_len, _P(self.pos_dev), _P(self.pending),
                       _P(self.fire), _P(self.reset_now), carry_id, c.window, c.seq_len,
                       _P(self.emb), _P(self.h), N, c.V, B, st)
            # depth history slot 0 = DepthAttn.project(h) (loomformer.py:3973), with
            # layer 0's qkv projection of the same h in the same launch
            self._multi("first", self.h, [dict(w=self.kvw, out=hist[:, 0]),
                                          dict(w=self.blocks[0]["qkv"], out=self.qkv)])
        sub = 0
        cache_sb = c.KVH * self.max_len * c.HD
        cache_st = c.HD
        cache_sh = self.max_len * c.HD
        carry_i = None          # index of the current depth carry in self.carry
        p_i = None              # index of the gate output p feeding the next block
        for bi, blk in enumerate(self.blocks):
            last = bi == L - 1
            kc, vc = self.k_cache[bi], self.v_cache[bi]
            # ---- attention step (loomformer.py:3300-3332): RoPE + cache append +
            # attention + chunk merge, one launch
            # with the depth read 2*bi of this token (loomformer.py:3999) in the same launch
            if self.depth_pair:
                # with the FFN sublayer's read (query sub + 1) over the same slots
                self._call("loom_gqa_decode_step_depth2", self.code, _P(self.qkv), _P(kc), _P(vc),
                           cache_sb, cache_st, cache_sh, _P(self.cos), _P(self.sin), _P(self.q),
                           _P(self.c), _P(self.kctx), N,
                           _P(self.ws), self.ws_bytes, B, self.max_len, _P(self.pos_dev), c.QH,
                           c.KVH, c.HD, _P(self.qp[sub]), _P(self.qp[sub + 1]), _P(self.hist),
                           _P(self.hist[:, :, N:]), 2 * L * 2 * N, 2 * N, sub + 1, _P(self.d),
                           _P(self.part_d), _P(self.part_lse), st)
            elif self.depth_rms is None:
                self._call("loom_gqa_decode_step_depth", self.code, _P(self.qkv), _P(kc), _P(vc),
                           cache_sb, cache_st, cache_sh, _P(self.cos), _P(self.sin), _P(self.q),
                           _P(self.c), _P(self.kctx), N,
                           _P(self.ws), self.ws_bytes, B, self.max_len, _P(self.pos_dev), c.QH,
                           c.KVH, c.HD, _P(self.qp[sub]), _P(self.hist), _P(self.hist[:, :, N:]),
                           2 * L * 2 * N, 2 * N, sub + 1, _P(self.d), st)
            else:
                self._call("loom_gqa_decode_step", self.code, _P(self.qkv), _P(kc), _P(vc),
                           cache_sb, cache_st, cache_sh, _P(self.cos), _P(self.sin), _P(self.q),
                           _P(self.c), _P(self.kctx), N, _P(self.ws), self.ws_bytes, B,
                           self.max_len, _P(self.pos_dev), c.QH, c.KVH, c.HD, st)
                self.depth_read(sub, self.hist, self.d, B)
            # ---- LN(o(c) + w_o(d)) (loomformer.py:3999-4000): both products
            # accumulate in one launch
            self._linear_ln(("attn", bi), self.c.view(B, N),
                            dict(w=blk["o"], w2=self.wo_for(sub), out=self.y), self.d.view(B, N),
                            blk["ln1_w"], blk["ln1_b"])
            # ---- history slot 2*bi+1 (loomformer.py:4004) and W_real of the same h
            # (+ IdentityAnchoredGate with the previous block's p, loomformer.py:2839;
            # + gate_proj(h), the amplitude source under paraplex_gate_proj, :2849)
            sub += 1
            real = dict(w=blk["w1r"], out=self.R, bias=blk["b1r"])
            if p_i is not None:
                real.update(gate_p=self.p[p_i], gate_alpha=blk["alpha"])
            segs = [dict(w=self.kvw, out=hist[:, sub]), real]
            if c.gate_proj:
                segs.append(dict(w=blk["gpw"], out=self.G, bias=blk["gpb"]))
            self._multi(("kvr", bi), self.h, segs, x_frag=self.h_frag)
            # ---- Paraplex FFN core (beta space, fused pointwise chain; loomformer.py:
            # 2818-2893, :2533-2560) and the Tria depth op (loomformer.py:4012-4040,
            # axis = bi % 3) of this token, one launch in bf16
            out_i = 0 if carry_i != 0 else 1
            gate = not last
            new_p = (0 if p_i != 0 else 1) if gate else None
            use_seed = bi == 0 and not first
            key = ("ffn_core", bi, use_seed)
            d = self._descs.get(key)
            if d is None:
                d = _lib.ffn_decode_desc(
                    u=self.h, q_h=self.q, k_ctx_h=self.kctx, c_h=self.c, d_h=self.dh,
                    w_compact=blk["w1i"], M=B, N=N, H=H, imag_in=c.imag_in, hidden_per_q_head=c.Hq,
                    head_dim=c.HD, n_q_heads=c.QH, open_sectors=1 if c.sectors == "open" else 0,
                    p_real=self.R, gate_src=self.G, imag_bias=blk["ib"], trace=self.trace[bi],
                    trace_w=blk["tw"],
                    powlu_m=float(c.powlu_m), act=self.act, s=self.s, beta=self.beta,
                    carry_prev=None if (carry_i is None or use_seed) else self.carry[carry_i],
                    seed=self.doc if use_seed else None,
                    seed_valid=self.pending if use_seed else None,
                    gate_w=blk["gate_w"] if gate else None, carry_out=self.carry[out_i],
                    p_out=self.p[new_p] if gate else None, alpha=float(c.tria_alpha), axis=bi % 3,
                    act_frag=self.act_frag,
                    u_frag=self.h_frag if (c.sectors != "open" and c.HD % 32 == 0) else None,
                    # the depth read of history slot `sub` (loomformer.py:4004-4006), d_h,
                    # computed by this launch
                    depth_q=self.qp[sub], depth_k=self.hist, depth_v=self.hist[:, :, N:],
                    depth_sbt=2 * L * 2 * N, depth_ss=2 * N, depth_S=sub + 1,
                    depth_rms=0 if self.depth_rms is None else 1,
                    depth_part_d=self.part_d, depth_part_lse=self.part_lse,
                    **({} if self.depth_rms is None else
                       dict(zip(("depth_qt", "depth_kt", "depth_vt"), self.depth_rms))))
                self._descs[key] = d
            self._call("loom_ffn_decode", self.code, _lib.ctypes.byref(d), st)
            carry_i, p_i = out_i, new_p
            # ---- LN(w_o(d_h) + W2(act) + b2) (loomformer.py:4045): one launch + LN
            self._linear_ln(("ffn", bi), self.dh.view(B, N),
                            dict(w=self.wo_for(sub), w2=blk["w2"], out=self.y, bias=blk["b2"]),
                            self.act, blk["ln2_w"], blk["ln2_b"], x2_frag=self.act_frag)
            if not last:
                # next history slot (loomformer.py:4050) and the next block's qkv
                sub += 1
                self._multi(("next", bi), self.h, [dict(w=self.kvw, out=hist[:, sub]),
                                                   dict(w=self.blocks[bi + 1]["qkv"], out=self.qkv)],
                            x_frag=self.h_frag)
            else:
                # the final-CA query of the last hidden state (tria.py:1580)
                self._multi(("next", bi), self.h, [dict(w=self.wqk, out=self.q_ca)],
                            x_frag=self.h_frag)
        # ---- temporal carry + PolARM on fires (loomformer.py:4053-4085), in place,
        # and the TriaAggregator readout of the new state (tria.py:1436-1441): one launch
        self._call("loom_decode_tria_readout", self.code, _P(self.carry[carry_i]),
                   None if first else _P(self.doc), None if first else _P(self.reset_now),
                   _P(self.fire), _P(self.doc), _P(self.score_w), _P(self.proj_w), _P(self.proj_b),
                   _P(self.up_w), _P(self.up_b), _P(self.a_t), _P(self.rd_ws), self.rd_ws_bytes, B, H, N,
                   float(c.polarm_beta), 1e-6, st)
        # ---- final cross-attention step (tria.py:1560-1595): stage k/v (computed
        # only on steps where a row fires, as the readout above), append on fire
        # (+ end-of-step bookkeeping), then attend over the appended keys
        self._multi("stage", self.a_t, [dict(w=self.wqk, out=self.stage_k),
                                        dict(w=self.wv, out=self.stage_v)], only_if=self.fire)
        self._call("loom_decode_epilogue", self.code, _P(self.stage_k), _P(self.stage_v),
                   _P(self.ca_k), _P(self.ca_v), _P(self.ca_valid), _P(self.ca_len), _P(self.fire),
                   _P(self.pending), _P(self.pos_dev), B, N, self.max_keys, st)
        self._call("loom_final_ca_sparse_strided", self.code, _P(self.q_ca), _P(self.ca_k),
                   _P(self.ca_v), self.max_keys * N, _P(self.ca_valid), self.max_keys,
                   _P(self.h), float(self.gamma), _P(self.h2), None, B, 1, self.max_keys,
                   _P(self.ca_len), N, float(N ** -0.5), st)
        self.head_logits(self.h2, self.logits, B)

    def _argmax(self) -> None:
        """ids = argmax(logits) per row (infer's greedy pick, loomformer.py:5306)."""
        self._call("loom_argmax_rows", self.code, _P(self.logits), self.B, self.cfg.V, _P(self.ids),
                   self._stream())

    def _check_ids(self, ids: torch.Tensor) -> None:
        """Token ids must index the embedding table (nn.Embedding raises otherwise)."""
        if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= self.cfg.V):
            raise ValueError(f"token ids must lie in [0, {self.cfg.V})")

    def _check_capacity(self, pos: int) -> None:
        if pos >= self.max_len:
            raise ValueError(f"generation exceeded seq_len={self.max_len}; no wraparound support")
        # hard fires up to and including `pos`: multiples of W in [1, min(pos+1, seq_len-1)]
        fires = min(pos + 1, self.cfg.seq_len - 1) // self.cfg.window
        if self.carry_token_id is None and fires > self.max_keys:
            raise ValueError("final-CA key cache is full")

    @torch.no_grad()
    def step(self, ids: torch.Tensor, pos: int) -> torch.Tensor:
        """Advance every sequence by one token at position ``pos`` (eager launches);
        returns logits [B, V]."""
        if pos == 0:
            self.reset()
        if pos != self.pos:
            raise ValueError(f"step expects position {self.pos}, got {pos}")
        self._check_capacity(pos)
        self._check_ids(ids)
        self.ids.copy_(ids.to(self.dev).view(-1))
        self._launch_step(first=pos == 0, prompt_len=0)
        self.pos = pos + 1
        return self.logits

    # ------------------------------------------------------------------ generation

    def _graph_for(self, prompt_len: int, steps: int = 1) -> torch.cuda.CUDAGraph:
        """Capture `steps` x (argmax -> ids, then one step for a position >= 1,
        reading the prompt while pos < prompt_len).  The position advances on the
        device, so several steps chain inside one graph and the gap between
        graph launches is paid once per `steps` tokens."""
        key = (prompt_len, steps)
        g = self._graphs.get(key)
        if g is None:
            torch.cuda.synchronize(self.dev)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(steps):
                    self._launch_step(first=False, prompt_len=prompt_len, argmax=True)
            self._graphs[key] = g
        return g

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, n_new: int, return_logits: bool = False,
                 use_graph: bool = True, chunked_prefill: bool = False):
        """Prefill ``prompt`` [B, P] token by token (the reference's infer loop) or,
        with ``chunked_prefill``, through the chunked forward; then ``n_new``
        greedy tokens.  Returns the new ids [B, n_new] (and with return_logits the
        logits after every step: [B, P + n_new, V] token by token, or
        [B, 1 + n_new, V] from the last prompt position on when chunked)."""
        B, P = prompt.shape
        if B != self.B:
            raise ValueError(f"prompt batch {B} != engine batch {self.B}")
        if P < 1:
            raise ValueError("prompt must hold at least one token")
        total = P + n_new
        self._check_capacity(total - 1)
        logits_all = [] if return_logits else None
        if chunked_prefill:
            self.prefill(prompt)
            first_pos = P
        else:
            self.reset()
            self._check_ids(prompt)
            self.prompt_buf[:, :P].copy_(prompt.to(self.dev))
            self._launch_step(first=True, prompt_len=P)
            first_pos = 1
        if return_logits:
            logits_all.append(self.logits.float().clone())
        graph = self._graph_for(P) if use_graph else None
        for _ in range(first_pos, total):
            if graph is not None:
                graph.replay()
            else:
                self._launch_step(first=False, prompt_len=P, argmax=True)
            if return_logits:
                logits_all.append(self.logits.float().clone())
        self.pos = total
        out = self.tokens[:, P:total].clone()
        if return_logits:
            return out, torch.stack(logits_all, 1)
        return out

    @torch.no_grad()
    def start(self, prompt: torch.Tensor) -> None:
        """Reset, load ``prompt`` [B, P] and run position 0 (eager)."""
        B, P = prompt.shape
        if B != self.B or P < 1:
            raise ValueError("prompt must be [batch, >=1]")
        self.reset()
        self._check_ids(prompt)
        self.prompt_buf[:, :P].copy_(prompt.to(self.dev))
        self._prompt_len = P
        self._launch_step(first=True, prompt_len=P)
        self.pos = 1

    def prefill(self, prompt: torch.Tensor) -> None:
        """Chunked prefill of ``prompt`` [B, P] (the reference's chunked forward,
        loomformer.py:3788-3883): afterwards the engine stands at position P
        with the last prompt token's logits, as token-by-token steps would leave
        it; ``replay_steps`` / ``generated`` continue from there."""
        from .prefill import prefill
        prefill(self, prompt)

    @torch.no_grad()
    def warm_graphs(self) -> None:
        """Capture both graphs ``replay_steps`` replays (the chained
        STEPS_PER_GRAPH-step graph and the single step) for the current prompt,
        so that later replays do no capture work on the host."""
        self._graph_for(self._prompt_len, self.STEPS_PER_GRAPH)
        self._graph_for(self._prompt_len)

    @torch.no_grad()
    def replay_steps(self, n: int) -> None:
        """Advance ``n`` positions with the captured step (prompt tokens while
        pos < P, greedy argmax after): n // STEPS_PER_GRAPH replays of the
        chained graph, then single-step replays for the rest."""
        self._check_capacity(self.pos + n - 1)
        if n >= self.STEPS_PER_GRAPH:
            g = self._graph_for(self._prompt_len, self.STEPS_PER_GRAPH)
            for _ in range(n // self.STEPS_PER_GRAPH):
                g.replay()
        if n % self.STEPS_PER_GRAPH:
            g = self._graph_for(self._prompt_len)
            for _ in range(n % self.STEPS_PER_GRAPH):
                g.replay()
        self.pos += n

    def generated(self) -> torch.Tensor:
        """Greedy tokens produced so far (positions >= P)."""
        return self.tokens[:, self._prompt_len:self.pos]
