"""Codebook-0 step on m3x kernels: cb0 head GEMM + one sampler kernel (controlled stop, per-seat settings).

Equivalent of Engine._cb0 (maya3/engine.py:652-694) and the per-slot sampler state Engine._build_fast allocates
(:208-233) and Engine._bind writes (:429-444). Where the engine draws Exp(1) noise with `row_exponential` and
takes argmax(q/E), this draws one Philox uniform per seat from the same (seed, frame counter, level 0) stream key
and inverts the CDF of the same renormalised top-k (then top-p) distribution (the kernel's contract is in
csrc/sample.hip).
"""
from __future__ import annotations

from types import SimpleNamespace

import torch

from . import ops
from ._lib import lib


class Cb0Sampler:
    def __init__(self, head_weight, max_seats, aeos=None, temp=0.9, top_k=64, rep=0.8, rep_win=12, stop=True,
                 top_p=1.0):
        """head_weight [V0, hidden] bf16 (Backbone.cb0_head, tts/model/backbone.py:121). aeos: the AEOS class
        (default 2048 when V0 == 2049, else none). stop=False skips the controlled-stop bookkeeping."""
        lib()
        self.w = head_weight
        with torch.inference_mode():
            self.pw = ops.pack_weight(head_weight)  # fragment-order copy for the head GEMM
            torch.cuda.current_stream(head_weight.device).synchronize()
        self.V = head_weight.shape[0]
        self.aeos = (2048 if self.V == 2049 else -1) if aeos is None else int(aeos)
        self.stop = bool(stop) and self.aeos >= 0
        self.rep_win = int(rep_win)
        dev = head_weight.device
        m = max_seats + 1
        self.max_seats = max_seats
        if not 0.0 < float(top_p) <= 1.0:
            raise ValueError("top_p must be in (0, 1]")
        # the configuration defaults a seat gets back when its request leaves a setting unset
        self.temp, self.top_k, self.top_p, self.rep = float(temp), int(top_k), float(top_p), float(rep)
        self.temp_t = torch.full((m,), self.temp, device=dev, dtype=torch.float32)
        self.topk_t = torch.full((m,), self.top_k, device=dev, dtype=torch.long)
        self.topp_t = torch.full((m,), self.top_p, device=dev, dtype=torch.float32)
        self.rep_t = torch.full((m,), float(rep), device=dev, dtype=torch.float32)
        self.seed_t = torch.zeros(m, device=dev, dtype=torch.int32)
        self.ctr_t = torch.zeros(m, device=dev, dtype=torch.int32)
        self.hist_t = torch.full((m, max(1, self.rep_win)), -1, device=dev, dtype=torch.long)
        self.frames_t = torch.zeros(m, device=dev, dtype=torch.long)
        self.min_t = torch.zeros(m, device=dev, dtype=torch.long)
        self.hazard_t = torch.zeros(m, device=dev, dtype=torch.float32)
        self.aeos_bias = torch.zeros(m, device=dev, dtype=torch.float32)

    @torch.inference_mode()
    def bind(self, slot, seed, temperature=None, top_k=None, top_p=None, repetition_penalty=None, min_frames=0):
        """Per-seat settings at admission (maya3/engine.py:429-444): a setting left unset (None, or 0 where the
        engine's `x or default` reads it so) takes the sampler's configured default, so a reused slot never
        inherits its previous seat's settings."""
        if top_p is not None and not 0.0 < float(top_p) <= 1.0:
            raise ValueError("top_p must be in (0, 1]")
        self.seed_t[slot] = int(seed)
        self.ctr_t[slot] = 0
        self.frames_t[slot] = 0
        self.min_t[slot] = int(min_frames)
        self.hazard_t[slot] = 0
        self.aeos_bias[slot] = 0
        self.hist_t[slot] = -1
        self.temp_t[slot] = float(temperature or self.temp)
        self.topk_t[slot] = int(top_k or self.top_k)
        self.topp_t[slot] = float(top_p or self.top_p)
        self.rep_t[slot] = float(self.rep if repetition_penalty is None else repetition_penalty)

    def make_buffers(self, B, h=None, codes=None):
        dev = self.w.device
        b = SimpleNamespace(B=B)
        b.slots = torch.full((B,), self.max_seats, dtype=torch.long, device=dev)
        b.h = h if h is not None else torch.zeros(B, self.w.shape[1], dtype=self.w.dtype, device=dev)
        b.logits = torch.empty(B, self.V, dtype=self.w.dtype, device=dev)
        b.u = torch.zeros(B, 1, dtype=torch.float32, device=dev)
        b.cb0 = torch.zeros(B, dtype=torch.long, device=dev)
        b.stop = torch.zeros(B, dtype=torch.long, device=dev)
        b.codes = codes
        return b

    def run(self, b, uniforms=True):
        """logits = h @ head^T; u from (seed_t, ctr_t, level 0); sample -> b.cb0 (and column 0 of b.codes)."""
        ops.linear(b.h, self.pw, b.logits)
        if uniforms:
            ops.philox_uniforms(self.seed_t, self.ctr_t, b.slots, b.u, 0)
        # with a history window the penalty always runs: a seat with penalty 0 subtracts exactly 0, so a graph
        # captured before any seat asked for a penalty still applies one bound later
        win = self.rep_win > 0
        ops.cb0_sample(b.logits, self.aeos, b.slots, b.u[:, 0], temp_t=self.temp_t, topk_t=self.topk_t,
                       topp_t=self.topp_t,
                       aeos_bias=self.aeos_bias if self.aeos >= 0 else None, rep_t=self.rep_t if win else None,
                       hist_t=self.hist_t if win else None,
                       frames_t=self.frames_t if self.stop else None, min_t=self.min_t if self.stop else None,
                       hazard_t=self.hazard_t if self.stop else None, ctr_t=self.ctr_t, cb0_out=b.cb0,
                       cb0_i32=None if b.codes is None else b.codes[:, 0], stop_out=b.stop)
        return b.stop, b.cb0

    @torch.inference_mode()
    def __call__(self, h, idx):
        """Eager step for seats idx with hidden states h [B, hidden]: returns (stop code [B], cb0 [B]) as int64."""
        b = self.make_buffers(h.shape[0])
        b.slots.copy_(idx)
        b.h.copy_(h)
        stop, cb0 = self.run(b)
        return stop.clone(), cb0.clone()
