"""Kernel-level helpers of the depth frame, on m3x kernels.

Drop-in for serve/fast_depth_kernels.py: `add_ln` (:35), `topk_sample` (:72), `row_exponential` (:95).
Sampling here inverts the CDF of the top-k softmax with one Philox uniform per row (counter (ctr, level),
key seed); the reference races Gumbel/exponential noise over the same distribution (:60-68).
"""
from __future__ import annotations

import torch

from .. import ops


def add_ln(x, a, ln, c=None):
    """x, a: [B, T, D] (last dim contiguous); c: [B, 1, D] or None; ln: LayerNorm- or RMSNorm-like module.
    Returns (x + a [+ c], norm(...)) as new contiguous tensors (rounded to the input dtype after each add)."""
    B, T, D = x.shape
    xo = torch.empty(B * T, D, device=x.device, dtype=x.dtype)
    y = torch.empty_like(xo)
    b = getattr(ln, 'bias', None)
    kind = ops.NORM_LAYER if b is not None else ops.NORM_RMS
    eps = getattr(ln, 'eps', None)
    eps = (1e-5 if kind == ops.NORM_LAYER else torch.finfo(x.dtype).eps) if eps is None else eps
    cc = None if c is None else c.reshape(B, D)
    ops.add_norm(x, a, cc, xo, y, ln.weight, b, eps, T, kind)
    return xo.view(B, T, D), y.view(B, T, D)


def topk_sample(logits, seed_t, level, temp, top_k, greedy=False, ctr_t=None):
    """seed_t [1] (engine-wide stream; counter = row) or, with ctr_t, per-row seeds [B] and counters [B].
    Returns int64 codes [B]."""
    B, V = logits.shape
    dev = logits.device
    out = torch.empty(B, device=dev, dtype=torch.long)
    u = None
    if not greedy:
        rows = torch.arange(B, device=dev)
        if ctr_t is not None:
            seeds, ctrs = seed_t.to(torch.int32).contiguous(), ctr_t.to(torch.int32).contiguous()
        else:
            seeds = seed_t.to(torch.int32).expand(B).contiguous()
            ctrs = rows.to(torch.int32)
        u = torch.empty(B, 1, device=dev, dtype=torch.float32)
        ops.philox_uniforms(seeds, ctrs, rows, u, int(level))
        u = u[:, 0]
    ops.topk_sample(logits.contiguous(), u, 1.0 / temp, top_k, greedy, out, out_i64=True)
    return out


def row_exponential(B, V, seeds, ctrs, level=0):
    """Out[row, :V] = Exp(1) noise from the row's own (seed, counter) stream."""
    out = torch.empty(B, V, device=seeds.device, dtype=torch.float32)
    ops.philox_exponential(seeds.to(torch.int32).contiguous(), ctrs.to(torch.int32).contiguous(), out, level)
    return out
