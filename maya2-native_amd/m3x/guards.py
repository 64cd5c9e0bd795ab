"""The engine's loop guard on the device (maya3/guards.py:80-107, used by the tick at maya3/engine.py:585-617).

loop_detect_batch keeps the reference's signature and results for a host history array. LoopGuard keeps every
slot's cb0 history on the device, so a frame graph can push the new codes and evaluate the rules without a host
copy of the history; the engine then reads one int32 code per seat with its other per-tick outputs.
"""
from __future__ import annotations

import numpy as np
import torch

from ._lib import check, lib
from .ops import _index, _need, _p, _stream


def _codes_to_hits(codes):
    return [None if c == 0 else ("stall" if c < 0 else f"period:{int(c)}") for c in codes]


def loop_guard(W, n, out, cfg, slots=None):
    """out[r] = 0 / -1 (stall) / p (period) for device history row W[slots[r]] with n[slots[r]] frames (W[r], n[r]
    without slots); W int32 [*, hist], n int64."""
    rows = n.numel() if slots is None else slots.numel()
    _index(slots=slots)
    _need(W, torch.int32, "W")
    _need(n, torch.long, "n")
    check(lib().m3x_loop_guard(_p(W), W.stride(0), _p(slots), _p(n), _p(out), rows, W.shape[1], int(cfg.stall),
                               int(cfg.period_win), float(cfg.period_thr), int(cfg.pmin), int(cfg.pmax), _stream()),
          "loop_guard")
    return out


def loop_detect_batch(W, n, cfg, device="cuda"):
    """W: [S, hist] int array, row i = the last `hist` cb0 codes of seat i, right-aligned (newest last; -1 = empty);
    n: [S] frames generated so far. Returns a list of None | 'stall' | 'period:<p>' (maya3/guards.py:80-107)."""
    W = np.asarray(W)
    S = W.shape[0]
    if S == 0:
        return []
    Wd = torch.as_tensor(np.ascontiguousarray(W, dtype=np.int32), device=device)
    nd = torch.as_tensor(np.asarray(n, dtype=np.int64), device=device)
    out = torch.empty(S, dtype=torch.int32, device=device)
    loop_guard(Wd, nd, out, cfg)
    return _codes_to_hits(out.cpu().tolist())


class LoopGuard:
    """Per-slot cb0 histories [max_slots + 1, hist] int32 (-1 = empty) and frame counts [max_slots + 1] int64 on
    the device: the engine's `s.hist` and `s.frames`."""

    def __init__(self, max_slots, cfg, device="cuda"):
        lib()
        self.cfg = cfg
        self.hist_len = int(getattr(cfg, "hist", 96))
        self.hist = torch.full((max_slots + 1, self.hist_len), -1, dtype=torch.int32, device=device)
        self.frames = torch.zeros(max_slots + 1, dtype=torch.int64, device=device)
        self.max_slots = max_slots

    def reset(self, slot):
        """A new seat on the slot (maya3/engine.py:447)."""
        self.hist[slot].fill_(-1)
        self.frames[slot] = 0

    def push(self, slots, codes):
        """Append codes[b] (int64, any row stride) to slot slots[b]'s history and count the frame."""
        ld = codes.stride(0) if codes.dim() > 1 else 1
        _index(slots=slots)
        _need(codes, torch.long, "codes")
        check(lib().m3x_hist_push(_p(self.hist), self.hist.stride(0), _p(self.frames), _p(slots), _p(codes), ld,
                                  slots.numel(), self.hist_len, _stream()), "hist_push")

    def detect(self, slots, out):
        """out[b] = 0 / -1 (stall) / p (period) for slot slots[b] (device tensors)."""
        return loop_guard(self.hist, self.frames, out, self.cfg, slots=slots)
