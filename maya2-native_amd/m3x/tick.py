"""The tick's readout (maya3/engine.py:558-573): every seat's stop code, cb0, optional loop-guard code, codes and
int16 PCM packed by one kernel into one device buffer, copied to pinned host memory in one transfer, and read
back as numpy views (the engine's `stop_l`, `cb0_l`, `pcm_np`).
"""
from __future__ import annotations

import numpy as np
import torch

from ._lib import check, lib
from .ops import _p, _stream


class TickReadout:
    def __init__(self, max_seats, frame=1920, nq=0, with_loop=False, device="cuda"):
        """frame: PCM samples per seat and tick (0: no PCM); nq: codes per seat to carry (0: none)."""
        self.width = int(lib().m3x_tick_pack_width(int(with_loop), nq, frame))
        self.frame, self.nq, self.with_loop = frame, nq, with_loop
        self.dev_buf = torch.empty(max_seats, self.width, dtype=torch.int64, device=device)
        self.host = torch.empty(max_seats, self.width, dtype=torch.int64).pin_memory()
        self.evt = None
        self.B = 0

    def pack(self, stop, cb0, loop=None, codes=None, pcm=None):
        """Packs B seats (stop, cb0 int64 [B]; loop int32 [B]; codes int32 [B, nq] rows; pcm float32 [B, frame]
        rows) and starts the copy to the pinned host buffer on the current stream."""
        B = stop.numel()
        if B > self.dev_buf.shape[0]:
            raise ValueError(f"tick readout: {B} seats exceed the {self.dev_buf.shape[0]} the buffer was built for")
        for name, t in (("cb0", cb0), ("loop", loop), ("codes", codes), ("pcm", pcm)):
            if t is not None and t.shape[0] < B:
                raise ValueError(f"tick readout: {name} has {t.shape[0]} rows for {B} seats")
        if codes is not None and (codes.dim() != 2 or codes.shape[1] < self.nq):
            raise ValueError(f"tick readout: codes must be [B, >= {self.nq}]")
        if pcm is not None and (pcm.dim() != 2 or pcm.shape[1] < self.frame):
            raise ValueError(f"tick readout: pcm must be [B, >= {self.frame}]")
        if (loop is not None) != self.with_loop or (codes is not None) != (self.nq > 0) or \
                (pcm is not None) != (self.frame > 0):
            raise ValueError("tick readout: the parts given differ from the layout built")
        if pcm is not None and (pcm.dtype != torch.float32 or pcm.stride(-1) != 1):
            raise ValueError("tick readout: pcm must be float32 rows")
        check(lib().m3x_tick_pack(_p(stop), _p(cb0), _p(loop), _p(codes), 0 if codes is None else codes.stride(0),
                                  self.nq, _p(pcm), 0 if pcm is None else pcm.stride(0), self.frame, _p(self.dev_buf),
                                  self.width, B, _stream()), "tick_pack")
        self.host[:B].copy_(self.dev_buf[:B], non_blocking=True)
        self.evt = torch.cuda.Event()
        self.evt.record()
        self.B = B

    def wait(self):
        """Waits for the copy; returns dict(stop, cb0, loop, codes, pcm) numpy views of the pinned buffer. Raises
        RuntimeError when a carried code is negative: a depth run that lost a step's input voids its codes to -1
        (m3x_depth_run_void), and the reference fails the engine on a GPU-side error (maya3/engine.py:375-385)."""
        self.evt.synchronize()
        hv = self.host[:self.B].numpy()
        col = 2
        out = {"stop": hv[:, 0], "cb0": hv[:, 1]}
        if self.with_loop:
            out["loop"] = hv[:, 2]
            col = 3
        if self.nq:
            w = (self.nq + 1) // 2
            out["codes"] = hv[:, col:col + w].view(np.int32)[:, :self.nq]
            col += w
            bad = np.flatnonzero((out["codes"] < 0).any(axis=1))
            if bad.size:
                raise RuntimeError(f"tick readout: the depth codes of seat rows {bad.tolist()} are void (a persistent "
                                   "depth run lost a step's input)")
        if self.frame:
            out["pcm"] = hv[:, col:col + (self.frame + 3) // 4].view(np.int16)[:, :self.frame]
        return out
