"""Host-side plumbing shared by every graphed surface (StaticBackbone, FastDepth, StaticMimi, FrameStep).

Three pieces, each used the same way by all of them:
  - `RowTable`: the per-row int64 columns a replay reads (slot, real-row flag, position offset, ...) live in one
    device tensor [fields, rows]; a host update goes through a small ring of pinned buffers as ONE async copy,
    and is skipped when its key equals the last staged one. A ring slot is reused only after the event of the
    copy that last read it has completed, so a queued copy never sees its source rewritten.
  - `Buckets`: the sorted bucket sizes of a surface and the smallest bucket that holds a request.
  - `capture`: warm-up runs on a side stream, then one capture into the surface's shared memory pool, with
    chosen per-slot state tensors put back afterwards (the warm-up and capture runs must not move live state).
"""
from __future__ import annotations

import bisect

import numpy as np
import torch


class Buckets:
    def __init__(self, sizes):
        self.sizes = tuple(sorted({int(s) for s in sizes}))
        if not self.sizes or self.sizes[0] <= 0:
            raise ValueError(f"bucket sizes must be positive, got {sizes}")

    def pick(self, n, what="batch"):
        """The smallest bucket >= n (ValueError when none is)."""
        i = bisect.bisect_left(self.sizes, n)
        if i == len(self.sizes):
            raise ValueError(f"{what} {n} exceeds the largest bucket {self.sizes[-1]}")
        return self.sizes[i]

    def largest_first(self, subset=None):
        """Capture order: a graph captured after a larger one reuses the pool blocks the larger one released."""
        return sorted({int(s) for s in (subset or self.sizes)}, reverse=True)


class Upload:
    """Host arrays into a fixed device tensor through a ring of pinned buffers, one async copy per send."""

    def __init__(self, dev, ring=4):
        self.dev = dev
        self._host = torch.empty((ring,) + tuple(dev.shape), dtype=dev.dtype).pin_memory()
        self._done = [None] * ring
        self._turn = 0

    def buffer(self):
        """The next pinned buffer (numpy view), once the copy that last read it has completed."""
        t = self._turn
        if self._done[t] is not None:
            self._done[t].synchronize()
        return self._host[t].numpy()

    def send(self, n=None):
        """Copies the first n elements (along dim 0; all when None) of the buffer from buffer() on the current
        stream and advances the ring."""
        t = self._turn
        src = self._host[t] if n is None else self._host[t][:n]
        dst = self.dev if n is None else self.dev[:n]
        dst.copy_(src, non_blocking=True)
        evt = torch.cuda.Event()
        evt.record()
        self._done[t] = evt
        self._turn = (t + 1) % len(self._done)


class RowTable:
    """Device columns [fields, rows] int64 staged from host lists through an Upload ring."""

    def __init__(self, fields, rows, device, pad, ring=4):
        """fields: column names; pad: name -> value of the rows past a staged list (e.g. the dummy slot)."""
        self.fields = tuple(fields)
        self.rows = int(rows)
        self.pad = np.array([int(pad.get(f, 0)) for f in self.fields], dtype=np.int64)
        self.dev = torch.from_numpy(np.repeat(self.pad[:, None], self.rows, 1)).to(device)
        self._up = Upload(self.dev, ring)
        self.key = None

    def __getitem__(self, field):
        """The device column of `field` (a contiguous [rows] view that a graph may capture)."""
        return self.dev[self.fields.index(field)]

    def stage(self, columns, key=None):
        """Uploads columns (name -> sequence of ints, at most `rows` long; missing names and the tail take their
        pad value) on the current stream. Returns False without a copy when `key` equals the last staged key."""
        if key is not None and key == self.key:
            return False
        buf = self._up.buffer()
        buf[:] = self.pad[:, None]
        for i, name in enumerate(self.fields):
            vals = columns.get(name)
            if vals is not None and len(vals):
                if len(vals) > self.rows:
                    raise ValueError(f"{len(vals)} rows exceed the table's {self.rows}")
                buf[i, :len(vals)] = np.asarray(vals, dtype=np.int64)
        self._up.send()
        self.key = key
        return True

    def forget(self):
        """The device columns were written by someone else: the next stage() uploads whatever its key."""
        self.key = None


class ErrorWatch:
    """The error word of a persistent kernel's sync block (sync[2]) seen by the host without a synchronisation:
    after() enqueues its copy into pinned memory behind the step that may set it; raise_if_set() raises once that
    copy has landed and shows the word set (a step's failure surfaces at the next call, or at the tick's readout,
    which sees the voided outputs in its own copy)."""

    def __init__(self, sync, what):
        self.sync, self.what = sync, what
        self.host = torch.zeros(1, dtype=sync.dtype).pin_memory()
        self.evt = None

    def after(self):
        self.host.copy_(self.sync[2:3], non_blocking=True)
        self.evt = torch.cuda.Event()
        self.evt.record()

    def raise_if_set(self):
        if self.evt is not None and self.evt.query() and int(self.host[0]):
            self.evt = None
            raise RuntimeError(f'{self.what} lost a step\'s input (its bounded waits ran out); that step\'s outputs '
                               'are void. clear_run_error() resets the error word')


def capture(body, pool, warm=2, keep=()):
    """Runs body() `warm` times on a side stream, then captures one run into a hipGraph on `pool`. The tensors in
    `keep` (per-slot counters and the like that a run advances) are restored after the runs. Returns the graph."""
    saved = [t.clone() for t in keep]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warm):
            body()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, pool=pool, stream=side):
        body()
    torch.cuda.current_stream().wait_stream(side)
    for t, v in zip(keep, saved):
        t.copy_(v)
    return graph


def check_slots(slots, limit, distinct=True):
    """ValueError for a repeated slot (distinct=True), then IndexError for one outside [0, limit)."""
    if distinct and len(set(slots)) != len(slots):
        raise ValueError("duplicate slots in one step")
    for s in slots:
        if not 0 <= s < limit:
            raise IndexError(f"slot {s} outside 0..{limit - 1}")
