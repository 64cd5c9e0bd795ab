"""One Maya3 frame step for a batch of decoding seats, captured as a single hipGraph.

Replay = x = feedback[slots] -> 28-layer backbone decode over the static KV cache (StaticBackbone.forward)
-> cb0 head + sampler (Cb0Sampler.run) -> depth levels 1..31 with sampling + feedback embedding (FastDepth.run)
-> the 32 codes of every row into an int32 device ring [depth, seats, 32] -> feedback[slots] = next input.
This joins what the engine's tick runs as separate graphs plus eager cb0 kernels (maya3/engine.py:538-556):
no host work, no synchronisation and no allocation between the stages. A depth built in another dtype than the
backbone (the engine's default depth is fp16, maya3/engine.py:53,192-199) gets the hidden state converted on the
way in; the feedback comes back in the backbone's dtype.
"""
from __future__ import annotations

import torch

from . import ops
from ._lib import lib
from .staging import capture, check_slots

N_CODEBOOKS = 32


class _FrameGraph:
    """Buffers of one (batch, context) frame, its graph, and the seats staged on it."""
    __slots__ = ("bufs", "graph", "ctx", "seats")

    def __init__(self, bufs, ctx):
        self.bufs, self.ctx, self.graph, self.seats = bufs, ctx, None, ()

    def __getitem__(self, key):  # ('bufs', 'graph', 'last') as a mapping, for callers that index the graph record
        return {"bufs": self.bufs, "graph": self.graph, "last": self.seats}[key]


class FrameStep:
    def __init__(self, backbone, cb0, depth, ring_depth=64, guard=None):
        """backbone: m3x StaticBackbone; cb0: Cb0Sampler; depth: m3x FastDepth (any of its dtypes); guard: an
        optional m3x.guards.LoopGuard. With it each frame appends the seats' cb0 codes to their device histories
        and writes each seat's loop-guard code (0, -1 stall, p period) to the buffer set's `loop`
        (maya3/engine.py:585-617 evaluates the rule on the host after the tick's copy)."""
        lib()
        self.bb, self.cb0, self.depth, self.guard = backbone, cb0, depth, guard
        dev = backbone.device
        S = backbone.max_slots
        self.feedback = torch.zeros(S + 1, backbone.hidden, dtype=backbone.dtype, device=dev)
        self.ring = torch.zeros(ring_depth, S, N_CODEBOOKS, dtype=torch.int32, device=dev)
        self.ring_head = torch.zeros(1, dtype=torch.int32, device=dev)
        self.graphs = {}
        self.pool = None

    def make_buffers(self, B, ctx):
        dev, dt = self.bb.device, self.bb.dtype
        bb = self.bb.make_buffers(B, ctx)
        codes = torch.zeros(B, N_CODEBOOKS, dtype=torch.int32, device=dev)
        cb = self.cb0.make_buffers(B, h=bb.out, codes=codes)
        same = self.depth.dtype == dt
        dp = self.depth.make_buffers(B, h=bb.out if same else None, codes=codes)
        # every stage reads the backbone's slot column
        cb.slots = dp.slots = bb.slots
        cb.loop = torch.zeros(B, dtype=torch.int32, device=dev)
        dp.fb_back = None if dp.feedback.dtype == dt else torch.empty(B, self.bb.hidden, dtype=dt, device=dev)
        return bb, cb, dp, codes

    def run(self, bufs):
        bb, cb, dp, codes = bufs
        ops.copy_rows(self.feedback, bb.x, src_idx=bb.slots)
        self.bb.forward(bb)
        self.cb0.run(cb)
        if self.guard is not None:
            self.guard.push(bb.slots, cb.cb0)
            self.guard.detect(bb.slots, cb.loop)
        if dp.h is not bb.out:
            ops.cast_rows(bb.out, dp.h)
        self.depth.run(dp)
        if self.bb._persistent_ok(bb.rows):
            # a one-row backbone run that lost a step's input voids the frame's codes (the readout raises on them)
            ops.depth_run_void(self.bb._run_sync, codes, bb.rows, 0, N_CODEBOOKS)
        ops.code_ring_write(codes, self.ring, self.ring_head, bb.rows)
        fb = dp.feedback if dp.fb_back is None else ops.cast_rows(dp.feedback, dp.fb_back)
        ops.copy_rows(fb, self.feedback, dst_idx=bb.slots)

    @torch.inference_mode()
    def capture(self, B, ctx, use_graph=True):
        key = (B, ctx)
        g = self.graphs.get(key)
        if g is not None:
            return g
        g = _FrameGraph(self.make_buffers(B, ctx), ctx)
        if use_graph:
            if self.pool is None:
                self.pool = torch.cuda.graph_pool_handle()
            # the warm-up and capture runs see only the dummy slot; every per-slot counter they move is put back
            state = [self.bb.lengths, self.cb0.ctr_t, self.cb0.hist_t, self.cb0.frames_t, self.cb0.hazard_t,
                     self.depth.row_ctr, self.ring_head]
            if self.guard is not None:
                state += [self.guard.hist, self.guard.frames]
            g.graph = capture(lambda: self.run(g.bufs), self.pool, warm=1, keep=state)
            torch.cuda.synchronize()
        self.graphs[key] = g
        return g

    def _check_room(self, g, seats):
        """Every staged seat must have room for one more position in the graph's context bucket and the cache."""
        room = min(g.ctx, self.bb.capacity)
        for s in seats:
            if self.bb.lengths_cpu[s] + 1 > room:
                raise ValueError(f'slot {s}: context {self.bb.lengths_cpu[s] + 1} exceeds the frame graph\'s '
                                 f'{room} positions')

    @torch.inference_mode()
    def set_slots(self, g, slots):
        """Stage the seats of graph g (padded with the dummy slot); every replay then advances each seat's length
        by one, on the device and in the backbone's host lengths."""
        bb = g.bufs[0]
        seats = tuple(int(s) for s in slots)
        if len(seats) > bb.rows:
            raise ValueError(f'{len(seats)} seats exceed the graph batch {bb.rows}')
        check_slots(seats, self.bb.max_slots)
        self._check_room(g, seats)
        bb.table.stage(dict(slot=seats, real=[1] * len(seats)), key=('frame', seats))
        g.seats = seats

    def replay(self, g):
        self._check_room(g, g.seats)
        if g.graph is not None:
            g.graph.replay()
        else:
            self.run(g.bufs)
        for s in g.seats:
            self.bb.lengths_cpu[s] += 1

    def codes(self, g):
        return g.bufs[3]

    def readout(self, g, rd, B=None, pcm=None):
        """Starts the tick's one host copy (m3x.tick.TickReadout rd, built with nq = 32 and with_loop = whether
        this frame has a guard): stop codes, cb0, loop codes, the 32 codes of the first B rows, and the seats'
        PCM rows if given (maya3/engine.py:558-563). B defaults to the staged seats. rd.wait() raises
        RuntimeError when the depth's persistent run failed this frame (its codes are voided to -1)."""
        bb, cb, dp, codes = g.bufs
        B = len(g.seats) if B is None else int(B)
        if pcm is not None and pcm.shape[0] < B:
            raise ValueError(f'pcm has {pcm.shape[0]} rows for {B} seats')
        rd.pack(cb.stop[:B], cb.cb0[:B], cb.loop[:B] if self.guard is not None else None, codes[:B],
                None if pcm is None else pcm[:B])
