"""One Maya3 frame step for a batch of decoding seats, captured as a single hipGraph.

Replay = x = feedback[slots] -> 28-layer backbone decode over the static KV cache (StaticBackbone.forward)
-> cb0 head + sampler (Cb0Sampler.run) -> depth levels 1..31 with sampling + feedback embedding (FastDepth.run)
-> the 32 codes of every row into an int32 device ring [depth, seats, 32] -> feedback[slots] = next input.
This joins what the engine's tick runs as separate graphs plus eager cb0 kernels (maya3/engine.py:538-556):
no host work, no synchronisation and no allocation between the stages.
"""
from __future__ import annotations

import torch

from . import ops
from ._lib import lib

N_CODEBOOKS = 32


class FrameStep:
    def __init__(self, backbone, cb0, depth, ring_depth=64, guard=None):
        """backbone: m3x StaticBackbone; cb0: Cb0Sampler; depth: m3x FastDepth (same dtype as the backbone);
        guard: an optional m3x.guards.LoopGuard. With it each frame appends the seats' cb0 codes to their device
        histories and writes each seat's loop-guard code (0, -1 stall, p period) to the buffer set's `loop`
        (maya3/engine.py:585-617 evaluates the rule on the host after the tick's copy)."""
        lib()
        if depth.dtype != backbone.dtype:
            raise ValueError('the frame graph runs the depth in the backbone dtype')
        self.bb, self.cb0, self.depth, self.guard = backbone, cb0, depth, guard
        dev = backbone.device
        S = backbone.max_slots
        self.feedback = torch.zeros(S + 1, backbone.hidden, dtype=backbone.dtype, device=dev)
        self.ring = torch.zeros(ring_depth, S, N_CODEBOOKS, dtype=torch.int32, device=dev)
        self.ring_head = torch.zeros(1, dtype=torch.int32, device=dev)
        self.graphs = {}
        self.pool = None

    def make_buffers(self, B, ctx):
        bb = self.bb.make_buffers(B, ctx)
        bb.real.fill_(0)
        codes = torch.zeros(B, N_CODEBOOKS, dtype=torch.int32, device=self.bb.device)
        cb = self.cb0.make_buffers(B, h=bb.out, codes=codes)
        dp = self.depth.make_buffers(B, h=bb.out, codes=codes)
        # one slot index tensor for every stage
        cb.slots = bb.slots
        dp.slots = bb.slots
        cb.loop = torch.zeros(B, dtype=torch.int32, device=self.bb.device)
        return bb, cb, dp, codes

    def run(self, bufs):
        bb, cb, dp, codes = bufs
        ops.copy_rows(self.feedback, bb.x, src_idx=bb.slots)
        self.bb.forward(bb)
        self.cb0.run(cb)
        if self.guard is not None:
            self.guard.push(bb.slots, cb.cb0)
            self.guard.detect(bb.slots, cb.loop)
        self.depth.run(dp)
        ops.code_ring_write(codes, self.ring, self.ring_head, bb.rows)
        ops.copy_rows(dp.feedback, self.feedback, dst_idx=bb.slots)

    @torch.inference_mode()
    def capture(self, B, ctx, use_graph=True):
        key = (B, ctx)
        if key in self.graphs:
            return self.graphs[key]
        bufs = self.make_buffers(B, ctx)
        g = {'bufs': bufs, 'graph': None, 'last': None}
        if use_graph:
            # warm-up replays touch only the dummy slot; restore every per-slot counter they move
            state = [self.bb.lengths, self.cb0.ctr_t, self.cb0.hist_t, self.cb0.frames_t, self.cb0.hazard_t,
                     self.depth.row_ctr, self.ring_head] + ([self.guard.hist, self.guard.frames]
                                                            if self.guard is not None else [])
            saved = [t.clone() for t in state]
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                self.run(bufs)
            torch.cuda.current_stream().wait_stream(stream)
            if self.pool is None:
                self.pool = torch.cuda.graph_pool_handle()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=self.pool, stream=stream):
                self.run(bufs)
            torch.cuda.synchronize()
            for t, v in zip(state, saved):
                t.copy_(v)
            g['graph'] = graph
        self.graphs[key] = g
        return g

    @torch.inference_mode()
    def set_slots(self, g, slots):
        """Stage the seat list of graph g (padded with the dummy slot); lengths advance by one per real row."""
        bb = g['bufs'][0]
        B = len(slots)
        if B > bb.rows:
            raise ValueError(f'{B} seats exceed the graph batch {bb.rows}')
        if len(set(slots)) != B:
            raise ValueError('duplicate slots in one step')
        for s in slots:
            if not 0 <= s < self.bb.max_slots:
                raise IndexError(s)
        pad = list(slots) + [self.bb.dummy] * (bb.rows - B)
        bb.slots.copy_(torch.tensor(pad, dtype=torch.long))
        bb.real.copy_(torch.tensor([1] * B + [0] * (bb.rows - B), dtype=torch.long))
        g['last'] = tuple(slots)

    def replay(self, g):
        if g['graph'] is not None:
            g['graph'].replay()
        else:
            self.run(g['bufs'])

    def codes(self, g):
        return g['bufs'][3]

    def readout(self, g, rd, B=None, pcm=None):
        """Starts the tick's one host copy (m3x.tick.TickReadout rd, built with nq = 32 and with_loop = whether
        this frame has a guard): stop codes, cb0, loop codes, the 32 codes of the first B rows, and the seats' PCM
        rows if given (maya3/engine.py:558-563)."""
        bb, cb, dp, codes = g['bufs']
        B = bb.rows if B is None else B
        rd.pack(cb.stop[:B], cb.cb0[:B], cb.loop[:B] if self.guard is not None else None, codes[:B],
                None if pcm is None else pcm[:B])
