"""The whole frame (backbone -> cb0 -> depth -> code ring -> feedback) as one hipGraph: replays match the eager
composition bit for bit, the codes land in the ring, lengths and per-slot streams advance once per frame, and
the cb0 codes equal the C-oracle sampler on the frame's own cb0 logits and uniform."""
import numpy as np
import pytest
import torch

from helpers import bf16_bits
from m3x import synth
from oracle import coracle as C

pytestmark = pytest.mark.gpu

S, CAP = 8, 256


def _frame(gpu, seed=61):
    from m3x.cb0 import Cb0Sampler
    from m3x.frame import FrameStep
    from m3x.serve.fast_backbone import StaticBackbone
    from m3x.serve.fast_depth import FastDepth
    bb = synth.qwen3_backbone(layers=2, seed=seed, device=gpu, affine=synth.AFFINE)
    sb = StaticBackbone(bb, S, capacity=CAP, batch_buckets=(4,), ctx_buckets=(CAP,), attention="triton",
                        fuse_rope=True)
    cb = Cb0Sampler(bb.cb0_head.weight, S, temp=0.9, top_k=50, rep=0.0)
    fd = FastDepth(synth.swiglu_depth(seed=seed + 1, device=gpu, affine=synth.AFFINE), S, dtype=torch.bfloat16, temp=0.9, top_k=50,
                   batch_buckets=(4,), fused=True)
    g = torch.Generator().manual_seed(seed + 2)
    lengths = [17, 0, 120, 3, 0, 64, 0, 0]
    with torch.inference_mode():
        _fill(sb, cb, fd, g, lengths)
    fs = FrameStep(sb, cb, fd, ring_depth=4)
    with torch.inference_mode():
        fs.feedback[:S].copy_(torch.randn(S, 1024, generator=g).to(torch.bfloat16))
    return fs


def _fill(sb, cb, fd, g, lengths):
    for i in range(2):
        sb.k[i][:S].copy_(torch.randn(S, 8, CAP, 128, generator=g).to(torch.bfloat16))
        sb.v[i][:S].copy_(torch.randn(S, 8, CAP, 128, generator=g).to(torch.bfloat16))
    sb.lengths[:S].copy_(torch.tensor(lengths))
    sb.lengths_cpu[:S] = lengths
    for s in range(S):
        cb.bind(s, seed=1000 + s)
    fd.row_seed.copy_(torch.arange(S + 1, dtype=torch.int32) * 31 + 7)


def test_frame_graph_equals_eager(gpu):
    a, b = _frame(gpu), _frame(gpu)
    ga = a.capture(4, CAP, use_graph=True)
    gb = b.capture(4, CAP, use_graph=False)
    slots = [2, 0, 5]
    a.set_slots(ga, slots)
    b.set_slots(gb, slots)
    for frame in range(3):
        a.replay(ga)
        b.replay(gb)
        torch.cuda.synchronize()
        # real rows only: the padding row runs the dummy slot, whose state is scratch by design
        assert torch.equal(a.codes(ga)[:3], b.codes(gb)[:3]), frame
        assert torch.equal(a.feedback[slots], b.feedback[slots]) and torch.equal(a.ring[:, :3], b.ring[:, :3])
    assert a.ring_head.item() == 3 and torch.equal(a.ring[2, :4], a.codes(ga))
    assert a.bb.lengths[:S].tolist() == [20, 0, 123, 3, 0, 67, 0, 0]
    assert a.cb0.ctr_t[[2, 0, 5]].tolist() == [3, 3, 3] and a.depth.row_ctr[[2, 0, 5]].tolist() == [3, 3, 3]
    assert a.cb0.ctr_t[1].item() == 0 and a.depth.row_ctr[1].item() == 0
    codes = a.codes(ga)[:3].cpu()
    assert codes.min() >= 0 and codes.max() < 2048


def test_frame_cb0_matches_oracle_sampler(gpu):
    fs = _frame(gpu, seed=71)
    g = fs.capture(4, CAP, use_graph=False)
    fs.set_slots(g, [1, 4, 6, 7])
    ctr0 = fs.cb0.ctr_t.cpu().clone()
    fs.replay(g)
    torch.cuda.synchronize()
    bbuf, cbuf, _, codes = g['bufs']
    logits = bf16_bits(cbuf.logits)
    for b, s in enumerate([1, 4, 6, 7]):
        u = C.philox_uniform(1000 + s, int(ctr0[s]), 0)
        assert u == cbuf.u[b, 0].item()
        ref, _ = C.cb0_sample(logits[b], -1, 0.9, 50, 0.0, 0.0, None, None, 0, None, None, u)
        assert ref == codes[b, 0].item() == cbuf.cb0[b].item()


def test_frame_loop_guard_in_graph(gpu):
    """With a LoopGuard, every replay appends the seats' cb0 codes to their device histories, counts the frame and
    writes each seat's loop code; the histories equal the cb0 column of the code ring and the codes equal the
    oracle's rule (maya3/guards.py:80-107) on those histories."""
    from types import SimpleNamespace
    from m3x.guards import LoopGuard
    from oracle import torch_oracle as O
    fs = _frame(gpu, seed=71)
    cfg = SimpleNamespace(stall=4, period_win=8, period_thr=0.5, pmin=2, pmax=4, hist=12)
    fs.guard = LoopGuard(S, cfg, device=gpu)
    slots = [2, 0, 5]
    with torch.inference_mode():
        g = fs.capture(4, CAP)
        fs.set_slots(g, slots)
        seen = {s: [] for s in slots}
        for t in range(16):
            fs.replay(g)
            torch.cuda.synchronize()
            cb0 = fs.codes(g)[:, 0].cpu().tolist()
            for i, s in enumerate(slots):
                seen[s].append(cb0[i])
            loop = g['bufs'][1].loop[:3].cpu().tolist()
            W = np.full((3, 12), -1)
            for i, s in enumerate(slots):
                h = seen[s][-12:]
                W[i, 12 - len(h):] = h
            want = O.loop_detect_batch(W, np.full(3, t + 1), 4, 8, 0.5, 2, 4)
            got = [None if c == 0 else ("stall" if c < 0 else f"period:{c}") for c in loop]
            assert got == want, t
        hist = fs.guard.hist.cpu().numpy()
        for i, s in enumerate(slots):
            assert hist[s].tolist() == seen[s][-12:]
        assert fs.guard.frames[slots].cpu().tolist() == [16] * 3


def test_frame_readout_matches_buffers(gpu):
    """FrameStep.readout copies the frame's stop codes, cb0 and 32 codes (and PCM rows given by the caller) to the
    host in one transfer, equal to the graph's own buffers."""
    from m3x.tick import TickReadout
    fs = _frame(gpu, seed=81)
    rd = TickReadout(4, frame=1920, nq=32, with_loop=False, device=gpu)
    with torch.inference_mode():
        g = fs.capture(4, CAP)
        fs.set_slots(g, [1, 6])
        fs.replay(g)
        pcm = torch.rand(4, 1920, device=gpu) * 2.4 - 1.2
        fs.readout(g, rd, B=2, pcm=pcm)
        got = rd.wait()
        bb, cb, dp, codes = g['bufs']
        assert got["cb0"].tolist() == cb.cb0[:2].cpu().tolist()
        assert got["stop"].tolist() == cb.stop[:2].cpu().tolist()
        assert np.array_equal(got["codes"], codes[:2].cpu().numpy())
        assert np.array_equal(got["pcm"], (pcm[:2].cpu().clamp(-1, 1) * 32767).round().to(torch.int16).numpy())
