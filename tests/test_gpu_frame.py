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
    bb = synth.qwen3_backbone(layers=2, seed=seed, device=gpu)
    sb = StaticBackbone(bb, S, capacity=CAP, batch_buckets=(4,), ctx_buckets=(CAP,), attention="triton",
                        fuse_rope=True)
    cb = Cb0Sampler(bb.cb0_head.weight, S, temp=0.9, top_k=50, rep=0.0)
    fd = FastDepth(synth.swiglu_depth(seed=seed + 1, device=gpu), S, dtype=torch.bfloat16, temp=0.9, top_k=50,
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
