"""The one-row backbone step as one persistent kernel (m3x_backbone_run: all layers in one launch, the steps handed
over in LL words) against the gather-path oracle, the launch path and its own graph replays, on the GPU."""
import numpy as np
import pytest
import torch

from helpers import close, convert, floor_check, report
from m3x import synth
from oracle import torch_oracle as O

pytestmark = pytest.mark.gpu

CAP = 4096


def _setup(gpu, layers, lengths, seed, persistent=True, use_graphs=True):
    """StaticBackbone over len(lengths) slots with random caches up to the given lengths (the same on the CPU)."""
    from m3x.serve.fast_backbone import StaticBackbone
    bb_g = synth.qwen3_backbone(layers=layers, seed=seed, device=gpu, affine=synth.AFFINE)
    bb_c = synth.qwen3_backbone(layers=layers, seed=seed, device="cpu", affine=synth.AFFINE)
    S = len(lengths)
    sb = StaticBackbone(bb_g, S, capacity=CAP, batch_buckets=(1, 2), ctx_buckets=(CAP,), attention="triton",
                        fuse_rope=True, use_graphs=use_graphs)
    sb.persistent = persistent
    g = torch.Generator().manual_seed(seed + 1)
    ctx = max(lengths) + 8
    kc = [torch.zeros(S + 1, 8, ctx, 128, dtype=torch.bfloat16) for _ in range(layers)]
    vc = [torch.zeros(S + 1, 8, ctx, 128, dtype=torch.bfloat16) for _ in range(layers)]
    for s, n in enumerate(lengths):
        kv = []
        for i in range(layers):
            k = torch.randn(1, 8, n, 128, generator=g).to(torch.bfloat16)
            v = torch.randn(1, 8, n, 128, generator=g).to(torch.bfloat16)
            kc[i][s, :, :n], vc[i][s, :, :n] = k[0], v[0]
            kv.append((k.to(gpu), v.to(gpu)))
        sb.load_prefix(s, kv, n)
    return sb, bb_c, kc, vc


def _oracles(bb_c, kc, vc, lengths):
    L = torch.tensor(list(lengths) + [0])
    ctx = kc[0].shape[2]
    c16, s16 = O.rope_tables(128, 1e6, ctx, torch.bfloat16)
    T = dict(bb=convert(bb_c, torch.float32), kc=[t.float() for t in kc], vc=[t.float() for t in vc], L=L.clone(),
             c=c16.float(), s=s16.float())
    return L, c16, s16, T


@pytest.mark.parametrize("layers,lengths", [(3, [0, 1, 37, 200, 1000, 4000]), (28, [2047, 4094])])
def test_one_row_run_matches_oracle(gpu, layers, lengths):
    """One-row steps of every slot in turn (positions 0 .. 4095: a single key, split boundaries, the longest
    context), two steps each: the hidden state and every layer's new K/V rows at the bf16 floor of the oracle,
    the lengths advanced, nothing else in the caches touched."""
    sb, bb_c, kc, vc = _setup(gpu, layers, lengths, 700 + layers)
    assert sb._persistent_ok(1)
    L, c16, s16, T = _oracles(bb_c, kc, vc, lengths)
    g = torch.Generator().manual_seed(701)
    before_k = [sb.k[i].clone() for i in range(layers)]
    for step in range(2):
        for s in range(len(lengths)):
            x = torch.randn(1, 1024, generator=g).to(torch.bfloat16)
            out = sb.step([s], x.to(gpu))
            ref = O.backbone_step(bb_c, kc, vc, L, torch.tensor([s]), x, c16, s16)
            truth = O.backbone_step(T["bb"], T["kc"], T["vc"], T["L"], torch.tensor([s]), x.float(), T["c"], T["s"])
            ok, info = floor_check(out, ref, truth)
            report(f"one-row run, {layers} layers, slot {s} at {int(L[s]) - 1}, step {step}", info)
            assert ok, (s, step, info)
    assert not sb.run_error()
    assert sb.lengths.cpu().tolist() == L.tolist() == sb.lengths_cpu
    for i in range(layers):
        for s, n in enumerate(lengths):
            for name, got, ref, tr in (("k", sb.k[i], kc[i], T["kc"][i]), ("v", sb.v[i], vc[i], T["vc"][i])):
                ok, info = floor_check(got[s, :, n:n + 2], ref[s, :, n:n + 2], tr[s, :, n:n + 2])
                assert ok, (name, i, s, info)
            # the prefix and the positions past the new ones are untouched
            assert torch.equal(sb.k[i][s, :, :n].cpu(), kc[i][s, :, :n])
            assert torch.equal(sb.k[i][s, :, n + 2:], before_k[i][s, :, n + 2:])
        assert torch.equal(sb.k[i][len(lengths)], before_k[i][len(lengths)])  # the dummy slot


def test_one_row_run_against_launch_path(gpu):
    """The persistent run and the launch path on the same inputs: both at the bf16 floor of the oracle, and no
    further from each other than two bf16 paths that sum in different orders (relative L2 within twice the floor)."""
    from helpers import rel_l2
    lengths = [300, 2500]
    a, bb_c, kc, vc = _setup(gpu, 4, lengths, 710, persistent=True)
    b, _, _, _ = _setup(gpu, 4, lengths, 710, persistent=False)
    L, c16, s16, T = _oracles(bb_c, kc, vc, lengths)
    g = torch.Generator().manual_seed(711)
    for t in range(3):
        for s in range(2):
            x = torch.randn(1, 1024, generator=g).to(torch.bfloat16)
            ya, yb = a.step([s], x.to(gpu)), b.step([s], x.to(gpu))
            ref = O.backbone_step(bb_c, kc, vc, L, torch.tensor([s]), x, c16, s16)
            truth = O.backbone_step(T["bb"], T["kc"], T["vc"], T["L"], torch.tensor([s]), x.float(), T["c"], T["s"])
            for y in (ya, yb):
                ok, info = floor_check(y, ref, truth)
                assert ok, (t, s, info)
            assert rel_l2(ya, yb) <= 2 * rel_l2(ref, truth), (t, s)
    for i in range(4):
        for s, n in enumerate(lengths):
            for ca, cb in ((a.k[i], b.k[i]), (a.v[i], b.v[i])):
                tr = (T["kc"] if ca is a.k[i] else T["vc"])[i][s, :, n:n + 3]
                ok, info = floor_check(ca[s, :, n:n + 3], cb[s, :, n:n + 3], tr)
                assert ok, (i, s, info)


def test_one_row_run_graph_replays_equal_eager(gpu):
    """Graph replays of the one-row step (the kernel's epoch moves every launch, so one replay never takes another's
    handover words) equal eager runs bit for bit, step after step."""
    lengths = [500, 900]
    a, _, _, _ = _setup(gpu, 3, lengths, 720, use_graphs=True)
    b, _, _, _ = _setup(gpu, 3, lengths, 720, use_graphs=False)
    g = torch.Generator().manual_seed(721)
    for t in range(4):
        x = torch.randn(1, 1024, generator=g).to(torch.bfloat16).to(gpu)
        ya, yb = a.step([t % 2], x), b.step([t % 2], x)
        assert torch.equal(ya, yb), t
    torch.cuda.synchronize()
    for i in range(3):
        assert torch.equal(a.k[i], b.k[i]) and torch.equal(a.v[i], b.v[i])


def test_one_row_run_failure_is_surfaced(gpu):
    """A run whose bounded waits give up (a spin limit of one polling round, forced from the host; every workgroup
    still exits) sets the error word; the next step raises RuntimeError; a frame graph over that backbone voids its
    codes to -1, which its tick readout refuses. After clear_run_error() with the default limit the step is whole
    again."""
    from m3x.cb0 import Cb0Sampler
    from m3x.frame import FrameStep
    from m3x.serve.fast_depth import FastDepth
    from m3x.tick import TickReadout
    lengths = [100, 50]
    sb, _, _, _ = _setup(gpu, 2, lengths, 730, use_graphs=False)
    ref, _, _, _ = _setup(gpu, 2, lengths, 730, use_graphs=False)
    g = torch.Generator().manual_seed(731)
    x = torch.randn(1, 1024, generator=g).to(torch.bfloat16).to(gpu)
    sb.spin_limit = 1
    sb.step([0], x)
    torch.cuda.synchronize()
    assert sb.run_error()
    with pytest.raises(RuntimeError):
        sb.step([1], x)
    # the frame graph at one seat over the failing backbone
    cb = Cb0Sampler(sb.backbone.cb0_head.weight, 2, temp=0.9, top_k=50, rep=0.0)
    fd = FastDepth(synth.swiglu_depth(seed=732, device=gpu, affine=synth.AFFINE), 2, dtype=torch.bfloat16, temp=0.9,
                   top_k=50, batch_buckets=(1,))
    fs = FrameStep(sb, cb, fd, ring_depth=2)
    fr = fs.capture(1, CAP)
    fs.set_slots(fr, [1])
    fs.replay(fr)
    rd = TickReadout(2, frame=0, nq=32, device=gpu)
    fs.readout(fr, rd)
    with pytest.raises(RuntimeError):
        rd.wait()
    assert (fs.codes(fr)[:1] == -1).all()
    # recovery, eager: the step equals a backbone that never failed
    sb.spin_limit = 0
    sb.clear_run_error()
    with torch.inference_mode():
        for s in (0, 1):
            sb.lengths[s] = ref.lengths[s]
            sb.lengths_cpu[s] = ref.lengths_cpu[s]
    y = sb.step([1], x)
    y_ref = ref.step([1], x)
    torch.cuda.synchronize()
    assert not sb.run_error()
    assert torch.equal(y, y_ref)
