"""The persistent depth run (m3x_depth_run: every level that continues a weight group in one kernel, the residual
stream and each (seat, head)'s K/V kept in LDS across the codebooks, steps handed over in LL words) against the
oracle and against the per-step launch path, on the GPU."""
import numpy as np
import pytest
import torch

from helpers import bf16_bits, close, convert, floor_check, report
from m3x import synth
from oracle import coracle as C
from oracle import torch_oracle as O

pytestmark = pytest.mark.gpu


def _eager(fd, B, slots, h, cb0, persistent):
    fd.persistent = persistent
    b = fd.make_buffers(B)
    b.slots.copy_(torch.tensor(slots))
    b.h.copy_(h)
    b.codes[:, 0].copy_(cb0)
    ctr = fd.row_ctr.clone()
    trace = []
    fd.run(b, trace=trace)
    torch.cuda.synchronize()
    fd.row_ctr.copy_(ctr)
    return b.codes.cpu().long(), b.feedback.cpu(), torch.stack([t.cpu() for t in trace], 1), b.u.cpu()


def _check_vs_oracle(label, model_c, h, cb0, codes, fb, logits, u, temp, top_k, dt, cross=None):
    for lv in range(1, 32):
        ref = C.topk_sample_rows(bf16_bits(logits[:, lv - 1]), 1.0 / temp, top_k, u[:, lv - 1].numpy(),
                                 is_f16=dt == torch.float16)
        assert np.array_equal(codes[:, lv].numpy(), ref), (label, lv)
    _, ref_l = O.depth_frame(model_c, h, cb0, u, temp, top_k, forced=codes, cross=cross, dt=dt)
    _, tru_l = O.depth_frame(convert(model_c, torch.float32), h.float(), cb0, u, temp, top_k, forced=codes,
                             cross=None if cross is None else cross.float(), dt=torch.float32)
    ok, info = floor_check(logits, ref_l, tru_l)
    report(f"{label} logits", info)
    assert ok, info
    ok, info = close(fb, O.feedback(model_c.audio_in, codes).float())
    assert ok, info


@pytest.mark.parametrize("B", [1, 5, 16])
def test_swiglu_run_matches_oracle_and_launch_path(gpu, B):
    """SwiGLU/RMSNorm trunk (levels 2..31 in one persistent kernel): every code equals the oracle sampler on the
    run's own logits and uniforms, the logits sit at the bf16 floor of the teacher-forced oracle, the feedback
    matches, no step's input went missing, and the logits agree with the launch path's within the same floor."""
    from m3x.serve.fast_depth import FastDepth
    model_g = synth.swiglu_depth(seed=611, device=gpu, affine=synth.AFFINE)
    model_c = synth.swiglu_depth(seed=611, device="cpu", affine=synth.AFFINE)
    fd = FastDepth(model_g, 20, dtype=torch.bfloat16, temp=0.9, top_k=50, batch_buckets=(B,))
    fd.PERSISTENT_SEATS = 16  # the kernel's own limit (serving switches to the launch path above 4 seats)
    fd.row_seed.copy_(torch.arange(21, dtype=torch.int32, device=gpu) * 7777 + 3)
    g = torch.Generator().manual_seed(612 + B)
    h = torch.randn(B, 1024, generator=g).to(torch.bfloat16)
    cb0 = torch.randint(0, 2048, (B,), generator=g)
    slots = list(range(3, 3 + B))
    assert fd._persistent_ok(B, 0)
    codes, fb, logits, u = _eager(fd, B, slots, h, cb0, True)
    assert not fd.run_error()
    _check_vs_oracle(f"persistent B={B}", model_c, h, cb0, codes, fb, logits, u, 0.9, 50, torch.bfloat16)
    # the launch path on the same inputs, teacher-forced to the persistent run's codes through the oracle bar
    codes2, _, logits2, u2 = _eager(fd, B, slots, h, cb0, False)
    assert torch.equal(u, u2) and torch.equal(codes[:, :2], codes2[:, :2])
    # levels up to the first code that differs (if any) see the same prefix: their logits agree closely
    same = (codes == codes2).all(0)
    first = int(torch.nonzero(~same)[0]) if (~same).any() else 32
    if first > 1:
        ok, info = close(logits[:, :first - 1], logits2[:, :first - 1], atol=2e-2)
        assert ok, info


def test_depthv2_runs_fp16_with_speaker(gpu):
    """The reference's DepthV2 geometry (LayerNorm + GELU, 16 x 64 heads, weight groups whose continuing levels
    form three persistent runs per frame, per-slot speaker constants) in fp16: codes and logits against the
    oracle, no missing input."""
    from m3x.serve.fast_depth import FastDepth
    gol = [None] + [0] * 3 + [1] * 8 + [2] * 20
    mk = lambda dev: synth.depthv2_like(group_of_level=gol, seed=621, device=dev, affine_std=0.1)  # noqa: E731
    model_g, model_c = mk(gpu), mk("cpu")
    B = 6
    fd = FastDepth(model_g, 8, dtype=torch.float16, temp=0.7, top_k=64, batch_buckets=(B,))
    fd.PERSISTENT_SEATS = 16  # the kernel's own limit: the run is tested past the seats serving gives it
    g = torch.Generator().manual_seed(622)
    mems = torch.randn(8, 1, 1, 1024, generator=g)
    for s in range(8):
        fd.set_speaker(s, mems[s].to(gpu), torch.ones(1, 1, device=gpu))
    fd.row_seed.copy_(torch.arange(9, dtype=torch.int32, device=gpu) * 131 + 5)
    h = torch.randn(B, 1024, generator=g).to(torch.float16)
    cb0 = torch.randint(0, 2048, (B,), generator=g)
    slots = [7, 0, 2, 5, 1, 6]
    assert fd._persistent_ok(B, 0) and fd._persistent_ok(B, 2)
    codes, fb, logits, u = _eager(fd, B, slots, h, cb0, True)
    assert not fd.run_error()
    cross = fd.cross_const[slots].cpu()
    _check_vs_oracle("persistent DepthV2 fp16", model_c, h, cb0, codes, fb, logits, u, 0.7, 64, torch.float16,
                     cross=cross)


def test_run_graph_replays_equal_eager(gpu):
    """Graph replays of a frame with a persistent run (the kernel's epoch moves every launch, so the LL tags of
    one replay never match another's) equal eager runs bit for bit, replay after replay."""
    from m3x.serve.fast_depth import FastDepth
    model_g = synth.swiglu_depth(seed=631, device=gpu, affine=synth.AFFINE)
    fd = FastDepth(model_g, 8, dtype=torch.bfloat16, temp=0.9, top_k=50, batch_buckets=(4,))
    fd.row_seed.copy_(torch.arange(9, dtype=torch.int32, device=gpu) * 7919 + 1)
    g = torch.Generator().manual_seed(632)
    h = torch.randn(3, 1024, generator=g).to(torch.bfloat16).to(gpu)
    cb0 = torch.randint(0, 2048, (3,), generator=g).to(gpu)
    fd.warmup()
    ctr = fd.row_ctr.clone()
    outs = [fd([5, 2, 7], h, cb0) for _ in range(4)]
    fd.row_ctr.copy_(ctr)
    eager = [fd._fn(torch.tensor([5, 2, 7], device=gpu), h, cb0) for _ in range(4)]
    torch.cuda.synchronize()
    assert not fd.run_error()
    for (c, f), (ce, fe) in zip(outs, eager):
        assert torch.equal(c, ce) and torch.equal(f, fe)
    assert not torch.equal(outs[0][0], outs[1][0])


def test_run_failure_is_surfaced(gpu):
    """A run whose bounded waits give up, forced from the host with a spin limit of one polling round (every
    workgroup still exits normally: a failed wait skips the rest of the run), sets the error word; the run's
    levels come back as code -1; the tick readout that carries the codes raises RuntimeError, and so does the next
    call of FastDepth._fn / __call__ (the host sees the word without a synchronisation). After clear_run_error()
    with the default limit, the next frame equals a run that never failed (the kernel's epoch moved on, so no stale
    handover word is taken)."""
    from m3x.serve.fast_depth import FastDepth
    from m3x.tick import TickReadout
    model_g = synth.swiglu_depth(seed=641, device=gpu, affine=synth.AFFINE)
    fd = FastDepth(model_g, 8, dtype=torch.bfloat16, temp=0.9, top_k=50, batch_buckets=(4,))
    fd.row_seed.copy_(torch.arange(9, dtype=torch.int32, device=gpu) * 613 + 9)
    g = torch.Generator().manual_seed(642)
    B, slots = 3, [4, 1, 6]
    h = torch.randn(B, 1024, generator=g).to(torch.bfloat16).to(gpu)
    cb0 = torch.randint(0, 2048, (B,), generator=g).to(gpu)
    assert fd._persistent_ok(B, 0)
    ref = _eager(fd, B, slots, h, cb0, True)
    assert not fd.run_error()
    ctr = fd.row_ctr.clone()
    fd.spin_limit = 1
    fd._fn(torch.tensor(slots, device=gpu), h, cb0)
    torch.cuda.synchronize()
    assert fd.run_error()
    with pytest.raises(RuntimeError):
        fd._fn(torch.tensor(slots, device=gpu), h, cb0)
    fd.row_ctr.copy_(ctr)
    b = fd.make_buffers(B)
    b.slots.copy_(torch.tensor(slots))
    b.h.copy_(h)
    b.codes[:, 0].copy_(cb0)
    fd.run(b)
    torch.cuda.synchronize()
    fd.row_ctr.copy_(ctr)
    codes = b.codes.cpu()
    assert (codes[:, 2:] == -1).all() and torch.equal(codes[:, 0], cb0.cpu().int())
    rd = TickReadout(8, frame=0, nq=32, device=gpu)
    rd.pack(torch.zeros(B, dtype=torch.int64, device=gpu), cb0.long(), codes=b.codes)
    with pytest.raises(RuntimeError):
        rd.wait()
    # the graph path (captured with the limit of one round) raises at the call after a failed replay
    fd.warmup()
    fd(slots, h, cb0)
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError):
        fd(slots, h, cb0)
    fd.row_ctr.copy_(ctr)
    # recovery
    fd.spin_limit = 0
    fd.clear_run_error()
    again = _eager(fd, B, slots, h, cb0, True)
    assert not fd.run_error()
    assert torch.equal(again[0], ref[0]) and torch.equal(again[1], ref[1]) and torch.equal(again[2], ref[2])
