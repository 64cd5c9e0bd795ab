"""FastDepth (drop-in of serve/fast_depth.py) on the GPU: sampled codes bit-exact against the C-oracle sampler on
the kernel's own logits and uniforms, logits within bf16 tolerance of the teacher-forced CPU oracle, feedback
within tolerance, graph replay identical to the eager body."""
import numpy as np
import pytest
import torch

from helpers import bf16_bits, close, convert, floor_check, rel_l2, report
from m3x import synth
from oracle import coracle as C
from oracle import torch_oracle as O

pytestmark = pytest.mark.gpu

B = 4
SLOTS = [3, 0, 6, 1]


def _run_eager(fd, h, cb0, gpu):
    b = fd.make_buffers(B)
    b.slots.copy_(torch.tensor(SLOTS))
    b.h.copy_(h.to(gpu))
    b.codes[:, 0].copy_(cb0.to(gpu))
    trace = []
    codes, fb = fd.run(b, trace=trace)
    torch.cuda.synchronize()
    return codes.cpu().long(), fb.cpu(), torch.stack([t.cpu() for t in trace], 1), b.u.cpu()


def _check(fd, model_c, h, cb0, gpu, dt, temp, top_k, cross=None, logit_tol=None):
    seeds = torch.randint(1, 2 ** 31 - 2, (fd.max_slots + 1,), generator=torch.Generator().manual_seed(5),
                          dtype=torch.int32)
    fd.row_seed.copy_(seeds.to(gpu))
    fd.row_ctr.copy_(torch.arange(fd.max_slots + 1, dtype=torch.int32).to(gpu) * 3)
    ctr0 = fd.row_ctr.cpu().clone()
    codes, fb, logits, u = _run_eager(fd, h, cb0, gpu)
    # uniforms: the slot's Philox stream, bit-exact
    ref_u = np.array([[C.philox_uniform(int(seeds[s]), int(ctr0[s]), 1 + j) for j in range(31)] for s in SLOTS],
                     np.float32)
    assert np.array_equal(u.numpy(), ref_u)
    assert (fd.row_ctr.cpu() - ctr0).tolist() == [1 if s in SLOTS else 0 for s in range(fd.max_slots + 1)]
    # sampling: bit-exact given the kernel's logits and uniforms
    for lv in range(1, 32):
        if dt == torch.float32:
            xs = logits[:, lv - 1].numpy() * np.float32(1.0 / temp)
            ref = np.array([C.topk_sample(xs[r], top_k, float(u[r, lv - 1])) for r in range(B)])
        else:
            ref = C.topk_sample_rows(bf16_bits(logits[:, lv - 1]), 1.0 / temp, top_k, u[:, lv - 1].numpy(),
                                     is_f16=dt == torch.float16)
        assert np.array_equal(codes[:, lv].numpy(), ref), lv
    assert torch.equal(codes[:, 0], cb0)
    if dt == torch.float32:
        return _check_f32(model_c, h, cb0, u, temp, top_k, codes, fb, logits, cross)
    # logits: teacher-forced CPU oracle on the same codes, against the fp32 evaluation's noise floor
    _, ref_logits = O.depth_frame(model_c, h, cb0, u, temp, top_k, forced=codes, cross=cross, dt=dt)
    m32 = convert(model_c, torch.float32)
    _, truth = O.depth_frame(m32, h.float(), cb0, u, temp, top_k, forced=codes,
                             cross=None if cross is None else cross.float(), dt=torch.float32)
    ok, info = floor_check(logits, ref_logits, truth)
    report(f"depth logits {dt}, {B} seats x 31 levels", info)
    assert ok, info
    ok, info = close(fb, O.feedback(model_c.audio_in, codes).float())
    report(f"depth feedback {dt}", info)
    assert ok, info
    return codes, fb


# fp32 bar: the kernel and the oracle evaluate the same fp32 math in different summation orders (MFMA 16x16x4
# f32 blocks against torch's CPU matmul), so they differ by fp32 rounding alone, ~sqrt(K) * 2^-24 relative per
# projection over 4 layers x 31 levels; the reference's fp32 FastDepth is its own precision baseline
# (maya3/tests/test_depth_fused.py:30-31).
F32_REL_L2, F32_MAX_ABS = 1e-5, 1e-5


def _check_f32(model_c, h, cb0, u, temp, top_k, codes, fb, logits, cross):
    _, ref_logits = O.depth_frame(model_c, h, cb0, u, temp, top_k, forced=codes, cross=cross, dt=torch.float32)
    err = rel_l2(logits, ref_logits)
    max_abs = (logits.float() - ref_logits.float()).abs().max().item()
    scale = ref_logits.abs().max().item()
    report("fastdepth fp32 logits", dict(rel_l2=err, max_abs=max_abs, max_logit=scale))
    assert err <= F32_REL_L2 and max_abs <= F32_MAX_ABS * max(1.0, scale), (err, max_abs, scale)
    ref_fb = O.feedback(model_c.audio_in, codes).float()
    ok, info = close(fb, ref_fb)
    assert ok, info
    return codes, fb


@pytest.mark.parametrize("affine", [synth.AFFINE, synth.AFFINE_WIDE])
def test_swiglu_depth_frame(gpu, affine):
    """The SwiGLU/RMSNorm trunk with non-unit norm weights: 1 + N(0, 0.1), and a wide log-normal spread
    (about 0.1x to 20x) that tests the folded norm's rounding (the norm weight multiplied into the packed
    weight, then rounded) on weights like trained ones."""
    from m3x.serve.fast_depth import FastDepth
    model_g = synth.swiglu_depth(seed=31, device=gpu, affine=affine)
    model_c = synth.swiglu_depth(seed=31, device="cpu", affine=affine)
    fd = FastDepth(model_g, 8, dtype=torch.bfloat16, temp=0.9, top_k=50, batch_buckets=(B,), fused=True)
    g = torch.Generator().manual_seed(32)
    h = torch.randn(B, 1024, generator=g).to(torch.bfloat16)
    cb0 = torch.randint(0, 2048, (B,), generator=g)
    _check(fd, model_c, h, cb0, gpu, torch.bfloat16, 0.9, 50)


def test_depthv2_geometry_fp16_with_speaker(gpu):
    """The reference's trunk shape: LayerNorm + GELU, 16 heads x 64, several weight groups with group starts and
    incremental levels, per-slot speaker constant (set_speaker), fp16."""
    from m3x.serve.fast_depth import FastDepth
    gol = [None] + [0] * 3 + [1] * 8 + [2] * 20
    mk = lambda dev: synth.depthv2_like(group_of_level=gol, seed=41, device=dev, affine_std=0.1)  # noqa: E731
    model_g, model_c = mk(gpu), mk("cpu")
    fd = FastDepth(model_g, 8, dtype=torch.float16, temp=0.7, top_k=64, batch_buckets=(B,), fused=True)
    g = torch.Generator().manual_seed(42)
    mems = torch.randn(8, 1, 1, 1024, generator=g)
    for s in range(8):
        fd.set_speaker(s, mems[s].to(gpu), torch.ones(1, 1, device=gpu))
    # the per-slot constant against o(v(mem)) on the CPU
    d = model_c.depth
    ref_cross = torch.stack([torch.stack([O.lin(O.lin(mems[s, 0].half(), c.kv.weight.half())[:, 1024:],
                                                c.o.weight.half())[0] for c in d.cross]) for s in range(8)])
    ok, info = close(fd.cross_const[:8], ref_cross.float(), atol=1e-3)
    assert ok, info
    h = torch.randn(B, 1024, generator=g).to(torch.float16)
    cb0 = torch.randint(0, 2048, (B,), generator=g)
    cross = fd.cross_const[SLOTS].cpu()
    _check(fd, model_c, h, cb0, gpu, torch.float16, 0.7, 64, cross=cross)


def test_swiglu_depth_frame_fp32(gpu):
    """FastDepth(dtype=torch.float32): the engine's depth_dtype="fp32" (maya3/engine.py:53,192-199) and the
    reference's own fp32 FastDepth (maya3/tests/test_depth_fused.py:30-31). Launch path, fp32 kernels throughout."""
    from m3x.serve.fast_depth import FastDepth
    model_g = convert(synth.swiglu_depth(seed=33, device=gpu, affine=synth.AFFINE), torch.float32)
    model_c = convert(synth.swiglu_depth(seed=33, device="cpu", affine=synth.AFFINE), torch.float32)
    fd = FastDepth(model_g, 8, dtype=torch.float32, temp=0.9, top_k=50, batch_buckets=(B,), fused=True)
    assert not fd._persistent_ok(B, 0)
    g = torch.Generator().manual_seed(34)
    h = torch.randn(B, 1024, generator=g)
    cb0 = torch.randint(0, 2048, (B,), generator=g)
    _check(fd, model_c, h, cb0, gpu, torch.float32, 0.9, 50)


def test_depthv2_geometry_fp32_with_speaker(gpu):
    """The reference's DepthV2 shape (LayerNorm + GELU, 16 x 64 heads, weight groups with group starts and
    incremental levels, speaker constants) in fp32, as the reference's fp32 FastDepth runs it."""
    from m3x.serve.fast_depth import FastDepth
    gol = [None] + [0] * 3 + [1] * 8 + [2] * 20
    mk = lambda dev: synth.depthv2_like(group_of_level=gol, seed=43, device=dev, affine_std=0.1)  # noqa: E731
    model_g, model_c = mk(gpu), mk("cpu")
    fd = FastDepth(model_g, 8, dtype=torch.float32, temp=0.7, top_k=64, batch_buckets=(B,), fused=True)
    g = torch.Generator().manual_seed(44)
    mems = torch.randn(8, 1, 1, 1024, generator=g)
    for s in range(8):
        fd.set_speaker(s, mems[s].to(gpu), torch.ones(1, 1, device=gpu))
    d = model_c.depth
    ref_cross = torch.stack([torch.stack([O.lin(O.lin(mems[s, 0], c.kv.weight)[:, 1024:], c.o.weight)[0]
                                          for c in d.cross]) for s in range(8)])
    assert rel_l2(fd.cross_const[:8], ref_cross) <= F32_REL_L2
    h = torch.randn(B, 1024, generator=g)
    cb0 = torch.randint(0, 2048, (B,), generator=g)
    cross = fd.cross_const[SLOTS].cpu()
    _check(fd, model_c, h, cb0, gpu, torch.float32, 0.7, 64, cross=cross)


def test_graph_replay_equals_eager(gpu):
    from m3x.serve.fast_depth import FastDepth
    model_g = synth.swiglu_depth(seed=51, device=gpu, affine=synth.AFFINE)
    fd = FastDepth(model_g, 8, dtype=torch.bfloat16, temp=0.9, top_k=50, batch_buckets=(2, 4), fused=True)
    fd.row_seed.copy_(torch.arange(9, dtype=torch.int32, device=gpu) * 7919 + 1)
    g = torch.Generator().manual_seed(52)
    h = torch.randn(3, 1024, generator=g).to(torch.bfloat16).to(gpu)
    cb0 = torch.randint(0, 2048, (3,), generator=g).to(gpu)
    fd.warmup()
    ctr = fd.row_ctr.clone()
    outs = [fd([5, 2, 7], h, cb0) for _ in range(2)]
    fd.row_ctr.copy_(ctr)
    e1 = fd._fn(torch.tensor([5, 2, 7], device=gpu), h, cb0)
    e2 = fd._fn(torch.tensor([5, 2, 7], device=gpu), h, cb0)
    for (c, f), (ce, fe) in zip(outs, (e1, e2)):
        assert torch.equal(c, ce) and torch.equal(f, fe)
    assert not torch.equal(outs[0][0], outs[1][0])  # the frame counter moved the streams
    with pytest.raises(ValueError):
        fd([1, 2], h, cb0)
    with pytest.raises(IndexError):
        fd([1, 2, 8], h, cb0)
