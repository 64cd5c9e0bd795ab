"""The drop-in surfaces the engine calls besides the frame step, each on the GPU through the C ABI:
row_exponential / add_ln / topk_sample (serve/fast_depth_kernels.py), load_slot with an HF cache from
serve/cache.py, StaticBackbone.warmup(mixed=True), the frame step with an fp16 depth under the bf16 backbone
(the engine's default depth dtype), Cb0Sampler.bind's defaults, FrameStep's host lengths and TickReadout's
argument checks."""
import math

import numpy as np
import pytest
import torch

from helpers import bf16_bits, close
from m3x import synth
from oracle import coracle as C
from oracle import torch_oracle as O

pytestmark = pytest.mark.gpu


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_row_exponential_matches_philox(gpu):
    """out[b, c] = -log(u) for u the Philox uniform of counter (ctr_b, level, c, 0) and key (seed_b, 0): the
    uniforms are the oracle's bit for bit, the logarithm within 1 ulp of the correctly rounded value; the noise is
    Exp(1) (mean and P(E > 1) over 262k draws), and levels and counters give different streams."""
    from m3x.serve.fast_depth_kernels import row_exponential
    g = _g(101)
    B, V = 5, 2049
    seeds = torch.randint(1, 2 ** 31 - 2, (B,), generator=g, dtype=torch.int32)
    ctrs = torch.randint(0, 5000, (B,), generator=g, dtype=torch.int32)
    for level in (0, 3):
        E = row_exponential(B, V, seeds.to(gpu), ctrs.to(gpu), level=level).cpu().numpy()
        for b in range(B):
            w = np.array([C.philox4x32_10([int(ctrs[b]), level, c, 0], [int(seeds[b]), 0])[0] for c in range(V)],
                         dtype=np.uint64)
            u = (w >> 8).astype(np.float64) * 2.0 ** -24
            ref = (-np.log(np.maximum(u, 1e-12))).astype(np.float32)
            ulp = np.spacing(np.abs(ref)).astype(np.float64)
            assert np.all(np.abs(E[b].astype(np.float64) - ref) <= 2 * ulp), (level, b)
    big = row_exponential(64, 4096, torch.arange(1, 65, dtype=torch.int32, device=gpu),
                          torch.zeros(64, dtype=torch.int32, device=gpu)).cpu()
    assert abs(big.mean().item() - 1.0) < 0.01 and abs((big > 1).float().mean().item() - math.exp(-1)) < 0.005
    a = row_exponential(2, 64, seeds[:2].to(gpu), ctrs[:2].to(gpu), level=1)
    b2 = row_exponential(2, 64, seeds[:2].to(gpu), (ctrs[:2] + 1).to(gpu), level=1)
    assert not torch.equal(a, b2)


@pytest.mark.parametrize("layer_norm", [True, False])
def test_add_ln_surface(gpu, layer_norm):
    """add_ln(x, a, ln, c) = (dt(dt(x + a) + c), norm(...)) (serve/fast_depth_kernels.py:14-45) for a LayerNorm
    (fp32 stats, one rounding) and an RMSNorm module, against the same arithmetic on the CPU."""
    from m3x.serve.fast_depth_kernels import add_ln
    g = _g(102 + layer_norm)
    B, T, D = 3, 5, 1024
    dt = torch.bfloat16
    x = torch.randn(B, T, D, generator=g).to(dt)
    a = torch.randn(B, T, D, generator=g).to(dt)
    c = torch.randn(B, 1, D, generator=g).to(dt)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(dt)
    bias = (0.1 * torch.randn(D, generator=g)).to(dt) if layer_norm else None
    ln = synth.Norm(w.to(gpu), 1e-5, None if bias is None else bias.to(gpu))
    xo, y = add_ln(x.to(gpu), a.to(gpu), ln, c.to(gpu))
    xr = (x.float() + a.float()).to(dt)
    xr = (xr.float() + c.float()).to(dt)
    assert torch.equal(xo.cpu(), xr)
    ref = O._norm(xr, synth.Norm(w, 1e-5, bias), dt)
    ok, info = close(y, ref, atol=0, rel_ulps=1)
    assert ok, info
    xo2, y2 = add_ln(x.to(gpu), a.to(gpu), ln)  # without the constant
    assert torch.equal(xo2.cpu(), (x.float() + a.float()).to(dt))


@pytest.mark.parametrize("per_row", [True, False])
def test_topk_sample_surface(gpu, per_row):
    """topk_sample(logits, seed_t, level, temp, top_k, greedy, ctr_t) draws one uniform per row from Philox
    (counter (ctr, level), key seed; the engine-wide stream uses counter = row) and returns the oracle sampler's
    code on those uniforms; greedy returns the argmax."""
    from m3x.serve.fast_depth_kernels import topk_sample
    g = _g(104 + per_row)
    B, V, level, temp, k = 7, 2048, 5, 0.8, 50
    logits = (torch.randn(B, V, generator=g) * 2).to(torch.bfloat16)
    if per_row:
        seeds = torch.randint(1, 2 ** 31 - 2, (B,), generator=g, dtype=torch.int32)
        ctrs = torch.randint(0, 99, (B,), generator=g, dtype=torch.int32)
        got = topk_sample(logits.to(gpu), seeds.to(gpu), level, temp, k, ctr_t=ctrs.to(gpu))
        u = np.array([C.philox_uniform(int(seeds[b]), int(ctrs[b]), level) for b in range(B)], np.float32)
    else:
        seed = torch.tensor([12345], dtype=torch.int32)
        got = topk_sample(logits.to(gpu), seed.to(gpu), level, temp, k)
        u = np.array([C.philox_uniform(12345, b, level) for b in range(B)], np.float32)
    assert got.dtype == torch.long
    ref = C.topk_sample_rows(bf16_bits(logits), 1.0 / temp, k, u)
    assert np.array_equal(got.cpu().numpy(), ref)
    greedy = topk_sample(logits.to(gpu), torch.ones(1, dtype=torch.int32, device=gpu), level, temp, k, greedy=True)
    assert torch.equal(greedy.cpu(), logits.float().argmax(-1))


def _small_backbone(gpu, layers=2, S=6, cap=256, use_graphs=True, buckets=(1, 2, 4, 8, 64), seed=111):
    from m3x.serve.fast_backbone import StaticBackbone
    bb = synth.qwen3_backbone(layers=layers, seed=seed, device=gpu, affine=synth.AFFINE)
    return StaticBackbone(bb, S, capacity=cap, batch_buckets=buckets, ctx_buckets=(cap,), attention="triton",
                          fuse_rope=True, use_graphs=use_graphs)


def test_load_slot_from_hf_cache(gpu):
    """load_slot(slot, cache, length) installs the first `length` positions of an HF cache built by
    cache_from_owned_tensors (serve/fast_backbone.py:158-165, serve/cache.py:7-20): the same state as load_prefix,
    so the next step of both slots gives the same bits; bad slots and lengths raise the reference's errors."""
    from m3x.serve.cache import cache_from_owned_tensors
    sb = _small_backbone(gpu)
    g = _g(106)
    T, n = 90, 77
    layers = [(torch.randn(1, 8, T, 128, generator=g).to(torch.bfloat16).to(gpu),
               torch.randn(1, 8, T, 128, generator=g).to(torch.bfloat16).to(gpu)) for _ in range(2)]
    cache = cache_from_owned_tensors(layers)
    assert cache.layers[0].keys is layers[0][0]  # owned, not copied
    sb.load_slot(2, cache, n)
    sb.load_prefix(4, [(k[:, :, :n], v[:, :, :n]) for k, v in layers], n)
    for i, (k, v) in enumerate(layers):
        assert torch.equal(sb.k[i][2, :, :n], k[0, :, :n]) and torch.equal(sb.v[i][2, :, :n], v[0, :, :n])
        assert not sb.k[i][2, :, n:].any()
    assert sb.lengths_cpu[2] == sb.lengths_cpu[4] == n and sb.lengths[2].item() == n
    x = torch.randn(1, 1024, generator=g).to(torch.bfloat16).to(gpu)
    a = sb.step([2], x)
    b = sb.step([4], x)
    assert torch.equal(a, b)
    with pytest.raises(IndexError):
        sb.load_slot(6, cache, n)
    with pytest.raises(ValueError):
        sb.load_slot(1, cache, 257)


def test_warmup_mixed_captures_step_mixed_graphs(gpu):
    """warmup(mixed=True) captures the inline-prefill graphs up front; step_mixed then replays them (no capture at
    step time) and gives the eager step's bits."""
    sa = _small_backbone(gpu, seed=112)
    sb = _small_backbone(gpu, seed=112, use_graphs=False)
    sa.warmup(batch_buckets=(64,), mixed=True)
    keys = set(sa.graphs)
    assert (64, 256, "mixed") in keys and (64, 256) in keys
    g = _g(107)
    for s in (sa, sb):
        s.load_prefix(1, [(torch.zeros(1, 8, 5, 128, dtype=torch.bfloat16, device=gpu),) * 2] * 2, 5)
    x = torch.randn(2, 1024, generator=g).to(torch.bfloat16).to(gpu)
    p = torch.randn(30, 1024, generator=g).to(torch.bfloat16).to(gpu)
    ra = sa.step_mixed([0, 1], x, [(3, p)])
    rb = sb.step_mixed([0, 1], x, [(3, p)])
    assert set(sa.graphs) == keys
    assert torch.equal(ra[0], rb[0]) and torch.equal(ra[1][0], rb[1][0])
    assert sa.lengths_cpu[:4] == [1, 6, 0, 30] == sa.lengths[:4].tolist()


def _frame(gpu, depth_dtype, use_guard=False, seed=121, S=8, cap=256):
    from m3x.cb0 import Cb0Sampler
    from m3x.frame import FrameStep
    from m3x.serve.fast_depth import FastDepth
    sb = _small_backbone(gpu, S=S, cap=cap, buckets=(4,), seed=seed)
    cb = Cb0Sampler(sb.backbone.cb0_head.weight, S, temp=0.9, top_k=50, rep=0.0)
    fd = FastDepth(synth.swiglu_depth(seed=seed + 1, device=gpu, dtype=depth_dtype, affine=synth.AFFINE), S, dtype=depth_dtype, temp=0.9,
                   top_k=50, batch_buckets=(4,))
    g = _g(seed + 2)
    with torch.inference_mode():
        for i in range(2):
            sb.k[i][:S].copy_(torch.randn(S, 8, cap, 128, generator=g).to(torch.bfloat16))
            sb.v[i][:S].copy_(torch.randn(S, 8, cap, 128, generator=g).to(torch.bfloat16))
        lengths = [17, 0, 120, 3, 0, 64, 0, 250]
        sb.lengths[:S].copy_(torch.tensor(lengths))
        sb.lengths_cpu[:S] = lengths
        for s in range(S):
            cb.bind(s, seed=1000 + s)
        fd.row_seed.copy_(torch.arange(S + 1, dtype=torch.int32) * 31 + 7)
    fs = FrameStep(sb, cb, fd, ring_depth=4)
    with torch.inference_mode():
        fs.feedback[:S].copy_(torch.randn(S, 1024, generator=g).to(torch.bfloat16))
    return fs


def test_frame_with_fp16_depth(gpu):
    """The engine's default depth dtype is fp16 under the bf16 backbone (maya3/engine.py:53,192-199): the frame
    graph converts the hidden state on the way in (the depth input equals the backbone output in fp16), keeps the
    feedback in bf16, replays equal eager runs bit for bit, and its depth codes equal the oracle sampler on the
    depth's own fp16 logits."""
    a, b = _frame(gpu, torch.float16), _frame(gpu, torch.float16)
    ga, gb = a.capture(4, 256), b.capture(4, 256, use_graph=False)
    slots = [2, 0, 5]
    a.set_slots(ga, slots)
    b.set_slots(gb, slots)
    for _ in range(2):
        a.replay(ga)
        b.replay(gb)
        torch.cuda.synchronize()
        assert torch.equal(a.codes(ga)[:3], b.codes(gb)[:3])
        assert torch.equal(a.feedback[slots], b.feedback[slots])
    bb, cb, dp, codes = ga.bufs
    assert dp.h.dtype == torch.float16 and torch.equal(dp.h[:3], bb.out[:3].half())
    assert a.feedback.dtype == torch.bfloat16
    assert a.bb.lengths_cpu[:6] == [19, 0, 122, 3, 0, 66] == a.bb.lengths[:6].tolist()
    # one frame's depth codes against the oracle sampler on the depth's own logits
    dp2 = a.depth.make_buffers(4)
    dp2.slots.copy_(bb.slots)
    dp2.h.copy_(dp.h)
    dp2.codes.copy_(codes)
    ctr = a.depth.row_ctr.clone()
    # the frame moved each row's counter once, the padding row's (the dummy slot) included
    a.depth.row_ctr.sub_(torch.bincount(bb.slots, minlength=9).int())
    trace = []
    a.depth.run(dp2, trace=trace)
    torch.cuda.synchronize()
    assert torch.equal(dp2.codes[:3], codes[:3]) and torch.equal(a.depth.row_ctr, ctr)
    for lv in range(1, 32):
        ref = C.topk_sample_rows(bf16_bits(trace[lv - 1][:3]), 1 / 0.9, 50, dp2.u[:3, lv - 1].cpu().numpy(),
                                 is_f16=True)
        assert np.array_equal(codes[:3, lv].cpu().numpy(), ref), lv


def test_frame_host_lengths_and_room(gpu):
    """FrameStep keeps the backbone's host lengths in step with the device (one per staged seat per replay), and
    refuses to stage or replay a seat whose next position does not fit the graph's context bucket."""
    fs = _frame(gpu, torch.bfloat16)
    g = fs.capture(4, 256)
    fs.set_slots(g, [7, 1])  # slot 7 holds 250 positions
    for _ in range(5):
        fs.replay(g)
    assert fs.bb.lengths_cpu[7] == 255 == fs.bb.lengths[7].item() and fs.bb.lengths_cpu[1] == 5
    fs.replay(g)
    assert fs.bb.lengths_cpu[7] == 256 == fs.bb.lengths[7].item()
    with pytest.raises(ValueError):
        fs.replay(g)  # position 256 does not fit a 256-position context
    with pytest.raises(ValueError):
        fs.set_slots(g, [1, 1])
    with pytest.raises(IndexError):
        fs.set_slots(g, [8])


def test_cb0_bind_restores_defaults(gpu):
    """bind with a setting unset gives the seat the sampler's configured default (maya3/engine.py:438-441), so a
    reused slot does not inherit the previous seat's temperature, top-k, top-p or penalty."""
    from m3x.cb0 import Cb0Sampler
    w = (torch.randn(2049, 1024, generator=_g(131)) * 0.02).to(torch.bfloat16).to(gpu)
    cb = Cb0Sampler(w, 4, temp=0.9, top_k=50, rep=0.8, top_p=0.95)
    cb.bind(2, seed=5, temperature=0.5, top_k=10, top_p=0.5, repetition_penalty=1.5, min_frames=3)
    assert cb.temp_t[2].item() == 0.5 and cb.topk_t[2].item() == 10 and cb.rep_t[2].item() == 1.5
    cb.bind(2, seed=6)
    assert cb.temp_t[2].item() == pytest.approx(0.9) and cb.topk_t[2].item() == 50
    assert cb.topp_t[2].item() == pytest.approx(0.95) and cb.rep_t[2].item() == pytest.approx(0.8)
    assert cb.min_t[2].item() == 0 and cb.seed_t[2].item() == 6
    cb.bind(1, seed=7, repetition_penalty=0.0)
    assert cb.rep_t[1].item() == 0.0


def test_tick_pack_checks_rows(gpu):
    """TickReadout.pack refuses more seats than its buffer and inputs with fewer rows than the seats."""
    from m3x.tick import TickReadout
    rd = TickReadout(4, frame=1920, nq=32, device=gpu)
    z = lambda n, *s, dt=torch.long: torch.zeros(n, *s, dtype=dt, device=gpu)  # noqa: E731
    with pytest.raises(ValueError):
        rd.pack(z(5), z(5), codes=z(5, 32, dt=torch.int32), pcm=z(5, 1920, dt=torch.float32))
    with pytest.raises(ValueError):
        rd.pack(z(3), z(3), codes=z(3, 32, dt=torch.int32), pcm=z(2, 1920, dt=torch.float32))
    with pytest.raises(ValueError):
        rd.pack(z(3), z(2), codes=z(3, 32, dt=torch.int32), pcm=z(3, 1920, dt=torch.float32))
    rd.pack(z(3), z(3), codes=z(3, 32, dt=torch.int32), pcm=z(3, 1920, dt=torch.float32))
    out = rd.wait()
    assert out["codes"].shape == (3, 32) and out["pcm"].shape == (3, 1920)
