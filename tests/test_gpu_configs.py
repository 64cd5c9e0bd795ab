"""Parity at the benchmark configurations' real workloads, through the C ABI on the GPU.

Every seat is independent, so each full-size step is checked two ways:
  - a few sampled seats against the CPU oracle (their cache rows copied out before the step; the bf16 noise floor
    bar of helpers.floor_check, figures printed);
  - properties on every seat: lengths advance by exactly the rows each seat ran, K/V change only at the positions
    written (per-position checksums of every layer before and after), the dummy slot stays untouched, and every
    sampled code equals the C oracle sampler on the kernel's own logits and uniforms (bit-exact).
C1: one Qwen3-0.6B-shaped layer, B=1, a 256-key cache, against the HF transformers golden fixture.
C2: the depth frame at 16 seats (31 codebooks, top-k 50, T 0.9).
C3: the 28-layer backbone step at 64 seats, capacity 4096, lengths U[64, 2048], + cb0.
C4: the mixed step: 216 decoding seats (lengths log-uniform in [128, 4096)) + 8 inline prefills of 256 tokens.
C5: the whole frame graph at 224 seats, lengths Poisson(2048) capped at 4096.
"""
import gc
import os
import sys

import numpy as np
import pytest
import torch

from helpers import bf16_bits, convert, floor_check, report, to_device
from m3x import synth
from oracle import coracle as C
from oracle import torch_oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(400)]

CAP = 4096
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))


@pytest.fixture(scope="module")
def models(gpu):
    """The 28-layer backbone and the 4-layer SwiGLU depth of the benchmark (seeded on the GPU), with CPU copies
    for the oracle."""
    bb = synth.qwen3_backbone(layers=28, seed=0, device=gpu, gen="cuda", affine=synth.AFFINE)
    dm = synth.swiglu_depth(seed=1, device=gpu, gen="cuda", affine=synth.AFFINE)
    yield bb, dm, to_device(bb, "cpu"), to_device(dm, "cpu")
    gc.collect()
    torch.cuda.empty_cache()


def _free():
    gc.collect()
    torch.cuda.empty_cache()


def _fill_cache(sb, seed):
    g = torch.Generator(device=sb.device).manual_seed(seed)
    for i in range(len(sb.layers)):
        sb.k[i].normal_(generator=g)
        sb.v[i].normal_(generator=g)


def _set_lengths(sb, lengths):
    n = len(lengths)
    sb.lengths[:n].copy_(torch.as_tensor(lengths))
    sb.lengths_cpu[:n] = [int(v) for v in lengths]


def _checksums(sb):
    """Per layer, per (slot, position): the fp32 sums of the K and V rows (deterministic reductions)."""
    return [(k.sum(dim=(1, 3), dtype=torch.float32), v.sum(dim=(1, 3), dtype=torch.float32))
            for k, v in zip(sb.k, sb.v)]


def _written_only_at(before, after, writes, slots_total):
    """Every (slot, position) whose K or V checksum changed is one of `writes` (slot -> positions), and every
    position in `writes` changed in every layer."""
    mask = torch.zeros(slots_total, before[0][0].shape[1], dtype=torch.bool)
    for s, ps in writes.items():
        mask[s, list(ps)] = True
    mask = mask.to(before[0][0].device)
    for i, ((kb, vb), (ka, va)) in enumerate(zip(before, after)):
        changed = (kb != ka) | (vb != va)
        assert not (changed & ~mask).any(), f"layer {i}: K/V changed outside the written positions"
        assert changed[mask].all(), f"layer {i}: a written position kept its old K/V"


def _sample_cache(sb, slots, ctx):
    """CPU copies [len(slots) + 1, KV, ctx, D] per layer of the sampled slots' first ctx positions (+ a zero row)."""
    kc, vc = [], []
    for i in range(len(sb.layers)):
        k = torch.zeros(len(slots) + 1, sb.kv_heads, ctx, sb.head_dim, dtype=torch.bfloat16)
        v = torch.zeros_like(k)
        k[:len(slots)] = sb.k[i][slots, :, :ctx].cpu()
        v[:len(slots)] = sb.v[i][slots, :, :ctx].cpu()
        kc.append(k)
        vc.append(v)
    return kc, vc


class _Oracle:
    """The bf16 oracle and its fp32 truth over compact caches of a few sampled slots (slot j of the compact caches
    is the j-th sampled slot; the last row is a zero dummy). step() may be called once per group of rows, since
    rows of different slots are independent: the caches and lengths carry over between calls."""

    def __init__(self, bb_c, kc, vc, lengths):
        self.bb16, self.bb32 = bb_c, convert(bb_c, torch.float32)
        self.kc16, self.vc16 = kc, vc
        self.kc32, self.vc32 = [t.float() for t in kc], [t.float() for t in vc]
        self.l16, self.l32 = lengths.clone(), lengths.clone()
        ctx = kc[0].shape[2]
        self.cos, self.sin = O.rope_tables(128, 1e6, ctx, torch.bfloat16)
        self.c32, self.s32 = O.rope_tables(128, 1e6, ctx, torch.float32)

    def step(self, rows_slot, x, offset=None, x_truth=None):
        """(bf16 output, fp32 truth) of rows at compact slots rows_slot with inputs x [rows, hidden] (the truth's
        own fp32 inputs x_truth if given)."""
        out16 = O.backbone_step(self.bb16, self.kc16, self.vc16, self.l16, rows_slot, x, self.cos, self.sin,
                                offset=offset)
        truth = O.backbone_step(self.bb32, self.kc32, self.vc32, self.l32, rows_slot,
                                x.float() if x_truth is None else x_truth, self.c32, self.s32, offset=offset)
        return out16, truth


def _check_new_kv(sb, orc, slots, positions, label):
    """The K/V rows the kernel wrote for the sampled slots at `positions` (per slot) vs the oracle's, all layers."""
    got, ref, tru = [], [], []
    for i in range(len(sb.layers)):
        for j, s in enumerate(slots):
            ps = list(positions[j])
            for cache, o16, o32 in ((sb.k[i], orc.kc16[i], orc.kc32[i]), (sb.v[i], orc.vc16[i], orc.vc32[i])):
                got.append(cache[s, :, ps].float().cpu().flatten())
                ref.append(o16[j, :, ps].float().flatten())
                tru.append(o32[j, :, ps].flatten())
    ok, info = floor_check(torch.cat(got), torch.cat(ref), torch.cat(tru))
    report(label, info)
    assert ok, info


def _cb0_exact(logits, u, temp, top_k):
    """cb0 codes of the C oracle sampler (no stop state, no penalty) on bf16 logits rows and uniforms."""
    bits = bf16_bits(logits)
    return np.array([C.cb0_sample(bits[b], -1, temp, top_k, 0.0, 0.0, None, None, 0, None, None, float(u[b]))[0]
                     for b in range(bits.shape[0])])


# ---------------------------------------------------------------- C1
@torch.inference_mode()
def test_c1_layer_vs_hf_golden(gpu):
    """C1 on the HIP path: one layer (bf16 weights and cache from the fixture's seeds), B=1, 256 cached keys,
    against HF transformers' fp32 Qwen3Model output (tests/golden/c1_qwen3_layer.npz) within the bf16 floor of the
    oracle run on the same bf16 inputs; the K/V rows written at position 256 likewise."""
    from m3x.serve.fast_backbone import StaticBackbone
    from make_golden import c1_inputs
    gold = np.load(os.path.join(HERE, "golden", "c1_qwen3_layer.npz"))
    _, k, v, x = c1_inputs()
    # the fixture's weights (the same seeded draws, wide-spread norm weights included) rounded to bf16
    bb16 = c1_inputs(torch.bfloat16)[0]
    sb = StaticBackbone(c1_inputs(torch.bfloat16, gpu)[0], 1, capacity=512,
                        batch_buckets=(1,), ctx_buckets=(512,), attention="triton", fuse_rope=True)
    sb.load_prefix(0, [(k.to(torch.bfloat16).to(gpu), v.to(torch.bfloat16).to(gpu))], 256)
    out = sb.step([0], x.to(torch.bfloat16).to(gpu))[0]
    kc = [torch.zeros(2, 8, 512, 128, dtype=torch.bfloat16)]
    vc = [torch.zeros(2, 8, 512, 128, dtype=torch.bfloat16)]
    kc[0][0, :, :256], vc[0][0, :, :256] = k[0].to(torch.bfloat16), v[0].to(torch.bfloat16)
    cos, sin = O.rope_tables(128, 1e6, 512, torch.bfloat16)
    ref16 = O.backbone_step(bb16, kc, vc, torch.tensor([256, 0]), torch.tensor([0]), x.to(torch.bfloat16), cos, sin)
    ok, info = floor_check(out, ref16[0], torch.from_numpy(gold["out"]))
    report("C1 hidden vs HF fp32 golden", info)
    assert ok, info
    for name, cache, key in (("K", sb.k[0], "k256"), ("V", sb.v[0], "v256")):
        ok, info = floor_check(cache[0, :, 256], (kc if name == "K" else vc)[0][0, :, 256],
                               torch.from_numpy(gold[key]))
        report(f"C1 {name} row 256 vs golden", info)
        assert ok, info
    assert sb.lengths_cpu[0] == 257 == sb.lengths[0].item()


# ---------------------------------------------------------------- C2
@torch.inference_mode()
def test_c2_depth_16_seats(gpu, models):
    """C2: FastDepth.__call__ over 16 seats (one graph replay); an eager rerun of the same frame traces every
    level's logits and gives the same codes; every code of every seat equals the oracle sampler on those logits
    and the seat's Philox uniforms; the logits of all seats against the teacher-forced CPU oracle; the feedback."""
    from m3x.serve.fast_depth import FastDepth
    _, dm, _, dm_c = models
    B = 16
    fd = FastDepth(dm, B, dtype=torch.bfloat16, temp=0.9, top_k=50, batch_buckets=(B,), fused=True)
    fd.row_seed.copy_(torch.arange(B + 1, dtype=torch.int32, device=gpu) * 69069 + 7)
    g = torch.Generator().manual_seed(202)
    h = torch.randn(B, 1024, generator=g).to(torch.bfloat16)
    cb0 = torch.randint(0, 2048, (B,), generator=g)
    slots = list(range(B))
    codes, fb = fd(slots, h.to(gpu), cb0.to(gpu))
    fd.row_ctr.sub_(torch.tensor([1] * B + [0], dtype=torch.int32, device=gpu))
    b = fd.make_buffers(B)
    b.slots.copy_(torch.tensor(slots))
    b.h.copy_(h)
    b.codes[:, 0].copy_(cb0)
    trace = []
    fd.run(b, trace=trace)
    torch.cuda.synchronize()
    assert torch.equal(b.codes.long(), codes) and torch.equal(b.feedback, fb)
    logits = torch.stack([t.cpu() for t in trace], 1)
    u = b.u.cpu()
    for lv in range(1, 32):
        ref = C.topk_sample_rows(bf16_bits(logits[:, lv - 1]), 1 / 0.9, 50, u[:, lv - 1].numpy())
        assert np.array_equal(codes[:, lv].cpu().numpy(), ref), lv
    codes_c = codes.cpu()
    _, ref_logits = O.depth_frame(dm_c, h, cb0, u, 0.9, 50, forced=codes_c)
    _, truth = O.depth_frame(convert(dm_c, torch.float32), h.float(), cb0, u, 0.9, 50, forced=codes_c,
                             dt=torch.float32)
    ok, info = floor_check(logits, ref_logits, truth)
    report("C2 depth logits, 16 seats x 31 levels", info)
    assert ok, info
    ok, info = floor_check(fb, O.feedback(dm_c.audio_in, codes_c), O.feedback(
        convert(dm_c.audio_in, torch.float32), codes_c))
    report("C2 feedback", info)
    assert ok, info
    del fd, b
    _free()


# ---------------------------------------------------------------- C3
@torch.inference_mode()
def test_c3_backbone_64_seats(gpu, models):
    """C3: StaticBackbone.step over 64 seats (28 layers, capacity 4096, lengths U[64, 2048]) + cb0: three sampled
    seats (shortest, median, longest) against the oracle, properties on all 64, cb0 bit-exact on all 64."""
    from m3x.cb0 import Cb0Sampler
    from m3x.serve.fast_backbone import StaticBackbone
    bb, _, bb_c, _ = models
    B = 64
    sb = StaticBackbone(bb, B, capacity=CAP, batch_buckets=(B,), ctx_buckets=(2048, 3072, CAP), attention="triton",
                        fuse_rope=True)
    sb.warmup()  # capture first: the warm-up runs write the dummy slot's position 0, the step must not
    _fill_cache(sb, 303)
    lengths = synth.c3_lengths(B)
    _set_lengths(sb, lengths)
    order = torch.argsort(lengths)
    sample = [int(order[0]), int(order[B // 2]), int(order[-1])]
    ctx = int(lengths[sample].max()) + 1
    kc, vc = _sample_cache(sb, sample, ctx)
    before = _checksums(sb)
    x = torch.randn(B, 1024, generator=torch.Generator().manual_seed(304)).to(torch.bfloat16)
    out = sb.step(list(range(B)), x.to(gpu))
    torch.cuda.synchronize()
    _written_only_at(before, _checksums(sb), {s: [int(lengths[s])] for s in range(B)}, B + 1)
    assert sb.lengths[:B].cpu().tolist() == (lengths + 1).tolist() == sb.lengths_cpu[:B] and sb.lengths[B] == 0
    orc = _Oracle(bb_c, kc, vc, torch.cat([lengths[sample], torch.tensor([0])]))
    out16, truth = orc.step(torch.arange(3), x[sample])
    ok, info = floor_check(out[sample], out16, truth)
    report("C3 hidden, 3 sampled seats, 28 layers", info)
    assert ok, info
    _check_new_kv(sb, orc, sample, [[int(lengths[s])] for s in sample], "C3 new K/V rows")
    cb = Cb0Sampler(bb.cb0_head.weight, B, temp=0.9, top_k=50, rep=0.0)
    for s in range(B):
        cb.bind(s, seed=500 + s)
    bufs = cb.make_buffers(B)
    bufs.slots.copy_(torch.arange(B))
    bufs.h.copy_(out)
    cb.run(bufs)
    torch.cuda.synchronize()
    assert np.array_equal(bufs.cb0.cpu().numpy(), _cb0_exact(bufs.logits, bufs.u[:, 0].cpu(), 0.9, 50))
    del sb, cb, bufs, before
    _free()


# ---------------------------------------------------------------- C4
@torch.inference_mode()
def test_c4_mixed_step_2264_rows(gpu, models):
    """C4: step_mixed with 216 decoding seats (lengths log-uniform in [128, 4096)) and 8 inline prefills of 256
    embedding rows (uniform ids over a 151,936-row table) from length 0 = 2264 rows in one graph replay: two
    decoding seats and one prefill against the oracle (the prefill's last hidden state and all 256 K/V rows of
    every layer), properties on all 224 seats, cb0 (top-k 50) bit-exact on all 224 outputs."""
    from m3x.cb0 import Cb0Sampler
    from m3x.serve.fast_backbone import StaticBackbone
    bb, _, bb_c, _ = models
    nd, npf, T = 216, 8, 256
    S = nd + npf
    sb = StaticBackbone(bb, S, capacity=CAP, batch_buckets=(nd + npf * T,), ctx_buckets=(CAP,), attention="triton",
                        fuse_rope=True)
    sb.warmup(mixed=True)  # capture first: the warm-up runs write the dummy slot's position 0, the step must not
    _fill_cache(sb, 404)
    lengths = torch.cat([synth.c4_decode_lengths(nd), torch.zeros(npf, dtype=torch.long)])
    _set_lengths(sb, lengths)
    g = torch.Generator(device=gpu).manual_seed(405)
    table = (torch.randn(151936, 1024, device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    ids = torch.randint(0, 151936, (npf, T), device=gpu, generator=g)
    pre = [(nd + j, table[ids[j]].contiguous()) for j in range(npf)]
    del table
    x = torch.randn(nd, 1024, device=gpu, generator=g).to(torch.bfloat16)
    order = torch.argsort(lengths[:nd])
    dec_sample = [int(order[0]), int(order[-1])]
    psl = nd + 3
    sample = dec_sample + [psl]
    ctx = int(lengths[dec_sample].max()) + 1
    kc, vc = _sample_cache(sb, sample, max(ctx, T))
    before = _checksums(sb)
    dec, last = sb.step_mixed(list(range(nd)), x, pre)
    torch.cuda.synchronize()
    writes = {s: [int(lengths[s])] for s in range(nd)}
    writes.update({nd + j: range(T) for j in range(npf)})
    _written_only_at(before, _checksums(sb), writes, S + 1)
    assert sb.lengths[:S].cpu().tolist() == (lengths + torch.tensor([1] * nd + [T] * npf)).tolist() == \
        sb.lengths_cpu[:S]
    orc = _Oracle(bb_c, kc, vc, torch.cat([lengths[sample], torch.tensor([0])]))
    # the two decoding rows and the prefill's 256 rows in separate oracle calls (different slots: independent)
    d16, dtr = orc.step(torch.tensor([0, 1]), x[dec_sample].cpu())
    p16, ptr = orc.step(torch.full((T,), 2), pre[3][1].cpu(), offset=torch.arange(T))
    got = torch.cat([dec[dec_sample], last[3][None]])
    ok, info = floor_check(got, torch.cat([d16, p16[-1:]]), torch.cat([dtr, ptr[-1:]]))
    report("C4 hidden, 2 decoding seats + a prefill's last row", info)
    assert ok, info
    _check_new_kv(sb, orc, sample, [[int(lengths[s])] for s in dec_sample] + [range(T)],
                  "C4 new K/V rows (2 decode rows + 256 prefill rows)")
    cb = Cb0Sampler(bb.cb0_head.weight, S, temp=0.9, top_k=50, rep=0.0)
    for s in range(S):
        cb.bind(s, seed=700 + s)
    bufs = cb.make_buffers(S)
    bufs.slots.copy_(torch.arange(S))
    bufs.h.copy_(torch.cat([dec, torch.stack(last)]))
    cb.run(bufs)
    torch.cuda.synchronize()
    assert np.array_equal(bufs.cb0.cpu().numpy(), _cb0_exact(bufs.logits, bufs.u[:, 0].cpu(), 0.9, 50))
    del sb, cb, bufs, pre, before
    _free()


# ---------------------------------------------------------------- C5
@torch.inference_mode()
def test_c5_frame_224_seats(gpu, models):
    """C5: the whole frame graph at 224 seats (lengths Poisson(2048) capped at 4096): backbone rows of three sampled
    seats against the oracle; cb0 of all 224 seats bit-exact against the oracle sampler on the graph's logits and
    uniforms; an eager rerun of the depth on the graph's own inputs gives the graph's codes, and all 224 x 31
    depth codes equal the oracle sampler on its traced logits; the sampled seats' depth logits against the
    teacher-forced oracle; the ring holds the frame's codes; K/V change only at each seat's position."""
    bb, dm, bb_c, dm_c = models
    B = 224
    sb, cb, fd, fs, g, lengths = _c5_frame(gpu, bb, dm, B)
    order = torch.argsort(lengths)
    sample = [int(order[0]), int(order[B // 2]), int(order[-1])]
    kc, vc = _sample_cache(sb, sample, int(lengths[sample].max()) + 1)
    x_in = fs.feedback[sample].cpu()
    before = _checksums(sb)
    ctr_depth = fd.row_ctr.clone()
    fs.replay(g)
    torch.cuda.synchronize()
    bbuf, cbuf, dbuf, codes = g.bufs
    _written_only_at(before, _checksums(sb), {s: [int(lengths[s])] for s in range(B)}, B + 1)
    assert sb.lengths[:B].cpu().tolist() == (lengths + 1).tolist() == sb.lengths_cpu[:B] and sb.lengths[B] == 0
    codes_c = codes.cpu().long()
    assert codes_c.min() >= 0 and codes_c.max() < 2048
    assert torch.equal(fs.ring[0].cpu(), codes.cpu()) and fs.ring_head.item() == 1
    # backbone rows of the sampled seats
    orc = _Oracle(bb_c, kc, vc, torch.cat([lengths[sample], torch.tensor([0])]))
    out16, truth = orc.step(torch.arange(3), x_in)
    ok, info = floor_check(bbuf.out[sample], out16, truth)
    report("C5 backbone hidden, 3 sampled seats", info)
    assert ok, info
    # cb0 of every seat
    assert np.array_equal(cbuf.cb0.cpu().numpy(), _cb0_exact(cbuf.logits, cbuf.u[:, 0].cpu(), 0.9, 50))
    assert torch.equal(codes_c[:, 0], cbuf.cb0.cpu())
    trace, u = _depth_rerun_exact(fd, bbuf, codes, ctr_depth)
    h_s = bbuf.out[sample].cpu()
    logits = torch.stack([t[sample].cpu() for t in trace], 1)
    _, ref_l = O.depth_frame(dm_c, h_s, codes_c[sample, 0], u[sample], 0.9, 50, forced=codes_c[sample])
    _, tru_l = O.depth_frame(convert(dm_c, torch.float32), h_s.float(), codes_c[sample, 0], u[sample], 0.9, 50,
                             forced=codes_c[sample], dt=torch.float32)
    ok, info = floor_check(logits, ref_l, tru_l)
    report("C5 depth logits, 3 sampled seats x 31 levels", info)
    assert ok, info
    del fs, sb, cb, fd, g, before
    _free()


def _c5_frame(gpu, bb, dm, B):
    """The C5 frame at B seats: cache N(0, 1), lengths Poisson(2048) capped, cb0 and depth streams seeded,
    random feedback rows, the frame graph captured with every seat staged."""
    from m3x.cb0 import Cb0Sampler
    from m3x.frame import FrameStep
    from m3x.serve.fast_backbone import StaticBackbone
    from m3x.serve.fast_depth import FastDepth
    sb = StaticBackbone(bb, B, capacity=CAP, batch_buckets=(B,), ctx_buckets=(CAP,), attention="triton",
                        fuse_rope=True)
    _fill_cache(sb, 505)
    lengths = synth.c5_lengths(B).clamp_max(CAP - 1)
    _set_lengths(sb, lengths)
    cb = Cb0Sampler(bb.cb0_head.weight, B, temp=0.9, top_k=50, rep=0.0)
    for s in range(B):
        cb.bind(s, seed=1 + s)
    fd = FastDepth(dm, B, dtype=torch.bfloat16, temp=0.9, top_k=50, batch_buckets=(B,), fused=True)
    fd.row_seed.copy_(torch.arange(B + 1, dtype=torch.int32, device=gpu) * 69069 + 1)
    fs = FrameStep(sb, cb, fd, ring_depth=4)
    fs.feedback.normal_(generator=torch.Generator(device=gpu).manual_seed(506))
    g = fs.capture(B, CAP)
    fs.set_slots(g, list(range(B)))
    return sb, cb, fd, fs, g, lengths


def _depth_rerun_exact(fd, bbuf, codes, ctr_before):
    """Rerun the depth of the frame just replayed, eagerly, on the graph's own inputs (the depth streams put back
    to ctr_before) with every level's logits traced: it must give the graph's codes, and every code of every seat
    must equal the C oracle sampler on those logits and the seat's uniforms. Returns (trace, uniforms)."""
    B = codes.shape[0]
    now = fd.row_ctr.clone()
    fd.row_ctr.copy_(ctr_before)
    d2 = fd.make_buffers(B)
    d2.slots.copy_(bbuf.slots)
    d2.h.copy_(bbuf.out)
    d2.codes[:, 0].copy_(codes[:, 0])
    trace = []
    fd.run(d2, trace=trace)
    torch.cuda.synchronize()
    assert torch.equal(d2.codes, codes) and torch.equal(fd.row_ctr, now)
    u = d2.u.cpu()
    codes_c = codes.cpu().long()
    for lv in range(1, 32):
        ref = C.topk_sample_rows(bf16_bits(trace[lv - 1]), 1 / 0.9, 50, u[:, lv - 1].numpy())
        assert np.array_equal(codes_c[:, lv].numpy(), ref), lv
    return trace, u


FRAMES = 8


@torch.inference_mode()
def test_c5_frames_through_the_feedback_loop(gpu, models):
    """C5 over FRAMES consecutive replays of the frame graph, each frame's codes feeding the next frame's input
    through the feedback embedding, as the engine's ticks run (the multi-step check of
    maya3/tests/test_backbone_fused.py:12-46 at full size). Three sampled seats run the same frames on the oracle,
    which keeps its own K/V history and takes the GPU's codes (teacher forcing): every frame, their backbone
    rows and the feedback rows the graph wrote are checked against it at the bf16 floor, so drift through the
    cache and the feedback loop shows; every frame, cb0 and all 224 x 31 depth codes are bit-exact against the
    oracle sampler on the frame's own logits and uniforms, the ring holds the frame's codes, and each seat's
    length moves by one. The last frame's depth logits of the sampled seats are checked against the oracle."""
    bb, dm, bb_c, dm_c = models
    B = 224
    sb, cb, fd, fs, g, lengths = _c5_frame(gpu, bb, dm, B)
    order = torch.argsort(lengths)
    sample = [int(order[0]), int(order[B // 2]), int(order[-1])]
    kc, vc = _sample_cache(sb, sample, int(lengths[sample].max()) + 1 + FRAMES)
    orc = _Oracle(bb_c, kc, vc, torch.cat([lengths[sample], torch.tensor([0])]))
    audio32 = convert(dm_c.audio_in, torch.float32)
    x16 = fs.feedback[sample].cpu()
    x32 = x16.float()
    bbuf, cbuf, dbuf, codes = g.bufs
    for t in range(FRAMES):
        ctr_depth = fd.row_ctr.clone()
        fs.replay(g)
        torch.cuda.synchronize()
        assert sb.lengths[:B].cpu().tolist() == (lengths + t + 1).tolist() == sb.lengths_cpu[:B]
        codes_c = codes.cpu().long()
        assert torch.equal(fs.ring[t % 4].cpu(), codes.cpu()) and fs.ring_head.item() == t + 1
        out16, truth = orc.step(torch.arange(3), x16, x_truth=x32)
        ok, info = floor_check(bbuf.out[sample], out16, truth)
        report(f"C5 frame {t}: backbone hidden, 3 sampled seats", info)
        assert ok, (t, info)
        assert np.array_equal(cbuf.cb0.cpu().numpy(), _cb0_exact(cbuf.logits, cbuf.u[:, 0].cpu(), 0.9, 50)), t
        assert torch.equal(codes_c[:, 0], cbuf.cb0.cpu())
        trace, u = _depth_rerun_exact(fd, bbuf, codes, ctr_depth)
        # the next input: the feedback of this frame's codes, oracle (bf16) and truth (fp32) chains
        x16 = O.feedback(dm_c.audio_in, codes_c[sample])
        x32 = O.feedback(audio32, codes_c[sample]).float()
        ok, info = floor_check(fs.feedback[sample], x16, x32)
        report(f"C5 frame {t}: feedback rows, 3 sampled seats", info)
        assert ok, (t, info)
    h_s = bbuf.out[sample].cpu()
    logits = torch.stack([tr[sample].cpu() for tr in trace], 1)
    _, ref_l = O.depth_frame(dm_c, h_s, codes_c[sample, 0], u[sample], 0.9, 50, forced=codes_c[sample])
    _, tru_l = O.depth_frame(convert(dm_c, torch.float32), h_s.float(), codes_c[sample, 0], u[sample], 0.9, 50,
                             forced=codes_c[sample], dt=torch.float32)
    ok, info = floor_check(logits, ref_l, tru_l)
    report(f"C5 frame {FRAMES - 1}: depth logits, 3 sampled seats x 31 levels", info)
    assert ok, info
    del fs, sb, cb, fd, g
    _free()
