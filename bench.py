#!/usr/bin/env python3
"""Headline benchmark: one Maya3 frame step on one MI355X, captured as a single hipGraph.

Workload (the full frame at B=224): Qwen3-0.6B-shaped 28-layer backbone decode over a static bf16 KV cache
(224 seats, capacity 4096, per-seat lengths Poisson(2048) capped at 4096, cache N(0,1)), codebook-0 head + top-k 50
sampling, the 4-layer SwiGLU depth transformer over codebooks 1..31 with top-k 50 / temperature 0.9 sampling, the
32 codes per seat into an int32 device ring and the feedback embedding for the next frame. Random-init weights
N(0, 0.02), seeded; per-seat Philox uniforms. Inputs are resident in HBM before the timed region.

Prints ONE JSON line: frames/s at B=224 (value), B=1 frame latency in us, the decode-attention roofline measured
live with HIP events on the launch stream, and the CPU baseline (the PyTorch-eager oracle on this host's cores).
Progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "maya2-native_amd"))
sys.path.insert(0, ROOT)

CAP = 4096


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def build_frame(torch, seats, lengths, seed_base=0, backbone=None, depth_model=None):
    from m3x import synth
    from m3x.cb0 import Cb0Sampler
    from m3x.frame import FrameStep
    from m3x.serve.fast_backbone import StaticBackbone
    from m3x.serve.fast_depth import FastDepth
    dev = torch.device("cuda:0")
    bb = backbone or synth.qwen3_backbone(layers=28, seed=0, device=dev, gen="cuda", affine=synth.AFFINE)
    dm = depth_model or synth.swiglu_depth(seed=1, device=dev, gen="cuda", affine=synth.AFFINE)
    sb = StaticBackbone(bb, seats, capacity=CAP, batch_buckets=(seats,), ctx_buckets=(CAP,), attention="triton",
                        fuse_rope=True)
    g = torch.Generator(device=dev).manual_seed(100 + seed_base)
    for i in range(len(sb.layers)):
        sb.k[i].normal_(generator=g)
        sb.v[i].normal_(generator=g)
    sb.lengths[:seats].copy_(lengths)
    sb.lengths_cpu[:seats] = lengths.tolist()
    cb = Cb0Sampler(bb.cb0_head.weight, seats, temp=0.9, top_k=50, rep=0.0)
    for s in range(seats):
        cb.bind(s, seed=1 + s)
    fd = FastDepth(dm, seats, dtype=torch.bfloat16, temp=0.9, top_k=50, batch_buckets=(seats,), fused=True)
    fd.row_seed.copy_(torch.arange(seats + 1, dtype=torch.int32, device=dev) * 69069 + 1)
    fs = FrameStep(sb, cb, fd, ring_depth=64)
    fs.feedback.normal_(generator=g)
    return fs, bb, dm


def secondary(torch, bb, dm, steps, only=None):
    """The other GPU configurations, timed through the reference surfaces on the frame's weights:
    C2 = FastDepth.__call__ over 16 seats (the 4-layer depth frame over codebooks 1..31, top-k 50, T 0.9, h N(0,1),
    cb0 uniform in [0, 2048)); C3 = StaticBackbone.step over 64 seats (lengths U[64, 2048]) + cb0; C4 =
    StaticBackbone.step_mixed with 216 decoding seats (lengths log-uniform in [128, 4096)) and 8 inline prefills of
    256 tokens (embedding rows of uniform ids from a [151936, 1024] N(0, 0.02) table, starting at length 0) = 2264
    rows + cb0 over the 224 seats. Lengths are reset before every step, so each timed step does the same work.
    only: "c2", "c3" or "c4" runs that line alone and returns."""
    from m3x import roofline
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(300)
    out = {}

    def run(label, sb, base, step, rows, attended, note):
        def reset():
            sb.lengths[:len(base)].copy_(base.to(dev), non_blocking=True)
            sb.lengths_cpu[:len(base)] = base.tolist()
        for _ in range(2):
            reset()
            step()
        torch.cuda.synchronize()
        t = 0.0
        for _ in range(steps):
            reset()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            step()
            torch.cuda.synchronize()
            t += time.perf_counter() - t0
        ms = t * 1e3 / steps
        byt = roofline.backbone_step_bytes(attended, rows)
        flo = roofline.backbone_step_flops(attended, rows)
        out[label] = {"rows": rows, "ms_per_step": round(ms, 3), "bytes_algorithmic": byt, "flops_algorithmic": flo,
                      "hbm_fraction": round(byt / (ms * 1e-3) / 1e9 / roofline.HBM_PEAK_GBS, 4),
                      "mfma_fraction": round(flo / (ms * 1e-3) / 1e12 / roofline.MFMA_BF16_TFLOPS, 4), "note": note}
        log(f"{label}: {rows} rows, {ms:.3f} ms/step ({out[label]['hbm_fraction']:.1%} of the HBM and "
            f"{out[label]['mfma_fraction']:.1%} of the MFMA roofline)")

    if only in (None, "c2"):
        _c2(torch, dm, steps, g, dev, out, roofline)
    if only in (None, "c3"):
        _c3(torch, bb, g, dev, run)
    if only in (None, "c4"):
        _c4(torch, bb, g, dev, run)
    if only is not None:
        return out
    return _rest(torch, bb, dev, g, out, steps)


def _c2(torch, dm, steps, g, dev, out, roofline):
    """C2: FastDepth.__call__ over 16 seats."""
    from m3x.serve.fast_depth import FastDepth
    B2 = 16
    fd = FastDepth(dm, B2, dtype=torch.bfloat16, temp=0.9, top_k=50, batch_buckets=(B2,), fused=True)
    fd.row_seed.copy_(torch.arange(B2 + 1, dtype=torch.int32, device=dev) * 69069 + 7)
    h2 = torch.randn(B2, 1024, device=dev, generator=g).to(torch.bfloat16)
    cb02 = torch.randint(0, 2048, (B2,), device=dev, generator=g)
    slots2 = list(range(B2))
    fd.warmup()
    for _ in range(3):
        fd(slots2, h2, cb02)
    torch.cuda.synchronize()
    t = 0.0
    for _ in range(steps * 4):
        t0 = time.perf_counter()
        fd(slots2, h2, cb02)
        torch.cuda.synchronize()
        t += time.perf_counter() - t0
    ms = t * 1e3 / (steps * 4)
    byt = roofline.depth_frame_bytes(seats=B2)
    flo = roofline.depth_frame_flops(B2)
    out["c2"] = {"rows": B2, "ms_per_step": round(ms, 3), "bytes_algorithmic": byt, "flops_algorithmic": flo,
                 "hbm_fraction": round(byt / (ms * 1e-3) / 1e9 / roofline.HBM_PEAK_GBS, 4),
                 "mfma_fraction": round(flo / (ms * 1e-3) / 1e12 / roofline.MFMA_BF16_TFLOPS, 4),
                 "note": "FastDepth.__call__ (host staging + one graph replay of the 31-codebook depth frame + clone); "
                         "the bytes stream the trunk once per codebook (its 98 MB stays in the 256 MB MALL)"}
    log(f"c2: {B2} seats, {ms:.3f} ms/frame ({out['c2']['hbm_fraction']:.1%} of the HBM and "
        f"{out['c2']['mfma_fraction']:.1%} of the MFMA roofline)")
    del fd
    torch.cuda.empty_cache()


def _c3(torch, bb, g, dev, run):
    """C3: StaticBackbone.step over 64 seats + cb0."""
    from m3x import synth
    from m3x.cb0 import Cb0Sampler
    from m3x.serve.fast_backbone import StaticBackbone
    B3 = 64
    sb = StaticBackbone(bb, B3, capacity=CAP, batch_buckets=(B3,), ctx_buckets=(CAP,), attention="triton",
                        fuse_rope=True)
    for i in range(len(sb.layers)):
        sb.k[i].normal_(generator=g)
        sb.v[i].normal_(generator=g)
    cb = Cb0Sampler(bb.cb0_head.weight, B3, temp=0.9, top_k=50, rep=0.0)
    len3 = synth.c3_lengths(B3)
    x3 = torch.randn(B3, 1024, device=dev, generator=g).to(torch.bfloat16)
    idx3 = torch.arange(B3, device=dev)
    slots3 = list(range(B3))
    run("c3", sb, len3, lambda: cb(sb.step(slots3, x3), idx3), B3, int(len3.sum()) + B3,
        "StaticBackbone.step (host staging + one graph replay + clone) + eager cb0 (head GEMM, Philox, sampler)")
    del sb, cb
    torch.cuda.empty_cache()


def _c4(torch, bb, g, dev, run):
    """C4: StaticBackbone.step_mixed over 216 decode rows and 8 inline prefills of 256 tokens + cb0."""
    from m3x import synth
    from m3x.cb0 import Cb0Sampler
    from m3x.serve.fast_backbone import StaticBackbone
    nd, npf, T = 216, 8, 256
    sb = StaticBackbone(bb, nd + npf, capacity=CAP, batch_buckets=(nd + npf * T,), ctx_buckets=(CAP,),
                        attention="triton", fuse_rope=True)
    for i in range(len(sb.layers)):
        sb.k[i].normal_(generator=g)
        sb.v[i].normal_(generator=g)
    cb = Cb0Sampler(bb.cb0_head.weight, nd + npf, temp=0.9, top_k=50, rep=0.0)
    len4 = torch.cat([synth.c4_decode_lengths(nd), torch.zeros(npf, dtype=torch.long)])
    x4 = torch.randn(nd, 1024, device=dev, generator=g).to(torch.bfloat16)
    table = (torch.randn(151936, 1024, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    ids = torch.randint(0, 151936, (npf, T), device=dev, generator=g)
    pre = [(nd + j, table[ids[j]]) for j in range(npf)]
    del table
    idx4 = torch.arange(nd + npf, device=dev)
    slots4 = list(range(nd))

    def c4_step():
        dec, last = sb.step_mixed(slots4, x4, pre)
        return cb(torch.cat([dec, torch.stack(last)]), idx4)
    run("c4", sb, len4, c4_step, nd + npf * T, int(len4[:nd].sum()) + nd + npf * T,
        "StaticBackbone.step_mixed (216 decode + 8 x 256 prefill rows, one graph replay) + eager cb0 over 224 "
        "seats; algorithmic bytes read each prefill key once")
    del sb, cb, pre
    torch.cuda.empty_cache()


def _rest(torch, bb, dev, g, out, steps):
    """The loop guard, the tick readout, time to first audio and the Mimi lines."""
    from m3x.serve.fast_backbone import StaticBackbone
    # the engine's loop guard for 224 seats (maya3/guards.py:80-107): device history push + rule, graph-timed,
    # beside the same rule on the host over the same histories (the engine evaluates it on the host each tick)
    from types import SimpleNamespace
    from m3x.guards import LoopGuard
    from oracle import torch_oracle as O
    gcfg = SimpleNamespace(stall=32, period_win=64, period_thr=0.7, pmin=2, pmax=16, hist=96)
    Bg = 224
    lg = LoopGuard(Bg, gcfg, device=dev)
    gslots = torch.arange(Bg, device=dev)
    gcodes = torch.randint(0, 2048, (Bg,), device=dev, generator=g)
    gout = torch.empty(Bg, dtype=torch.int32, device=dev)
    for _ in range(100):
        lg.push(gslots, gcodes)
    stream = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    gg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gg, stream=side):
        for _ in range(20):
            lg.push(gslots, gcodes)
            lg.detect(gslots, gout)
    gg.replay()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(5):
        gg.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    gpu_us = e0.elapsed_time(e1) * 1e3 / 100
    Wh, nh = lg.hist[:Bg].cpu().numpy(), lg.frames[:Bg].cpu().numpy()
    t0 = time.perf_counter()
    for _ in range(5):
        O.loop_detect_batch(Wh, nh)
    cpu_us = (time.perf_counter() - t0) / 5 * 1e6
    out["loop_guard"] = {"seats": Bg, "gpu_us": round(gpu_us, 2), "cpu_us": round(cpu_us, 1),
                         "note": "push + rule per frame in the graph, against the rule over the same histories on "
                                 "one host thread"}
    log(f"loop guard, {Bg} seats: {gpu_us:.2f} us on the GPU (push + rule), {cpu_us:.0f} us on the host")
    del lg

    # the tick's readout for 224 seats: stop, cb0, loop code, 32 codes and 1920 PCM samples packed by one kernel
    # and copied to pinned host memory in one transfer (maya3/engine.py:558-563), wall time to the host
    from m3x.tick import TickReadout
    rd = TickReadout(Bg, frame=1920, nq=32, with_loop=True, device=dev)
    tstop = torch.zeros(Bg, dtype=torch.int64, device=dev)
    tcb0 = torch.randint(0, 2048, (Bg,), device=dev, generator=g)
    tcodes = torch.randint(0, 2048, (Bg, 32), device=dev, generator=g).to(torch.int32)
    tpcm = torch.randn(Bg, 1920, device=dev, generator=g) * 0.3
    ts = []
    for i in range(22):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        rd.pack(tstop, tcb0, gout, tcodes, tpcm)
        rd.wait()
        if i >= 2:
            ts.append(time.perf_counter() - t0)
    out["tick_readout"] = {"seats": Bg, "bytes": Bg * rd.width * 8,
                           "us": round(sorted(ts)[len(ts) // 2] * 1e6, 1),
                           "note": "one pack kernel + one pinned D2H copy + event wait, median wall time"}
    log(f"tick readout, {Bg} seats ({Bg * rd.width * 8 / 1e3:.0f} kB): {out['tick_readout']['us']:.0f} us")
    del rd

    # time to first audio: a 512-token prompt prefilled onto one empty seat through the graphed inline-prefill
    # step (StaticBackbone.prefill), beside the eager HF forward the engine falls back to (maya3/engine.py:497-502)
    Tp = 512
    sb = StaticBackbone(bb, 2, capacity=CAP, batch_buckets=(Tp,), ctx_buckets=(CAP,), attention="triton",
                        fuse_rope=True)
    xp = (torch.randn(Tp, 1024, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    sb.prefill(0, xp)
    ts = []
    for _ in range(steps):
        sb.free(0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        sb.prefill(0, xp)
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    pre_ms = sorted(ts)[len(ts) // 2] * 1e3
    out["ttfa_prefill"] = {"tokens": Tp, "ms": round(pre_ms, 3),
                           "note": "StaticBackbone.prefill of 512 tokens onto an empty seat (one graph replay), median"}
    try:
        out["ttfa_prefill"]["hf_eager_ms"] = round(_hf_eager_prefill_ms(torch, bb, xp, steps), 3)
    except Exception as e:  # the comparison is informative only
        log(f"HF eager prefill comparison skipped: {e}")
    log(f"prefill of {Tp} tokens: {pre_ms:.2f} ms (HF eager: {out['ttfa_prefill'].get('hf_eager_ms')})")
    del sb
    torch.cuda.empty_cache()
    out["depthv2_geometry"] = depthv2_frame(torch, max(steps * 4, 20))
    out["mimi_decode"] = mimi_decode(torch, dev, max(steps, 20))
    return out


def depthv2_frame(torch, steps, seat_counts=(1, 16)):
    """The reference's own depth geometry, timed: a DepthV2-shaped trunk (LayerNorm + GELU 3072, 16 heads x 64, 4
    layers, the 11 weight groups of GROUP_OF_LEVEL, rank-128 code embeddings, per-layer speaker cross constants set
    for every seat) as an fp16 FastDepth (the engine's default depth dtype, maya3/engine.py:53) with the reference's
    sampling defaults (temp 0.7, top-k 64). Graph-timed depth frame (HIP events over replays of the FastDepth graph)
    and the wall time of __call__, at 1 and 16 seats, beside the reference's published depth stage of its
    one-seat frame: 6.5 ms on an H100 NVL (docs/ENGINE.md:211, its real 555M decoder of this geometry)."""
    from m3x import roofline, synth
    from m3x.serve.fast_depth import FastDepth
    dev = torch.device("cuda:0")
    model = synth.depthv2_like(seed=2, device=dev, dtype=torch.float16, affine_std=0.1)
    S = max(seat_counts)
    fd = FastDepth(model, S, dtype=torch.float16, temp=0.7, top_k=64, batch_buckets=tuple(seat_counts), fused=True)
    g = torch.Generator(device=dev).manual_seed(400)
    for s in range(S):
        fd.set_speaker(s, torch.randn(1, 1, 1024, device=dev, generator=g), torch.ones(1, 1, device=dev))
    fd.row_seed.copy_(torch.arange(S + 1, dtype=torch.int32, device=dev) * 7919 + 3)
    fd.warmup()
    stream = torch.cuda.current_stream()
    res = {"geometry": "DepthV2: LayerNorm + GELU 3072, 16 x 64 heads, 4 layers, 11 weight groups "
                       "(GROUP_OF_LEVEL), speaker constants; fp16; temp 0.7, top-k 64",
           "reference_b1_depth_ms": 6.5, "reference_hardware": "1x H100 NVL (docs/ENGINE.md:211)"}
    for B in seat_counts:
        h = torch.randn(B, 1024, device=dev, generator=g).to(torch.float16)
        cb0 = torch.randint(0, 2048, (B,), device=dev, generator=g)
        slots = list(range(B))
        for _ in range(3):
            fd(slots, h, cb0)
        torch.cuda.synchronize()
        ts = []
        for _ in range(steps):
            t0 = time.perf_counter()
            fd(slots, h, cb0)
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        gr = fd._graph(fd.bucket_for(B))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            gr.graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        gms = e0.elapsed_time(e1) / steps
        byt = roofline.depth_frame_bytes(ffn=3072, ffn_mats=2, seats=B)
        res[f"b{B}"] = {"seats": B, "graph_ms": round(gms, 4), "call_wall_ms": round(sorted(ts)[len(ts) // 2] * 1e3, 4),
                        "persistent_levels": bool(fd._persistent_ok(B, 10)), "bytes_algorithmic": byt,
                        "hbm_fraction": round(byt / (gms * 1e-3) / 1e9 / roofline.HBM_PEAK_GBS, 4)}
        log(f"DepthV2 geometry fp16, {B} seats: {gms:.3f} ms per depth frame in the graph "
            f"(reference: 6.5 ms at one seat on an H100 NVL)")
    del fd, model
    torch.cuda.empty_cache()
    return res


def mimi_decode(torch, dev, steps):
    """One 80 ms Mimi frame per seat (32 codes -> 1920 PCM samples) through StaticMimi's graph at 1, 64 and 224
    seats (HIP-event time of the replay, and the wall time of decode() with its slot/code uploads and the owned
    output), beside one frame of the fp32 streaming oracle on the host at one seat. The headline figures compute in
    float32, the Mimi module's dtype and so the reference's precision (serve/fast_codec.py:47-49,
    maya3/engine.py:165,201); the `fp16` object is the opt-in float16 variant."""
    from m3x import synth
    from oracle.mimi_oracle import MimiStream
    res = _mimi_variant(torch, dev, steps, torch.float32)
    res["fp16"] = _mimi_variant(torch, dev, steps, torch.float16)
    mc = synth.mimi(seed=7)
    st = MimiStream(mc, 1)
    c = synth.mimi_codes(1, 4, seed=8)
    with torch.no_grad():
        st.decode_frame(c[:, :, 0])
        t0 = time.perf_counter()
        for t in range(1, 4):
            st.decode_frame(c[:, :, t])
    res["cpu_oracle_ms_b1"] = round((time.perf_counter() - t0) / 3 * 1e3, 2)
    res["cpu_cores"] = torch.get_num_threads()
    res["note"] = ("StaticMimi in float32 (the reference's precision; the fp16 object: float16 storage with fp32 "
                   "accumulation); realtime_x = seconds of audio per second of GPU time; CPU: the fp32 streaming "
                   "oracle, one seat")
    return res


def _mimi_variant(torch, dev, steps, dtype):
    from m3x import synth
    from m3x.serve.fast_codec import StaticMimi
    sm = StaticMimi(synth.mimi(seed=7, device=dev), 224, batch_buckets=(1, 64, 224), dtype=dtype)
    res = {"dtype": str(dtype).replace("torch.", "")}
    stream = torch.cuda.current_stream()
    with torch.inference_mode():
        sm.warmup()
        for B in (1, 64, 224):
            codes = synth.mimi_codes(B, 1, seed=8)[:, :, 0].to(dev)
            slots = list(range(B))
            for _ in range(3):
                sm.decode(slots, codes)
            bucket = sm._buckets[B]
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(steps):
                bucket.graph.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            gpu_ms = e0.elapsed_time(e1) / steps
            ts = []
            for _ in range(steps):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                sm.decode(slots, codes)
                torch.cuda.synchronize()
                ts.append(time.perf_counter() - t0)
            wall_ms = sorted(ts)[len(ts) // 2] * 1e3
            res[f"b{B}"] = {"seats": B, "graph_ms": round(gpu_ms, 4), "decode_wall_ms": round(wall_ms, 4),
                            "frames_per_s": round(B / gpu_ms * 1e3, 1),
                            "realtime_x": round(B * 80.0 / gpu_ms, 1)}
            log(f"Mimi decode ({res['dtype']}), {B} seats: {gpu_ms:.3f} ms per frame in the graph, "
                f"decode() {wall_ms:.3f} ms wall")
    del sm
    torch.cuda.empty_cache()
    return res


def _hf_eager_prefill_ms(torch, bb, x, steps):
    """The reference's eager fallback for a long prompt (`self.model.backbone(prompt, use_cache=True)`): HF
    transformers' Qwen3Model on the same weights, bf16, on this GPU; median ms."""
    from transformers import Qwen3Config, Qwen3Model
    L0 = bb.lm.model.layers
    cfg = Qwen3Config(hidden_size=1024, intermediate_size=3072, num_hidden_layers=len(L0), num_attention_heads=16,
                      num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6, rope_theta=1e6, vocab_size=16,
                      max_position_embeddings=4096)
    dev = x.device
    m = Qwen3Model(cfg).to(device=dev, dtype=torch.bfloat16).eval()
    sd = {"norm.weight": bb.lm.model.norm.weight}
    for i, L in enumerate(L0):
        a, f = L.self_attn, L.mlp
        for name, w in (("self_attn.q_proj", a.q_proj), ("self_attn.k_proj", a.k_proj), ("self_attn.v_proj", a.v_proj),
                        ("self_attn.o_proj", a.o_proj), ("mlp.gate_proj", f.gate_proj), ("mlp.up_proj", f.up_proj),
                        ("mlp.down_proj", f.down_proj)):
            sd[f"layers.{i}.{name}.weight"] = w.weight
        sd[f"layers.{i}.self_attn.q_norm.weight"] = a.q_norm.weight
        sd[f"layers.{i}.self_attn.k_norm.weight"] = a.k_norm.weight
        sd[f"layers.{i}.input_layernorm.weight"] = L.input_layernorm.weight
        sd[f"layers.{i}.post_attention_layernorm.weight"] = L.post_attention_layernorm.weight
    m.load_state_dict(sd, strict=False)
    ts = []
    with torch.inference_mode():
        for i in range(steps + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            m(inputs_embeds=x[None], use_cache=True)
            torch.cuda.synchronize()
            if i:
                ts.append(time.perf_counter() - t0)
    del m
    torch.cuda.empty_cache()
    return sorted(ts)[len(ts) // 2] * 1e3


def _cpu_frames(torch, O, bb, dm, seats, seconds, seed, tiled=False, min_frames=2):
    """Seconds per eager oracle frame (backbone + cb0 + depth + feedback) at `seats` seats of the C5 shapes, over
    the frames that fit in `seconds` after one untimed frame (at least min_frames, at most 50). tiled: every slot's K/V is
    one random slot's, copied (drawing ~60 GB of normals for 224 seats would take minutes on one thread; the
    arithmetic and the bytes streamed are the same)."""
    from m3x import synth
    lengths = synth.c5_lengths(seats, seed=seed)
    cap = int(lengths.max()) + 64
    g = torch.Generator().manual_seed(200 + seats)
    if tiled:
        def cache():
            one = torch.randn(1, 8, cap, 128, generator=g).to(torch.bfloat16)
            return one.expand(seats + 1, 8, cap, 128).contiguous()
        kc = [cache() for _ in range(28)]
        vc = [cache() for _ in range(28)]
    else:
        kc = [torch.randn(seats + 1, 8, cap, 128, generator=g).to(torch.bfloat16) for _ in range(28)]
        vc = [torch.randn(seats + 1, 8, cap, 128, generator=g).to(torch.bfloat16) for _ in range(28)]
    L = torch.cat([lengths, torch.zeros(1, dtype=torch.long)])
    cos, sin = O.rope_tables(128, 1e6, cap, torch.bfloat16)
    x = torch.randn(seats, 1024, generator=g).to(torch.bfloat16)
    slots = torch.arange(seats)
    frames, t0 = -1, 0.0
    while True:
        h = O.backbone_step(bb, kc, vc, L, slots, x, cos, sin)
        u = torch.rand(seats, 32, generator=g)
        cb0, _ = O.cb0_step(bb.cb0_head.weight, h, u[:, 0], 0.9, 50)
        codes, _ = O.depth_frame(dm, h, cb0, u[:, 1:], 0.9, 50)
        x = O.feedback(dm.audio_in, codes)
        frames += 1
        if frames == 0:
            t0 = time.perf_counter()
            continue
        el = time.perf_counter() - t0
        log(f"cpu baseline, {seats} seats, frame {frames}: {el:.1f}s")
        if (el >= seconds and frames >= min_frames) or frames >= 50:
            return el / frames, frames, lengths.tolist()


def _host_ram_gib():
    try:
        return round(os.sysconf("SC_PAGE_SIZE") * os.sysconf("SC_PHYS_PAGES") / 2 ** 30, 1)
    except (ValueError, OSError):
        return None


# host RAM that the full 224-seat CPU frame asks for: 2x its ~58 GB KV cache (its KV history is max length + 64
# positions per slot, not the GPU cache's 4096)
FULL_CPU_RAM_GIB = 120


def cpu_baseline(torch, seconds, sizes=(2, 10)):
    """The oracle's eager frame (backbone + cb0 + depth) on the host cores at the C5 shapes. With at least
    FULL_CPU_RAM_GIB of host RAM the full 224-seat frame is timed (cpu_full_frame: one untimed frame, then one or
    more timed frames filling about seconds / 2; ~40 s of wall time with the cache fill). Otherwise it is timed at
    two seat counts and fitted as t(B) = a + b B: the fixed part a (weights streamed and converted once per frame,
    whatever the seats) and the per-seat part b (the seat's KV history, its rows through every projection, its
    sampling) both measured, then the 224-seat frame time a + 224 b, labelled extrapolated (the fit overstates the
    per-seat cost: the full frame measured 12.5 s on 16 host threads where the fit gave ~23 s)."""
    ram_gb = _host_ram_gib()
    if ram_gb is not None and ram_gb >= FULL_CPU_RAM_GIB:
        out = cpu_full_frame(torch, seconds / 2, min_frames=1)
        out.update(host_ram_gib=ram_gb, host_cpus=os.cpu_count())
        return out
    from m3x import synth
    from oracle import torch_oracle as O
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    bb = synth.qwen3_backbone(layers=28, seed=0, device="cpu", affine=synth.AFFINE)
    dm = synth.swiglu_depth(seed=1, device="cpu", affine=synth.AFFINE)
    pts = [(s,) + _cpu_frames(torch, O, bb, dm, s, seconds / len(sizes), 5) for s in sizes]
    (s1, t1, n1, l1), (s2, t2, n2, l2) = pts
    b = (t2 - t1) / (s2 - s1)
    a = t1 - b * s1
    t224 = a + 224 * b
    return dict(value=round(224 / t224, 4), unit="frames/s", cores=threads, kind="port", extrapolated=True,
                host_ram_gib=ram_gb, host_cpus=os.cpu_count(),
                fit={"fixed_s_per_frame": round(a, 4), "s_per_seat_frame": round(b, 5),
                     "points": [{"seats": s1, "s_per_frame": round(t1, 4), "frames": n1},
                                {"seats": s2, "s_per_frame": round(t2, 4), "frames": n2}]},
                sample=f"the PyTorch-eager oracle's frame (28 layers, cb0, depth over 31 codebooks) on {threads} host "
                       f"threads at {s1} seats (KV lengths {l1}: {t1:.2f} s per frame over {n1} frames) and {s2} "
                       f"seats ({t2:.2f} s over {n2} frames), fitted as {a:.3f} s + {b:.4f} s per seat: a 224-seat "
                       f"frame takes {t224:.1f} s on this host (not run in full: the host has {ram_gb} GiB of RAM, "
                       f"under the {FULL_CPU_RAM_GIB} GiB the full frame's KV cache asks for)")


def cpu_full_frame(torch, seconds, min_frames=2):
    """The oracle's eager frame on the host cores at all 224 seats of the C5 shapes (the KV lengths of the GPU
    frame, synth.c5_lengths(224)), timed in full rather than fitted from seat subsets: one untimed frame, then
    timed frames until `seconds` have passed, at least min_frames (the KV cache alone is ~58 GB of host memory)."""
    from m3x import synth
    from oracle import torch_oracle as O
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    bb = synth.qwen3_backbone(layers=28, seed=0, device="cpu", affine=synth.AFFINE)
    dm = synth.swiglu_depth(seed=1, device="cpu", affine=synth.AFFINE)
    lengths = synth.c5_lengths(224)
    t0 = time.perf_counter()
    t, n, _ = _cpu_frames(torch, O, bb, dm, 224, seconds, 5, tiled=True, min_frames=min_frames)  # c5_lengths' seed
    return dict(value=round(224 / t, 4), unit="frames/s", cores=threads, kind="port", extrapolated=False,
                s_per_frame=round(t, 3), frames=n, wall_s=round(time.perf_counter() - t0, 1),
                sample=f"the PyTorch-eager oracle's full frame (28 layers, cb0, depth over 31 codebooks) at 224 seats "
                       f"(KV lengths synth.c5_lengths(224), mean {float(lengths.float().mean()):.0f}) on {threads} "
                       f"host threads: {t:.2f} s per frame over {n} timed frames after one untimed; every slot's K/V "
                       f"is one random slot's, copied")


def c1_cpu(torch, reps=20):
    """C1: one Qwen3-0.6B-shaped decoder layer (+ final norm), one decode step at B=1 over a 256-token cache, fp32,
    through the oracle's eager restatement of the reference path on the host cores (CPU-only by definition)."""
    from m3x import synth
    from oracle import torch_oracle as O
    bb = synth.qwen3_backbone(layers=1, seed=0, dtype=torch.float32)
    g = torch.Generator().manual_seed(10)
    kc = [torch.zeros(2, 8, 512, 128)]
    vc = [torch.zeros(2, 8, 512, 128)]
    kc[0][0, :, :256] = torch.randn(8, 256, 128, generator=g)
    vc[0][0, :, :256] = torch.randn(8, 256, 128, generator=g)
    x = torch.randn(1, 1024, generator=g)
    cos, sin = O.rope_tables(128, 1e6, 512, torch.float32)
    slots = torch.tensor([0])
    t = 0.0
    for i in range(reps + 2):
        lengths = torch.tensor([256, 0])
        t0 = time.perf_counter()
        O.backbone_step(bb, kc, vc, lengths, slots, x, cos, sin)
        if i >= 2:
            t += time.perf_counter() - t0
    return {"ms_per_step": round(t * 1e3 / reps, 3), "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{reps} steps of one fp32 layer at B=1, cache 256 tokens"}


def _traffic_ratio():
    """HBM bytes per algorithmic byte of the decode attention, measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, each scaled by the counts of a plain copy of known size) on this workload and recorded in
    profiles/; None if the record is absent."""
    path = os.path.join(ROOT, "profiles", "decode_attn_b224_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_per_algorithmic_byte:"):
            return float(line.split(":", 1)[1].split()[0])
    return None


def b1_latency(torch, replays, bb=None, dm=None):
    """Median latency (us) of the frame graph at one seat (KV length 2048), over `replays` replays."""
    log("B=1 frame latency (length 2048)")
    stream = torch.cuda.current_stream()
    fs1, _, _ = build_frame(torch, 1, torch.tensor([2048]), seed_base=1, backbone=bb, depth_model=dm)
    g1 = fs1.capture(1, CAP)
    fs1.set_slots(g1, [0])
    for _ in range(5):
        fs1.replay(g1)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
    for a, b in ev:
        a.record(stream)
        fs1.replay(g1)
        b.record(stream)
    torch.cuda.synchronize()
    lat = sorted(a.elapsed_time(b) * 1e3 for a, b in ev)
    log(f"B=1: median {lat[len(lat) // 2]:.0f} us over {len(lat)} replays")
    return lat[len(lat) // 2]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=224)
    ap.add_argument("--b1-replays", type=int, default=200)
    ap.add_argument("--attn-iters", type=int, default=56)
    ap.add_argument("--copy-probe", action="store_true", help="also run one 256 MiB device copy (counter scale)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-b1", action="store_true")
    ap.add_argument("--no-secondary", action="store_true", help="skip the C3 / C4 backbone-step lines")
    ap.add_argument("--secondary-steps", type=int, default=5)
    ap.add_argument("--mimi-only", action="store_true", help="print only the Mimi decode line (for profiling)")
    ap.add_argument("--b1-only", action="store_true", help="print only the B=1 frame latency (for profiling)")
    ap.add_argument("--only", choices=("c2", "c3", "c4"), help="print only that configuration's line (for profiling)")
    ap.add_argument("--cpu-full", action="store_true",
                    help="print only the oracle's full 224-seat frame on the host cores (minutes, ~60 GB of RAM)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the frame step shards by seats with no collectives, and the benchmark "
              "runs on a single MI355X (run with --gpus 1).", file=sys.stderr)
        sys.exit(2)

    import torch
    from m3x import roofline, synth
    from m3x import ops
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.cpu_full:
        log("the oracle's full 224-seat frame on the host cores")
        print(json.dumps({"cpu_full_frame": cpu_full_frame(torch, args.cpu_seconds)}), flush=True)
        return
    if args.mimi_only:
        print(json.dumps({"mimi_decode": mimi_decode(torch, torch.device("cuda:0"), max(args.secondary_steps, 20))}),
              flush=True)
        return
    B = args.batch
    K, W = args.steps, args.warmup
    dev = torch.device("cuda:0")
    if args.b1_only:
        with torch.inference_mode():
            print(json.dumps({"b1_frame_us": round(b1_latency(torch, args.b1_replays), 1)}), flush=True)
        return
    if args.only:
        with torch.inference_mode():
            bb = synth.qwen3_backbone(layers=28, seed=0, device=dev, gen="cuda", affine=synth.AFFINE)
            dm = synth.swiglu_depth(seed=1, device=dev, gen="cuda", affine=synth.AFFINE)
            print(json.dumps({"backbone_configs": secondary(torch, bb, dm, args.secondary_steps, only=args.only)}),
                  flush=True)
        return
    log(f"device {torch.cuda.get_device_name(0)}; building the B={B} frame (KV {B + 1} slots x {CAP})")
    lengths = synth.c5_lengths(B)
    if int(lengths.max()) + W + K + 1 > CAP:
        raise SystemExit("lengths + steps exceed the KV capacity")
    with torch.inference_mode():
        fs, bb, dm = build_frame(torch, B, lengths)
        torch.cuda.synchronize()
        log(f"KV cache {fs.bb.memory_bytes() / 1e9:.1f} GB; capturing the frame graph")
        g = fs.capture(B, CAP)
        fs.set_slots(g, list(range(B)))
        for _ in range(W):
            fs.replay(g)
        torch.cuda.synchronize()
        attended0 = int(fs.bb.lengths[:B].sum()) + B  # keys attended in the first timed step
        log(f"timing {K} frame steps")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(K):
            fs.replay(g)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        ms = (t1 - t0) * 1e3 / K
        fps = B / (ms / 1e3)
        log(f"B={B}: {ms:.3f} ms/frame, {fps:.0f} frames/s")
        codes = fs.codes(g)[:B]
        if not (codes.min().item() >= 0 and codes.max().item() < 2048):
            raise SystemExit("codes out of range")
        attended = attended0 + (K - 1) * B // 2  # mean over the timed steps

        # decode attention alone, live, on the launch stream: the frame's own buffers, each layer over its own
        # cache as in the frame (a cache is 1.9 GB, far above the 256 MB MALL, so every launch streams from HBM)
        bufs = g["bufs"][0]
        sb = fs.bb
        o = torch.empty_like(bufs.q)
        att_keys = int((bufs.pos[:B].long() + 1).sum())
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        nl = len(sb.k)

        def attn_launch(i):
            ops.decode_attn(bufs.q, sb.k[i % nl], sb.v[i % nl], o, bufs.slots, bufs.pos, sb.scaling, bufs.ctx,
                            bufs.chunk, bufs.attn_ws, sb.heads, sb.kv_heads)
        for i in range(3):
            attn_launch(i)
        e0.record(stream)
        for i in range(args.attn_iters):
            attn_launch(i)
        e1.record(stream)
        torch.cuda.synchronize()
        attn_us = e0.elapsed_time(e1) * 1e3 / args.attn_iters
        attn_bytes = roofline.decode_attn_bytes(att_keys, B)
        attn_gbs = attn_bytes / (attn_us * 1e-6) / 1e9
        log(f"decode attention: {attn_us:.1f} us/launch, {attn_gbs:.0f} GB/s ({attn_gbs / roofline.HBM_PEAK_GBS:.1%})")
        # fused residual add + RMSNorm (the backbone's norm kernel): at the frame's 224 rows, over rotating
        # buffer sets, launched from a graph as in the frame, and at a streaming size (2 GB per launch) where
        # launch latency is amortised
        norm = {}
        hw = torch.ones(1024, dtype=torch.bfloat16, device=dev)
        for label, rows, sets, iters in (("frame", B, 8, 64), ("stream", 262144, 1, 8)):
            bufsets = [[torch.randn(rows, 1024, device=dev).to(torch.bfloat16) for _ in range(4)] for _ in range(sets)]

            def norms():
                for i in range(iters):
                    bs = bufsets[i % sets]
                    ops.add_rms(bs[0], bs[1], hw, 1e-6, bs[2], bs[3])
            side = torch.cuda.Stream()
            side.wait_stream(stream)
            with torch.cuda.stream(side):
                norms()
            stream.wait_stream(side)
            ng = torch.cuda.CUDAGraph()
            with torch.cuda.graph(ng, stream=side):
                norms()
            ng.replay()
            e0.record(stream)
            for _ in range(3):
                ng.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            n_us = e0.elapsed_time(e1) * 1e3 / (3 * iters)
            n_gbs = roofline.add_norm_bytes(rows) / (n_us * 1e-6) / 1e9
            norm[label] = {"rows": rows, "launch_us": round(n_us, 2), "achieved": round(n_gbs, 1),
                           "frac": round(n_gbs / roofline.HBM_PEAK_GBS, 4)}
            log(f"add+RMSNorm {label} ({rows} rows): {n_us:.2f} us/launch, {n_gbs:.0f} GB/s "
                f"({n_gbs / roofline.HBM_PEAK_GBS:.1%})")
            del bufsets
        torch.cuda.empty_cache()
        if args.copy_probe:
            # a plain device copy of known size: what FETCH_SIZE / WRITE_SIZE read for it scales their counts
            src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
            dst = torch.empty_like(src)
            dst.copy_(src)
            torch.cuda.synchronize()
            del src, dst
        step_bytes = roofline.backbone_step_bytes(attended, B) + roofline.depth_frame_bytes(seats=B)
        del fs, g, bufs, o
        torch.cuda.empty_cache()

        b1_us = None
        if not args.no_b1:
            b1_us = b1_latency(torch, args.b1_replays, bb, dm)
        sec = None
        if not args.no_secondary:
            sec = secondary(torch, bb, dm, args.secondary_steps)
        del bb, dm
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        log(f"CPU baseline (~{args.cpu_seconds:.0f} s)")
        cpu = cpu_baseline(torch, args.cpu_seconds)
        cpu["c1"] = c1_cpu(torch)
        log(f"c1 (one fp32 decoder layer, B=1, CPU): {cpu['c1']['ms_per_step']:.2f} ms")

    ratio = _traffic_ratio()
    out = {
        "metric": "audio frames/sec at B=224 frame step; B=1 frame µs; % HBM/MFMA roofline",
        "value": round(fps, 1),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded random-init weights N(0,0.02), KV cache and feedback N(0,1), Philox uniforms",
        "config": {"workload": "full Maya3 frame step, one hipGraph: 28-layer Qwen3-0.6B-shaped backbone decode "
                               "(hidden 1024, 16q/8kv x 128, SwiGLU 3072) over a static KV cache (224 seats, cap "
                               "4096, lengths Poisson(2048)), cb0 top-k 50, 4-layer SwiGLU-2816 depth over "
                               "codebooks 1..31 (top-k 50, T 0.9), int32 [224,32] code ring",
                   "seats": B, "kv_capacity": CAP, "mean_kv_len": round(float(lengths.float().mean()), 1),
                   "parallelism": "single GPU (seats are data-parallel within the GPU)"},
        "b1_frame_us": None if b1_us is None else round(b1_us, 1),
        "audio_s_per_s": round(fps * 0.08, 1),
        "frame_bytes_algorithmic": step_bytes,
        "frame_hbm_fraction": round(step_bytes / (ms * 1e-3) / 1e9 / roofline.HBM_PEAK_GBS, 4),
        "roofline": {"kernel": "decode_attn over the B=224 step's caches (layers in turn)", "bound": "hbm",
                     "achieved": round(attn_gbs, 1), "peak": roofline.HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(attn_gbs / roofline.HBM_PEAK_GBS, 4), "traffic": None if ratio is None else int(ratio * attn_bytes),
                     "launch_us": round(attn_us, 2), "bytes_per_launch": attn_bytes},
        "norm_roofline": {"kernel": "add_rms (residual add + RMSNorm, hidden 1024)", "bound": "hbm", "unit": "GB/s",
                          "peak": roofline.HBM_PEAK_GBS, **norm},
        "backbone_configs": sec,
        "cpu_baseline": cpu,
    }
    md = (sec or {}).get("mimi_decode", {}).get(f"b{B}")
    tr = (sec or {}).get("tick_readout")
    if md and tr:
        # the whole tick at the headline batch: frame graph, then the codec on its codes, then the host readout
        tick_ms = ms + md["graph_ms"] + tr["us"] * 1e-3
        out["tick"] = {"seats": B, "frame_ms": round(ms, 4), "codec_ms": md["graph_ms"],
                       "readout_ms": round(tr["us"] * 1e-3, 4), "tick_ms": round(tick_ms, 4),
                       "audio_s_per_s": round(B * 0.08 / (tick_ms * 1e-3), 1),
                       "note": "sum of the three parts measured separately (frame graph, StaticMimi graph at the "
                               "same seat count, pack + pinned copy)"}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
