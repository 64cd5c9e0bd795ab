"""Writes tests/golden/depth_v2_frame.npz: one depth frame computed by the reference's own FastDepth._compute
(serve/fast_depth.py:84-141) over the reference's DepthV2 (tts/model/depth_v2.py:145-230) and AudioInputEmbed
(tts/model/audio_io.py:17-35), in fp32, greedy, on the CPU. The reference's depth path is plain torch (its
Triton parts are the fused variant, not used here), so it runs here as written.

This script imports /root/reference and runs only in the build container; the fixture it writes is data (inputs
and outputs), and the tests regenerate the weights from the seed instead of storing them.

Weights: m3x.synth.depthv2_like(seed=SEED, affine_std=0.1) in fp32 (all 11 weight groups, the reference's
GROUP_OF_LEVEL), copied parameter by parameter into DepthV2(d_backbone=1024) and AudioInputEmbed(1024); the
feedback table is the synth's bf16 table widened to fp32.
Inputs (torch.Generator seed SEED + 1, in order): h [B, 1024] N(0, 1), cb0 [B] in [0, 2048), speaker memories
[B, 1, 1, 1024] N(0, 1) installed with set_speaker on slots SLOTS.
Outputs: codes [B, 32] (int64), the 31 head outputs [B, 31, 2048] (fp32, captured by forward hooks on the heads
of FastDepth's private copy), feedback [B, 1024], cross_const rows of SLOTS [B, 4, 1024].
Run: python tests/golden/make_depth_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.join(HERE, "..", "..")
sys.path.insert(0, os.path.join(ROOT, "maya2-native_amd"))

SEED = 401
B = 2
SLOTS = [3, 0]
MAX_SLOTS = 4


def golden_inputs():
    """(synth model, h, cb0, mems) exactly as this script and the tests build them."""
    from m3x import synth
    model = synth.depthv2_like(seed=SEED, affine_std=0.1, dtype=torch.float32)
    g = torch.Generator().manual_seed(SEED + 1)
    h = torch.randn(B, 1024, generator=g)
    cb0 = torch.randint(0, 2048, (B,), generator=g)
    mems = torch.randn(B, 1, 1, 1024, generator=g)
    return model, h, cb0, mems


def _reference_model(model):
    sys.path.insert(0, "/root/reference")
    from tts.model.audio_io import AudioInputEmbed
    from tts.model.depth_v2 import DepthV2
    s = model.depth
    ref = DepthV2(d_backbone=1024).eval()
    put = lambda dst, src: dst.data.copy_(src.detach().float())  # noqa: E731
    put(ref.in_proj.weight, s.in_proj.weight)
    put(ref.code_lo.weight, s.code_lo.weight)
    put(ref.code_up.weight, s.code_up.weight)
    put(ref.level_emb.weight, s.level_emb.weight)
    for g_ref, g_syn in zip(ref.groups, s.groups):
        for blk, sb in zip(g_ref, g_syn):
            for name in ("n1", "n2"):
                put(getattr(blk, name).weight, getattr(sb, name).weight)
                put(getattr(blk, name).bias, getattr(sb, name).bias)
            for name in ("qkv", "o", "f1", "f2"):
                put(getattr(blk, name).weight, getattr(sb, name).weight)
    for c_ref, c_syn in zip(ref.cross, s.cross):
        put(c_ref.kv.weight, c_syn.kv.weight)
        put(c_ref.o.weight, c_syn.o.weight)
    put(ref.norm.weight, s.norm.weight)
    put(ref.norm.bias, s.norm.bias)
    for h_ref, h_syn in zip(ref.heads, s.heads):
        put(h_ref.weight, h_syn.weight)
    audio = AudioInputEmbed(1024).eval()
    put(audio.table.weight, model.audio_in.table.weight)
    put(audio.norm.weight, model.audio_in.norm.weight)
    from types import SimpleNamespace
    return SimpleNamespace(depth=ref, audio_in=audio)


def main():
    model, h, cb0, mems = golden_inputs()
    ref_model = _reference_model(model)
    from serve.fast_depth import FastDepth
    with torch.inference_mode():
        fd = FastDepth(ref_model, MAX_SLOTS, dtype=torch.float32, greedy=True)
        for b, slot in enumerate(SLOTS):
            fd.set_speaker(slot, mems[b], torch.ones(1, 1))
        logits = []
        hooks = [head.register_forward_hook(lambda mod, inp, out: logits.append(out.detach().clone()))
                 for head in fd.depth.heads]
        codes, feedback = fd._compute(torch.tensor(SLOTS), h, cb0)
        for hk in hooks:
            hk.remove()
    assert len(logits) == 31
    np.savez_compressed(os.path.join(HERE, "depth_v2_frame.npz"), codes=codes.numpy().astype(np.int64),
                        logits=torch.stack(logits, 1).numpy().astype(np.float32),
                        feedback=feedback.float().numpy(), cross=fd.cross_const[SLOTS].float().numpy())
    print("codes", codes.tolist())


if __name__ == "__main__":
    main()
