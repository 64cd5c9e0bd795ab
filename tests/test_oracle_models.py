"""Pins of the PyTorch CPU oracle (oracle/torch_oracle.py) against HF transformers (the reference's backbone
dependency), the committed C1 golden fixture, and the depth invariants the reference itself asserts. CPU only."""
import math
import os
import sys

import numpy as np
import pytest
import torch

from m3x import synth
from oracle import torch_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from make_golden import c1_inputs, hf_c1  # noqa: E402


def _c1_oracle(bb, k, v, x):
    kc = [torch.zeros(2, 8, 512, 128)]
    vc = [torch.zeros(2, 8, 512, 128)]
    kc[0][0, :, :256] = k[0]
    vc[0][0, :, :256] = v[0]
    lengths = torch.tensor([256, 0])
    cos, sin = O.rope_tables(128, 1e6, 512, torch.float32)
    out = O.backbone_step(bb, kc, vc, lengths, torch.tensor([0]), x, cos, sin)
    return out[0], kc[0][0, :, 256], vc[0][0, :, 256], lengths


def test_c1_layer_matches_golden_fixture():
    """Config 1 (one Qwen3-0.6B-shaped layer, B=1, KV length 256, fp32): the gather-path oracle reproduces HF's
    decoder layer (fixture written by tests/golden/make_golden.py)."""
    ref = np.load(os.path.join(HERE, "golden", "c1_qwen3_layer.npz"))
    out, k256, v256, lengths = _c1_oracle(*c1_inputs())
    assert np.abs(out.numpy() - ref["out"]).max() < 1e-4
    assert np.abs(k256.numpy() - ref["k256"]).max() < 1e-5
    assert np.array_equal(v256.numpy(), ref["v256"])
    assert lengths.tolist() == [257, 0]


def test_c1_layer_matches_hf_live():
    bb, k, v, x = c1_inputs()
    out_hf, k_hf, v_hf = hf_c1(bb, k, v, x)
    out, k256, v256, _ = _c1_oracle(bb, k, v, x)
    assert (out - out_hf).abs().max() < 1e-4 and (k256 - k_hf).abs().max() < 1e-5 and torch.equal(v256, v_hf)


def test_rope_tables_match_hf():
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    cfg = Qwen3Config(hidden_size=1024, num_attention_heads=16, num_key_value_heads=8, head_dim=128, rope_theta=1e6,
                      max_position_embeddings=4096)
    hf = Qwen3RotaryEmbedding(cfg)
    pos = torch.arange(4096)[None]
    for dt in (torch.float32, torch.bfloat16):
        c_hf, s_hf = hf(torch.zeros(1, 1, 1024, dtype=dt), pos)
        c_m, s_m = synth.Rotary(128, 1e6)(torch.zeros(1, 1, 1024, dtype=dt), pos)
        c_o, s_o = O.rope_tables(128, 1e6, 4096, dt)
        assert torch.equal(c_hf[0], c_m[0]) and torch.equal(s_hf[0], s_m[0])
        assert torch.equal(c_hf[0], c_o) and torch.equal(s_hf[0], s_o)


def test_backbone_gather_path_prefill_equals_decode():
    """Inline prefill rows of one slot at consecutive positions (step_mixed) give the same hidden states as
    decoding them one per step (serve/fast_backbone.py:327-333: K/V written before attention, causal by pos)."""
    bb = synth.qwen3_backbone(layers=2, hidden=1024, seed=5, dtype=torch.float32)
    cos, sin = O.rope_tables(128, 1e6, 64, torch.float32)
    g = torch.Generator().manual_seed(6)
    xs = torch.randn(5, 1024, generator=g)
    kc = [torch.zeros(2, 8, 64, 128) for _ in range(2)]
    vc = [torch.zeros(2, 8, 64, 128) for _ in range(2)]
    L = torch.tensor([3, 0])
    kc2, vc2, L2 = [t.clone() for t in kc], [t.clone() for t in vc], L.clone()
    pre = O.backbone_step(bb, kc, vc, L, torch.zeros(5, dtype=torch.long), xs, cos, sin, offset=torch.arange(5))
    dec = torch.cat([O.backbone_step(bb, kc2, vc2, L2, torch.tensor([0]), xs[i:i + 1], cos, sin) for i in range(5)])
    assert (pre - dec).abs().max() < 1e-4 and L.tolist() == L2.tolist() == [8, 0]


def _small_depth(seed=11):
    return synth.swiglu_depth(layers=4, d=256, heads=2, ffn=512, n_codes=256, d_backbone=256, seed=seed,
                              dtype=torch.float32)


def test_depth_incremental_equals_full_recompute():
    """Within one weight group, position L of a longer causal prefix equals the level-L pass
    (tts/model/depth_v2.py:284-295; self-test :604-607 asserts grouped vs loop within 1e-5 in fp32)."""
    m = _small_depth()
    g = torch.Generator().manual_seed(12)
    B = 3
    h = torch.randn(B, 256, generator=g)
    forced = torch.randint(0, 256, (B, 32), generator=g)
    u = torch.rand(B, 31, generator=g)
    _, inc = O.depth_frame(m, h, forced[:, 0], u, 0.9, 50, forced=forced, dt=torch.float32)
    blocks = m.depth.groups[0]
    m.depth.groups = [blocks] * 31
    m.depth.group_of_level = [None] + list(range(31))
    _, full = O.depth_frame(m, h, forced[:, 0], u, 0.9, 50, forced=forced, dt=torch.float32)
    assert (inc - full).abs().max() < 1e-5


def test_depthv2_within_frame_causality():
    """cb0 steers level 1; cb_k steers level k+1 but never levels <= k (tts/model/depth_v2.py:575-585)."""
    m = synth.depthv2_like(d_backbone=256, d=256, heads=4, ffn=512, n_codes=128, rank=32, dtype=torch.float32)
    g = torch.Generator().manual_seed(13)
    B = 2
    h = torch.randn(B, 256, generator=g)
    forced = torch.randint(0, 128, (B, 32), generator=g)
    u = torch.rand(B, 31, generator=g)
    cross = torch.randn(B, 4, 256, generator=g) * 0.1
    _, l1 = O.depth_frame(m, h, forced[:, 0], u, 0.9, 50, forced=forced, cross=cross, dt=torch.float32)
    f2 = forced.clone()
    f2[:, 0] = (f2[:, 0] + 7) % 128
    _, l2 = O.depth_frame(m, h, f2[:, 0], u, 0.9, 50, forced=f2, cross=cross, dt=torch.float32)
    assert not torch.allclose(l1[:, 0], l2[:, 0])
    f3 = forced.clone()
    f3[:, 2] = (f3[:, 2] + 7) % 128
    _, l3 = O.depth_frame(m, h, forced[:, 0], u, 0.9, 50, forced=f3, cross=cross, dt=torch.float32)
    assert torch.equal(l1[:, :2], l3[:, :2]) and not torch.allclose(l1[:, 2], l3[:, 2])


def test_feedback_closed_form():
    """norm(sum_l table[c_l + 2048 l] / sqrt(32)) with torch's nn.RMSNorm(eps=None) (tts/model/audio_io.py:27-35)."""
    g = torch.Generator().manual_seed(14)
    table = (torch.randn(32 * 64, 256, generator=g) * 0.02).to(torch.bfloat16)
    audio_in = synth.SimpleNamespace(n_codes=64, table=synth.Lin(table),
                                     norm=synth.Norm(torch.ones(256, dtype=torch.bfloat16), None))
    codes = torch.randint(0, 64, (5, 32), generator=g)
    got = O.feedback(audio_in, codes)
    e = table[codes + torch.arange(32) * 64].float().sum(1).to(torch.bfloat16)
    x = (e.float() / math.sqrt(32)).to(torch.bfloat16)
    # eps=None means finfo(input dtype).eps; the reference's input is bf16
    ref = torch.nn.RMSNorm(256, eps=torch.finfo(torch.bfloat16).eps, dtype=torch.float32)(x.float())
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(1e-30))) - 7)
    assert ((got.float() - ref).abs() / ulp).max() <= 1.0
