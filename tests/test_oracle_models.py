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


def _swap(a, b, attr="weight"):
    ta, tb = getattr(a, attr), getattr(b, attr)
    setattr(a, attr, tb)
    setattr(b, attr, ta)


def test_c1_golden_detects_planted_norm_mistakes():
    """The golden's norm weights are wide-spread (about 0.1x to 20x), so each wiring mistake a norm can suffer
    moves the oracle's output far beyond the fixture's 1e-4 tolerance: input/post-attention norms swapped, q/k
    norms swapped, the final norm's weight dropped (planted in the oracle's inputs, on the CPU)."""
    ref = torch.from_numpy(np.load(os.path.join(HERE, "golden", "c1_qwen3_layer.npz"))["out"])
    for plant in ("swap_in_post", "swap_qk", "drop_final"):
        bb, k, v, x = c1_inputs()
        L = bb.lm.model.layers[0]
        if plant == "swap_in_post":
            _swap(L.input_layernorm, L.post_attention_layernorm)
        elif plant == "swap_qk":
            _swap(L.self_attn.q_norm, L.self_attn.k_norm)
        else:
            bb.lm.model.norm.weight = torch.ones_like(bb.lm.model.norm.weight)
        out = _c1_oracle(bb, k, v, x)[0]
        assert (out - ref).abs().max() > 1e-2, plant


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


def _small_depth(seed=11, dtype=torch.float32):
    return synth.swiglu_depth(layers=4, d=256, heads=2, ffn=512, n_codes=256, d_backbone=256, seed=seed,
                              dtype=dtype, affine=synth.AFFINE)


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
    w = (1 + 0.1 * torch.randn(256, generator=g)).to(torch.bfloat16)
    audio_in = synth.SimpleNamespace(n_codes=64, table=synth.Lin(table), norm=synth.Norm(w, None))
    codes = torch.randint(0, 64, (5, 32), generator=g)
    got = O.feedback(audio_in, codes)
    e = table[codes + torch.arange(32) * 64].float().sum(1).to(torch.bfloat16)
    x = (e.float() / math.sqrt(32)).to(torch.bfloat16)
    # eps=None means finfo(input dtype).eps; the reference's input is bf16
    rms = torch.nn.RMSNorm(256, eps=torch.finfo(torch.bfloat16).eps, dtype=torch.float32)
    with torch.no_grad():
        rms.weight.copy_(w.float())
        ref = rms(x.float())
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(1e-30))) - 7)
    assert ((got.float() - ref).abs() / ulp).max() <= 1.0


def test_depth_oracle_matches_reference_fast_depth_golden():
    """The oracle's depth frame against tests/golden/depth_v2_frame.npz, written by the reference's own
    FastDepth._compute (serve/fast_depth.py:84-141) over its DepthV2 (all 11 weight groups, LayerNorm + GELU, 16 x 64
    heads, speaker cross constants from set_speaker :73-82) in fp32 and greedy mode: the speaker constants, every
    level's head logits, the 32 codes and the feedback. Randomised norm affines make a misplaced weight or bias, a
    wrong epsilon, GELU form or cross-constant placement show."""
    import os
    import sys
    import numpy as np
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    from make_depth_golden import golden_inputs
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "depth_v2_frame.npz"))
    model, h, cb0, mems = golden_inputs()
    d = model.depth
    cross = torch.stack([torch.stack([O.lin(O.lin(mems[b, 0], c.kv.weight)[:, 1024:], c.o.weight)[0]
                                      for c in d.cross]) for b in range(h.shape[0])])
    assert (cross - torch.from_numpy(gold["cross"])).abs().max() < 1e-5
    u = torch.zeros(h.shape[0], 31)
    codes, logits = O.depth_frame(model, h, cb0, u, 0.7, 64, greedy=True, cross=cross, dt=torch.float32)
    ref_logits = torch.from_numpy(gold["logits"])
    assert (logits - ref_logits).abs().max() < 2e-5, (logits - ref_logits).abs().max()
    assert torch.equal(codes, torch.from_numpy(gold["codes"]))
    table32 = synth.SimpleNamespace(n_codes=2048, table=synth.Lin(model.audio_in.table.weight.float()),
                                    norm=synth.Norm(model.audio_in.norm.weight.float(), None))
    fb = O.feedback(table32, codes)
    assert (fb - torch.from_numpy(gold["feedback"])).abs().max() < 1e-5


def test_depth_oracle_golden_detects_planted_mistakes():
    """The golden pins the trunk: a LayerNorm without its bias, or the speaker constants left out, moves the logits
    far beyond the tolerance above (the mistakes are planted in the oracle's inputs, on the CPU)."""
    import os
    import sys
    import numpy as np
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    from make_depth_golden import golden_inputs
    gold = torch.from_numpy(np.load(os.path.join(os.path.dirname(__file__), "golden", "depth_v2_frame.npz"))["logits"])
    model, h, cb0, mems = golden_inputs()
    d = model.depth
    cross = torch.stack([torch.stack([O.lin(O.lin(mems[b, 0], c.kv.weight)[:, 1024:], c.o.weight)[0]
                                      for c in d.cross]) for b in range(h.shape[0])])
    u = torch.zeros(h.shape[0], 31)
    d.groups[0][1].n2.bias = torch.zeros_like(d.groups[0][1].n2.bias)
    _, lg = O.depth_frame(model, h, cb0, u, 0.7, 64, greedy=True, cross=cross, dt=torch.float32)
    assert (lg[:, 0] - gold[:, 0]).abs().max() > 1e-3
    _, lg2 = O.depth_frame(model, h, cb0, u, 0.7, 64, greedy=True, cross=cross * 0, dt=torch.float32)
    assert (lg2[:, 0] - gold[:, 0]).abs().max() > 1e-3


def _hf_qwen3_bf16(bb, layers):
    from transformers import Qwen3Config, Qwen3Model
    cfg = Qwen3Config(hidden_size=1024, intermediate_size=3072, num_hidden_layers=layers, num_attention_heads=16,
                      num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6, rope_theta=1e6, vocab_size=16,
                      max_position_embeddings=4096, attn_implementation="eager")
    m = Qwen3Model(cfg).eval().to(torch.bfloat16)
    sd = {"norm.weight": bb.lm.model.norm.weight}
    for i, L in enumerate(bb.lm.model.layers):
        a, mm = L.self_attn, L.mlp
        for name, mod in (("self_attn.q_proj", a.q_proj), ("self_attn.k_proj", a.k_proj),
                          ("self_attn.v_proj", a.v_proj), ("self_attn.o_proj", a.o_proj),
                          ("self_attn.q_norm", a.q_norm), ("self_attn.k_norm", a.k_norm),
                          ("mlp.gate_proj", mm.gate_proj), ("mlp.up_proj", mm.up_proj),
                          ("mlp.down_proj", mm.down_proj), ("input_layernorm", L.input_layernorm),
                          ("post_attention_layernorm", L.post_attention_layernorm)):
            sd[f"layers.{i}.{name}.weight"] = mod.weight
    missing, _ = m.load_state_dict(sd, strict=False)
    assert set(missing) <= {"embed_tokens.weight"}, missing
    return m


def test_backbone_oracle_bf16_rounding_points_match_hf():
    """The backbone oracle's bf16 rounding points against HF transformers' Qwen3 modules in bf16 (the reference's
    eager backbone, serve/fast_backbone.py:204-228): on identical bf16 inputs, RMSNorm (Qwen3RMSNorm) and q/k norm +
    RoPE (apply_rotary_pos_emb on HF's own bf16 cos/sin) are bit-identical; over a 4-layer prefill + decode step
    the oracle stays as close to HF's bf16 eager forward as both are to the fp32 evaluation of the same weights
    (two bf16 paths that round in the same places differ only by GEMM accumulation order)."""
    from transformers import DynamicCache, Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, Qwen3RotaryEmbedding, apply_rotary_pos_emb
    from helpers import convert, rel_l2
    g = torch.Generator().manual_seed(91)
    # RMSNorm, bit for bit
    w = (1 + 0.1 * torch.randn(1024, generator=g)).to(torch.bfloat16)
    x = (3 * torch.randn(64, 1024, generator=g)).to(torch.bfloat16)
    hf_norm = Qwen3RMSNorm(1024, eps=1e-6).to(torch.bfloat16)
    hf_norm.weight.data.copy_(w)
    assert torch.equal(hf_norm(x), O.rms_hf(x, w, 1e-6))
    # q/k norm + RoPE at positions spread over the cache, bit for bit
    cfg = Qwen3Config(hidden_size=1024, num_attention_heads=16, num_key_value_heads=8, head_dim=128, rope_theta=1e6,
                      max_position_embeddings=4096)
    pos = torch.randint(0, 4096, (64,), generator=g)
    cos, sin = Qwen3RotaryEmbedding(cfg)(torch.zeros(1, 1, 1024, dtype=torch.bfloat16), pos[None])
    q = torch.randn(64, 16, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(64, 8, 128, generator=g).to(torch.bfloat16)
    wq, wk = [(1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16) for _ in range(2)]
    qn, kn = Qwen3RMSNorm(128).to(torch.bfloat16), Qwen3RMSNorm(128).to(torch.bfloat16)
    qn.weight.data.copy_(wq)
    kn.weight.data.copy_(wk)
    q_hf, k_hf = apply_rotary_pos_emb(qn(q).transpose(0, 1), kn(k).transpose(0, 1), cos[0], sin[0], unsqueeze_dim=0)
    c, s = cos[0][:, None], sin[0][:, None]
    q_o = O.rms_hf(q, wq, 1e-6)
    k_o = O.rms_hf(k, wk, 1e-6)
    assert torch.equal(q_hf.transpose(0, 1), q_o * c + O.rotate_half(q_o) * s)
    assert torch.equal(k_hf.transpose(0, 1), k_o * c + O.rotate_half(k_o) * s)
    # 4 layers: 64-token prefill then one decode step, HF bf16 eager against the oracle; norm weights spread like
    # trained ones (about 0.1x to 20x), so the bf16 rounding of every norm's output and weight product counts
    L, T = 4, 64
    bb = synth.qwen3_backbone(layers=L, seed=92, dtype=torch.bfloat16, affine=synth.AFFINE_WIDE)
    m = _hf_qwen3_bf16(bb, L)
    xs = torch.randn(1, T + 1, 1024, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        cache = DynamicCache()
        m(inputs_embeds=xs[:, :T], past_key_values=cache, use_cache=True)
        out_hf = m(inputs_embeds=xs[:, T:], past_key_values=cache, use_cache=True).last_hidden_state[0, 0]
    ctab, stab = O.rope_tables(128, 1e6, 128, torch.bfloat16)
    kc = [torch.zeros(2, 8, 128, 128, dtype=torch.bfloat16) for _ in range(L)]
    vc = [torch.zeros(2, 8, 128, 128, dtype=torch.bfloat16) for _ in range(L)]
    lens = torch.tensor([0, 0])
    O.backbone_step(bb, kc, vc, lens, torch.zeros(T, dtype=torch.long), xs[0, :T], ctab, stab, offset=torch.arange(T),
                    attention="gather")
    out_o = O.backbone_step(bb, kc, vc, lens, torch.tensor([0]), xs[0, T:], ctab, stab, attention="gather")[0]
    b32 = convert(bb, torch.float32)
    c32, s32 = O.rope_tables(128, 1e6, 128, torch.float32)
    k3 = [torch.zeros(2, 8, 128, 128) for _ in range(L)]
    v3 = [torch.zeros(2, 8, 128, 128) for _ in range(L)]
    l3 = torch.tensor([0, 0])
    O.backbone_step(b32, k3, v3, l3, torch.zeros(T, dtype=torch.long), xs[0, :T].float(), c32, s32,
                    offset=torch.arange(T))
    truth = O.backbone_step(b32, k3, v3, l3, torch.tensor([0]), xs[0, T:].float(), c32, s32)[0]
    floor = max(rel_l2(out_o, truth), rel_l2(out_hf, truth))
    assert rel_l2(out_o, out_hf) <= 1.5 * floor, (rel_l2(out_o, out_hf), floor)
    cos_sim = torch.nn.functional.cosine_similarity(out_o.float()[None], out_hf.float()[None]).item()
    # the cosine the rel-L2 bound allows (with wide norm weights both bf16 paths sit ~3 % off the fp32
    # evaluation after 4 layers, the q/k norm weights scaling the attention scores up to ~400x)
    assert cos_sim >= 1 - (1.5 * floor) ** 2 / 2, (cos_sim, rel_l2(out_o, out_hf), floor)
    # the V rows the step wrote are the v projection of identical bf16 inputs at layer 0: GEMM order only
    v0 = cache.layers[0].values[0, :, T]
    assert (vc[0][0, :, T].float() - v0.float()).abs().max() <= 2 * torch.exp2(torch.floor(torch.log2(
        v0.float().abs().max())) - 7)


def test_depth_swiglu_rms_branch_matches_hf_modules():
    """The oracle's SwiGLU/RMSNorm depth trunk is the golden-pinned LayerNorm/GELU trunk (same residual, attention
    and schedule code) with two pieces swapped in; each is pinned here against the HF Qwen3 module it restates:
      - _norm's RMS branch against Qwen3RMSNorm on the same bf16 rows and weights: bit for bit (bf16), and within
        fp32 rounding (fp32);
      - _ffn's SwiGLU against Qwen3MLP with gate = the first half of gate_up and up = the second: the bf16 rounding
        point after silu, then the product, bit for bit on the same bf16 gate/up values; the whole block within
        fp32 rounding in fp32 (torch's CPU GEMMs order the sums their own way)."""
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3MLP, Qwen3RMSNorm
    g = torch.Generator().manual_seed(95)
    d, ffn = 256, 512
    for dt in (torch.bfloat16, torch.float32):
        w = torch.exp(0.8 * torch.randn(d, generator=g)).to(dt)
        x = (3 * torch.randn(33, d, generator=g)).to(dt)
        hf = Qwen3RMSNorm(d, eps=1e-6).to(dt)
        hf.weight.data.copy_(w)
        got = O._norm(x, synth.Norm(w, 1e-6), dt)
        if dt == torch.bfloat16:
            assert torch.equal(got, hf(x))
        else:
            assert (got - hf(x)).abs().max() <= 4e-7 * x.abs().max() * w.abs().max()
    cfg = Qwen3Config(hidden_size=d, intermediate_size=ffn, hidden_act="silu")
    for dt in (torch.bfloat16, torch.float32):
        gu = (0.05 * torch.randn(2 * ffn, d, generator=g)).to(dt)
        dn = (0.05 * torch.randn(d, ffn, generator=g)).to(dt)
        mlp = Qwen3MLP(cfg).to(dt)
        mlp.gate_proj.weight.data.copy_(gu[:ffn])
        mlp.up_proj.weight.data.copy_(gu[ffn:])
        mlp.down_proj.weight.data.copy_(dn)
        y = torch.randn(17, d, generator=g).to(dt)
        blk = synth.SimpleNamespace(gate_up=synth.Lin(gu), down=synth.Lin(dn))
        got = O._ffn(blk, y, dt)
        with torch.no_grad():
            ref = mlp(y)
            if dt == torch.bfloat16:
                # the rounding points: silu(gate) rounded, times up, rounded, on identical bf16 gate/up values
                gate, up = O.lin(y, gu[:ffn]), O.lin(y, gu[ffn:])
                assert torch.equal(mlp.act_fn(gate) * up, torch.nn.functional.silu(gate.float()).to(dt) * up)
                # the block: as close as two bf16 GEMM orders allow (torch's CPU bf16 GEMM vs fp32 sums)
                assert ((got.float() - ref.float()).norm() / ref.float().norm()).item() < 1e-2
            else:
                assert (got - ref).abs().max() <= 1e-5 * ref.abs().max()


def test_depth_swiglu_trunk_detects_planted_norm_mistakes():
    """With non-unit norm weights the SwiGLU trunk's logits move well beyond the bf16 bar when n1 and n2 are
    swapped in a layer or the final norm's weight is dropped (planted in the oracle's inputs, on the CPU)."""
    m = _small_depth(dtype=torch.float32)
    g = torch.Generator().manual_seed(96)
    B = 3
    h = torch.randn(B, 256, generator=g)
    forced = torch.randint(0, 256, (B, 32), generator=g)
    u = torch.rand(B, 31, generator=g)
    _, base = O.depth_frame(m, h, forced[:, 0], u, 0.9, 50, forced=forced, dt=torch.float32)
    blk = m.depth.groups[0][2]
    _swap(blk.n1, blk.n2)
    _, l1 = O.depth_frame(m, h, forced[:, 0], u, 0.9, 50, forced=forced, dt=torch.float32)
    _swap(blk.n1, blk.n2)
    m.depth.norm.weight = torch.ones_like(m.depth.norm.weight)
    _, l2 = O.depth_frame(m, h, forced[:, 0], u, 0.9, 50, forced=forced, dt=torch.float32)
    scale = base.abs().max()
    assert (l1 - base).abs().max() > 0.05 * scale and (l2 - base).abs().max() > 0.05 * scale
