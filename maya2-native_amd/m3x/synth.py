"""Seeded synthetic models and inputs for the benchmark/parity workloads (no checkpoints, no network).

The holders below expose the attribute names the drop-in surfaces read from real modules:
  backbone: `backbone.lm.model.{layers[i].{self_attn.{q,k,v,o}_proj, self_attn.{q,k}_norm, mlp.{gate,up,down}_proj,
            input_layernorm, post_attention_layernorm}, norm, rotary_emb}`, `backbone.lm.config`,
            `backbone.cb0_head` (HF Qwen3 via tts/model/backbone.py:59-98);
  depth:    `model.depth.{in_proj, groups[g][l].{n1,n2,qkv,o,...}, norm, heads, ...}`, `model.audio_in.{table,norm}`
            (tts/model/depth_v2.py:145-230, tts/model/audio_io.py:17-35).
Draw order is fixed per builder (documented inline), so a seed reproduces the same weights on any host.
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import torch


class Lin:
    """nn.Linear-shaped holder: .weight [out, in], no bias."""

    def __init__(self, w):
        self.weight = w
        self.bias = None


class Norm:
    """Norm-shaped holder (RMSNorm when b is None, else LayerNorm)."""

    def __init__(self, w, eps, b=None):
        self.weight = w
        self.bias = b
        self.eps = eps
        self.variance_epsilon = eps


class Rotary:
    """HF Qwen3RotaryEmbedding default rope: inv_freq = 1/theta^(2i/D); cos/sin of cat(freqs, freqs) in fp32, cast
    to the input dtype (transformers models/qwen3/modeling_qwen3.py Qwen3RotaryEmbedding.forward)."""

    def __init__(self, head_dim, theta):
        self.inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))

    def __call__(self, x, position_ids):
        inv = self.inv_freq[None, :, None].float().expand(position_ids.shape[0], -1, 1).to(x.device)
        pos = position_ids[:, None, :].float()
        freqs = (inv.float() @ pos.float()).transpose(1, 2)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(x.dtype), emb.sin().to(x.dtype)


def _normal(g, shape, std, device, dtype):
    return (torch.randn(*shape, generator=g, dtype=torch.float32, device=g.device) * std).to(device=device,
                                                                                          dtype=dtype)


def _norm_weights(g, norms, affine, device):
    """Draw the weights of `norms` (Norm holders, in order) from generator g: "normal:s" -> 1 + N(0, s),
    "lognormal:s" -> exp(N(0, s)) (at s = 0.8 a 1024-wide vector spans about 0.1x to 20x, like trained
    Qwen3 norm weights). Drawn in fp32, then cast to each holder's dtype; a LayerNorm holder also gets a bias
    N(0, s)."""
    kind, s = affine.split(":")
    s = float(s)
    if kind not in ("normal", "lognormal"):
        raise ValueError(f"affine kind {kind!r}")
    for n in norms:
        d, dt = n.weight.shape[0], n.weight.dtype
        z = _normal(g, (d,), s, "cpu", torch.float32)
        w = 1 + z if kind == "normal" else torch.exp(z)
        n.weight = w.to(device=device, dtype=dt)
        if n.bias is not None:
            n.bias = _normal(g, (d,), s, device, dt)


def qwen3_backbone(layers=28, hidden=1024, heads=16, kv_heads=8, head_dim=128, inter=3072, v0=2048, theta=1e6,
                   eps=1e-6, seed=0, device="cpu", dtype=torch.bfloat16, std=0.02, gen="cpu", affine=None):
    """Qwen3-0.6B-shaped backbone (gen: the device of the generator; "cpu" reproduces across hosts). Per layer, in
    order: q [H*D, hid], k [KV*D, hid], v [KV*D, hid], o [hid, H*D], gate [I, hid], up [I, hid], down [hid, I], all
    N(0, std); then cb0 head [v0, hid]. RMSNorm weights 1 (HF init) when affine is None; otherwise ("normal:s" or
    "lognormal:s", see _norm_weights) drawn after everything else, per layer input_layernorm,
    post_attention_layernorm, q_norm, k_norm, then the final norm, so the other weights do not change."""
    g = torch.Generator(device=gen).manual_seed(seed)
    ones = lambda n: torch.ones(n, dtype=dtype, device=device)  # noqa: E731
    L = []
    for _ in range(layers):
        attn = SimpleNamespace(
            q_proj=Lin(_normal(g, (heads * head_dim, hidden), std, device, dtype)),
            k_proj=Lin(_normal(g, (kv_heads * head_dim, hidden), std, device, dtype)),
            v_proj=Lin(_normal(g, (kv_heads * head_dim, hidden), std, device, dtype)),
            o_proj=Lin(_normal(g, (hidden, heads * head_dim), std, device, dtype)),
            q_norm=Norm(ones(head_dim), eps), k_norm=Norm(ones(head_dim), eps))
        mlp = SimpleNamespace(gate_proj=Lin(_normal(g, (inter, hidden), std, device, dtype)),
                              up_proj=Lin(_normal(g, (inter, hidden), std, device, dtype)),
                              down_proj=Lin(_normal(g, (hidden, inter), std, device, dtype)))
        L.append(SimpleNamespace(self_attn=attn, mlp=mlp, input_layernorm=Norm(ones(hidden), eps),
                                 post_attention_layernorm=Norm(ones(hidden), eps)))
    cb0 = Lin(_normal(g, (v0, hidden), std, device, dtype))
    cfg = SimpleNamespace(num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=head_dim,
                          hidden_size=hidden, rms_norm_eps=eps, intermediate_size=inter, num_hidden_layers=layers,
                          rope_theta=theta)
    model = SimpleNamespace(layers=L, norm=Norm(ones(hidden), eps), rotary_emb=Rotary(head_dim, theta))
    if affine:
        _norm_weights(g, [n for layer in L for n in (layer.input_layernorm, layer.post_attention_layernorm,
                                                     layer.self_attn.q_norm, layer.self_attn.k_norm)]
                      + [model.norm], affine, device)
    params = [t for layer in L for t in (layer.self_attn.q_proj.weight, layer.self_attn.k_proj.weight)]
    model.parameters = lambda: iter(params)
    lm = SimpleNamespace(model=model, config=cfg)
    return SimpleNamespace(lm=lm, cb0_head=cb0, d_model=hidden)


def swiglu_depth(layers=4, d=1024, heads=8, ffn=2816, n_q=32, n_codes=2048, d_backbone=1024, seed=1,
                 device="cpu", dtype=torch.bfloat16, std=0.02, eps=1e-6, gen="cpu", affine=None):
    """Depth transformer of the 4-layer SwiGLU/RMSNorm trunk shared by every level (one weight group).
    Draw order: in_proj [d, d_backbone], level0 [d], embed [n_q-1, n_codes, d] (per-codebook table, level
    embedding folded in), per layer qkv [3d, d], o [d, d], gate|up [2*ffn, d], down [d, ffn]; heads
    [n_q-1, n_codes, d]; then the backbone-side feedback table [n_q*n_codes, d_backbone]. Norm weights 1 when
    affine is None; otherwise ("normal:s" / "lognormal:s", see _norm_weights) drawn after everything else, per
    layer n1, n2, then the final norm, then the feedback RMSNorm."""
    g = torch.Generator(device=gen).manual_seed(seed)
    ones = lambda n: torch.ones(n, dtype=dtype, device=device)  # noqa: E731
    in_proj = Lin(_normal(g, (d, d_backbone), std, device, dtype))
    level0 = _normal(g, (d,), std, device, dtype)
    embed = _normal(g, (n_q - 1, n_codes, d), std, device, dtype)
    blocks = []
    for _ in range(layers):
        blocks.append(SimpleNamespace(n1=Norm(ones(d), eps), n2=Norm(ones(d), eps),
                                      qkv=Lin(_normal(g, (3 * d, d), std, device, dtype)),
                                      o=Lin(_normal(g, (d, d), std, device, dtype)),
                                      gate_up=Lin(_normal(g, (2 * ffn, d), std, device, dtype)),
                                      down=Lin(_normal(g, (d, ffn), std, device, dtype))))
    heads_w = _normal(g, (n_q - 1, n_codes, d), std, device, dtype)
    table = _normal(g, (n_q * n_codes, d_backbone), std, device, dtype)
    depth = SimpleNamespace(n_q=n_q, n_codes=n_codes, n_heads=heads, in_proj=in_proj, level0=level0, embed=embed,
                            groups=[blocks], group_of_level=[None] + [0] * (n_q - 1), norm=Norm(ones(d), eps),
                            heads=[Lin(heads_w[i]) for i in range(n_q - 1)], cross=None)
    audio_in = SimpleNamespace(n_q=n_q, n_codes=n_codes, table=Lin(table),
                               norm=Norm(torch.ones(d_backbone, dtype=dtype, device=device),
                                         torch.finfo(dtype).eps))
    if affine:
        _norm_weights(g, [n for blk in blocks for n in (blk.n1, blk.n2)] + [depth.norm, audio_in.norm], affine,
                      device)
    return SimpleNamespace(depth=depth, audio_in=audio_in)


# the norm-weight draws of the end-to-end tests and the benchmark: every RMSNorm / q_norm / k_norm weight
# 1 + N(0, 0.1), so that a swapped, dropped or misplaced norm weight changes the outputs
AFFINE = "normal:0.1"
# a wide spread (about 0.1x .. 20x over a 1024-wide vector), like trained norm weights
AFFINE_WIDE = "lognormal:0.8"


REFERENCE_GROUP_OF_LEVEL = [None] + list(range(8)) + [8] * 8 + [9] * 8 + [10] * 7


def depthv2_like(d_backbone=1024, d=1024, heads=16, ffn=3072, layers=4, n_q=32, n_codes=2048, rank=128, seed=2,
                 device="cpu", dtype=torch.float32, std=0.02, group_of_level=None, affine_std=0.0):
    """The reference's DepthV2 geometry (tts/model/depth_v2.py:145-230): LayerNorm + GELU trunks, 16 heads x 64,
    11 weight groups, shared per-layer speaker cross-attention, rank-128 factorised code embeddings. Draw order:
    in_proj, code_lo [(n_q-1)*n_codes, rank], code_up [d, rank], level_emb [n_q, d], per group per layer
    qkv/o/f1/f2, per layer cross kv [2d, d] / o [d, d], heads [n_q-1][n_codes, d], feedback table. Norm affines:
    weights 1 and biases 0 (the nn.LayerNorm init) when affine_std is 0; otherwise, drawn after everything else in
    module order (per group per layer n1, n2; final norm; feedback RMSNorm), weight 1 + N(0, affine_std) and bias
    N(0, affine_std), so that a misplaced affine term shows in the outputs."""
    gol = group_of_level or REFERENCE_GROUP_OF_LEVEL
    n_groups = max(x for x in gol if x is not None) + 1
    g = torch.Generator().manual_seed(seed)
    ln = lambda: Norm(torch.ones(d, dtype=dtype, device=device), 1e-5, torch.zeros(d, dtype=dtype, device=device))  # noqa: E731
    in_proj = Lin(_normal(g, (d, d_backbone), std, device, dtype))
    code_lo = Lin(_normal(g, ((n_q - 1) * n_codes, rank), std, device, dtype))
    code_up = Lin(_normal(g, (d, rank), std, device, dtype))
    level_emb = Lin(_normal(g, (n_q, d), std, device, dtype))
    groups = []
    for _ in range(n_groups):
        groups.append([SimpleNamespace(n1=ln(), n2=ln(), qkv=Lin(_normal(g, (3 * d, d), std, device, dtype)),
                                       o=Lin(_normal(g, (d, d), std, device, dtype)),
                                       f1=Lin(_normal(g, (ffn, d), std, device, dtype)),
                                       f2=Lin(_normal(g, (d, ffn), std, device, dtype))) for _ in range(layers)])
    cross = [SimpleNamespace(kv=Lin(_normal(g, (2 * d, d), std, device, dtype)),
                             o=Lin(_normal(g, (d, d), std, device, dtype))) for _ in range(layers)]
    heads_l = [Lin(_normal(g, (n_codes, d), std, device, dtype)) for _ in range(n_q - 1)]
    # the backbone-side feedback embedding lives at the engine dtype (bf16), whatever the depth's
    table = _normal(g, (n_q * n_codes, d_backbone), std, device, torch.bfloat16)
    depth = SimpleNamespace(n_q=n_q, n_codes=n_codes, n_heads=heads, in_proj=in_proj, code_lo=code_lo,
                            code_up=code_up, level_emb=level_emb, groups=groups, group_of_level=list(gol),
                            norm=ln(), heads=heads_l, cross=cross)
    audio_in = SimpleNamespace(n_q=n_q, n_codes=n_codes, table=Lin(table),
                               norm=Norm(torch.ones(d_backbone, dtype=torch.bfloat16, device=device),
                                         torch.finfo(torch.bfloat16).eps))
    if affine_std:
        norms = [n for blocks in groups for blk in blocks for n in (blk.n1, blk.n2)] + [depth.norm]
        for n in norms:
            n.weight = (1 + _normal(g, (d,), affine_std, "cpu", torch.float32)).to(device=device, dtype=dtype)
            n.bias = _normal(g, (d,), affine_std, device, dtype)
        audio_in.norm.weight = (1 + _normal(g, (d_backbone,), affine_std, "cpu", torch.float32)).to(
            device=device, dtype=torch.bfloat16)
    return SimpleNamespace(depth=depth, audio_in=audio_in)


# ---------------------------------------------------------------- workload inputs
def c3_lengths(B, seed=3):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(64, 2049, (B,), generator=g)


def c4_decode_lengths(n=216, seed=4):
    g = torch.Generator().manual_seed(seed)
    u = torch.rand(n, generator=g, dtype=torch.float64)
    return torch.floor(torch.exp(math.log(128) + u * (math.log(4096) - math.log(128)))).long().clamp_max(4095)


def c5_lengths(B, seed=5, mean=2048, cap=4096):
    g = torch.Generator().manual_seed(seed)
    lam = torch.full((B,), float(mean), dtype=torch.float64)
    return torch.poisson(lam, generator=g).long().clamp(1, cap)


def uniforms(shape, seed=7):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(*shape, generator=g, dtype=torch.float32)


def mimi(seed=0, device="cpu", dtype=torch.float32):
    """A Mimi codec (transformers MimiModel, default MimiConfig: 32 codebooks of 2048 x 256, an 8-layer 512-wide
    sliding-window decoder transformer, SEANet decoder with ratios 8/6/5/4, 1920 samples per 12.5 Hz frame) with
    seeded random weights: codebook rows N(0, 1); every conv and linear weight N(0, 1 / fan_in); biases and the
    norms' affine terms N(0, 0.02) around their init; layer scales 0.1. There is no network for the kyutai weights."""
    from transformers import MimiConfig, MimiModel
    g = torch.Generator().manual_seed(seed)
    m = MimiModel(MimiConfig()).eval()
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("layer_scale.scale") or name.endswith("_layer_scale.scale"):
                p.fill_(0.1)
            elif p.dim() >= 2:
                mod = _owner(m, name)
                if isinstance(mod, torch.nn.ConvTranspose1d):  # [C_in, C_out / groups, k]: inputs per output
                    fan_in = max(1, p.shape[0] // mod.groups * p.shape[2] // mod.stride[0])
                else:
                    fan_in = p[0].numel()
                p.copy_(torch.randn(p.shape, generator=g) / math.sqrt(fan_in))
            elif name.endswith("weight"):  # norm scales
                p.copy_(1 + 0.02 * torch.randn(p.shape, generator=g))
            else:  # biases
                p.copy_(0.02 * torch.randn(p.shape, generator=g))
        for name, b in m.named_buffers():
            if name.endswith("embed_sum"):
                b.copy_(torch.randn(b.shape, generator=g))
            elif name.endswith("cluster_usage"):
                b.fill_(1.0)
        for mod in m.modules():
            if hasattr(mod, "_embed"):
                mod._embed = None
    return m.to(device=device, dtype=dtype)


def _owner(model, pname):
    mod = model
    for part in pname.split(".")[:-1]:
        mod = getattr(mod, part)
    return mod


def mimi_codes(B, frames, seed=0):
    """Uniform codes [B, 32, frames] in [0, 2048)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 2048, (B, 32, frames), generator=g)
