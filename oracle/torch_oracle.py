"""PyTorch-eager CPU restatement of the Maya3 frame step (floating-point parts).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use this as the
checker / CPU baseline; the product package never imports it.

Follows, op for op:
  backbone_step   StaticBackbone._forward with attention='gather' (serve/fast_backbone.py:176-234, gather branch
                  :204-228) on HF Qwen3 semantics: Qwen3RMSNorm (w * bf16(x * rsqrt(mean x^2 + eps))),
                  rotate_half RoPE rounded after each op, K/V written before attention, bf16 scores -> fp32
                  softmax -> bf16 probabilities @ V, MLP down(silu(gate) * up)
                  (transformers models/qwen3/modeling_qwen3.py Qwen3RMSNorm/Qwen3MLP/apply_rotary_pos_emb).
  depth_frame     FastDepth._compute_fused (serve/fast_depth.py:143-203) with _add_ln's rounding
                  (serve/fast_depth_kernels.py:14-45): x' = dt(x + a) [+ c], next norm fused; group schedule
                  from GROUP_OF_LEVEL (tts/model/depth_v2.py:45); last trunk layer only at the last position at a
                  group start; sampling by the C oracle's top-k contract on the bf16/fp16 head logits.
  feedback        serve/fast_depth.py:200-203 + tts/model/audio_io.py:27-35.
  loop_detect_batch  maya3/guards.py:80-107 (the engine's stall / period loop guard).
Parity of each piece is pinned in tests/test_oracle_models.py (HF decoder layer, incremental-vs-full depth,
closed forms).
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from . import coracle

N_LEVELS = 32


# ---------------------------------------------------------------- backbone (gather path)
def rms_hf(x, w, eps):
    xf = x.float()
    var = xf.pow(2).mean(-1, keepdim=True)
    return w * (xf * torch.rsqrt(var + eps)).to(x.dtype)


def rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), -1)


def lin(x, w):
    """nn.Linear on 16-bit tensors: fp32 accumulation, one rounding to the input dtype."""
    return (x.float() @ w.float().t()).to(x.dtype)


def rope_tables(head_dim, theta, cap, dtype):
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = (inv[None, :, None].float() @ torch.arange(cap)[None, None, :].float()).transpose(1, 2)[0]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def backbone_step(bb, kc, vc, lengths, slots, x, cos, sin, offset=None, real=None, ctx=None, attention='triton'):
    """One decode step. bb: synth/HF-shaped backbone (CPU tensors); kc/vc: lists of [S+1, KV, cap, D] caches
    (updated in place); lengths [S+1] long (updated); slots [R] long; x [R, hidden]. Returns the normed hidden.
    attention='triton': the engine's attention (`_decode_attn`, serve/fast_backbone.py:31-58: fp32 scores, fp32
    softmax and fp32 P.V, one rounding of the output) — the configuration the reference's own parity test uses as
    its unfused baseline (maya3/tests/test_backbone_fused.py:16-17); attention='gather': the eager gather branch
    (:215-218: bf16 scores, bf16 probabilities)."""
    cfg = bb.lm.config
    H, KV = cfg.num_attention_heads, cfg.num_key_value_heads
    D = getattr(cfg, 'head_dim', None) or cfg.hidden_size // H
    G = H // KV
    eps = cfg.rms_norm_eps
    scaling = D ** -0.5
    B = x.shape[0]
    pos = lengths[slots]
    if offset is not None:
        pos = pos + offset
    c = cos[pos][:, None]
    s = sin[pos][:, None]
    if ctx is None:
        ctx = int(pos.max()) + 1
    bias = torch.zeros(B, ctx, dtype=torch.float32).masked_fill_(
        torch.arange(ctx)[None] > pos[:, None], float('-inf')).view(B, 1, 1, ctx)
    h = x
    for i, layer in enumerate(bb.lm.model.layers):
        a = layer.self_attn
        y = rms_hf(h, layer.input_layernorm.weight, eps)
        q = rms_hf(lin(y, a.q_proj.weight).view(B, H, D), a.q_norm.weight, eps)
        k = rms_hf(lin(y, a.k_proj.weight).view(B, KV, D), a.k_norm.weight, eps)
        v = lin(y, a.v_proj.weight).view(B, KV, D)
        q = q * c + rotate_half(q) * s
        k = k * c + rotate_half(k) * s
        kc[i][slots, :, pos] = k
        vc[i][slots, :, pos] = v
        K = kc[i][:, :, :ctx].index_select(0, slots)
        V = vc[i][:, :, :ctx].index_select(0, slots)
        scores = torch.matmul(q.view(B, KV, G, D).float(), K.float().transpose(-1, -2))
        if attention == 'gather':
            scores = scores.to(q.dtype).float() * scaling + bias
            o = torch.matmul(scores.softmax(-1).to(q.dtype).float(), V.float()).to(q.dtype).reshape(B, H * D)
        else:
            scores = scores * scaling + bias
            o = torch.matmul(scores.softmax(-1), V.float()).to(q.dtype).reshape(B, H * D)
        h = h + lin(o, a.o_proj.weight)
        y2 = rms_hf(h, layer.post_attention_layernorm.weight, eps)
        m = layer.mlp
        h = h + lin(F.silu(lin(y2, m.gate_proj.weight)) * lin(y2, m.up_proj.weight), m.down_proj.weight)
    out = rms_hf(h, bb.lm.model.norm.weight, eps)
    lengths.index_add_(0, slots, real if real is not None else torch.ones_like(slots))
    return out


# ---------------------------------------------------------------- depth (fused body)
def _norm(x, mod, dt):
    """LayerNorm (fp32 stats, one rounding) when the module has a bias, else Qwen-style RMSNorm."""
    b = getattr(mod, 'bias', None)
    eps = getattr(mod, 'eps', None)
    xf = x.float()
    if b is not None:
        eps = 1e-5 if eps is None else eps
        mu = xf.mean(-1, keepdim=True)
        d = xf - mu
        var = (d * d).mean(-1, keepdim=True)
        return (d / torch.sqrt(var + eps) * mod.weight.float() + b.float()).to(dt)
    eps = torch.finfo(dt).eps if eps is None else eps
    inv = 1.0 / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return ((xf * inv).to(dt).float() * mod.weight.float()).to(dt)


def _attend(q, k, v, causal_from):
    """q [B, Tq, H, hd], k/v [B, n, H, hd]; query j attends keys 0..causal_from+j. fp32 softmax, output rounded."""
    B, Tq, H, hd = q.shape
    n = k.shape[1]
    s = torch.einsum('bthd,bnhd->bhtn', q.float(), k.float()) * hd ** -0.5
    mask = torch.arange(n)[None, :] > (causal_from + torch.arange(Tq))[:, None]
    s = s.masked_fill(mask[None, None], float('-inf'))
    p = s.softmax(-1)
    return torch.einsum('bhtn,bnhd->bthd', p, v.float()).to(q.dtype)


def depth_weights(model, dt):
    """Flatten a synth/reference-shaped depth model into plain CPU tensors of dtype dt."""
    d = model.depth
    cv = lambda t: t.detach().to('cpu', dt)  # noqa: E731
    if hasattr(d, 'embed'):
        embed, level0 = cv(d.embed), cv(d.level0)
    else:
        table = (cv(d.code_lo.weight).float() @ cv(d.code_up.weight).float().t()).to(dt)
        table = table.view(N_LEVELS - 1, d.n_codes, -1)
        lvl = cv(d.level_emb.weight)
        embed = (table + lvl[1:N_LEVELS, None]).to(dt)
        level0 = lvl[0]
    return dict(d=d, embed=embed, level0=level0, in_proj=cv(d.in_proj.weight),
                gol=list(getattr(d, 'group_of_level', [None] + list(range(8)) + [8] * 8 + [9] * 8 + [10] * 7)),
                H=int(getattr(d, 'n_heads', 16)), heads=[cv(h.weight) for h in d.heads], dt=dt)


def _ffn(blk, y, dt):
    cv = lambda t: t.detach().to('cpu', dt)  # noqa: E731
    if hasattr(blk, 'gate_up'):
        gu = lin(y, cv(blk.gate_up.weight))
        F_ = gu.shape[-1] // 2
        return lin(F.silu(gu[..., :F_].float()).to(dt) * gu[..., F_:], cv(blk.down.weight))
    return lin(F.gelu(lin(y, cv(blk.f1.weight)).float()).to(dt), cv(blk.f2.weight))


def depth_frame(model, h, cb0, u, temp, top_k, greedy=False, cross=None, forced=None, dt=torch.bfloat16):
    """h [B, d_bb], cb0 [B] long, u [B, 31] uniforms. cross: [B, LAYERS, D] speaker constants or None.
    forced: [B, 32] codes to feed the prefix instead of the sampled ones (teacher forcing).
    Returns (codes [B, 32] long, logits [B, 31, V] in dt)."""
    W = depth_weights(model, dt)
    d = W['d']
    cv = lambda t: t.detach().to('cpu', dt)  # noqa: E731
    B = h.shape[0]
    D = W['in_proj'].shape[0]
    H = W['H']
    hd = D // H
    prefix = torch.zeros(B, N_LEVELS, D, dtype=dt)
    prefix[:, 0] = (lin(h.to(dt), W['in_proj']).float() + W['level0'].float()).to(dt)
    prefix[:, 1] = W['embed'][0][cb0]
    codes = torch.zeros(B, N_LEVELS, dtype=torch.long)
    codes[:, 0] = cb0
    logits_all = []
    kv = {}
    previous = None
    for level in range(1, N_LEVELS):
        group = W['gol'][level]
        n = level + 1
        incremental = group == previous
        T, p0 = (1, level) if incremental else (n, 0)
        blocks = d.groups[group]
        x = prefix[:, p0:p0 + T]
        y = _norm(x, blocks[0].n1, dt)
        for li, blk in enumerate(blocks):
            qkv = lin(y, cv(blk.qkv.weight)).view(B, T, 3, H, hd)
            if li not in kv:
                kv[li] = (torch.zeros(B, N_LEVELS, H, hd, dtype=dt), torch.zeros(B, N_LEVELS, H, hd, dtype=dt))
            kv[li][0][:, p0:p0 + T] = qkv[:, :, 1]
            kv[li][1][:, p0:p0 + T] = qkv[:, :, 2]
            last_only = li == len(blocks) - 1 and not incremental
            tq0 = T - 1 if last_only else 0
            a = _attend(qkv[:, tq0:, 0], kv[li][0][:, :p0 + T], kv[li][1][:, :p0 + T], p0 + tq0)
            x = x[:, tq0:]
            Tq = T - tq0
            x = (x.float() + lin(a.reshape(B, Tq, D), cv(blk.o.weight)).float()).to(dt)
            y2 = _norm(x, blk.n2, dt)
            f = _ffn(blk, y2, dt)
            x = (x.float() + f.float()).to(dt)
            if cross is not None:
                x = (x.float() + cross[:, li, None].float()).to(dt)
            nxt = blocks[li + 1].n1 if li + 1 < len(blocks) else d.norm
            y = _norm(x, nxt, dt)
            T, p0 = Tq, p0 + tq0
        logits = lin(y[:, -1], W['heads'][level - 1])
        logits_all.append(logits)
        if dt == torch.float32:
            xs = logits.numpy() * np.float32(1.0 / temp)
            code = torch.tensor([coracle.topk_sample(xs[b], top_k, float(u[b, level - 1]), greedy)
                                 for b in range(B)], dtype=torch.long)
        else:
            bits = logits.view(torch.int16).numpy().view(np.uint16)
            code = torch.from_numpy(coracle.topk_sample_rows(bits, 1.0 / temp, top_k, u[:, level - 1].numpy(),
                                                             greedy=greedy, is_f16=dt == torch.float16)).long()
        codes[:, level] = code
        feed = forced[:, level] if forced is not None else code
        if n < N_LEVELS:
            prefix[:, n] = W['embed'][level][feed]
        previous = group
    return codes, torch.stack(logits_all, 1)


def feedback(audio_in, codes):
    """norm(sum_l table[codes_l + n_codes*l] / sqrt(32)) with an fp32 sum and fp32 RMSNorm, one final rounding."""
    table = audio_in.table.weight.detach().cpu()
    dt = table.dtype
    n_codes = audio_in.n_codes
    idx = codes.long() + torch.arange(codes.shape[1]) * n_codes
    e = table[idx].float().sum(1).to(dt)
    x = (e.float() / math.sqrt(codes.shape[1])).to(dt).float()
    eps = getattr(audio_in.norm, 'eps', None)
    eps = torch.finfo(dt).eps if eps is None else eps
    inv = 1.0 / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return (x * inv * audio_in.norm.weight.detach().cpu().float()).to(dt)


def cb0_step(head_w, h, u, temp, top_k, aeos=-1):
    """cb0 with the BASELINE settings (no penalty/stop state): logits = h @ head^T (bf16), C-oracle sampler."""
    logits = lin(h, head_w.detach().cpu())
    bits = logits.view(torch.int16).numpy().view(np.uint16)
    out = [coracle.cb0_sample(bits[b], aeos, temp, top_k, 0.0, 0.0, None, None, 0, None, None, float(u[b]))[0]
           for b in range(h.shape[0])]
    return torch.tensor(out, dtype=torch.long), logits


def loop_detect_batch(W, n, stall=32, period_win=64, period_thr=0.7, pmin=2, pmax=16):
    """The engine's loop guard (maya3/guards.py:80-107): W [S, hist] int (newest last, -1 = empty), n [S] frames.
    A row stalls when its last `stall` codes all equal the first of them (n >= max(12, stall)); otherwise it has
    period p for the smallest p in pmin..pmax whose lag-p match fraction over the last period_win codes, a float64
    mean, reaches period_thr (n >= max(12, stall, period_win)). Returns None | 'stall' | 'period:<p>' per row."""
    W = np.asarray(W)
    n = np.asarray(n)
    out = []
    for i in range(W.shape[0]):
        row, frames = W[i], int(n[i])
        if frames < max(12, stall):
            out.append(None)
            continue
        tail = row[-stall:]
        if np.all(tail == tail[0]):
            out.append("stall")
            continue
        hit = None
        if frames >= max(12, stall, period_win):
            win = row[-period_win:]
            for p in range(pmin, pmax + 1):
                if np.mean(win[p:] == win[:-p]) >= period_thr:
                    hit = p
                    break
        out.append(None if hit is None else f"period:{hit}")
    return out
