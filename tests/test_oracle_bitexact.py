"""Pins of the C oracle (oracle/m3x_oracle.c) against independent references: torch, math, closed forms,
known-answer vectors and the distribution the reference samples from. CPU only."""
import math

import numpy as np
import pytest
import torch

from oracle import coracle as C


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ---------------------------------------------------------------- bf16 rounding
def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    u = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    # every bf16 pattern with its halfway / just-below / just-above fp32 neighbours
    base = (np.arange(1 << 16, dtype=np.uint32) << 16)
    u = np.concatenate([u, base, base | 0x7fff, base | 0x8000, base | 0x8001, base | 0x17fff & 0xffff])
    x = u.view(np.float32)
    x = x[~np.isnan(x)]
    got = C.bf16_round(x)
    ref = _bits(torch.from_numpy(x.copy()).to(torch.bfloat16))
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- exp
def test_expf_accuracy_and_special_values():
    x = np.linspace(-87.0, 0.0, 1_000_001, dtype=np.float32)
    y = C.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(y - ref) / ulp).max() <= 1.0
    assert C.expf(np.zeros(1, np.float32))[0] == 1.0
    assert C.expf(np.array([-87.5, -200.0, -np.inf], np.float32)).tolist() == [0.0, 0.0, 0.0]
    # e^(k ln 2) lands within an ulp of 2^k (the scaling step is exact)
    k = np.arange(-120, 1)
    xs = (k * np.log(2.0)).astype(np.float32)
    got = C.expf(xs).astype(np.float64)
    assert np.all(np.abs(got - np.exp(xs.astype(np.float64))) <= np.spacing(got.astype(np.float32)))


# ---------------------------------------------------------------- Philox4x32-10 known answers (Random123 kat_vectors)
@pytest.mark.parametrize("ctr,key,out", [
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
])
def test_philox_known_answers(ctr, key, out):
    assert C.philox4x32_10(ctr, key) == out


def test_philox_uniform_range_and_moments():
    u = np.array([C.philox_uniform(12345, c, l) for c in range(200) for l in range(32)])
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.02 and abs(u.var() - 1 / 12) < 0.01
    # distinct streams per (seed, counter, level)
    assert C.philox_uniform(1, 0, 0) != C.philox_uniform(2, 0, 0) != C.philox_uniform(1, 1, 0)


# ---------------------------------------------------------------- add + RMSNorm
def _hf_rms(x, w, eps):
    xf = x.float()
    return w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)


@pytest.mark.parametrize("n", [1024, 2048])
def test_add_rms_vs_torch(n):
    g = torch.Generator().manual_seed(n)
    h = torch.randn(64, n, generator=g).to(torch.bfloat16)
    a = torch.randn(64, n, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)
    ho, y = C.add_rms(_bits(h), _bits(a), _bits(w), 1e-6)
    s = h + a  # torch bf16 add: fp32 add, one rounding
    assert np.array_equal(ho, _bits(s))
    ref = _hf_rms(s, w, 1e-6).float()
    got = torch.from_numpy(C.bf16_to_f32(y)).view(ref.shape)
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(1e-30))) - 7)
    diff = (got - ref).abs() / ulp
    assert diff.max() <= 1.0 and (diff > 0).float().mean() < 0.02
    # plain norm (a == NULL) is the HF module on h
    _, y0 = C.add_rms(_bits(h), None, _bits(w), 1e-6)
    ref0 = _hf_rms(h, w, 1e-6).float()
    d0 = (torch.from_numpy(C.bf16_to_f32(y0)).view(ref0.shape) - ref0).abs()
    assert d0.max() <= (torch.exp2(torch.floor(torch.log2(ref0.abs().clamp_min(1e-30))) - 7)).max()


def test_add_rms_constant_row_closed_form():
    n = 1024
    c = np.float32(1.5)
    h = np.full((1, n), C.bf16_round(np.array([c]))[0], np.uint16)
    w = C.bf16_round(np.full(n, 0.75, np.float32))
    _, y = C.add_rms(h, None, w, 1e-6)
    inv = np.float32(1.0) / np.sqrt(np.float32(c * c) + np.float32(1e-6), dtype=np.float32)
    expect = C.bf16_round(C.bf16_to_f32(C.bf16_round(np.array([c * inv], np.float32))) * np.float32(0.75))
    assert np.all(y == expect[0])


# ---------------------------------------------------------------- q/k norm + RoPE
def _rope_tables(cap, D, theta=1e6):
    inv = 1.0 / (theta ** (torch.arange(0, D, 2).float() / D))
    fr = torch.arange(cap).float()[:, None] * inv[None]
    emb = torch.cat([fr, fr], -1)
    return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)


def _rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), -1)


def test_qk_norm_rope_vs_hf_formula():
    # the reference's own check (maya3/tests/test_rope_kernel.py:6-26): rel L2 < 1e-2 vs HF q/k-norm + RoPE
    g = torch.Generator().manual_seed(0)
    B, H, KV, D, CAP = 5, 16, 8, 128, 512
    qkv = (torch.randn(B, (H + 2 * KV) * D, generator=g) * 2).to(torch.bfloat16)
    wq = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    wk = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    pos = torch.tensor([0, 7, 100, 300, 511], dtype=torch.int32)
    cos, sin = _rope_tables(CAP, D)
    q, k = C.qk_norm_rope(_bits(qkv), H, KV, D, pos.numpy(), _bits(cos), _bits(sin), _bits(wq), _bits(wk), 1e-6)
    q_, k_, _ = qkv.split([H * D, KV * D, KV * D], -1)
    c, s = cos[pos.long()][:, None], sin[pos.long()][:, None]
    qn = _hf_rms(q_.view(B, H, D), wq, 1e-6)
    kn = _hf_rms(k_.view(B, KV, D), wk, 1e-6)
    qr = qn * c + _rotate_half(qn) * s
    kr = kn * c + _rotate_half(kn) * s
    rel = lambda a, b: ((a - b.float()).norm() / b.float().norm()).item()  # noqa: E731
    qg = torch.from_numpy(C.bf16_to_f32(q))
    kg = torch.from_numpy(C.bf16_to_f32(k))
    assert rel(qg, qr) < 1e-2 and rel(kg, kr) < 1e-2
    # position 0: cos = 1, sin = 0, the rotation is the identity: the output is the normed head (HF rounding,
    # at most one bf16 ulp apart where the fp32 sum of squares is associated differently)
    ref0 = qn[0].float()
    ulp0 = torch.exp2(torch.floor(torch.log2(ref0.abs().clamp_min(1e-30))) - 7)
    d0 = (qg[0] - ref0).abs() / ulp0
    assert d0.max() <= 1.0 and (d0 > 0).float().mean() < 0.02
    # each (i, i + D/2) pair keeps its norm under the rotation (up to bf16 rounding)
    half = D // 2
    pn = qg[..., :half] ** 2 + qg[..., half:] ** 2
    pr = qn.float()[..., :half] ** 2 + qn.float()[..., half:] ** 2
    assert ((pn - pr).abs() / pr.clamp_min(1e-6)).median() < 1e-2


# ---------------------------------------------------------------- samplers
def _exact_topk_probs(x, k):
    kth = np.sort(x)[::-1][k - 1]
    p = np.where(x >= kth, np.exp(x.astype(np.float64) - x.max()), 0.0)
    return p / p.sum()


def test_topk_sampler_distribution():
    # the reference's sampler test recipe (maya3/tests/test_depth_fused.py:12-23): TV < 0.03 over 200k draws,
    # zero mass outside the top-k set
    rng = np.random.default_rng(0)
    logits = (rng.standard_normal(2048) * 3).astype(np.float32)
    x = (logits * np.float32(1 / 0.7)).astype(np.float32)
    u = rng.random(200_000, dtype=np.float32)
    d = C.topk_sample_many(x, 64, u)
    emp = np.bincount(d, minlength=2048) / d.size
    p = _exact_topk_probs(x, 64)
    assert 0.5 * np.abs(emp - p).sum() < 0.03
    assert emp[p == 0].sum() == 0


def test_topk_sampler_special_cases():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(2048).astype(np.float32)
    top = int(np.argmax(x))
    assert C.topk_sample(x, 50, 0.0) == top                         # u = 0 -> the top candidate
    assert all(C.topk_sample(x, 1, float(v)) == top for v in rng.random(20))  # k = 1 -> argmax
    assert C.topk_sample(x, 50, 0.9, greedy=True) == top
    # ties at the k-th value are all kept (x >= kth), lowest index first among equals
    y = np.full(16, -1.0, np.float32)
    y[[3, 7, 11]] = 2.0
    y[[1, 5]] = 5.0
    draws = C.topk_sample_many(y, 3, np.linspace(0, 0.999999, 2001, dtype=np.float32))
    assert set(np.unique(draws)) == {1, 3, 5, 7, 11}
    assert C.topk_sample(y, 3, 0.0) == 1 and C.topk_sample(y, 3, 0.0, greedy=True) == 1
    # the inverse CDF is monotone in u along the (x desc, index asc) order
    order = [1, 5, 3, 7, 11]
    ranks = [order.index(v) for v in draws]
    assert ranks == sorted(ranks)


def _engine_cb0_reference(logits, temp, aeos_bias, rep, hist, frames, min_t, hazard, top_k, aeos=2048, top_p=None):
    """maya3/engine.py:657-686 in torch (deterministic part): probs, pa, arg, hazard, stop code, q."""
    lg = logits.float() / temp[:, None]
    lg[:, aeos] += aeos_bias
    pen = torch.zeros_like(lg)
    pen.scatter_add_(1, hist.clamp_min(0), (hist >= 0).float())
    pen[:, aeos] = 0
    lg = lg - rep[:, None] * (pen > 0).float()
    srt = lg.sort(-1, descending=True).values
    kth = srt.gather(1, (top_k - 1).clamp(0, lg.shape[1] - 1)[:, None])
    lg = lg.masked_fill(lg < kth, -float('inf'))
    if top_p is not None:  # :669-672
        sp_, si = lg.softmax(-1).sort(-1, descending=True)
        drop = (sp_.cumsum(-1) - sp_) > top_p[:, None]
        lg = lg.masked_fill(torch.zeros_like(drop).scatter(1, si, drop), -float('inf'))
    probs = lg.softmax(-1)
    pa = probs[:, aeos]
    arg = probs.argmax(-1)
    can = frames >= min_t
    hz = torch.where(can, 1 - (1 - hazard) * (1 - pa), hazard)
    code = torch.zeros_like(arg)
    code = torch.where(can & (hz >= .6), torch.full_like(code, 4), code)
    code = torch.where(can & (pa >= .35), torch.full_like(code, 3), code)
    code = torch.where(can & (arg == aeos), torch.full_like(code, 2), code)
    q = probs.clone()
    q[:, aeos] = 0
    q = q / q.sum(-1, keepdim=True).clamp_min(1e-12)
    return code, hz, q


def test_cb0_stop_logic_vs_engine():
    g = torch.Generator().manual_seed(2)
    B, V = 64, 2049
    logits = (torch.randn(B, V, generator=g) * 2).to(torch.bfloat16)
    logits[:16, 2048] = 9.0   # AEOS is the argmax
    logits[16:32, 2048] = 4.0  # AEOS mass near the thresholds
    temp = torch.full((B,), 0.9)
    bias = torch.zeros(B)
    bias[40:48] = 3.0
    rep = torch.full((B,), 0.8)
    hist = torch.randint(-1, V - 1, (B, 12), generator=g)
    frames = torch.randint(0, 10, (B,), generator=g)
    min_t = torch.full((B,), 4)
    hazard = torch.rand(B, generator=g) * 0.7
    code, hz, _ = _engine_cb0_reference(logits, temp, bias, rep, hist, frames, min_t, hazard, torch.full((B,), 64))
    for b in range(B):
        h = hist[b].numpy().astype(np.int64).copy()
        fr = np.array([frames[b].item()], np.int64)
        hzb = np.array([hazard[b].item()], np.float32)
        ctr = np.zeros(1, np.int32)
        cb0, stop = C.cb0_sample(_bits(logits[b]), 2048, 0.9, 64, float(bias[b]), 0.8, h, fr, 4, hzb, ctr, 0.5)
        assert stop == code[b].item(), b
        assert abs(hzb[0] - hz[b].item()) < 1e-5
        assert fr[0] == frames[b].item() + 1 and ctr[0] == 1 and h[-1] == cb0 and cb0 != 2048


def test_cb0_sample_distribution_excludes_aeos():
    g = torch.Generator().manual_seed(3)
    logits = (torch.randn(1, 2049, generator=g) * 2).to(torch.bfloat16)
    logits[0, 2048] = 5.0
    z = torch.zeros(1)
    _, _, q = _engine_cb0_reference(logits, torch.full((1,), 0.9), z, z, torch.full((1, 12), -1), torch.zeros(1),
                                    torch.zeros(1), z, torch.full((1,), 50))
    rng = np.random.default_rng(4)
    bits = _bits(logits[0])
    draws = np.array([C.cb0_sample(bits, 2048, 0.9, 50, 0.0, 0.0, None, None, 0, None, None, float(u))[0]
                      for u in rng.random(40_000, dtype=np.float32)])
    emp = np.bincount(draws, minlength=2049) / draws.size
    tv = 0.5 * np.abs(emp - q[0].double().numpy()).sum()
    assert tv < 0.04 and emp[2048] == 0 and emp[q[0].numpy() == 0].sum() == 0


def _distinct_head_logits(g, B, V, n_head=96):
    """bf16 logits whose n_head largest are distinct multiples of 1/16 in (1, 7] (exact in bf16, no ties for the
    top-k and top-p sorts) over a body below 1."""
    body = (torch.randn(B, V, generator=g) * 0.3).clamp(-3, 0.9)
    for b in range(B):
        idx = torch.randperm(V, generator=g)[:n_head]
        body[b, idx] = 7.0 - torch.arange(n_head, dtype=torch.float32) / 16
    return body.to(torch.bfloat16)


def test_cb0_top_p_matches_engine_mask():
    """The oracle's top-p cut against maya3/engine.py:669-672: with no AEOS class, the codes drawn over a fine
    grid of uniforms are exactly the engine's kept set, and the stop statistics (pa, hazard, stop code) and the
    renormalised AEOS-free distribution agree when an AEOS class is present."""
    g = torch.Generator().manual_seed(11)
    B, V = 6, 2049
    logits = _distinct_head_logits(g, B, V)
    top_p = torch.tensor([0.05, 0.3, 0.5, 0.75, 0.9, 0.99])
    top_k = torch.full((B,), 64)
    z = torch.zeros(B)
    none_hist = torch.full((B, 12), -1)
    grid = (np.arange(4_000, dtype=np.float32) + 0.5) / 4_000
    # no AEOS class: compare kept sets (the engine formula with aeos pointing at a class it never keeps)
    logits_na = logits.clone()
    logits_na[:, 2048] = -8.0
    _, _, q = _engine_cb0_reference(logits_na, torch.full((B,), 0.9), z, z, none_hist, torch.zeros(B), torch.zeros(B),
                                    z, top_k, top_p=top_p)
    for b in range(B):
        bits = _bits(logits_na[b])
        drawn = {C.cb0_sample(bits, -1, 0.9, 64, 0.0, 0.0, None, None, 0, None, None, float(u), float(top_p[b]))[0]
                 for u in grid}
        kept = set(torch.nonzero(q[b] > 0).flatten().tolist())
        assert drawn == kept, (b, sorted(drawn ^ kept))
        assert len(kept) < 64
    # top_p = 1 is the plain top-k draw; a tiny top_p keeps the argmax alone
    bits = _bits(logits[0])
    for u in (0.0, 0.3, 0.97):
        assert (C.cb0_sample(bits, -1, 0.9, 64, 0.0, 0.0, None, None, 0, None, None, u, 1.0) ==
                C.cb0_sample(bits, -1, 0.9, 64, 0.0, 0.0, None, None, 0, None, None, u))
        assert C.cb0_sample(bits, -1, 0.9, 64, 0.0, 0.0, None, None, 0, None, None, u, 1e-6)[0] == \
            int(logits[0].float().argmax())
    # with an AEOS class inside the top-p set: stop code and hazard as the engine computes them on the cut set
    logits_a = logits.clone()
    logits_a[:, 2048] = torch.tensor([7.03125, 6.5, 5.0, 6.96875, 1.0, 4.0])  # distinct from the head values
    frames = torch.full((B,), 5)
    min_t = torch.full((B,), 4)
    hazard = torch.full((B,), 0.3)
    code, hz, q = _engine_cb0_reference(logits_a, torch.full((B,), 0.9), z, z, none_hist, frames, min_t, hazard, top_k,
                                        top_p=top_p)
    for b in range(B):
        fr = np.array([5], np.int64)
        hzb = np.array([0.3], np.float32)
        bits = _bits(logits_a[b])
        _, stop = C.cb0_sample(bits, 2048, 0.9, 64, 0.0, 0.0, None, fr, 4, hzb, None, 0.5, float(top_p[b]))
        assert stop == code[b].item() and abs(hzb[0] - hz[b].item()) < 1e-5, b
        drawn = {C.cb0_sample(bits, 2048, 0.9, 64, 0.0, 0.0, None, None, 0, None, None, float(u),
                              float(top_p[b]))[0] for u in grid}
        kept = set(torch.nonzero(q[b] > 0).flatten().tolist())
        assert drawn == kept or (not kept and drawn == {0}), (b, sorted(drawn ^ kept))
