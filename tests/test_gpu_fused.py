"""Projections fused with the residual stream (m3x_linear_resid) and with the norm that follows it, folded into the
consumer (m3x_linear_normed with ops.fold_norm weights), against the launch chain they replace (projection, then
add+norm, then projection) and against fp32 torch references."""
import pytest
import torch

from helpers import floor_check, report

pytestmark = pytest.mark.gpu


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _tile_stats(v, kind):
    """fp32 (sum, second moment) per 16-column tile of rows v [M, N]: sum of squares (RMS) or of squared deviations
    from the tile mean (LayerNorm)."""
    t = v.float().view(v.shape[0], -1, 16)
    s = t.sum(-1)
    q = (t * t).sum(-1) if kind == 1 else ((t - t.mean(-1, keepdim=True)) ** 2).sum(-1)
    return torch.stack([s, q], -1)


@pytest.mark.parametrize("M,N,K", [(1, 1024, 1024), (5, 1024, 2816), (16, 1024, 3072), (64, 1024, 1024),
                                   (224, 1024, 1024), (224, 1024, 2816), (224, 1024, 3072), (250, 1024, 2048),
                                   (100, 2048, 1024), (600, 1024, 3072), (2264, 1024, 1024), (2264, 1024, 3072)])
@pytest.mark.parametrize("kind", [0, 1])
def test_linear_resid_bf16(gpu, M, N, K, kind):
    """h_out = dt(h + dt(x W^T)) bit for bit against the plain projection plus a bf16 add (same plan, same sums);
    h read through a strided view and updated in place; tile statistics against fp32 sums of the stored row."""
    from m3x import ops
    g = _g(M * 13 + K + kind)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(gpu)
    w = ops.pack_weight((torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu))
    big = torch.randn(M, 3 * N, generator=g).to(torch.bfloat16).to(gpu)
    h = big[:, N:2 * N]
    h0, big0 = h.clone(), big.clone()
    part = torch.full((ops.tile_stats_elems(M, N),), float("nan"), device=gpu)
    ops.linear_resid(x, w, h, h, part, kind)
    ref = (h0.float() + ops.linear(x, w).float()).to(torch.bfloat16)
    assert torch.equal(h.cpu(), ref.cpu())
    assert torch.equal(big[:, :N].cpu(), big0[:, :N].cpu()) and torch.equal(big[:, 2 * N:].cpu(), big0[:, 2 * N:].cpu())
    st = part.view(M, N // 16, 2).cpu()
    exp = _tile_stats(ref.cpu(), kind)
    assert torch.allclose(st, exp, rtol=1e-5, atol=1e-4), (st - exp).abs().max()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T", [(4, 3), (224, 1), (16, 31)])
def test_linear_resid_cross_term(gpu, dtype, B, T):
    """The per-seat constant c[m // T] (the depth trunk's speaker term) is added after the residual, rounded once
    more, as add_norm does with its c."""
    from m3x import ops
    g = _g(B * 7 + T)
    M, N, K = B * T, 1024, 2816
    x = torch.randn(M, K, generator=g).to(dtype).to(gpu)
    w = ops.pack_weight((torch.randn(N, K, generator=g) * 0.02).to(dtype).to(gpu))
    h = torch.randn(M, N, generator=g).to(dtype).to(gpu)
    cross = torch.randn(B, 4 * N, generator=g).to(dtype).to(gpu)
    c = cross[:, 2 * N:3 * N]
    out = torch.empty(M, N, dtype=dtype, device=gpu)
    part = torch.empty(ops.tile_stats_elems(M, N), device=gpu)
    ops.linear_resid(x, w, h, out, part, 0, c=c, tc=T)
    lin = ops.linear(x, w).float()
    ref = ((h.float() + lin).to(dtype).float() + c.repeat_interleave(T, 0).float()).to(dtype)
    assert torch.equal(out.cpu(), ref.cpu())
    exp = _tile_stats(ref.cpu(), 0)
    assert torch.allclose(part.view(M, N // 16, 2).cpu(), exp, rtol=1e-5, atol=1e-4)


def _norm_f32(h, w, b, eps, kind):
    """The norm in fp32 with no rounding (the truth both bf16 orders are measured against)."""
    x = h.float()
    if kind == 0:
        return torch.nn.functional.layer_norm(x, (x.shape[1],), w.float(), b.float(), eps)
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w.float()


def _act_ref(a, u, act, dtype):
    if act == 0:
        return torch.nn.functional.silu(a.to(dtype).float()).to(dtype).float() * u.to(dtype).float()
    if act == 1:
        return torch.nn.functional.gelu(a.to(dtype).float())
    return a


@pytest.mark.parametrize("M", [1, 3, 16, 64, 130, 224, 600, 2264])
@pytest.mark.parametrize("act,kind", [(-1, 1), (0, 1), (1, 0), (-1, 0)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_linear_normed(gpu, M, act, kind, dtype):
    """norm(h) . W^T with the norm folded (weights from fold_norm, row scale and shift from linear_resid's tile
    statistics) against an fp32 evaluation of norm-then-project at the bf16 bar, and no further from it than the
    two-launch chain it replaces (add+norm kernel, rounded normed rows, projection). Norm weights 1 + N(0, 0.1)."""
    _normed_case(gpu, M, act, kind, dtype, wide=False)


@pytest.mark.parametrize("M", [1, 16, 224, 2264])
@pytest.mark.parametrize("act,kind", [(-1, 1), (0, 1), (1, 0)])
def test_linear_normed_wide_norm_weights(gpu, M, act, kind):
    """The same bar with norm weights spread like trained ones: exp(N(0, 0.8)), about 0.1x to 20x. The folded
    weight rounds W * w to bf16 once, so its relative error stays that of a bf16 weight at every scale of w."""
    _normed_case(gpu, M, act, kind, torch.bfloat16, wide=True)


def _normed_case(gpu, M, act, kind, dtype, wide):
    from m3x import ops
    g = _g(M * 31 + act * 5 + kind + 1000 * wide)
    D = 1024
    N = {-1: 3072, 0: 2816, 1: 3072}[act]
    eps = 1e-6 if kind == 1 else 1e-5
    x = torch.randn(M, 2816, generator=g).to(dtype).to(gpu)
    wd = ops.pack_weight((torch.randn(D, 2816, generator=g) * 0.02).to(dtype).to(gpu))
    h = (2 * torch.randn(M, D, generator=g) + 0.5).to(dtype).to(gpu)
    z = torch.randn(D, generator=g)
    nw = (torch.exp(0.8 * z) if wide else 1 + 0.1 * z).to(dtype).to(gpu)
    nb = (0.1 * torch.randn(D, generator=g)).to(dtype).to(gpu) if kind == 0 else None
    part = torch.empty(ops.tile_stats_elems(M, D), device=gpu)
    hn = ops.linear_resid(x, wd, h, torch.empty_like(h), part, kind)
    W = (torch.randn(2 * N if act == 0 else N, D, generator=g) * 0.02).to(dtype).to(gpu)
    pf, u, v = ops.fold_norm(W, nw, nb)
    if act == 0:
        got = ops.linear_normed(hn, part, eps, kind, pf.rows(0, N), pf.rows(N, 2 * N), act, u=u, v=v)
    else:
        got = ops.linear_normed(hn, part, eps, kind, pf, None, act, u=u, v=v)
    # the two-launch chain: add+norm kernel, then the projection of the rounded normed rows
    y = torch.empty_like(hn)
    ops.add_norm(hn, None, None, None, y, nw, nb, eps, 1, kind)
    pw = ops.pack_weight(W)
    if act == 0:
        two = ops.linear_act(y, pw.rows(0, N), pw.rows(N, 2 * N), act)
    else:
        two = ops.linear(y, pw) if act == -1 else ops.linear_act(y, pw, None, act)
    yr = _norm_f32(hn.cpu(), nw.cpu(), None if nb is None else nb.cpu(), eps, kind)
    Wc = W.float().cpu()
    a = yr @ Wc[:N].t()
    truth = _act_ref(a, yr @ Wc[N:].t() if act == 0 else None, act, dtype)
    # the bf16 floor against the truth, with the launch chain as the bf16 reference path (rel-L2 within 1.25x its
    # own, max-abs within 2e-2 or twice its own, cosine to it >= 0.9995), and no worse than it in rel-L2 by > 25 %
    ok, info = floor_check(got, two, truth)
    report(f"linear_normed M={M} act={act} kind={kind} {dtype} wide={wide}", info)
    assert ok, info
    e_got = (got.float().cpu() - truth).norm().item()
    e_two = (two.float().cpu() - truth).norm().item()
    assert e_got <= 1.25 * e_two + 1e-4 * truth.norm().item(), (e_got, e_two)


def test_linear_normed_rejects_bad_args(gpu):
    from m3x import ops
    x = torch.zeros(4, 1024, dtype=torch.bfloat16, device=gpu)
    w = ops.pack_weight(torch.zeros(64, 1024, dtype=torch.bfloat16, device=gpu))
    nw = torch.ones(1024, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        ops.linear_normed(x, torch.zeros(10, device=gpu), 1e-6, 1, w)
    with pytest.raises(ValueError):  # LayerNorm without the folded weight's column vectors
        ops.linear_normed(x, torch.zeros(ops.tile_stats_elems(4, 1024), device=gpu), 1e-5, 0, w)
    w2 = ops.pack_weight(torch.zeros(64, 2048, dtype=torch.bfloat16, device=gpu))
    x2 = torch.zeros(4, 2048, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError):  # the norm prologue covers rows of width 1024 only
        ops.linear_normed(x2, torch.zeros(ops.tile_stats_elems(4, 2048), device=gpu), 1e-6, 1, w2)


@pytest.mark.parametrize("M", [1, 3, 16, 17, 100, 200, 224, 256, 300, 513, 700, 2264])
@pytest.mark.parametrize("normed", [False, True])
def test_linear_qk_rope(gpu, M, normed):
    """The q|k|v projection with the q/k norm, RoPE and cache writes: the same bits as the projection
    (linear / linear_normed) followed by qk_norm_rope_cache, in one launch where the plan holds whole heads
    (193..256 rows and above 512: qkv left untouched) and through qkv elsewhere; cache entries other than the
    rows' own (slot, pos) unchanged."""
    from m3x import ops
    g = _g(M * 3 + normed)
    H, KV, D, K, eps = 16, 8, 128, 1024, 1e-6
    N = (H + 2 * KV) * D
    S, cap = 40, 192
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(gpu)
    W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
    part = None
    if normed:
        # rows with tile statistics, as the previous layer's down projection leaves them
        wd = ops.pack_weight((torch.randn(K, 2816, generator=g) * 0.02).to(torch.bfloat16).to(gpu))
        a = torch.randn(M, 2816, generator=g).to(torch.bfloat16).to(gpu)
        part = torch.empty(ops.tile_stats_elems(M, K), device=gpu)
        x = ops.linear_resid(a, wd, x, torch.empty_like(x), part, ops.NORM_RMS)
        nw = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16).to(gpu)
        w, u, v = ops.fold_norm(W, nw)
    else:
        w = ops.pack_weight(W)
    rows = torch.arange(M)
    slots = (rows % S).to(gpu)                          # distinct (slot, pos) per row
    pos = ((rows // S) * 3 + rows % 5).int().to(gpu)
    cosb = torch.randn(cap, D, generator=g).to(torch.bfloat16).to(gpu)
    sinb = torch.randn(cap, D, generator=g).to(torch.bfloat16).to(gpu)
    wq = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(gpu)
    wk = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(gpu)
    kc0 = torch.randn(S + 1, KV, cap, D, generator=g).to(torch.bfloat16).to(gpu)
    vc0 = torch.randn(S + 1, KV, cap, D, generator=g).to(torch.bfloat16).to(gpu)
    # the two-launch chain
    qkv_ref = ops.linear_normed(x, part, eps, ops.NORM_RMS, w, u=u, v=v) if normed else ops.linear(x, w)
    q_ref = torch.empty(M, H, D, dtype=torch.bfloat16, device=gpu)
    kc_ref, vc_ref = kc0.clone(), vc0.clone()
    ops.qk_norm_rope_cache(qkv_ref, q_ref, kc_ref, vc_ref, slots, pos, cosb, sinb, wq, wk, eps, H, KV)
    # fused
    qkv = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
    q = torch.full((M, H, D), float("nan"), dtype=torch.bfloat16, device=gpu)
    kc, vc = kc0.clone(), vc0.clone()
    ops.linear_qk_rope(x, w, qkv, q, kc, vc, slots, pos, cosb, sinb, wq, wk, eps, H, KV, part=part, eps_in=eps)
    torch.cuda.synchronize()
    assert torch.equal(q.cpu(), q_ref.cpu())
    assert torch.equal(kc.cpu(), kc_ref.cpu()) and torch.equal(vc.cpu(), vc_ref.cpu())
    fused = 192 < M <= 256 or M > 512
    if fused:
        assert bool(torch.isnan(qkv.float()).all()), "the fused plan leaves qkv untouched"
    else:
        assert torch.equal(qkv.cpu(), qkv_ref.cpu())
