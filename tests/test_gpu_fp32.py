"""fp32 instances of the depth kernels (FastDepth(dtype=torch.float32), the engine's depth_dtype="fp32",
maya3/engine.py:53,192-199): projections on v_mfma_f32_16x16x4_f32 over fp32 packed fragments, add+norm, depth
attention, the sampler on fp32 logits (bit-exact against the C oracle) and the feedback / row kernels.

Bar: the kernels evaluate the fp32 math the reference's torch ops evaluate, in another summation order, so they
are compared with a float64 evaluation: every element within 1e-5 absolute plus 1e-5 relative, i.e. a few hundred
fp32 ulps, far above the ~sqrt(K) * 2^-24 relative rounding of a K-term fp32 sum and far below any bf16 error
(2^-8 relative)."""
import numpy as np
import pytest
import torch

from oracle import coracle as C

pytestmark = pytest.mark.gpu

F32_ATOL = F32_RTOL = 1e-5


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _close32(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    err = (got - ref).abs()
    bound = F32_ATOL + F32_RTOL * ref.abs()
    return bool((err <= bound).all()), dict(max_abs=err.max().item(), worst=(err - bound).max().item())


@pytest.mark.parametrize("M,N,K", [(1, 1024, 1024), (4, 3072, 1024), (16, 2816, 1024), (5, 1024, 2816),
                                   (33, 2049, 1024), (224, 1024, 2816), (3, 512, 96), (40, 1024, 1056),
                                   (700, 3072, 1024), (1, 2048, 1024), (3584, 512, 512)])
def test_linear_f32(gpu, M, N, K):
    from m3x import ops
    g = _g(M * 5 + N + K)
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.02
    pw = ops.pack_weight(w.to(gpu))
    assert pw.dtype == torch.float32
    y = ops.linear(x.to(gpu), pw)
    ok, info = _close32(y, x.double() @ w.double().t())
    assert ok, info


def test_pack_weight_f32_layout(gpu):
    """Fragment (t, s), lane l, element e holds w[16 t + l % 16][32 s + 8 (l / 16) + e]; rows past N are zero."""
    from m3x import ops
    N, K = 20, 64
    w = torch.arange(N * K, dtype=torch.float32).view(N, K)
    p = ops.pack_weight(w.to(gpu)).data.cpu().view(2, K // 32, 64, 8)
    for t in range(2):
        for s in range(K // 32):
            for lane in (0, 5, 17, 63):
                n = 16 * t + lane % 16
                ref = w[n, 32 * s + 8 * (lane // 16):32 * s + 8 * (lane // 16) + 8] if n < N else torch.zeros(8)
                assert torch.equal(p[t, s, lane], ref)


@pytest.mark.parametrize("M,I,K,kind", [(1, 2816, 1024, "swiglu"), (16, 2816, 1024, "swiglu"),
                                        (224, 2816, 1024, "swiglu"), (4, 3072, 1024, "gelu"),
                                        (31, 3072, 1024, "gelu")])
def test_linear_act_f32(gpu, M, I, K, kind):
    from m3x import ops
    g = _g(M + I)
    x = torch.randn(M, K, generator=g)
    if kind == "swiglu":
        wgu = torch.randn(2 * I, K, generator=g) * 0.02
        p = ops.pack_weight(wgu.to(gpu))
        y = ops.linear_act(x.to(gpu), p.rows(0, I), p.rows(I, 2 * I), ops.ACT_SWIGLU)
        gg = x.double() @ wgu[:I].double().t()
        ref = torch.nn.functional.silu(gg) * (x.double() @ wgu[I:].double().t())
    else:
        w1 = torch.randn(I, K, generator=g) * 0.02
        y = ops.linear_act(x.to(gpu), ops.pack_weight(w1.to(gpu)), None, ops.ACT_GELU)
        ref = torch.nn.functional.gelu(x.double() @ w1.double().t())
    ok, info = _close32(y, ref)
    assert ok, info


@pytest.mark.parametrize("rows,T,n,kind", [(4, 1, 1024, 1), (3, 5, 1024, 0), (40, 2, 1024, 1), (7, 1, 2048, 0),
                                           (64, 4, 512, 0)])
def test_add_norm_f32(gpu, rows, T, n, kind):
    """x' = x + a + c[b]; y = LayerNorm(x') (kind 0) or RMSNorm(x') (kind 1), all in fp32."""
    from m3x import ops
    g = _g(rows * 3 + n)
    B = rows
    x = torch.randn(B, T, n, generator=g)
    a = torch.randn(B * T, n, generator=g)
    c = torch.randn(B, n, generator=g)
    w = 1 + 0.1 * torch.randn(n, generator=g)
    b = 0.1 * torch.randn(n, generator=g) if kind == 0 else None
    xo = torch.empty(B * T, n, device=gpu)
    y = torch.empty(B * T, n, device=gpu)
    ops.add_norm(x.to(gpu), a.to(gpu), c.to(gpu), xo, y, w.to(gpu), None if b is None else b.to(gpu), 1e-5, T, kind)
    xp = x.reshape(B * T, n).double() + a.double() + c.double().repeat_interleave(T, 0)
    if kind == 0:
        ref = torch.nn.functional.layer_norm(xp, (n,), w.double(), b.double(), 1e-5)
    else:
        ref = xp * torch.rsqrt(xp.pow(2).mean(-1, keepdim=True) + 1e-5) * w.double()
    ok, info = _close32(xo, xp)
    assert ok, info
    ok, info = _close32(y, ref)
    assert ok, info


@pytest.mark.parametrize("B,T,p0,tq0,H,hd", [(4, 1, 7, 0, 8, 128), (3, 9, 0, 0, 16, 64), (2, 12, 0, 11, 8, 128),
                                             (5, 1, 30, 0, 16, 64)])
def test_depth_attn_f32(gpu, B, T, p0, tq0, H, hd):
    """Causal SDPA over the frame's positions: cached keys 0..p0-1 from the scratch, this call's T rows from qkv
    (stored to the scratch), queries tq0..T-1."""
    from m3x import ops
    g = _g(B * 11 + T + p0)
    D = H * hd
    np_ = 32
    qkv = torch.randn(B, T, 3 * D, generator=g)
    kd = torch.randn(B, H, np_, hd, generator=g)
    vd = torch.randn(B, H, np_, hd, generator=g)
    kd_g, vd_g = kd.to(gpu), vd.to(gpu)
    out = torch.empty(B * (T - tq0), D, device=gpu)
    ops.depth_attn(qkv.to(gpu).view(B * T, 3 * D), kd_g, vd_g, out, B, T, p0, tq0, H, hd, hd ** -0.5, True)
    q = qkv[:, :, :D].view(B, T, H, hd).transpose(1, 2).double()
    kn = qkv[:, :, D:2 * D].view(B, T, H, hd).transpose(1, 2)
    vn = qkv[:, :, 2 * D:].view(B, T, H, hd).transpose(1, 2)
    K = torch.cat([kd[:, :, :p0], kn], 2).double()
    V = torch.cat([vd[:, :, :p0], vn], 2).double()
    s = (q @ K.transpose(-1, -2)) * hd ** -0.5
    pos_q = torch.arange(p0, p0 + T)[:, None]
    s = s.masked_fill(torch.arange(p0 + T)[None, :] > pos_q, float("-inf"))
    ref = (s.softmax(-1) @ V)[:, :, tq0:].transpose(1, 2).reshape(B * (T - tq0), D)
    ok, info = _close32(out, ref)
    assert ok, info
    assert torch.equal(kd_g[:, :, p0:p0 + T].cpu(), kn)
    assert torch.equal(vd_g[:, :, p0:p0 + T].cpu(), vn)
    assert torch.equal(kd_g[:, :, :p0].cpu(), kd[:, :, :p0])


def test_topk_sample_f32_bitexact(gpu):
    """The sampler on fp32 logits draws exactly the C oracle's code from x = logit * inv_temp, and the embed
    variant writes the drawn code's row and its RMSNorm in fp32."""
    from m3x import ops
    g = _g(71)
    B, V, k, temp = 64, 2048, 50, 0.9
    logits = torch.randn(B, V, generator=g) * 3
    logits[5, 100:110] = logits[5].max() + 1  # ties at the top
    u = torch.rand(B, generator=g)
    out = torch.zeros(B, dtype=torch.int32, device=gpu)
    ops.topk_sample(logits.to(gpu), u.to(gpu), 1.0 / temp, k, False, out)
    xs = logits.numpy() * np.float32(1.0 / temp)
    ref = np.array([C.topk_sample(xs[r], k, float(u[r])) for r in range(B)])
    assert np.array_equal(out.cpu().numpy(), ref)
    table = torch.randn(V, 1024, generator=g)
    w = 1 + 0.1 * torch.randn(1024, generator=g)
    prefix = torch.zeros(B, 2, 1024, device=gpu)
    xo = torch.empty(B, 1024, device=gpu)
    y = torch.empty(B, 1024, device=gpu)
    out2 = torch.zeros(B, dtype=torch.int32, device=gpu)
    ops.topk_sample_embed(logits.to(gpu), u.to(gpu), 1.0 / temp, k, False, out2, table.to(gpu), prefix[:, 1],
                          x_out=xo, y=y, w=w.to(gpu), eps=1e-6, kind=ops.NORM_RMS)
    assert np.array_equal(out2.cpu().numpy(), ref)
    rows = table[torch.from_numpy(ref).long()]
    assert torch.equal(prefix[:, 1].cpu(), rows) and torch.equal(xo.cpu(), rows)
    r64 = rows.double()
    ok, info = _close32(y, r64 * torch.rsqrt(r64.pow(2).mean(-1, keepdim=True) + 1e-6) * w.double())
    assert ok, info


def test_feedback_and_rows_f32(gpu):
    from m3x import ops
    g = _g(81)
    B, nq, nc, n = 6, 32, 2048, 1024
    table = torch.randn(nq * nc, n, generator=g) * 0.02
    codes = torch.randint(0, nc, (B, nq), generator=g, dtype=torch.int32)
    w = 1 + 0.1 * torch.randn(n, generator=g)
    out = torch.empty(B, n, device=gpu)
    eps = float(torch.finfo(torch.float32).eps)
    ops.feedback(table.to(gpu), codes.to(gpu), out, w.to(gpu), eps, nq ** 0.5, nq, nc)
    idx = codes.long() + torch.arange(nq) * nc
    x = table[idx].double().sum(1) / nq ** 0.5
    ok, info = _close32(out, x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w.double())
    assert ok, info
    # bias rows and row copies in fp32
    xr = torch.randn(B, n, generator=g)
    bias = torch.randn(n, generator=g)
    o = torch.empty(B, n, device=gpu)
    ops.add_rows(xr.to(gpu), bias.to(gpu), o)
    assert torch.equal(o.cpu(), xr + bias)
    dst = torch.zeros(4, n, device=gpu)
    ops.copy_rows(table.to(gpu), dst, src_idx=torch.tensor([3, 0, 9, 3], device=gpu))
    assert torch.equal(dst.cpu(), table[[3, 0, 9, 3]])
