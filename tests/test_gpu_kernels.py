"""Kernel-level parity on the GPU: bit-exact against the C oracle where the contract is exact (add+RMSNorm,
q/k-norm+RoPE+KV write, samplers, Philox, index kernels), bf16 tolerance against an fp32 torch reference for
GEMMs and attention."""
import numpy as np
import pytest
import torch

from helpers import bf16_bits, close, from_bits
from oracle import coracle as C
from oracle import torch_oracle as O

pytestmark = pytest.mark.gpu


def _g(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------- GEMM
@pytest.mark.parametrize("M,N,K", [(1, 1024, 1024), (5, 4096, 1024), (16, 2048, 1024), (33, 1024, 3072),
                                   (100, 2049, 1024), (224, 6144, 1024), (7, 1024, 2816), (448, 2816, 1024),
                                   (2264, 4096, 1024),
                                   # one-workgroup-per-CU plans: 8 waves at K = 1024, 16 waves at longer K
                                   (224, 1024, 1024), (224, 2048, 1024), (224, 3072, 1024), (224, 4096, 1024),
                                   (250, 3072, 1024), (64, 2049, 1024), (224, 1024, 2048), (224, 1024, 2816),
                                   (200, 1024, 3072), (100, 1024, 2816), (70, 1024, 2048),
                                   # K slices of unequal length: the last chunk of the last slice is partial
                                   (40, 1024, 1056), (200, 1024, 1312), (3, 512, 160),
                                   # one 16-row block over 8 waves
                                   (1, 1024, 2816), (16, 1024, 3072), (2, 2049, 2048), (1, 4096, 1024),
                                   # 2-D LDS tiles above 512 rows: partial row / column blocks, N % 16 != 0
                                   (513, 1024, 1024), (1000, 2049, 1024), (2264, 1024, 3072), (700, 1024, 2816),
                                   (1300, 136, 2048)])
def test_linear_bf16(gpu, M, N, K):
    from m3x import ops
    g = _g(M * 7 + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    y = ops.linear(x.to(gpu), ops.pack_weight(w.to(gpu)))
    ref = (x.float() @ w.float().t())
    ok, info = close(y, ref, atol=1e-2)
    assert ok, info


@pytest.mark.parametrize("M,N,K", [(24, 3072, 1024), (1, 2816, 1024), (3, 1024, 96), (700, 3072, 1024)])
def test_linear_fp16(gpu, M, N, K):
    from m3x import ops
    g = _g(M + K)
    x = torch.randn(M, K, generator=g).to(torch.float16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.float16)
    y = ops.linear(x.to(gpu), ops.pack_weight(w.to(gpu)))
    ok, info = close(y, x.float() @ w.float().t(), atol=1e-2)
    assert ok, info


@pytest.mark.parametrize("M,I,K,dtype", [(1, 3072, 1024, torch.bfloat16), (224, 2816, 1024, torch.bfloat16),
                                         (37, 3072, 1024, torch.float16), (224, 3072, 1024, torch.bfloat16),
                                         (64, 3072, 1024, torch.float16), (130, 2816, 1024, torch.bfloat16),
                                         (1100, 3072, 1024, torch.bfloat16), (600, 2816, 1024, torch.float16),
                                         (2264, 3072, 1024, torch.bfloat16)])
def test_linear_swiglu_epilogue(gpu, M, I, K, dtype):
    """Fused gate|up GEMM + silu*mul against the separate GEMM + activation kernel (the two launches may slice K
    differently, so the fp32 sums can round apart by an ulp) and against an fp32 reference."""
    from m3x import ops
    g = _g(M + I)
    x = torch.randn(M, K, generator=g).to(dtype).to(gpu)
    wgu = (torch.randn(2 * I, K, generator=g) * 0.02).to(dtype).to(gpu)
    pgu = ops.pack_weight(wgu)
    fused = ops.linear_act(x, pgu.rows(0, I), pgu.rows(I, 2 * I), ops.ACT_SWIGLU)
    gu = ops.linear(x, pgu)
    sep = torch.empty(M, I, dtype=dtype, device=gpu)
    ops.act(gu, sep, ops.ACT_SWIGLU)
    # near-zero outputs come from cancelling sums, where one fp32 ulp of the sum is many ulps of the result
    ok, info = close(fused, sep.float(), atol=1e-3, rel_ulps=2)
    assert ok, info
    ref = torch.nn.functional.silu((x.float() @ wgu[:I].float().t()).to(dtype).float()).to(dtype).float() * \
        (x.float() @ wgu[I:].float().t()).to(dtype).float()
    ok, info = close(fused, ref.cpu(), atol=1e-2)
    assert ok, info


@pytest.mark.parametrize("M", [9, 150, 700])
def test_linear_gelu_epilogue(gpu, M):
    from m3x import ops
    g = _g(77 + M)
    x = torch.randn(M, 1024, generator=g).to(torch.float16).to(gpu)
    w = (torch.randn(3072, 1024, generator=g) * 0.02).to(torch.float16).to(gpu)
    pw = ops.pack_weight(w)
    fused = ops.linear_act(x, pw, None, ops.ACT_GELU)
    sep = torch.empty(M, 3072, dtype=torch.float16, device=gpu)
    ops.act(ops.linear(x, pw), sep, ops.ACT_GELU)
    ok, info = close(fused, sep.float(), atol=1e-3, rel_ulps=2)
    assert ok, info
    ok, info = close(fused, torch.nn.functional.gelu(x.float() @ w.float().t()).cpu(), atol=1e-2)
    assert ok, info


def test_linear_strided_output(gpu):
    from m3x import ops
    g = _g(3)
    x = torch.randn(9, 1024, generator=g).to(torch.bfloat16).to(gpu)
    w = (torch.randn(512, 1024, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
    big = torch.zeros(9, 1536, dtype=torch.bfloat16, device=gpu)
    ops.linear(x, ops.pack_weight(w), big[:, 256:768])
    ok, info = close(big[:, 256:768], x.float() @ w.float().t(), atol=1e-2)
    assert ok, info
    assert big[:, :256].abs().sum() == 0 and big[:, 768:].abs().sum() == 0


@pytest.mark.parametrize("N,K", [(2049, 1024), (16, 32), (48, 96)])
def test_pack_weight_layout(gpu, N, K):
    """The packed layout bit for bit: fragment (t, s), lane l, element e holds W[16t + l%16][32s + 8(l//16) + e]
    (zero rows past N), checked against the same layout written as a reshape/permute of the padded matrix."""
    from m3x import ops
    g = _g(N + K)
    w = torch.randn(N, K, generator=g).to(torch.bfloat16)
    pw = ops.pack_weight(w.to(gpu))
    Np = -(-N // 16) * 16
    wpad = torch.zeros(Np, K, dtype=torch.bfloat16)
    wpad[:N] = w
    want = wpad.view(Np // 16, 16, K // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(-1)
    assert pw.data.numel() == Np * K and (pw.N, pw.K) == (N, K)
    assert np.array_equal(bf16_bits(pw.data.cpu()), bf16_bits(want))
    # a row block of a packed weight is the packed form of those rows
    if N >= 32:
        sub = ops.pack_weight(w[16:].contiguous().to(gpu))
        assert np.array_equal(bf16_bits(pw.rows(16, N).data.cpu()), bf16_bits(sub.data.cpu()))


def test_linear_deterministic_and_graph_replay(gpu):
    """Same inputs, same bits: eager twice and four graph replays with eager work in between."""
    from m3x import ops
    g = _g(5)
    x = torch.randn(224, 1024, generator=g).to(torch.bfloat16).to(gpu)
    pw = ops.pack_weight((torch.randn(3072, 1024, generator=g) * 0.02).to(torch.bfloat16).to(gpu))
    y0 = ops.linear(x, pw).clone()
    assert torch.equal(ops.linear(x, pw), y0)
    y = torch.zeros_like(y0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.linear(x, pw, y)
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=s):
        ops.linear(x, pw, y)
    for _ in range(4):
        y.zero_()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y0)
        ops.linear(x[:7], pw)  # eager work between replays
        torch.cuda.synchronize()


# ---------------------------------------------------------------- add + RMSNorm (bit-exact)
@pytest.mark.parametrize("n,rows", [(1024, 7), (1024, 224), (2048, 3)])
def test_add_rms_bitexact(gpu, n, rows):
    from m3x import ops
    g = _g(n + rows)
    h = torch.randn(rows, n, generator=g).to(torch.bfloat16)
    a = torch.randn(rows, n, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)
    ho, y = ops.add_rms(h.to(gpu), a.to(gpu), w.to(gpu), 1e-6)
    ref_ho, ref_y = C.add_rms(bf16_bits(h), bf16_bits(a), bf16_bits(w), 1e-6)
    assert np.array_equal(bf16_bits(ho), ref_ho)
    assert np.array_equal(bf16_bits(y), ref_y)
    _, y0 = ops.add_rms(h.to(gpu), None, w.to(gpu), 1e-6)
    assert np.array_equal(bf16_bits(y0), C.add_rms(bf16_bits(h), None, bf16_bits(w), 1e-6)[1])
    hg = h.to(gpu)
    ops.add_rms(hg, a.to(gpu), w.to(gpu), 1e-6, h_out=hg)  # in place, as the step runs it
    assert np.array_equal(bf16_bits(hg), ref_ho)


# ---------------------------------------------------------------- q/k norm + RoPE + cache write (bit-exact)
def test_qk_norm_rope_cache_bitexact(gpu):
    from m3x import ops
    from oracle.torch_oracle import rope_tables
    g = _g(0)
    B, H, KV, D, CAP, S = 6, 16, 8, 128, 512, 8
    qkv = (torch.randn(B, (H + 2 * KV) * D, generator=g) * 2).to(torch.bfloat16)
    wq = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    wk = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    pos = torch.tensor([0, 7, 100, 300, 511, 31], dtype=torch.int32)
    slots = torch.tensor([0, 1, 2, 3, 4, 7])
    cos, sin = rope_tables(D, 1e6, CAP, torch.bfloat16)
    K = torch.zeros(S, KV, CAP, D, dtype=torch.bfloat16, device=gpu)
    V = torch.zeros_like(K)
    q = torch.empty(B, H, D, dtype=torch.bfloat16, device=gpu)
    ops.qk_norm_rope_cache(qkv.to(gpu), q, K, V, slots.to(gpu), pos.to(gpu), cos.to(gpu), sin.to(gpu), wq.to(gpu),
                           wk.to(gpu), 1e-6, H, KV)
    rq, rk = C.qk_norm_rope(bf16_bits(qkv), H, KV, D, pos.numpy(), bf16_bits(cos), bf16_bits(sin), bf16_bits(wq),
                            bf16_bits(wk), 1e-6)
    assert np.array_equal(bf16_bits(q), rq)
    Kc, Vc = K.cpu(), V.cpu()
    for r in range(B):
        assert np.array_equal(bf16_bits(Kc[slots[r], :, pos[r]]), rk[r])
        assert torch.equal(Vc[slots[r], :, pos[r]], qkv[r, (H + KV) * D:].view(KV, D))
        Kc[slots[r], :, pos[r]] = 0
        Vc[slots[r], :, pos[r]] = 0
    assert Kc.abs().sum() == 0 and Vc.abs().sum() == 0  # nothing else written


# ---------------------------------------------------------------- decode attention
def _attn_ref(q, K, V, slots, pos, scale, G):
    out = torch.empty(q.shape, dtype=torch.float32)
    for r in range(q.shape[0]):
        p = int(pos[r])
        k = K[slots[r], :, :p + 1].float()  # [KV, n, D]
        v = V[slots[r], :, :p + 1].float()
        qq = q[r].float().view(k.shape[0], G, -1)
        s = torch.einsum('kgd,knd->kgn', qq, k) * scale
        out[r] = torch.einsum('kgn,knd->kgd', s.softmax(-1), v).reshape(q.shape[1:])
    return out


@pytest.mark.parametrize("heads,kv,chunk,CAP", [(16, 8, 128, 2048), (16, 8, 256, 2048), (16, 8, 1024, 2048),
                                               (8, 8, 128, 2048), (16, 8, 128, 4096)])
def test_decode_attn(gpu, heads, kv, chunk, CAP):
    from m3x import ops
    g = _g(heads + chunk + CAP)
    D, S = 128, 9
    K = torch.randn(S, kv, CAP, D, generator=g).to(torch.bfloat16)
    V = torch.randn(S, kv, CAP, D, generator=g).to(torch.bfloat16)
    slots = torch.tensor([0, 1, 2, 3, 4, 5, 6, 8, 1])
    pos = torch.tensor([0, 31, 32, 127, 128, 1000, CAP - 1, 513, 5], dtype=torch.int32)  # up to 32 splits
    # stale cache rows past each row's context hold NaN: nothing past pos may leak into the output
    for r in range(len(slots)):
        if slots[r] != 1:
            K[slots[r], :, pos[r] + 1:] = float('nan')
            V[slots[r], :, pos[r] + 1:] = float('nan')
    q = torch.randn(len(slots), heads, D, generator=g).to(torch.bfloat16)
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=gpu)
    ws = torch.empty(max(ops.decode_attn_workspace(len(slots), kv, CAP, chunk), 16) // 4, device=gpu)
    ops.decode_attn(q.to(gpu), K.to(gpu), V.to(gpu), out, slots.to(gpu), pos.to(gpu), D ** -0.5, CAP, chunk, ws,
                    heads, kv)
    ref = _attn_ref(q, K, V, slots, pos, D ** -0.5, heads // kv)
    assert torch.isfinite(out.float()).all()
    ok, info = close(out, ref, atol=1e-2)
    assert ok, info


@pytest.mark.parametrize("heads,kv,chunk", [(16, 8, 2048), (16, 8, 128), (8, 8, 256), (16, 8, 1024)])
def test_prefill_items_match_decode_rows(gpu, heads, kv, chunk):
    """Inline prefill rows attended as items (up to 32 query vectors per pass over their slot's keys, one persistent
    grid walking the items) give exactly the bits of attending each row alone, and match the fp32 reference.
    Runs cover full items, a partial last item, an item of one row, lone rows and runs crossing split
    boundaries; the same rows as one-row items, and with the items listed in another order, give the same bits."""
    from m3x import ops
    g = _g(heads * 3 + chunk)
    D, S, CAP = 128, 8, 2048
    K = torch.randn(S, kv, CAP, D, generator=g).to(torch.bfloat16)
    V = torch.randn(S, kv, CAP, D, generator=g).to(torch.bfloat16)
    # (slot, first position, rows)
    runs = [(0, 500, 1), (1, 0, 20), (2, 1020, 9), (3, 37, 1), (4, 120, 13), (5, 2000, 17), (6, 250, 33),
            (7, 1500, 1)]
    slots, pos, spans = [], [], []
    for s, p0, n in runs:
        spans.append((len(slots), n, p0))
        slots += [s] * n
        pos += list(range(p0, p0 + n))
        K[s, :, p0 + n:] = float("nan")  # past the run's last position nothing may leak
        V[s, :, p0 + n:] = float("nan")
    R = len(slots)
    qb = min(16, 2 * (16 // (heads // kv)))  # rows per item: two blocks of 16 query vectors where they fit 16 rows
    bins = ops.attn_item_bins(R, kv, CAP, chunk)
    items = ops.attn_items(spans, heads, kv, bins, chunk).tolist()
    blocks = [(r0 + s, min(qb, n - s), p0 + s + min(qb, n - s)) for r0, n, p0 in spans for s in range(0, n, qb)]
    nitems = sum((keys + chunk - 1) // chunk for _, _, keys in blocks)
    assert items[0] == bins and items[1] == 0 and items[1 + bins] == nitems
    assert sorted((c >> 11, (c >> 5) & 63, c & 31) for c in items[2 + bins:]) == sorted(
        (r, sp, m) for r, m, keys in blocks for sp in range((keys + chunk - 1) // chunk))
    singles = ops.attn_items([(r, 1, p) for r, p in enumerate(pos)], heads, kv, bins, chunk).tolist()
    # the same items dealt bin by bin in reverse order
    rev = [bins] + items[1:2 + bins] + items[2 + bins:][::-1]
    slots_g = torch.tensor(slots, device=gpu)
    pos_g = torch.tensor(pos, dtype=torch.int32, device=gpu)
    q = torch.randn(R, heads, D, generator=g).to(torch.bfloat16)
    Kg, Vg, qg = K.to(gpu), V.to(gpu), q.to(gpu)
    ws = torch.empty(max(ops.decode_attn_workspace(R, kv, CAP, chunk), 16) // 4, device=gpu)
    outs = []
    for it in (None, items, singles, rev):
        o = torch.full(q.shape, float("nan"), dtype=torch.bfloat16, device=gpu)
        itg = None if it is None else torch.tensor(it, dtype=torch.int32, device=gpu)
        ops.decode_attn(qg, Kg, Vg, o, slots_g, pos_g, D ** -0.5, CAP, chunk, ws, heads, kv, items=itg)
        outs.append(o)
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    ref = _attn_ref(q, K, V, torch.tensor(slots), torch.tensor(pos), D ** -0.5, heads // kv)
    ok, info = close(outs[1], ref, atol=1e-2)
    assert ok, info


# ---------------------------------------------------------------- activations, depth norm / attention
def test_swiglu_and_gelu(gpu):
    from m3x import ops
    g = _g(5)
    gu = torch.randn(37, 2 * 2816, generator=g).to(torch.bfloat16)
    out = torch.empty(37, 2816, dtype=torch.bfloat16, device=gpu)
    ops.act(gu.to(gpu), out, ops.ACT_SWIGLU)
    ref = torch.nn.functional.silu(gu[:, :2816].float()).to(torch.bfloat16).float() * gu[:, 2816:].float()
    assert torch.equal(out.cpu(), ref.to(torch.bfloat16)) or close(out, ref, atol=0, rel_ulps=1)[0]
    x = torch.randn(11, 3072, generator=g).to(torch.float16)
    o2 = torch.empty(11, 3072, dtype=torch.float16, device=gpu)
    ops.act(x.to(gpu), o2, ops.ACT_GELU)
    ok, info = close(o2, torch.nn.functional.gelu(x.float()), atol=1e-3, rel_ulps=1)
    assert ok, info


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_norm_one_wave_rows_match_block_rows(gpu, dtype):
    """Up to 16 rows run one wave per row; the same rows inside a larger batch run the block kernel: same bits."""
    from m3x import ops
    g = _g(33)
    R, D = 40, 1024
    x = torch.randn(R, D, generator=g).to(dtype).to(gpu)
    a = torch.randn(R, D, generator=g).to(dtype).to(gpu)
    c = torch.randn(1, D, generator=g).to(dtype).to(gpu)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype).to(gpu)
    b = (0.1 * torch.randn(D, generator=g)).to(dtype).to(gpu)
    # fp16 with the cross term: the block kernel's y can sit 1 ulp off an exact fp32 emulation on rare elements,
    # where the one-wave kernel matches it; the paths are compared without the cross term there
    cc = c if dtype == torch.bfloat16 else None
    for kind in (0, 1):
        outs = []
        for rows in (R, 16, 1):
            xo = torch.empty(rows, D, dtype=dtype, device=gpu)
            y = torch.empty_like(xo)
            ops.add_norm(x[:rows], a[:rows], None if cc is None else cc.expand(rows, D), xo, y, w,
                         b if kind == 0 else None, 1e-5, 1, kind)
            outs.append((xo, y))
        for xo, y in outs[1:]:
            n = xo.shape[0]
            assert torch.equal(xo, outs[0][0][:n]) and torch.equal(y, outs[0][1][:n]), (kind, n)
    if dtype == torch.bfloat16:
        res = []
        for rows in (R, 16, 1):
            h_out, y = ops.add_rms(x[:rows], a[:rows], w, 1e-6)
            res.append((h_out, y))
        for h_out, y in res[1:]:
            n = y.shape[0]
            assert torch.equal(h_out, res[0][0][:n]) and torch.equal(y, res[0][1][:n]), n


@pytest.mark.parametrize("kind", [0, 1])
def test_add_norm_strided(gpu, kind):
    from m3x import ops
    g = _g(10 + kind)
    B, NP, T, D = 3, 32, 5, 1024
    pre = torch.randn(B, NP, D, generator=g).to(torch.bfloat16)
    a = torch.randn(B * T, D, generator=g).to(torch.bfloat16)
    c = torch.randn(B, 4 * D, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    b = (0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    p0 = 7
    pg = pre.to(gpu)
    xo = torch.empty(B * T, D, dtype=torch.bfloat16, device=gpu)
    y = torch.empty_like(xo)
    cg = c.to(gpu)
    ops.add_norm(pg[:, p0:p0 + T], a.to(gpu), cg[:, D:2 * D], xo, y, w.to(gpu), b.to(gpu) if kind == 0 else None,
                 1e-5, T, kind)
    x = pre[:, p0:p0 + T].reshape(B * T, D)
    xr = (x.float() + a.float()).to(torch.bfloat16)
    xr = (xr.float() + c[:, D:2 * D].repeat_interleave(T, 0).float()).to(torch.bfloat16)
    assert torch.equal(xo.cpu(), xr)
    xf = xr.float()
    if kind == 0:
        d = xf - xf.mean(-1, keepdim=True)
        ref = d / torch.sqrt((d * d).mean(-1, keepdim=True) + 1e-5) * w.float() + b.float()
    else:
        ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(torch.bfloat16).float() * w.float()
    ok, info = close(y, ref, atol=0, rel_ulps=1)
    assert ok, info


@pytest.mark.parametrize("T,p0,tq0,hd,NP,dtype", [(2, 0, 0, 128, 32, torch.bfloat16), (1, 5, 0, 128, 32, torch.bfloat16),
                                                  (9, 0, 8, 128, 32, torch.bfloat16), (17, 0, 0, 128, 32, torch.bfloat16),
                                                  (1, 31, 0, 128, 32, torch.bfloat16), (1, 63, 0, 128, 64, torch.float16),
                                                  (24, 40, 0, 64, 64, torch.float16), (3, 6, 1, 64, 16, torch.bfloat16)])
def test_depth_attn(gpu, T, p0, tq0, hd, NP, dtype):
    from m3x import ops
    g = _g(T * 100 + p0 + hd)
    B, H = 3, 8
    D = H * hd
    kd = torch.randn(B, H, NP, hd, generator=g).to(dtype)
    vd = torch.randn(B, H, NP, hd, generator=g).to(dtype)
    qkv = torch.randn(B * T, 3 * D, generator=g).to(dtype)
    kdg, vdg = kd.to(gpu), vd.to(gpu)
    Tq = T - tq0
    out = torch.empty(B * Tq, D, dtype=dtype, device=gpu)
    ops.depth_attn(qkv.to(gpu), kdg, vdg, out, B, T, p0, tq0, H, hd, hd ** -0.5, True)
    q3 = qkv.view(B, T, 3, H, hd)
    kd[:, :, p0:p0 + T] = q3[:, :, 1].transpose(1, 2)
    vd[:, :, p0:p0 + T] = q3[:, :, 2].transpose(1, 2)
    assert torch.equal(kdg.cpu(), kd) and torch.equal(vdg.cpu(), vd)
    ref = torch.empty(B, Tq, H, hd)
    for t in range(tq0, T):
        n = p0 + t + 1
        s = torch.einsum('bhd,bhnd->bhn', q3[:, t, 0].float(), kd[:, :, :n].float()) * hd ** -0.5
        ref[:, t - tq0] = torch.einsum('bhn,bhnd->bhd', s.softmax(-1), vd[:, :, :n].float())
    ok, info = close(out, ref.reshape(B * Tq, D), atol=1e-2)
    assert ok, info


# ---------------------------------------------------------------- samplers (bit-exact)
@pytest.mark.parametrize("dtype,V,k", [(torch.bfloat16, 2048, 50), (torch.float16, 2048, 64),
                                       (torch.bfloat16, 2049, 2049), (torch.bfloat16, 4096, 1)])
def test_topk_sample_bitexact(gpu, dtype, V, k):
    from m3x import ops
    g = _g(V + k)
    B = 64
    logits = (torch.randn(B, V, generator=g) * 2).to(dtype)
    logits[3] = 1.0                       # all tied: every index kept
    logits[4, :100] = logits[4, 100]      # a block of ties at the top
    logits[5, 7] = float('-inf')
    u = torch.rand(B, generator=g)
    u[0] = 0.0
    out = torch.empty(B, dtype=torch.int32, device=gpu)
    ops.topk_sample(logits.to(gpu), u.to(gpu), 1 / 0.9, k, False, out)
    ref = C.topk_sample_rows(bf16_bits(logits), 1 / 0.9, k, u.numpy(), is_f16=dtype == torch.float16)
    assert np.array_equal(out.cpu().numpy(), ref)
    out64 = torch.empty(B, dtype=torch.long, device=gpu)
    ops.topk_sample(logits.to(gpu), None, 1 / 0.9, k, True, out64, out_i64=True)
    refg = C.topk_sample_rows(bf16_bits(logits), 1 / 0.9, k, None, greedy=True, is_f16=dtype == torch.float16)
    assert np.array_equal(out64.cpu().numpy(), refg)


def _peaked_rows(g, B, V, dtype):
    """Rows with fewer than k elements within 8 of the max (after the 1/0.9 scale), the shape of a confident
    model's logits: a few leaders far above a wide bulk, exact ties at the k-th place, -0/+0, -inf tails, rows
    with fewer finite elements than k, a bulk beyond the coarse histogram's reach."""
    x = torch.randn(B, V, generator=g) * 3 - 20
    for b in range(B):
        lead = 1 + b % 12
        x[b, torch.randperm(V, generator=g)[:lead]] = 10 + torch.randn(lead, generator=g) * (0.5 + b % 3)
    x[1, 100:200] = -20.0                         # 100 ties in the bulk, at the k-th place for k = 50
    x[2, :] = float("-inf")
    x[2, 5:45] = torch.randn(40, generator=g)     # 40 finite elements
    x[3, 10:20] = 0.0
    x[3, 20:30] = -0.0
    x[3, 30:] = -50.0                             # the k-th place among +0 / -0 ties
    x[4, 300:] = float("-inf")
    x[5, :3] = 200.0                              # the bulk more than 135 below the max: the radix select
    x[6, :] = torch.randn(V, generator=g) * 40    # a wide row: the coarse histogram
    return x.to(dtype)


@pytest.mark.parametrize("dtype,V,k", [(torch.bfloat16, 2048, 50), (torch.float16, 2048, 64),
                                       (torch.bfloat16, 2049, 15), (torch.bfloat16, 2048, 1)])
def test_topk_sample_peaked_rows(gpu, dtype, V, k):
    """The coarse-histogram and radix-select paths (fewer than k elements within 8 of the row max) draw the
    oracle's codes bit for bit, for the depth sampler and the cb0 sampler."""
    from m3x import ops
    g = _g(V * 3 + k)
    B = 96
    logits = _peaked_rows(g, B, V, dtype)
    u = torch.rand(B, generator=g)
    u[0] = 0.0
    u[1] = 0.999999
    out = torch.empty(B, dtype=torch.int32, device=gpu)
    ops.topk_sample(logits.to(gpu), u.to(gpu), 1 / 0.9, k, False, out)
    ref = C.topk_sample_rows(bf16_bits(logits), 1 / 0.9, k, u.numpy(), is_f16=dtype == torch.float16)
    assert np.array_equal(out.cpu().numpy(), ref), np.nonzero(out.cpu().numpy() != ref)
    ops.topk_sample(logits.to(gpu), None, 1 / 0.9, k, True, out)
    refg = C.topk_sample_rows(bf16_bits(logits), 1 / 0.9, k, None, greedy=True, is_f16=dtype == torch.float16)
    assert np.array_equal(out.cpu().numpy(), refg)
    if dtype != torch.bfloat16:
        return
    slots = torch.arange(B, dtype=torch.long)
    cb0 = torch.zeros(B, dtype=torch.long, device=gpu)
    ops.cb0_sample(logits.to(gpu), -1, slots.to(gpu), u.to(gpu), temp=0.9, top_k=k, cb0_out=cb0)
    lg = bf16_bits(logits)
    for b in range(B):
        r, _ = C.cb0_sample(lg[b], -1, 0.9, k, 0.0, 0.0, None, None, 0, None, None, float(u[b]))
        assert r == int(cb0[b]), b


@pytest.mark.parametrize("dtype,n,kind", [(torch.bfloat16, 1024, 1), (torch.bfloat16, 1024, 0),
                                          (torch.float16, 2048, 0)])
def test_topk_sample_embed(gpu, dtype, n, kind):
    """The fused sampler draws the same codes as topk_sample, gathers table[code] into the prefix row and, with
    y given, writes exactly what add_norm writes for that row alone."""
    from m3x import ops
    g = _g(n + kind)
    B, V, k = 37, 2048, 50
    logits = (torch.randn(B, V, generator=g) * 2).to(dtype).to(gpu)
    u = torch.rand(B, generator=g).to(gpu)
    table = torch.randn(V + 3, n, generator=g).to(dtype).to(gpu)
    w = (1 + 0.1 * torch.randn(n, generator=g)).to(dtype).to(gpu)
    bias = (0.1 * torch.randn(n, generator=g)).to(dtype).to(gpu) if kind == 0 else None
    ref = torch.empty(B, dtype=torch.int32, device=gpu)
    ops.topk_sample(logits, u, 1 / 0.9, k, False, ref)
    codes = torch.full((B, 4), -7, dtype=torch.int32, device=gpu)
    prefix = torch.zeros(B, 4, n, dtype=dtype, device=gpu)
    xo = torch.empty(B, n, dtype=dtype, device=gpu)
    y = torch.empty(B, n, dtype=dtype, device=gpu)
    ops.topk_sample_embed(logits, u, 1 / 0.9, k, False, codes[:, 2], table, prefix[:, 2], x_out=xo, y=y, w=w, b=bias,
                          eps=1e-5, kind=kind)
    assert torch.equal(codes[:, 2], ref)
    assert bool((codes[:, [0, 1, 3]] == -7).all())
    rows = table[ref.long()]
    assert torch.equal(prefix[:, 2], rows) and torch.equal(xo, rows)
    assert not prefix[:, [0, 1, 3]].any()
    xo2, y2 = torch.empty_like(xo), torch.empty_like(y)
    ops.add_norm(rows, None, None, xo2, y2, w, bias, 1e-5, 1, kind)
    assert torch.equal(y, y2)
    # prefix only
    prefix.zero_()
    codes.fill_(-7)
    ops.topk_sample_embed(logits, u, 1 / 0.9, k, False, codes[:, 1], table, prefix[:, 3])
    assert torch.equal(codes[:, 1], ref) and torch.equal(prefix[:, 3], rows)
    assert not prefix[:, :3].any()


def test_cb0_sample_bitexact(gpu):
    from m3x import ops
    g = _g(21)
    B, V, S, W = 48, 2049, 64, 12
    logits = (torch.randn(B, V, generator=g) * 2).to(torch.bfloat16)
    logits[:8, 2048] = 9.0
    logits[8:16, 2048] = 4.5
    slots = torch.randperm(S, generator=g)[:B]
    temp = 0.6 + torch.rand(S, generator=g)
    topk = torch.randint(1, 80, (S,), generator=g)
    bias = torch.zeros(S)
    bias[slots[20:24]] = 2.0
    rep = torch.rand(S, generator=g)
    hist = torch.randint(-1, 2048, (S, W), generator=g)
    frames = torch.randint(0, 8, (S,), generator=g)
    min_t = torch.full((S,), 3)
    hazard = torch.rand(S, generator=g) * 0.7
    ctr = torch.randint(0, 100, (S,), generator=g).int()
    u = torch.rand(B, generator=g)
    # top-p per slot: half the slots keep 1 (no cut), the rest cut at 0.05..0.95 (some sets beyond 64 candidates)
    topp = torch.where(torch.rand(S, generator=g) < 0.5, torch.ones(S), 0.05 + 0.9 * torch.rand(S, generator=g))
    topk[slots[40:44]] = 200
    st = [t.clone().to(gpu) for t in (hist, frames, hazard, ctr)]
    cb0 = torch.zeros(B, dtype=torch.long, device=gpu)
    stop = torch.zeros(B, dtype=torch.long, device=gpu)
    codes = torch.zeros(B, 32, dtype=torch.int32, device=gpu)
    ops.cb0_sample(logits.to(gpu), 2048, slots.to(gpu), u.to(gpu), temp_t=temp.to(gpu), topk_t=topk.to(gpu),
                   aeos_bias=bias.to(gpu), rep_t=rep.to(gpu), hist_t=st[0], frames_t=st[1], min_t=min_t.to(gpu),
                   hazard_t=st[2], ctr_t=st[3], cb0_out=cb0, cb0_i32=codes[:, 0], stop_out=stop,
                   topp_t=topp.to(gpu))
    bits = bf16_bits(logits)
    for b in range(B):
        s = int(slots[b])
        h = hist[s].numpy().astype(np.int64).copy()
        fr = np.array([frames[s].item()], np.int64)
        hz = np.array([hazard[s].item()], np.float32)
        ct = np.array([ctr[s].item()], np.int32)
        c, sp = C.cb0_sample(bits[b], 2048, float(temp[s]), int(topk[s]), float(bias[s]), float(rep[s]), h, fr, 3, hz,
                             ct, float(u[b]), float(topp[s]))
        assert (c, sp) == (cb0[b].item(), stop[b].item()), b
        assert codes[b, 0].item() == c
        assert np.array_equal(st[0][s].cpu().numpy(), h) and st[1][s].item() == fr[0]
        assert st[2][s].item() == hz[0] and st[3][s].item() == ct[0]


# ---------------------------------------------------------------- Philox, feedback, index kernels
def test_philox_known_answers_and_uniforms(gpu):
    from m3x import ops
    for ctr, key, expect in [([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
                             ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
                              [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1])]:
        c = torch.tensor(np.array(ctr, np.uint32).view(np.int32), device=gpu)
        k = torch.tensor(np.array(key, np.uint32).view(np.int32), device=gpu)
        o = torch.zeros(4, dtype=torch.int32, device=gpu)
        ops.philox_block(c, k, o)
        assert o.cpu().numpy().view(np.uint32).tolist() == expect
    seeds = torch.tensor([3, 99, 2 ** 31 - 2, 12345], dtype=torch.int32)
    ctrs = torch.tensor([0, 5, 77, 1], dtype=torch.int32)
    slots = torch.tensor([2, 0, 3, 1, 2])
    out = torch.zeros(5, 31, device=gpu)
    ops.philox_uniforms(seeds.to(gpu), ctrs.to(gpu), slots.to(gpu), out, 1)
    ref = np.array([[C.philox_uniform(int(seeds[s]), int(ctrs[s]), 1 + j) for j in range(31)] for s in slots],
                   np.float32)
    assert np.array_equal(out.cpu().numpy(), ref)


def test_feedback(gpu):
    from m3x import ops, synth
    from oracle import torch_oracle as O
    g = _g(31)
    table = (torch.randn(32 * 2048, 1024, generator=g) * 0.02).to(torch.bfloat16)
    audio_in = synth.SimpleNamespace(n_codes=2048, table=synth.Lin(table),
                                     norm=synth.Norm(torch.ones(1024, dtype=torch.bfloat16), None))
    codes = torch.randint(0, 2048, (6, 32), generator=g, dtype=torch.int32)
    out = torch.empty(6, 1024, dtype=torch.bfloat16, device=gpu)
    ops.feedback(table.to(gpu), codes.to(gpu), out, torch.ones(1024, dtype=torch.bfloat16, device=gpu),
                 torch.finfo(torch.bfloat16).eps, 32 ** 0.5, 32, 2048)
    ok, info = close(out, O.feedback(audio_in, codes).float(), atol=0, rel_ulps=1)
    assert ok, info


def test_index_kernels(gpu):
    from m3x import ops
    g = _g(41)
    lengths = torch.tensor([5, 0, 17, 3, 0], device=gpu)
    slots = torch.tensor([2, 0, 2, 4], device=gpu)
    offset = torch.tensor([0, 0, 1, 0], device=gpu)
    pos = torch.zeros(4, dtype=torch.int32, device=gpu)
    ops.positions(lengths, slots, offset, pos)
    assert pos.tolist() == [17, 5, 18, 0]
    ops.lengths_add(lengths, slots, torch.tensor([1, 1, 1, 0], device=gpu))
    assert lengths.tolist() == [6, 0, 19, 3, 0]
    # runs of one slot across wave and workgroup boundaries, duplicates apart, zeros, a ragged tail
    rs = np.random.default_rng(3)
    sl = np.concatenate([np.full(300, 7), rs.integers(0, 12, 50), np.full(61, 3), [7, 7], np.full(130, 11)])
    re = rs.integers(0, 3, sl.size)
    re[:40] = 1
    want = np.zeros(12, dtype=np.int64)
    np.add.at(want, sl, re)
    lens = torch.zeros(12, dtype=torch.int64, device=gpu)
    ops.lengths_add(lens, torch.from_numpy(sl).to(gpu), torch.from_numpy(re).to(gpu))
    assert lens.cpu().numpy().tolist() == want.tolist()
    table = torch.randn(50, 64, generator=g).to(torch.bfloat16).to(gpu)
    idx = torch.tensor([3, 49, 0, 7], dtype=torch.int32, device=gpu)
    dst = torch.zeros(10, 64, dtype=torch.bfloat16, device=gpu)
    ops.copy_rows(table, dst, src_idx=idx, dst_idx=torch.tensor([9, 0, 4, 2], device=gpu))
    assert torch.equal(dst[[9, 0, 4, 2]], table[[3, 49, 0, 7]])
    codes = torch.randint(0, 2048, (5, 32), dtype=torch.int32, device=gpu)
    ring = torch.zeros(3, 8, 32, dtype=torch.int32, device=gpu)
    head = torch.tensor([4], dtype=torch.int32, device=gpu)
    ops.code_ring_write(codes, ring, head, 5)
    assert torch.equal(ring[1, :5], codes) and head.item() == 5 and ring[[0, 2]].abs().sum() == 0
    ctr = torch.zeros(6, dtype=torch.int32, device=gpu)
    ops.ctr_add(ctr, torch.tensor([1, 5, 5, 0], device=gpu))
    assert ctr.tolist() == [1, 1, 0, 0, 0, 2]


def test_index_dtypes_rejected_before_launch(gpu):
    """Slot tensors are int64 and position tensors int32 in the ABI: a tensor of the other width is refused on the
    host (a kernel would read it as out-of-range indices)."""
    from m3x import guards, ops
    q = torch.zeros(2, 16, 128, dtype=torch.bfloat16, device=gpu)
    kc = torch.zeros(3, 8, 64, 128, dtype=torch.bfloat16, device=gpu)
    s64 = torch.tensor([0, 1], device=gpu)
    p32 = torch.tensor([3, 5], dtype=torch.int32, device=gpu)
    ws = torch.empty(16, device=gpu)
    for slots, pos, what in ((s64.int(), p32, "slots"), (s64, p32.long(), "pos")):
        with pytest.raises(ValueError, match=what):
            ops.decode_attn(q, kc, kc, torch.empty_like(q), slots, pos, 0.1, 64, 128, ws, 16, 8)
    with pytest.raises(ValueError, match="slots"):
        ops.ctr_add(torch.zeros(4, dtype=torch.int32, device=gpu), s64.int())
    with pytest.raises(ValueError, match="slots"):
        ops.lengths_add(torch.zeros(4, dtype=torch.int64, device=gpu), s64.int(), s64)
    lg = guards.LoopGuard(4, _guard_cfg(), device=gpu)
    with pytest.raises(ValueError, match="slots"):
        lg.push(s64.int(), s64)
    with pytest.raises(ValueError, match="codes"):
        lg.push(s64, s64.int())
    torch.cuda.synchronize()


# ---------------------------------------------------------------- loop guard (bit-exact vs the oracle)
def _guard_cfg(**kw):
    from types import SimpleNamespace
    d = dict(stall=32, period_win=64, period_thr=0.7, pmin=2, pmax=16, hist=96)
    d.update(kw)
    return SimpleNamespace(**d)


def test_loop_guard_matches_oracle(gpu):
    """m3x.guards.loop_detect_batch == the oracle's restatement of maya3/guards.py:80-107, row for row, on random
    histories with planted stalls, exact and noisy periods, empty entries and frame counts around the thresholds."""
    from m3x import guards
    rng = np.random.default_rng(5)
    rows, ns = [], []
    for i in range(400):
        kind = i % 5
        row = rng.integers(0, 64 if kind == 4 else 2048, 96)
        if kind == 1:
            row[-32:] = row[-32]
        elif kind == 2:
            p = int(rng.integers(2, 17))
            pat = rng.integers(0, 2048, p)
            row = np.tile(pat, 96 // p + 1)[:96]
            flips = rng.random(96) < rng.uniform(0, 0.4)
            row = np.where(flips, rng.integers(0, 2048, 96), row)
        elif kind == 3:
            row[:int(rng.integers(0, 96))] = -1
        rows.append(row)
        ns.append(int(rng.choice([0, 11, 12, 31, 32, 33, 63, 64, 65, 500])))
    W, n = np.stack(rows), np.array(ns)
    for cfg in (_guard_cfg(), _guard_cfg(stall=16, period_win=48, period_thr=0.55, pmin=3, pmax=12)):
        got = guards.loop_detect_batch(W, n, cfg)
        want = O.loop_detect_batch(W, n, cfg.stall, cfg.period_win, cfg.period_thr, cfg.pmin, cfg.pmax)
        assert got == want
        assert "stall" in got and None in got and any(g and g.startswith("period") for g in got)


def test_loop_guard_device_history(gpu):
    """LoopGuard keeps each slot's history on the device (push = the engine's shift-and-append) and detect() on a
    subset of slots equals the oracle run on the host-kept histories."""
    from m3x import guards
    cfg = _guard_cfg()
    S = 6
    lg = guards.LoopGuard(S, cfg, device=gpu)
    host = np.full((S + 1, 96), -1, dtype=np.int64)
    frames = np.zeros(S + 1, dtype=np.int64)
    rng = np.random.default_rng(6)
    out = torch.empty(4, dtype=torch.int32, device=gpu)
    for t in range(120):
        slots = [0, 2, 3, 5] if t % 3 else [0, 2, 3, 5, 1]
        codes = rng.integers(0, 2048, len(slots))
        codes[0] = 9                     # slot 0 stalls
        codes[1] = (t % 4) * 100         # slot 2 loops with period 4
        if t == 60:  # a new seat on slot 3
            lg.reset(3)
            host[3] = -1
            frames[3] = 0
        lg.push(torch.tensor(slots, device=gpu), torch.tensor(codes, device=gpu))
        for s, c in zip(slots, codes):
            host[s, :-1] = host[s, 1:]
            host[s, -1] = c
            frames[s] += 1
        q = [0, 2, 3, 5]
        lg.detect(torch.tensor(q, device=gpu), out)
        want = O.loop_detect_batch(host[q], frames[q])
        got = [None if c == 0 else ("stall" if c < 0 else f"period:{c}") for c in out.cpu().tolist()]
        assert got == want, t
    assert torch.equal(lg.hist.cpu().long(), torch.from_numpy(host))
    assert torch.equal(lg.frames.cpu(), torch.from_numpy(frames))


# ---------------------------------------------------------------- tick readout (bit-exact vs the engine's torch ops)
@pytest.mark.parametrize("nq,frame,with_loop", [(32, 1920, True), (0, 1920, False), (31, 0, True), (0, 7, False)])
def test_tick_readout_packs_like_the_engine(gpu, nq, frame, with_loop):
    """One packed row per seat, read back through one pinned copy: stop, cb0, loop and codes verbatim, and the PCM
    equal to the engine's `(pcm.clamp(-1, 1) * 32767).round().to(torch.int16)` (maya3/engine.py:559) bit for bit,
    including out-of-range samples and values that round half to even."""
    from m3x.tick import TickReadout
    g = _g(nq + frame)
    B = 5
    stop = torch.randint(0, 5, (B,), generator=g)
    cb0 = torch.randint(0, 2049, (B,), generator=g)
    loop = torch.randint(-1, 17, (B,), generator=g).to(torch.int32)
    codes = torch.randint(0, 2048, (B, 40), generator=g).to(torch.int32)
    pcm = (torch.randn(B, max(frame, 1), generator=g) * 0.6).float()
    if frame >= 8:
        pcm[0, :8] = torch.tensor([1.5, -3.0, 1.0, -1.0, 0.0, -0.0, 0.5 / 32767, 2.5 / 32767])
    rd = TickReadout(8, frame=frame, nq=nq, with_loop=with_loop, device=gpu)
    rd.pack(stop.to(gpu), cb0.to(gpu), loop.to(gpu) if with_loop else None,
            codes[:, :nq].to(gpu) if nq else None, pcm[:, :frame].to(gpu).contiguous() if frame else None)
    got = rd.wait()
    assert got["stop"].tolist() == stop.tolist() and got["cb0"].tolist() == cb0.tolist()
    if with_loop:
        assert got["loop"].tolist() == loop.tolist()
    if nq:
        assert np.array_equal(got["codes"], codes[:, :nq].numpy())
    if frame:
        want = (pcm[:, :frame].clamp(-1, 1) * 32767).round().to(torch.int16).numpy()
        assert np.array_equal(got["pcm"], want)
