"""m3x_decode_attn_noalloc (the allocation-free decode attention) against m3x_decode_attn with a caller workspace,
through the C ABI on the GPU: two calls in a row, the second with a smaller input, each bit-identical to the
workspace entry point on the same inputs; a step with inline prefill rows through the work-item list, likewise;
a size past the scratch limit is refused before anything launches."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _case(gpu, rows, ctx, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    S, KV, H, D, cap = rows + 1, 8, 16, 128, 4096
    kc = torch.randn(S, KV, cap, D, device=gpu, generator=g).to(torch.bfloat16)
    vc = torch.randn(S, KV, cap, D, device=gpu, generator=g).to(torch.bfloat16)
    q = torch.randn(rows, H, D, device=gpu, generator=g).to(torch.bfloat16)
    slots = torch.randperm(S, device=gpu, generator=g)[:rows].long()
    pos = torch.randint(ctx // 2, ctx, (rows,), device=gpu, generator=g).int()
    return kc, vc, q, slots, pos


def _call(L, kc, vc, q, slots, pos, out, ctx, chunk, ws=None, stream=None, items=None):
    common = [_p(q), q.stride(0), q.stride(1), _p(kc), _p(vc), kc.stride(0), kc.stride(1), kc.stride(2),
              kc.shape[2], _p(out), out.stride(0), out.stride(1), _p(slots), _p(pos),
              None if items is None else _p(items),
              ctypes.c_float(128 ** -0.5), q.shape[0], 16, 8, 128, ctx, chunk]
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if ws is None:
        return L.m3x_decode_attn_noalloc(*common, st)
    return L.m3x_decode_attn(*common, _p(ws), ws.numel() * 4, st)


def test_noalloc_decode_attn_matches_workspace_entry(gpu):
    from m3x._lib import lib
    L = lib()
    # first call: 4 rows over 2048 keys in 128-key splits (16 splits, 540 KB of partials); second: 1 row over 512
    for rows, ctx, chunk, seed in ((4, 2048, 128, 1), (1, 512, 128, 2)):
        kc, vc, q, slots, pos = _case(gpu, rows, ctx, seed)
        ref = torch.empty_like(q)
        ws = torch.empty(max(L.m3x_decode_attn_workspace(rows, 8, ctx, chunk), 16) // 4, dtype=torch.float32,
                         device=gpu)
        assert _call(L, kc, vc, q, slots, pos, ref, ctx, chunk, ws=ws) == 0
        got = torch.full_like(q, float("nan"))
        assert _call(L, kc, vc, q, slots, pos, got, ctx, chunk) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (rows, ctx)
    # 64 rows over 4096 keys in 128-key splits need 17 MB of partials: refused before anything reads the caches or
    # launches, so one-slot caches stand in
    kc = torch.zeros(1, 8, 4096, 128, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    q = torch.zeros(64, 16, 128, dtype=torch.bfloat16, device=gpu)
    slots = torch.zeros(64, dtype=torch.long, device=gpu)
    pos = torch.full((64,), 4095, dtype=torch.int32, device=gpu)
    out = torch.zeros_like(q)
    assert _call(L, kc, vc, q, slots, pos, out, 4096, 128) == -3
    torch.cuda.synchronize()
    assert not out.any()


def test_noalloc_decode_attn_items_match_workspace_entry(gpu):
    """A mixed step's work items (two decode rows and a 20-row inline prefill of one slot, 128-key splits) through
    both entry points: the same bits."""
    from m3x import ops
    from m3x._lib import lib
    L = lib()
    g = torch.Generator(device=gpu).manual_seed(4)
    S, KV, H, D, cap, ctx, chunk = 4, 8, 16, 128, 1024, 1024, 128
    kc = torch.randn(S, KV, cap, D, device=gpu, generator=g).to(torch.bfloat16)
    vc = torch.randn(S, KV, cap, D, device=gpu, generator=g).to(torch.bfloat16)
    rows = 22
    q = torch.randn(rows, H, D, device=gpu, generator=g).to(torch.bfloat16)
    slots = torch.tensor([0, 2] + [1] * 20, dtype=torch.long, device=gpu)
    pos = torch.tensor([700, 130] + list(range(300, 320)), dtype=torch.int32, device=gpu)
    bins = ops.attn_item_bins(rows, KV, ctx, chunk)
    items = torch.from_numpy(ops.attn_items([(0, 1, 700), (1, 1, 130), (2, 20, 300)], H, KV, bins, chunk)).to(gpu)
    ref = torch.empty_like(q)
    ws = torch.empty(max(L.m3x_decode_attn_workspace(rows, KV, ctx, chunk), 16) // 4, dtype=torch.float32,
                     device=gpu)
    assert _call(L, kc, vc, q, slots, pos, ref, ctx, chunk, ws=ws, items=items) == 0
    got = torch.full_like(q, float("nan"))
    assert _call(L, kc, vc, q, slots, pos, got, ctx, chunk, items=items) == 0
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
