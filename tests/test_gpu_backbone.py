"""StaticBackbone (drop-in of serve/fast_backbone.py) on the GPU vs the gather-path oracle on the CPU."""
import pytest
import torch

from helpers import close, convert, floor_check, report
from m3x import synth
from oracle import torch_oracle as O

pytestmark = pytest.mark.gpu

LAYERS, S, CAP = 3, 6, 512
PREFIX = [0, 1, 37, 200, 300, 0]


def _setup(gpu, use_graphs=True, affine=synth.AFFINE):
    from m3x.serve.fast_backbone import StaticBackbone
    bb_g = synth.qwen3_backbone(layers=LAYERS, seed=21, device=gpu, affine=affine)
    bb_c = synth.qwen3_backbone(layers=LAYERS, seed=21, device="cpu", affine=affine)
    sb = StaticBackbone(bb_g, S, capacity=CAP, batch_buckets=(1, 2, 4, 8, 64), ctx_buckets=(256, 512),
                        attention="triton", fuse_rope=True, use_graphs=use_graphs)
    g = torch.Generator().manual_seed(22)
    kc = [torch.zeros(S + 1, 8, CAP, 128, dtype=torch.bfloat16) for _ in range(LAYERS)]
    vc = [torch.zeros(S + 1, 8, CAP, 128, dtype=torch.bfloat16) for _ in range(LAYERS)]
    for s, n in enumerate(PREFIX):
        kv = []
        for i in range(LAYERS):
            k = torch.randn(1, 8, n, 128, generator=g).to(torch.bfloat16)
            v = torch.randn(1, 8, n, 128, generator=g).to(torch.bfloat16)
            kc[i][s, :, :n] = k[0]
            vc[i][s, :, :n] = v[0]
            kv.append((k.to(gpu), v.to(gpu)))
        sb.load_prefix(s, kv, n)
    lengths = torch.tensor(PREFIX + [0])
    cos, sin = O.rope_tables(128, 1e6, CAP, torch.bfloat16)
    # fp32 evaluation of the same math on the same (bf16-valued) weights and cache: the truth for the floor
    truth = dict(bb=convert(bb_c, torch.float32), kc=[t.float() for t in kc], vc=[t.float() for t in vc],
                 lengths=lengths.clone(), cos=cos.float(), sin=sin.float())
    return sb, bb_c, kc, vc, lengths, cos, sin, truth


def _truth_step(T, slots, x, offset=None):
    return O.backbone_step(T["bb"], T["kc"], T["vc"], T["lengths"], slots, x.float(), T["cos"], T["sin"],
                           offset=offset)


@pytest.mark.parametrize("affine", [synth.AFFINE, synth.AFFINE_WIDE])
def test_step_matches_oracle(gpu, affine):
    """Three decode steps with non-unit norm weights (1 + N(0, 0.1), and a log-normal spread of about 0.1x to 20x
    that tests the folded input/post-attention norms and the q/k norms on weights like trained ones)."""
    sb, bb_c, kc, vc, lengths, cos, sin, T = _setup(gpu, affine=affine)
    g = torch.Generator().manual_seed(23)
    slots = [0, 2, 3, 4]
    for t in range(3):
        x = torch.randn(len(slots), 1024, generator=g).to(torch.bfloat16)
        out = sb.step(slots, x.to(gpu))
        ref = O.backbone_step(bb_c, kc, vc, lengths, torch.tensor(slots), x, cos, sin)
        truth = _truth_step(T, torch.tensor(slots), x)
        ok, info = floor_check(out, ref, truth)
        report(f"backbone step {t} ({affine})", info)
        assert ok, (t, info)
    assert sb.lengths.cpu().tolist() == lengths.tolist() and sb.lengths_cpu == lengths.tolist()
    assert sb.lengths[S].item() == 0
    for i in range(LAYERS):
        for s in slots:
            n0, n = PREFIX[s], int(lengths[s])
            assert torch.equal(sb.k[i][s, :, :n0].cpu(), kc[i][s, :, :n0])  # the prefix is untouched
            for name, got, ref, tr in (("k", sb.k[i], kc[i], T["kc"][i]), ("v", sb.v[i], vc[i], T["vc"][i])):
                ok, info = floor_check(got[s, :, n0:n], ref[s, :, n0:n], tr[s, :, n0:n])
                assert ok, (name, i, s, info)
        # slots that did not step are untouched
        assert torch.equal(sb.k[i][1].cpu(), kc[i][1]) and torch.equal(sb.k[i][5].cpu(), kc[i][5])


def test_step_mixed_prefill_matches_oracle(gpu):
    sb, bb_c, kc, vc, lengths, cos, sin, T = _setup(gpu)
    g = torch.Generator().manual_seed(24)
    x = torch.randn(2, 1024, generator=g).to(torch.bfloat16)
    p5 = (torch.randn(20, 1024, generator=g) * 0.5).to(torch.bfloat16)
    p1 = (torch.randn(7, 1024, generator=g) * 0.5).to(torch.bfloat16)
    dec, last = sb.step_mixed([0, 3], x.to(gpu), [(5, p5.to(gpu)), (1, p1.to(gpu))])
    slots = torch.tensor([0, 3] + [5] * 20 + [1] * 7)
    offset = torch.tensor([0, 0] + list(range(20)) + list(range(7)))
    ref = O.backbone_step(bb_c, kc, vc, lengths, slots, torch.cat([x, p5, p1]), cos, sin, offset=offset)
    truth = _truth_step(T, slots, torch.cat([x, p5, p1]), offset=offset)
    ok, info = floor_check(torch.cat([dec, torch.stack(last)]), ref[[0, 1, 21, 28]], truth[[0, 1, 21, 28]])
    assert ok, info
    assert sb.lengths_cpu[:S] == [1, 8, 37, 201, 300, 20] == lengths[:S].tolist()
    # every prefill row's attention shows in the next layer's K/V writes at its position
    for i in range(1, LAYERS):
        for s, n0, n in ((5, 0, 20), (1, 1, 8)):
            for name, got, rf, tr in (("k", sb.k[i], kc[i], T["kc"][i]), ("v", sb.v[i], vc[i], T["vc"][i])):
                ok, info = floor_check(got[s, :, n0:n], rf[s, :, n0:n], tr[s, :, n0:n])
                assert ok, (name, i, s, info)
    # the next decode step of the prefilled slot continues from its new length
    y = torch.randn(1, 1024, generator=g).to(torch.bfloat16)
    out = sb.step([5], y.to(gpu))
    ok, info = floor_check(out, O.backbone_step(bb_c, kc, vc, lengths, torch.tensor([5]), y, cos, sin),
                           _truth_step(T, torch.tensor([5]), y))
    assert ok, info


def test_prefill_in_pieces_and_prefix_export(gpu):
    """StaticBackbone.prefill runs a long prompt through the graphed inline-prefill step in pieces of the largest
    row bucket (150 tokens over 64-row pieces here) and matches the oracle's one-shot causal prefill; its KV,
    exported and installed into another slot, is bit-identical there and decodes identically."""
    sb, bb_c, kc, vc, lengths, cos, sin, T = _setup(gpu)
    g = torch.Generator().manual_seed(27)
    x = (torch.randn(150, 1024, generator=g) * 0.5).to(torch.bfloat16)
    last = sb.prefill(5, x.to(gpu))
    slots = torch.tensor([5] * 150)
    offset = torch.arange(150)
    ref = O.backbone_step(bb_c, kc, vc, lengths, slots, x, cos, sin, offset=offset)
    truth = _truth_step(T, slots, x, offset=offset)
    ok, info = floor_check(last[None], ref[-1:], truth[-1:])
    assert ok, info
    assert sb.lengths_cpu[5] == 150 and int(sb.lengths[5]) == 150
    for i in range(LAYERS):
        for name, got, rf, tr in (("k", sb.k[i], kc[i], T["kc"][i]), ("v", sb.v[i], vc[i], T["vc"][i])):
            ok, info = floor_check(got[5, :, :150], rf[5, :, :150], tr[5, :, :150])
            assert ok, (name, i, info)
    kv = sb.export_prefix(5)
    assert len(kv) == LAYERS and tuple(kv[0][0].shape) == (1, 8, 150, 128)
    sb.load_prefix(4, kv, 150)
    for i in range(LAYERS):
        assert torch.equal(sb.k[i][4, :, :150], sb.k[i][5, :, :150])
        assert torch.equal(sb.v[i][4, :, :150], sb.v[i][5, :, :150])
    y = torch.randn(1, 1024, generator=g).to(torch.bfloat16).to(gpu)
    out = sb.step([5, 4], torch.cat([y, y]))
    assert torch.equal(out[0], out[1])
    with pytest.raises(ValueError):
        sb.prefill(5, torch.zeros(CAP, 1024, dtype=torch.bfloat16, device=gpu))
    with pytest.raises(IndexError):
        sb.prefill(S, x.to(gpu))


def test_graph_replay_equals_eager(gpu):
    a = _setup(gpu, use_graphs=True)[0]
    b = _setup(gpu, use_graphs=False)[0]
    g = torch.Generator().manual_seed(25)
    for slots in ([0, 2, 3, 4], [0, 2, 3, 4], [1], [4, 0]):
        x = torch.randn(len(slots), 1024, generator=g).to(torch.bfloat16).to(gpu)
        assert torch.equal(a.step(slots, x), b.step(slots, x))
    for i in range(LAYERS):
        assert torch.equal(a.k[i], b.k[i]) and torch.equal(a.v[i], b.v[i])


def test_spread_decode_step_takes_item_launch(gpu):
    """A decode step of 40 seats whose contexts are spread out (the longest above 1.5x the mean) runs its attention
    as the item launch (splits dealt longest-first over one round of workgroups), its item list kept across steps
    until a row crosses a split boundary. With the per-row launch's split size the outputs and caches equal that
    launch's bit for bit, step after step (across a rebuild); with its own 1024-key splits the
    outputs differ only by the split combine's rounding (the merge order of the fp32 partials). A step with
    near-equal contexts, or of 16 rows, keeps the per-row launch."""
    import m3x.serve.fast_backbone as fb
    from m3x.serve.fast_backbone import StaticBackbone
    bb = synth.qwen3_backbone(layers=2, seed=41, device=gpu, affine=synth.AFFINE)
    B, cap = 40, 1024
    lengths = torch.randint(8, 900, (B,), generator=torch.Generator().manual_seed(42))
    lengths[0] = 950  # longest context: 950 + 1 keys against a mean near 450
    lengths[1] = 510  # crosses a 512-key split boundary on the third step: the cached item list is rebuilt

    def backbone(item_chunk=None):
        saved = fb.item_chunk
        if item_chunk is not None:
            fb.item_chunk = item_chunk
        try:
            sb = StaticBackbone(bb, B, capacity=cap, batch_buckets=(48,), ctx_buckets=(cap,), attention="triton",
                                fuse_rope=True)
            sb.warmup()
        finally:
            fb.item_chunk = saved
        g = torch.Generator(device=gpu).manual_seed(43)
        with torch.inference_mode():  # the caches are inference tensors
            for i in range(2):
                sb.k[i].normal_(generator=g)
                sb.v[i].normal_(generator=g)
            sb.lengths[:B].copy_(lengths)
        sb.lengths_cpu[:B] = lengths.tolist()
        return sb

    per_row_chunk = fb.attn_chunk(48, 8, cap)
    same, own, ref = backbone(lambda rows: per_row_chunk), backbone(), backbone()
    assert any(k[-1] == "items" for k in same.graphs)  # warmup captured both launches of the 48-row bucket
    assert same._graph(48, cap, items=True).bufs.chunk == per_row_chunk and own._graph(48, cap, items=True).bufs.chunk == 1024
    g = torch.Generator().manual_seed(44)
    slots = list(range(B))
    skew = fb.ITEM_SKEW
    for t in range(3):
        x = torch.randn(B, 1024, generator=g).to(torch.bfloat16).to(gpu)
        runs = [(r, 1, same.lengths_cpu[s]) for r, s in enumerate(slots)]
        assert same._spread(48, runs) and own._spread(48, runs)
        y_same, y_own = same.step(slots, x), own.step(slots, x)
        try:
            fb.ITEM_SKEW = float("inf")  # the per-row launch for ref
            assert not ref._spread(48, runs)
            y_ref = ref.step(slots, x)
        finally:
            fb.ITEM_SKEW = skew
        assert torch.equal(y_same, y_ref), t
        # the list is rebuilt only when a row's split count changes (the 512-key lists at step 3)
        assert same._graph(48, cap, items=True).items_key[1][1] == (same.lengths_cpu[1] - 1 + per_row_chunk) // per_row_chunk
        ok, info = close(y_own, y_ref, atol=2e-2)
        assert ok, (t, info)
    for i in range(2):
        assert torch.equal(same.k[i], ref.k[i]) and torch.equal(same.v[i], ref.v[i])
    even = [(r, 1, 500 + r % 7) for r in range(B)]
    assert not same._spread(48, even) and not same._spread(16, runs)


def test_errors_match_reference_conventions(gpu):
    sb = _setup(gpu)[0]
    x = torch.zeros(2, 1024, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        sb.step([1, 1], x)
    with pytest.raises(IndexError):
        sb.step([0, S], x)
    with pytest.raises(ValueError):
        sb.step_mixed([], None, [(1, torch.zeros(CAP, 1024, dtype=torch.bfloat16, device=gpu))])
    with pytest.raises(IndexError):
        sb.load_prefix(S, [], 0)
    with pytest.raises(ValueError):
        type(sb)(synth.qwen3_backbone(layers=1, device=gpu), 2, attention="flash")
