"""Host-side logic that needs no GPU: launch planning, workload formulas, cache interop, surface errors."""
import os
import subprocess
import sys

import pytest
import torch

from m3x import roofline, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_attn_chunk_plan():
    from m3x.serve.fast_backbone import attn_chunk
    assert attn_chunk(1, 8, 4096) == 128          # one row: 128-key splits spread over the chip
    assert attn_chunk(16, 8, 4096) == 512
    assert attn_chunk(224, 8, 2048) == 4096       # 224 rows: 1792 workgroups unsplit, no combine launch
    for rows, ctx in [(1, 512), (64, 2048), (2264, 4096)]:
        c = attn_chunk(rows, 8, ctx)
        assert c % 128 == 0 and 128 <= c <= 4096


def test_attn_items_cover_every_row_once():
    """The work list of a mixed step: every split of every row in exactly one item of one slot's run, items of at
    most min(16, 2 (16 / G)) rows that start at a run's start or a multiple of that into it and cover one chunk of the block's
    keys, bins listed back to back, and the longest processing time deal (no bin exceeds the lightest by more than
    its largest item)."""
    from m3x import ops
    runs = [(0, 1, 3000), (1, 1, 10), (2, 20, 0), (22, 9, 700), (31, 1, 4000), (32, 256, 100)]
    rows = 288
    for heads, kv, bins, chunk in [(16, 8, 96, 4096), (8, 8, 7, 1024), (16, 8, 1, 512), (16, 8, 40, 128)]:
        qb = min(16, 2 * (16 // (heads // kv)))
        it = ops.attn_items(runs, heads, kv, bins, chunk).tolist()
        assert it[0] == bins and it[1] == 0
        start = it[1:2 + bins]
        codes = it[2 + bins:]
        assert start == sorted(start) and start[-1] == len(codes)
        covered = []
        cost = {}
        for c in codes:
            r0, sp, m = c >> 11, (c >> 5) & 63, c & 31
            assert 1 <= m <= qb
            run = [r for r in runs if r[0] <= r0 < r[0] + r[1]][0]
            assert r0 + m <= run[0] + run[1] and (r0 - run[0]) % qb == 0
            keys = run[2] + (r0 - run[0]) + m  # keys of the block's last row
            assert sp * chunk < keys
            cost[c] = min(chunk, keys - sp * chunk) + 64
            covered += [(r, sp) for r in range(r0, r0 + m)]
        want = []
        for r0, n, p0 in runs:
            for s0 in range(0, n, qb):
                m = min(qb, n - s0)
                want += [(r, sp) for r in range(r0 + s0, r0 + s0 + m) for sp in range((p0 + s0 + m + chunk - 1) // chunk)]
        assert sorted(covered) == sorted(want) and len({r for r, _ in covered}) == rows
        loads = [sum(cost[c] for c in codes[start[b]:start[b + 1]]) for b in range(bins)]
        assert max(loads) - min(loads) <= max(cost.values())


def _items_restated(runs, heads, kv_heads, bins, chunk):
    """The item list restated: blocks of min(16, 2 (16 // G)) rows, splits of `chunk` keys, cost keys + 64, a stable
    longest-first order and each item to the least loaded bin (lowest index on ties)."""
    import heapq
    qb = min(16, 2 * (16 // (heads // kv_heads)))
    costs, codes = [], []
    for r0, n, p0 in runs:
        for s in range(0, n, qb):
            m = min(qb, n - s)
            keys = p0 + s + m
            for sp in range((keys + chunk - 1) // chunk):
                costs.append(min(chunk, keys - sp * chunk) + 64)
                codes.append(2048 * (r0 + s) + 32 * sp + m)
    order = sorted(range(len(costs)), key=lambda i: -costs[i])
    per = [[] for _ in range(bins)]
    heap = [(0, b) for b in range(bins)]
    for i in order:
        load, b = heapq.heappop(heap)
        per[b].append(codes[i])
        heapq.heappush(heap, (load + costs[i], b))
    start = [0]
    for p in per:
        start.append(start[-1] + len(p))
    return [bins] + start + [c for p in per for c in p]


def test_attn_items_deal_order():
    """The library's item list is exactly the restated deal (what the GPU's bins walk), and splits past the code's
    64 are refused."""
    import numpy as np
    from m3x import ops
    rng = np.random.default_rng(5)
    for trial in range(40):
        runs, row = [], 0
        for _ in range(int(rng.integers(1, 120))):
            n = 1 if rng.random() < 0.8 else int(rng.integers(1, 300))
            runs.append((row, n, int(rng.integers(0, 3000))))
            row += n
        heads, kv = (16, 8) if trial % 2 else (16, 16)
        bins, chunk = int(rng.integers(1, 100)), int(rng.choice([128, 512, 4096]))
        assert ops.attn_items(runs, heads, kv, bins, chunk).tolist() == _items_restated(runs, heads, kv, bins, chunk)
    with pytest.raises(ValueError):
        ops.attn_items([(0, 1, 65 * 128)], 16, 8, 4, 128)


def test_roofline_matches_published_shapes():
    # BASELINE: backbone weights 880,803,840 B; 112 KiB of KV per token per seat
    assert roofline.backbone_weight_bytes() == 880_803_840
    assert roofline.decode_attn_bytes(1, 0) * 28 == 112 * 1024
    # per depth codebook step: trunk 102,760,448 B + head 4,194,304 B
    assert roofline.depth_frame_bytes(seats=0) == 31 * (102_760_448 + 4_194_304) + 1024 * 1024 * 2


def test_synth_is_seeded_and_shaped():
    a = synth.qwen3_backbone(layers=1, seed=3)
    b = synth.qwen3_backbone(layers=1, seed=3)
    la, lb = a.lm.model.layers[0], b.lm.model.layers[0]
    assert torch.equal(la.self_attn.q_proj.weight, lb.self_attn.q_proj.weight)
    assert la.self_attn.q_proj.weight.shape == (2048, 1024) and la.mlp.down_proj.weight.shape == (1024, 3072)
    assert a.cb0_head.weight.shape == (2048, 1024)
    lens = synth.c5_lengths(224)
    assert lens.shape == (224,) and 1900 < float(lens.float().mean()) < 2200 and int(lens.max()) <= 4096
    c4 = synth.c4_decode_lengths()
    assert c4.min() >= 128 and c4.max() < 4096


def test_cache_pack_split_roundtrip():
    from m3x.serve.cache import cache_from_owned_tensors, pack_caches, split_cache
    g = torch.Generator().manual_seed(1)
    caches = []
    for n in (3, 0, 5):
        if n == 0:
            caches.append(None)
            continue
        caches.append(cache_from_owned_tensors([(torch.randn(1, 2, n, 4, generator=g), torch.randn(1, 2, n, 4,
                                                                                              generator=g))
                                                for _ in range(2)]))
    packed, mask, lengths = pack_caches(caches, 2, "cpu")
    assert lengths == [3, 0, 5] and packed.layers[0].keys.shape == (3, 2, 5, 4)
    assert mask.shape == (3, 7) and mask[0].tolist() == [False, False, True, True, True, True, True]
    rows = split_cache(packed, lengths)
    for c, r, n in zip(caches, rows, lengths):
        if n:
            for la, lb in zip(c.layers, r.layers):
                assert torch.equal(la.keys, lb.keys) and torch.equal(la.values, lb.values)


def test_surfaces_reject_host_models():
    from m3x.serve.fast_backbone import StaticBackbone
    from m3x.serve.fast_depth import FastDepth
    with pytest.raises(ValueError):
        StaticBackbone(synth.qwen3_backbone(layers=1), 2, attention="gather")
    with pytest.raises(ValueError):
        StaticBackbone(synth.qwen3_backbone(layers=1), 2, attention="flash")
    with pytest.raises(ValueError):
        StaticBackbone(synth.qwen3_backbone(layers=1, dtype=torch.float32), 2)
    small = synth.swiglu_depth(d=1024, n_q=16)
    with pytest.raises(ValueError):
        FastDepth(small, 2)
    from m3x.serve.fast_codec import StaticMimi
    with pytest.raises(ValueError):  # a host-resident Mimi: the product path has no CPU fallback
        StaticMimi(synth.mimi(seed=1), 2)


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_frame_step_room_check_on_host():
    """FrameStep refuses a seat whose next position does not fit the graph's context bucket or the cache, at the
    bucket edge exactly (host logic; no kernel runs)."""
    from types import SimpleNamespace
    from m3x.frame import FrameStep, _FrameGraph
    bb = SimpleNamespace(device=torch.device("cpu"), max_slots=4, hidden=8, dtype=torch.bfloat16, capacity=300,
                         lengths_cpu=[0, 255, 256, 299, 0], dummy=4)
    fs = FrameStep(bb, None, SimpleNamespace(), ring_depth=2)
    g = _FrameGraph(None, 256)
    fs._check_room(g, [0, 1])  # 256 positions after the step: fits
    with pytest.raises(ValueError):
        fs._check_room(g, [2])  # 257 > the 256-position bucket
    g2 = _FrameGraph(None, 512)
    fs._check_room(g2, [3])  # 300 = capacity
    bb.lengths_cpu[3] = 300
    with pytest.raises(ValueError):
        fs._check_room(g2, [3])  # 301 > the 300-position cache


def test_row_table_staging_and_buckets():
    """Buckets picks the smallest bucket that holds a request and raises past the largest; check_slots raises the
    reference's errors (ValueError for a repeated slot, IndexError for one out of range)."""
    from m3x.staging import Buckets, check_slots
    b = Buckets((8, 1, 4, 4))
    assert b.sizes == (1, 4, 8) and b.pick(3) == 4 and b.pick(8) == 8 and b.largest_first() == [8, 4, 1]
    with pytest.raises(ValueError):
        b.pick(9)
    with pytest.raises(ValueError):
        check_slots([1, 1], 4)
    with pytest.raises(IndexError):
        check_slots([4], 4)
    check_slots([1, 1], 4, distinct=False)


def test_mixed_step_rows_layout():
    """The host side of StaticBackbone.step_mixed (serve/fast_backbone.py:326-359): the decoding seats' rows first,
    then each prefill's T rows on its slot at offsets 0..T-1; one attention run per decode row (row, 1, its
    position) and one per prefill (its first row, T, its first position); the context needed is the longest of
    them, and a step past the capacity raises. Checked on random mixes against the rows spelled out one by one."""
    import numpy as np
    from types import SimpleNamespace
    from m3x.serve.fast_backbone import StaticBackbone
    rng = np.random.default_rng(17)
    for _ in range(100):
        S = 64
        lengths = [int(v) for v in rng.integers(0, 900, S + 1)]
        perm = [int(v) for v in rng.permutation(S)]
        nd, npf = int(rng.integers(0, 12)), int(rng.integers(0, 4))
        if nd + npf == 0:
            continue
        slots = perm[:nd]
        prefills = [(s, torch.empty(int(rng.integers(1, 40)), 1)) for s in perm[nd:nd + npf]]
        host = SimpleNamespace(lengths_cpu=lengths, max_slots=S, capacity=1000)
        row_slot, row_off, runs, need = StaticBackbone._rows_of(host, slots, prefills)
        want_slot, want_off, want_runs, want_need = [], [], [], 0
        for s in slots:
            want_runs.append([len(want_slot), 1, lengths[s]])
            want_slot.append(s)
            want_off.append(0)
            want_need = max(want_need, lengths[s] + 1)
        for s, t in prefills:
            want_runs.append([len(want_slot), t.shape[0], lengths[s]])
            for j in range(t.shape[0]):
                want_slot.append(s)
                want_off.append(j)
            want_need = max(want_need, lengths[s] + t.shape[0])
        assert row_slot.tolist() == want_slot and row_off.tolist() == want_off
        assert runs.dtype == np.int32 and runs.tolist() == want_runs and need == want_need
    host = SimpleNamespace(lengths_cpu=[995] + [0] * 8, max_slots=8, capacity=1000)
    with pytest.raises(ValueError):
        StaticBackbone._rows_of(host, [1], [(0, torch.empty(6, 1))])
