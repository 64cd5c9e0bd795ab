"""Static-KV single-token decode of the Qwen3 backbone with per-seat positions, on m3x gfx950 kernels.

Drop-in for serve/fast_backbone.py (StaticBackbone, :111-362): same constructor, methods, attributes, errors and
static KV layout — per layer `k[i], v[i]: [max_slots+1, kv_heads, capacity, head_dim]` in the model dtype, slot
`max_slots` a dummy whose length stays 0 and pads a batch up to its bucket (:3-4,146-150). One hipGraph per
(row bucket, context bucket), all graphs in one memory pool; q|k|v and gate|up are concatenated once and the HF
weights re-viewed into them (:130-141), and every projection weight gets one packed copy in MFMA fragment order
(ops.pack_weight) that the projection kernels stream with fully contiguous loads.

Per layer the step runs: [add+]RMSNorm -> q|k|v GEMM -> q/k-norm + RoPE + K/V cache write -> decode attention
over the cache in place -> o GEMM -> add+RMSNorm -> gate|up GEMM -> SwiGLU -> down GEMM (deferred into the next
layer's add+RMSNorm), i.e. the reference's fuse_rope path (:187-203). `attention`, `fuse_proj`, `fuse_rope` and
`fused_norm` are accepted for construction-site compatibility; there is one kernel path.
"""
from __future__ import annotations

from types import SimpleNamespace

import torch

from .. import ops
from .._lib import lib


def attn_chunk(rows: int, kv_heads: int, ctx: int) -> int:
    """Keys per split of the decode attention: about 1024 workgroups over the context bucket, 128..4096 keys each.

    Measured on MI355X (graph-timed, 8 kv heads, head_dim 128): 224 rows at 2048 keys run best unsplit (one
    workgroup per (row, kv head), no combine launch); a single row at 2048 keys runs best at 128-key splits
    (8.2 us with the combine, against 9.5 at 256), 16 rows at 512."""
    want = rows * kv_heads * ctx / 1024.0
    c = 128
    while c < want and c < 4096:
        c *= 2
    return c


class _Graph:
    __slots__ = ('graph', 'slots', 'slots_cpu', 'x', 'real', 'real_cpu', 'out', 'last', 'offset', 'offset_cpu',
                 'offset_dirty', 'evt', 'bufs', 'items_cpu')


class StaticBackbone:
    def __init__(self, backbone, max_slots, capacity=1536,
                 batch_buckets=(1, 2, 4, 8, 16, 24, 32, 48, 64, 80, 96), ctx_buckets=(512, 768, 1024, 1536),
                 attention='gather', fused_norm=False, use_graphs=True, fuse_proj=False, fuse_rope=False):
        if attention not in ('gather', 'triton'):
            raise ValueError('attention must be gather or triton')
        lib()  # the kernels are the only path: fail here if the library is missing
        with torch.inference_mode():
            self.backbone = backbone
            self.lm = backbone.lm.model
            cfg = backbone.lm.config
            self.layers = list(self.lm.layers)
            self.norm = self.lm.norm
            p = next(self.lm.parameters())
            self.dtype = p.dtype
            self.device = p.device
            if self.dtype != torch.bfloat16:
                raise ValueError('fused add+norm kernel is bf16-only')
            if self.device.type != 'cuda':
                raise ValueError('StaticBackbone runs on the GPU; the model is on ' + str(self.device))
            self.heads = cfg.num_attention_heads
            self.kv_heads = cfg.num_key_value_heads
            self.head_dim = getattr(cfg, 'head_dim', None) or cfg.hidden_size // cfg.num_attention_heads
            self.groups = self.heads // self.kv_heads
            self.hidden = cfg.hidden_size
            self.scaling = self.head_dim ** -0.5
            self.eps = cfg.rms_norm_eps
            self.max_slots = max_slots
            self.capacity = capacity
            self.dummy = max_slots
            self.attention = attention
            self.fused_norm = fused_norm
            self.use_graphs = use_graphs
            self.fuse_proj = True
            self.fuse_rope = True
            self.wqkv = []
            self.wgu = []
            for layer in self.layers:
                a = layer.self_attn
                m = layer.mlp
                if a.q_proj.bias is not None or getattr(m.gate_proj, 'bias', None) is not None:
                    raise ValueError('fuse_proj expects bias-free projections')
                w = torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]).contiguous()
                nq, nk = a.q_proj.weight.shape[0], a.k_proj.weight.shape[0]
                _reweight(a.q_proj, w[:nq])
                _reweight(a.k_proj, w[nq:nq + nk])
                _reweight(a.v_proj, w[nq + nk:])
                self.wqkv.append(w)
                g = torch.cat([m.gate_proj.weight, m.up_proj.weight]).contiguous()
                ng = m.gate_proj.weight.shape[0]
                _reweight(m.gate_proj, g[:ng])
                _reweight(m.up_proj, g[ng:])
                self.wgu.append(g)
            self.inter = self.wgu[0].shape[0] // 2
            # MFMA fragment-order copies for the projection kernels (the module weights stay as they are)
            I = self.inter
            self.pqkv = [ops.pack_weight(w) for w in self.wqkv]
            pgu = [ops.pack_weight(g) for g in self.wgu]
            self.pgate = [p.rows(0, I) for p in pgu]
            self.pup = [p.rows(I, 2 * I) for p in pgu]
            self.po = [ops.pack_weight(layer.self_attn.o_proj.weight) for layer in self.layers]
            self.pdown = [ops.pack_weight(layer.mlp.down_proj.weight) for layer in self.layers]
            torch.cuda.current_stream(self.device).synchronize()
            self.batch_buckets = tuple(sorted(set(batch_buckets)))
            if self.batch_buckets[-1] < max_slots:
                self.batch_buckets += (max_slots,)
            self.ctx_buckets = tuple(sorted({min(c, capacity) for c in ctx_buckets} | {capacity}))
            # the kernels read 32-key tiles: the slot extent is the capacity rounded up to a multiple of 32
            cap_alloc = -(-capacity // 32) * 32
            shape = (max_slots + 1, self.kv_heads, cap_alloc, self.head_dim)
            self.k = [torch.zeros(shape, dtype=self.dtype, device=self.device) for _ in self.layers]
            self.v = [torch.zeros(shape, dtype=self.dtype, device=self.device) for _ in self.layers]
            self.lengths = torch.zeros(max_slots + 1, dtype=torch.long, device=self.device)
            self.lengths_cpu = [0] * (max_slots + 1)
            positions = torch.arange(cap_alloc, device=self.device)[None]
            cos, sin = self.lm.rotary_emb(torch.zeros(1, 1, self.hidden, dtype=self.dtype, device=self.device),
                                          positions)
            self.cos = cos[0].contiguous()  # [cap, head_dim], model dtype (as HF)
            self.sin = sin[0].contiguous()
            self.graphs = {}
            self.pool = None

    # ---------------------------------------------------------------- slots
    @torch.inference_mode()
    def load_slot(self, slot, hf_cache, length):
        if not 0 <= slot < self.max_slots:
            raise IndexError(slot)
        if length > self.capacity:
            raise ValueError(f'length {length} exceeds capacity {self.capacity}')
        for i in range(len(self.layers)):
            layer = hf_cache.layers[i]
            self.k[i][slot, :, :length].copy_(layer.keys[0, :, :length])
            self.v[i][slot, :, :length].copy_(layer.values[0, :, :length])
        self.lengths[slot] = length
        self.lengths_cpu[slot] = length

    @torch.inference_mode()
    def free(self, slot):
        self.lengths[slot] = 0
        self.lengths_cpu[slot] = 0

    @torch.inference_mode()
    def load_prefix(self, slot, kv, length):
        """Install a stored reference-prefix KV (list of per-layer (k,v) [1,KV,length,D]) into a slot."""
        if not 0 <= slot < self.max_slots:
            raise IndexError(slot)
        for i, (k, v) in enumerate(kv):
            self.k[i][slot, :, :length].copy_(k[0])
            self.v[i][slot, :, :length].copy_(v[0])
        self.lengths[slot] = length
        self.lengths_cpu[slot] = length

    @torch.inference_mode()
    def export_prefix(self, slot, length=None):
        """The slot's first `length` (default: all) cached positions in load_prefix's format: a list of per-layer
        (k, v) [1, kv_heads, length, head_dim] copies, e.g. a voice prefix computed once and installed into other
        slots (the `voice.kv` of maya3/engine.py:276-277)."""
        if not 0 <= slot < self.max_slots:
            raise IndexError(slot)
        n = self.lengths_cpu[slot] if length is None else int(length)
        if not 0 <= n <= self.lengths_cpu[slot]:
            raise ValueError(f'length {n} outside the slot\'s {self.lengths_cpu[slot]} cached positions')
        return [(self.k[i][slot:slot + 1, :, :n].clone(), self.v[i][slot:slot + 1, :, :n].clone())
                for i in range(len(self.layers))]

    @torch.inference_mode()
    def prefill(self, slot, x):
        """Causal prefill of x [T, hidden] onto the slot's cached prefix, through the graphed inline-prefill step
        (step_mixed with no decoding seats) in pieces of at most the largest row bucket; returns the last position's
        hidden state [hidden]. Replaces the eager HF prefill that the engine falls back to for prompts longer than a
        tick's row budget and that computes a voice's prefix KV (maya3/engine.py:270-279,497-506)."""
        if not 0 <= slot < self.max_slots:
            raise IndexError(slot)
        if x.dim() != 2 or x.shape[1] != self.hidden or x.shape[0] == 0:
            raise ValueError(f'x must be [T>0, {self.hidden}], got {tuple(x.shape)}')
        if self.lengths_cpu[slot] + x.shape[0] > self.capacity:
            raise ValueError(f'context {self.lengths_cpu[slot] + x.shape[0]} exceeds capacity {self.capacity}')
        piece = self.batch_buckets[-1]
        last = None
        for t0 in range(0, x.shape[0], piece):
            _, out = self.step_mixed([], None, [(slot, x[t0:t0 + piece])])
            last = out[0]
        return last

    # ---------------------------------------------------------------- math
    def make_buffers(self, rows, ctx, mixed=False):
        """Static buffers of one (row bucket, context bucket) step; reused by every replay of its graph.
        mixed: the step may hold inline prefill rows (step_mixed), whose attention runs in blocks of consecutive
        rows; a decode-only step (step, the frame step) leaves that launch out."""
        dev, dt = self.device, self.dtype
        H, KV, D, hid, I = self.heads, self.kv_heads, self.head_dim, self.hidden, self.inter
        b = SimpleNamespace(rows=rows, ctx=ctx, mixed=mixed)
        b.slots = torch.full((rows,), self.dummy, dtype=torch.long, device=dev)
        b.real = torch.zeros(rows, dtype=torch.long, device=dev)
        b.offset = torch.zeros(rows, dtype=torch.long, device=dev)
        b.items = None
        b.pos = torch.zeros(rows, dtype=torch.int32, device=dev)
        b.x = torch.zeros(rows, hid, dtype=dt, device=dev)
        b.h = torch.empty(rows, hid, dtype=dt, device=dev)
        b.y = torch.empty(rows, hid, dtype=dt, device=dev)
        b.qkv = torch.empty(rows, (H + 2 * KV) * D, dtype=dt, device=dev)
        b.q = torch.empty(rows, H, D, dtype=dt, device=dev)
        b.o = torch.empty(rows, H * D, dtype=dt, device=dev)
        b.a = torch.empty(rows, hid, dtype=dt, device=dev)
        b.act = torch.empty(rows, I, dtype=dt, device=dev)
        b.pend = torch.empty(rows, hid, dtype=dt, device=dev)
        b.out = torch.empty(rows, hid, dtype=dt, device=dev)
        b.chunk = attn_chunk(rows, KV, ctx)
        if mixed:
            # attention work items of a mixed step (ops.attn_items): prefill rows attended 16 // G at a time; until
            # a step stages its own, every row is an item of its own
            b.item_bins = ops.attn_item_bins(rows, KV, ctx, b.chunk)
            items = ops.attn_items([(r, 1, 0) for r in range(rows)], H, KV, b.item_bins, b.chunk)
            b.items = torch.zeros(2 + b.item_bins + rows * ((ctx + b.chunk - 1) // b.chunk), dtype=torch.int32,
                                  device=dev)
            b.items[:len(items)] = torch.from_numpy(items)
        ws = ops.decode_attn_workspace(rows, KV, ctx, b.chunk)
        b.attn_ws = torch.empty(max(ws, 16) // 4, dtype=torch.float32, device=dev)
        return b

    def forward(self, b):
        """One decode step over the rows of buffer set `b` (positions from lengths[slots] + offset); returns b.out."""
        H, KV, D, eps = self.heads, self.kv_heads, self.head_dim, self.eps
        R = b.rows
        ops.positions(self.lengths, b.slots, b.offset, b.pos)
        o3 = b.o.view(R, H, D)
        for i, layer in enumerate(self.layers):
            attn = layer.self_attn
            if i == 0:
                ops.add_rms(b.x, None, layer.input_layernorm.weight, eps, y=b.y)
            else:
                ops.add_rms(b.h, b.pend, layer.input_layernorm.weight, eps, h_out=b.h, y=b.y)
            ops.linear(b.y, self.pqkv[i], b.qkv)
            ops.qk_norm_rope_cache(b.qkv, b.q, self.k[i], self.v[i], b.slots, b.pos, self.cos, self.sin,
                                   attn.q_norm.weight, attn.k_norm.weight, eps, H, KV)
            ops.decode_attn(b.q, self.k[i], self.v[i], o3, b.slots, b.pos, self.scaling, b.ctx, b.chunk, b.attn_ws,
                            H, KV, items=b.items)
            ops.linear(b.o, self.po[i], b.a)
            ops.add_rms(b.x if i == 0 else b.h, b.a, layer.post_attention_layernorm.weight, eps, h_out=b.h, y=b.y)
            ops.linear_act(b.y, self.pgate[i], self.pup[i], ops.ACT_SWIGLU, b.act)
            ops.linear(b.act, self.pdown[i], b.pend)
        ops.add_rms(b.h, b.pend, self.norm.weight, eps, h_out=b.h, y=b.out)
        ops.lengths_add(self.lengths, b.slots, b.real)
        return b.out

    # ---------------------------------------------------------------- graphs
    def _bucket(self, values, need, what):
        for b in values:
            if b >= need:
                return b
        raise ValueError(f'{what} {need} exceeds largest bucket {values[-1]}')

    @torch.inference_mode()
    def _capture(self, bb, cb, mixed=False):
        g = _Graph()
        g.bufs = self.make_buffers(bb, cb, mixed)
        g.slots, g.real, g.offset, g.x = g.bufs.slots, g.bufs.real, g.bufs.offset, g.bufs.x
        g.offset_cpu = torch.zeros(bb, dtype=torch.long, pin_memory=True)
        g.offset_dirty = False
        g.slots_cpu = torch.full((bb,), self.dummy, dtype=torch.long, pin_memory=True)
        g.real_cpu = torch.zeros(bb, dtype=torch.long, pin_memory=True)
        g.items_cpu = torch.zeros_like(g.bufs.items, device='cpu').pin_memory() if mixed else None
        g.last = None
        g.graph = None
        g.evt = None
        g.out = g.bufs.out
        if self.use_graphs:
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                for _ in range(2):
                    self.forward(g.bufs)  # all-dummy rows: touches only the dummy slot
            torch.cuda.current_stream().wait_stream(stream)
            if self.pool is None:
                self.pool = torch.cuda.graph_pool_handle()
            g.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g.graph, pool=self.pool):
                self.forward(g.bufs)
        self.graphs[(bb, cb, 'mixed') if mixed else (bb, cb)] = g
        return g

    @torch.inference_mode()
    def warmup(self, batch_buckets=None, ctx_buckets=None, mixed=False):
        """Captures the decode graphs of the buckets (and with mixed=True also the graphs step_mixed uses for steps
        with inline prefills; otherwise those are captured on their first use)."""
        # largest first so later (smaller) captures reuse the shared pool's blocks
        for bb in sorted(batch_buckets or self.batch_buckets, reverse=True):
            for cb in sorted(ctx_buckets or self.ctx_buckets, reverse=True):
                cb = min(cb, self.capacity)
                if (bb, cb) not in self.graphs:
                    self._capture(bb, cb)
                if mixed and (bb, cb, 'mixed') not in self.graphs:
                    self._capture(bb, cb, True)
        torch.cuda.synchronize()

    def _run(self, g):
        if g.graph is not None:
            g.graph.replay()
        else:
            self.forward(g.bufs)
        return g.out

    @torch.inference_mode()
    def step(self, slots, x):
        B = len(slots)
        if B == 0:
            return x.new_zeros(0, self.hidden)
        if len(set(slots)) != B:
            raise ValueError('duplicate slots in one step')
        need = 0
        for s in slots:
            if not 0 <= s < self.max_slots:
                raise IndexError(s)
            need = max(need, self.lengths_cpu[s] + 1)
        if need > self.capacity:
            raise ValueError(f'context {need} exceeds capacity {self.capacity}')
        if tuple(x.shape) != (B, self.hidden):
            raise ValueError(f'x must be [{B}, {self.hidden}], got {tuple(x.shape)}')
        bb = self._bucket(self.batch_buckets, B, 'batch')
        cb = self._bucket(self.ctx_buckets, need, 'context')
        g = self.graphs.get((bb, cb)) or self._capture(bb, cb)
        key = tuple(slots)
        if g.offset_dirty:
            g.offset.zero_()
            g.offset_dirty = False
            g.last = None
        if g.last != key:
            if g.evt is not None:
                g.evt.synchronize()  # pinned staging may still feed an earlier async copy
            g.slots_cpu[:B] = torch.tensor(slots, dtype=torch.long)
            g.slots_cpu[B:] = self.dummy
            g.real_cpu[:B] = 1
            g.real_cpu[B:] = 0
            g.slots.copy_(g.slots_cpu, non_blocking=True)
            g.real.copy_(g.real_cpu, non_blocking=True)
            g.evt = torch.cuda.Event()
            g.evt.record()
            g.last = key
        g.x[:B].copy_(x)
        out = self._run(g)[:B].clone()
        for s in slots:
            self.lengths_cpu[s] += 1
        return out

    @torch.inference_mode()
    def step_mixed(self, slots, x, prefills):
        """One graphed step for decoding seats plus inline prefills.

        prefills: list of (slot, x_tokens [T,hidden]); the slot must already hold its prefix. Each prefill
        contributes T rows of the same slot at consecutive positions: every layer writes all rows' K/V before
        attention, and row i only reads keys <= its own position, so this is an exact causal prefill.
        Returns (decode hidden [B,hidden], [last hidden per prefill]) (serve/fast_backbone.py:326-359).
        """
        B = len(slots)
        rows = B + sum(t.shape[0] for _, t in prefills)
        if rows == 0:
            return x.new_zeros(0, self.hidden), []
        if len(set(slots) | {s for s, _ in prefills}) != B + len(prefills):
            raise ValueError('duplicate slots in one step')
        for s in list(slots) + [s for s, _ in prefills]:
            if not 0 <= s < self.max_slots:
                raise IndexError(s)
        need = max([self.lengths_cpu[s] + 1 for s in slots] + [self.lengths_cpu[s] + t.shape[0] for s, t in prefills])
        if need > self.capacity:
            raise ValueError(f'context {need} exceeds capacity {self.capacity}')
        bb = self._bucket(self.batch_buckets, rows, 'batch')
        cb = self._bucket(self.ctx_buckets, need, 'context')
        key = (bb, cb, 'mixed') if prefills else (bb, cb)
        g = self.graphs.get(key) or self._capture(bb, cb, bool(prefills))
        if g.evt is not None:
            g.evt.synchronize()
        index = list(slots)
        offsets = [0] * B
        for s, t in prefills:
            index += [s] * t.shape[0]
            offsets += range(t.shape[0])
        g.slots_cpu[:rows] = torch.tensor(index, dtype=torch.long)
        g.slots_cpu[rows:] = self.dummy
        g.offset_cpu[:rows] = torch.tensor(offsets, dtype=torch.long)
        g.offset_cpu[rows:] = 0
        g.real_cpu[:rows] = 1
        g.real_cpu[rows:] = 0
        g.slots.copy_(g.slots_cpu, non_blocking=True)
        g.real.copy_(g.real_cpu, non_blocking=True)
        g.offset.copy_(g.offset_cpu, non_blocking=True)
        if g.items_cpu is not None:
            runs = [(i, 1, self.lengths_cpu[s]) for i, s in enumerate(slots)]
            at = B
            for s, t in prefills:
                runs.append((at, t.shape[0], self.lengths_cpu[s]))
                at += t.shape[0]
            runs += [(r, 1, 0) for r in range(rows, bb)]  # padding rows on the dummy slot
            items = ops.attn_items(runs, self.heads, self.kv_heads, g.bufs.item_bins, g.bufs.chunk)
            g.items_cpu[:len(items)] = torch.from_numpy(items)
            g.bufs.items.copy_(g.items_cpu, non_blocking=True)
        g.last = None
        g.offset_dirty = bool(prefills)
        g.evt = torch.cuda.Event()
        g.evt.record()
        if B:
            g.x[:B].copy_(x)
        at = B
        for _, t in prefills:
            g.x[at:at + t.shape[0]].copy_(t)
            at += t.shape[0]
        out = self._run(g)
        decoded = out[:B].clone()
        last = []
        at = B
        for s, t in prefills:
            at += t.shape[0]
            last.append(out[at - 1].clone())
            self.lengths_cpu[s] += t.shape[0]
        for s in slots:
            self.lengths_cpu[s] += 1
        return decoded, last

    def memory_bytes(self):
        return sum(t.numel() * t.element_size() for t in self.k + self.v)


def _reweight(module, view):
    """Point a Linear-like module's weight at `view` (nn.Parameter .data or a plain holder attribute)."""
    w = module.weight
    if isinstance(w, torch.nn.Parameter):
        w.data = view
    else:
        module.weight = view
