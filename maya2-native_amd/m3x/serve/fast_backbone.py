"""Static-KV decode of the Qwen3 backbone with per-seat positions, on m3x gfx950 kernels.

Drop-in for serve/fast_backbone.py (StaticBackbone, :111-362). The surface is the reference's: constructor
arguments, `step`, `step_mixed`, `load_slot`, `load_prefix`, `free`, `warmup`, `memory_bytes`, the attributes the
engine and its tests read (`k`, `v`, `lengths`, `lengths_cpu`, `kv_heads`, `head_dim`, `layers`, `max_slots`,
`capacity`, `dummy`), and its exception types. The KV layout is the reference's contract: per layer
`k[i], v[i]: [max_slots + 1, kv_heads, capacity, head_dim]` in the model dtype, slot `max_slots` a dummy whose
length stays 0 and that pads a step up to its row bucket (:3-4,146-150).

How a step runs here:
  - A step is a list of rows. Decoding seats give one row each; an inline prefill of T tokens gives T rows of
    one slot at offsets 0..T-1 from the slot's length. The row layout (slot, real-row flag, offset) is one
    int64 table staged in a single async copy (m3x.staging.RowTable); a decode step with the same seats as the
    previous one on its graph stages nothing.
  - Each (row bucket, context bucket) has one hipGraph over its own buffers; steps with inline prefills use a
    separate graph whose attention walks a host-built list of work items (prefill rows of one slot share one
    pass over its keys).
  - The graph body per layer (the reference's fuse_rope path, :187-203): q|k|v GEMM with the input RMSNorm
    folded in (the norm weight in the packed weight, each row's 1 / rms in the epilogue) -> q/k-norm + RoPE + K/V
    cache write -> decode attention in place over the cache -> o GEMM that adds into the residual and leaves the
    row's tile statistics -> gate|up GEMM with the post-attention RMSNorm folded in and SwiGLU behind -> down GEMM
    that adds into the residual. Only the first
    layer's input norm and the final norm run as add+norm kernels (widths other than 1024 keep the separate
    add+RMSNorm launches).
  - q|k|v and gate|up are joined into one weight each, with the model's modules re-pointed at row views of
    the joined tensors (no second copy of the HF weights, as the reference's fuse_proj does, :130-141), and every
    projection also gets a copy in MFMA fragment order (ops.pack_weight).
`attention`, `fuse_proj`, `fuse_rope` and `fused_norm` are accepted for construction-site compatibility; there is
one kernel path.
"""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import torch

from .. import ops
from .._lib import lib
from ..staging import Buckets, ErrorWatch, RowTable, Upload, capture, check_slots

TILE = 32  # keys per attention tile: the per-slot extent of the cache allocation is a multiple of this


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


# Decode steps whose contexts are spread out take the item launch of the attention: each row's keys cut into splits
# and the splits dealt longest-first into one round of workgroups, so no long row is left running alone at the end
# of the grid. Measured on MI355X (graph-timed, 8 kv heads, head_dim 128, lengths U[64, 2048]): 24-192 rows 1-16 %
# faster than the per-row launch, bit-identical (the same arithmetic per row); with near-equal contexts (Poisson
# 2048) the per-row launch stays 3-8 % faster, so a step takes the item launch only when its longest context exceeds
# ITEM_SKEW times the mean, and only from ITEM_MIN_ROWS rows (at 16 rows the per-row launch wins either way).
ITEM_MIN_ROWS = 24
ITEM_SKEW = 1.5


def item_chunk(rows: int) -> int:
    """Keys per split of a decode step's item launch (1024 up to 96 rows, 2048 above: measured best)."""
    return 1024 if rows <= 96 else 2048


def _retarget(module, view):
    """Point a Linear-like module's weight at `view` (nn.Parameter .data or a plain holder attribute)."""
    w = module.weight
    if isinstance(w, torch.nn.Parameter):
        w.data = view
    else:
        module.weight = view


def _join(modules):
    """One contiguous [sum of outs, in] tensor of the modules' weights, each module re-pointed at its rows."""
    joint = torch.cat([m.weight for m in modules]).contiguous()
    at = 0
    for m in modules:
        n = m.weight.shape[0]
        _retarget(m, joint[at:at + n])
        at += n
    return joint


class _StepGraph:
    """One (row bucket, context bucket[, inline prefills | item launch]) step: buffers, row table, item upload,
    graph, and the key of the decode item list last uploaded."""
    __slots__ = ("bufs", "items", "graph", "items_key")

    def __init__(self, bufs):
        self.bufs, self.items, self.graph, self.items_key = bufs, None, None, None


class StaticBackbone:
    def __init__(self, backbone, max_slots, capacity=1536,
                 batch_buckets=(1, 2, 4, 8, 16, 24, 32, 48, 64, 80, 96), ctx_buckets=(512, 768, 1024, 1536),
                 attention='gather', fused_norm=False, use_graphs=True, fuse_proj=False, fuse_rope=False):
        if attention not in ('gather', 'triton'):
            raise ValueError('attention must be gather or triton')
        lib()  # the kernels are the only path: fail here if the library is missing
        self.attention, self.fused_norm, self.use_graphs = attention, fused_norm, use_graphs
        self.fuse_proj = self.fuse_rope = True
        with torch.inference_mode():
            self._read_model(backbone)
            self.max_slots, self.capacity, self.dummy = int(max_slots), int(capacity), int(max_slots)
            self._pack_weights()
            rows = Buckets(batch_buckets)
            if rows.sizes[-1] < self.max_slots:  # a step of every seat must have a row bucket
                rows = Buckets(rows.sizes + (self.max_slots,))
            self._rows = rows
            self._ctx = Buckets({min(int(c), self.capacity) for c in ctx_buckets} | {self.capacity})
            self.batch_buckets, self.ctx_buckets = rows.sizes, self._ctx.sizes
            self._alloc_cache()
        self.graphs = {}
        self.pool = None
        # the one-row step as one persistent kernel (m3x_backbone_run): its exchange area and epoch / error words;
        # spin_limit: polling rounds before a wait gives up (0: the kernel's default)
        self.persistent = True
        self.spin_limit = 0
        self._run_xchg = torch.zeros(ops.backbone_run_xchg_bytes() // 8, dtype=torch.int64, device=self.device)
        self._run_sync = torch.zeros(4, dtype=torch.int32, device=self.device)
        self._run_table = None
        self._nwg = torch.cuda.get_device_properties(self.device).multi_processor_count
        self._watch = ErrorWatch(self._run_sync, 'StaticBackbone: a persistent one-row step')

    # ---------------------------------------------------------------- construction
    def _read_model(self, backbone):
        self.backbone = backbone
        self.lm = backbone.lm.model
        cfg = backbone.lm.config
        self.layers = list(self.lm.layers)
        self.norm = self.lm.norm
        p = next(self.lm.parameters())
        self.dtype, self.device = p.dtype, p.device
        if self.dtype != torch.bfloat16:
            raise ValueError('fused add+norm kernel is bf16-only')
        if self.device.type != 'cuda':
            raise ValueError('StaticBackbone runs on the GPU; the model is on ' + str(self.device))
        self.heads, self.kv_heads = cfg.num_attention_heads, cfg.num_key_value_heads
        self.head_dim = getattr(cfg, 'head_dim', None) or cfg.hidden_size // cfg.num_attention_heads
        self.groups = self.heads // self.kv_heads
        self.hidden = cfg.hidden_size
        self.scaling = self.head_dim ** -0.5
        self.eps = cfg.rms_norm_eps
        # width 1024 (Qwen3-0.6B): the o and down projections add into the residual and leave its tile statistics,
        # and the q|k|v and gate|up projections, whose packed weights carry the RMSNorm weight, scale each row of
        # their product by the row's 1 / rms (no add+norm launch)
        self.fused_norms = self.hidden == 1024

    def _pack_weights(self):
        self.wqkv, self.wgu = [], []
        self.pqkv, self.pgate, self.pup, self.po, self.pdown = [], [], [], [], []
        for i, layer in enumerate(self.layers):
            a, m = layer.self_attn, layer.mlp
            if a.q_proj.bias is not None or getattr(m.gate_proj, 'bias', None) is not None:
                raise ValueError('fuse_proj expects bias-free projections')
            self.wqkv.append(_join([a.q_proj, a.k_proj, a.v_proj]))
            self.wgu.append(_join([m.gate_proj, m.up_proj]))
            inter = m.gate_proj.weight.shape[0]
            # with fused norms the RMSNorm weight in front of q|k|v (after the first layer) and of gate|up is folded
            # into the packed copy; the HF modules keep their own weights
            if self.fused_norms and i > 0:
                self.pqkv.append(ops.fold_norm(self.wqkv[-1], layer.input_layernorm.weight)[0])
            else:
                self.pqkv.append(ops.pack_weight(self.wqkv[-1]))
            if self.fused_norms:
                gu = ops.fold_norm(self.wgu[-1], layer.post_attention_layernorm.weight)[0]
            else:
                gu = ops.pack_weight(self.wgu[-1])
            self.pgate.append(gu.rows(0, inter))
            self.pup.append(gu.rows(inter, 2 * inter))
            self.po.append(ops.pack_weight(a.o_proj.weight))
            self.pdown.append(ops.pack_weight(m.down_proj.weight))
        self.inter = self.pgate[0].N
        torch.cuda.current_stream(self.device).synchronize()  # packing ran on the current stream

    def _alloc_cache(self):
        # the allocation's per-slot extent is a whole number of attention tiles; k[i] / v[i] are views of exactly
        # `capacity` positions, as the reference's tensors are
        self._extent = -(-self.capacity // TILE) * TILE
        full = (self.max_slots + 1, self.kv_heads, self._extent, self.head_dim)
        self._kfull = [torch.zeros(full, dtype=self.dtype, device=self.device) for _ in self.layers]
        self._vfull = [torch.zeros(full, dtype=self.dtype, device=self.device) for _ in self.layers]
        self.k = [t[:, :, :self.capacity] for t in self._kfull]
        self.v = [t[:, :, :self.capacity] for t in self._vfull]
        self.lengths = torch.zeros(self.max_slots + 1, dtype=torch.long, device=self.device)
        self.lengths_cpu = [0] * (self.max_slots + 1)
        cos, sin = self.lm.rotary_emb(torch.zeros(1, 1, self.hidden, dtype=self.dtype, device=self.device),
                                      torch.arange(self._extent, device=self.device)[None])
        self.cos, self.sin = cos[0].contiguous(), sin[0].contiguous()  # [extent, head_dim], model dtype (as HF)

    # ---------------------------------------------------------------- slots
    def _set_length(self, slot, n):
        self.lengths[slot] = n
        self.lengths_cpu[slot] = n

    def _install(self, slot, length, pairs):
        """Copy the first `length` positions of per-layer (keys, values) [kv_heads, >= length, head_dim]."""
        check_slots([slot], self.max_slots)
        if length > self.capacity:
            raise ValueError(f'length {length} exceeds capacity {self.capacity}')
        for i, (keys, values) in enumerate(pairs):
            self.k[i][slot, :, :length].copy_(keys[:, :length])
            self.v[i][slot, :, :length].copy_(values[:, :length])
        self._set_length(slot, length)

    @torch.inference_mode()
    def load_slot(self, slot, hf_cache, length):
        """Install an HF cache's first `length` positions (serve/fast_backbone.py:158-165; m3x.serve.cache builds
        such caches)."""
        self._install(slot, length, [(hf_cache.layers[i].keys[0], hf_cache.layers[i].values[0])
                                     for i in range(len(self.layers))])

    @torch.inference_mode()
    def free(self, slot):
        self._set_length(slot, 0)

    @torch.inference_mode()
    def load_prefix(self, slot, kv, length):
        """Install a stored reference-prefix KV (list of per-layer (k, v) [1, KV, length, D]) into a slot."""
        self._install(slot, length, [(k[0], v[0]) for k, v in kv])

    @torch.inference_mode()
    def export_prefix(self, slot, length=None):
        """The slot's first `length` (default: all) cached positions in load_prefix's format: a list of per-layer
        (k, v) [1, kv_heads, length, head_dim] copies, e.g. a voice prefix computed once and installed into other
        slots (the `voice.kv` of maya3/engine.py:276-277)."""
        check_slots([slot], self.max_slots)
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
        check_slots([slot], self.max_slots)
        if x.dim() != 2 or x.shape[1] != self.hidden or x.shape[0] == 0:
            raise ValueError(f'x must be [T>0, {self.hidden}], got {tuple(x.shape)}')
        if self.lengths_cpu[slot] + x.shape[0] > self.capacity:
            raise ValueError(f'context {self.lengths_cpu[slot] + x.shape[0]} exceeds capacity {self.capacity}')
        piece = self.batch_buckets[-1]
        last = None
        for t0 in range(0, x.shape[0], piece):
            last = self.step_mixed([], None, [(slot, x[t0:t0 + piece])])[1][0]
        return last

    # ---------------------------------------------------------------- math
    def make_buffers(self, rows, ctx, mixed=False, items=False):
        """Static buffers of one (row bucket, context bucket) step; reused by every replay of its graph.
        b.table holds the per-row columns slot / real / offset (b.slots, b.real, b.offset are its device columns).
        mixed: the step may hold inline prefill rows (step_mixed), whose attention runs in blocks of consecutive
        rows; a decode-only step (step, the frame step) leaves that launch out unless items is set (a decode step
        whose contexts are spread out: its rows' keys in splits dealt over one round of workgroups)."""
        dev, dt = self.device, self.dtype
        H, KV, D, hid, I = self.heads, self.kv_heads, self.head_dim, self.hidden, self.inter
        b = SimpleNamespace(rows=rows, ctx=ctx, mixed=mixed, decode_items=items and not mixed)
        b.table = RowTable(('slot', 'real', 'offset'), rows, dev, pad=dict(slot=self.dummy))
        b.slots, b.real, b.offset = b.table['slot'], b.table['real'], b.table['offset']
        b.pos = torch.zeros(rows, dtype=torch.int32, device=dev)
        b.x = torch.zeros(rows, hid, dtype=dt, device=dev)
        for name, width in (('h', hid), ('y', hid), ('qkv', (H + 2 * KV) * D), ('o', H * D), ('a', hid),
                            ('act', I), ('pend', hid), ('out', hid)):
            setattr(b, name, torch.empty(rows, width, dtype=dt, device=dev))
        # the 16-column tile statistics the residual projections leave for the next norm
        b.part = torch.empty(ops.tile_stats_elems(rows, hid), dtype=torch.float32, device=dev)
        b.q = torch.empty(rows, H, D, dtype=dt, device=dev)
        b.chunk = item_chunk(rows) if b.decode_items else attn_chunk(rows, KV, ctx)
        b.items = None
        if mixed or b.decode_items:
            # work items (ops.attn_items): until a step stages its own, every row is its own item
            b.item_bins = ops.attn_item_bins(rows, KV, ctx, b.chunk)
            cap_items = 2 + b.item_bins + rows * -(-ctx // b.chunk)
            b.items = torch.zeros(cap_items, dtype=torch.int32, device=dev)
            first = ops.attn_items([(r, 1, 0) for r in range(rows)], H, KV, b.item_bins, b.chunk)
            b.items[:len(first)] = torch.from_numpy(first).to(dev)
        ws = ops.decode_attn_workspace(rows, KV, ctx, b.chunk)
        b.attn_ws = torch.empty(max(ws, 16) // 4, dtype=torch.float32, device=dev)
        return b

    # ---------------------------------------------------------------- one-row persistent run
    def _persistent_ok(self, rows):
        """Whether a step of `rows` rows runs as one persistent kernel: one row (the one-seat frame), the
        Qwen3-0.6B geometry the kernel implements (hidden 1024 with the folded norms, 16 q / 8 kv heads of 128,
        SwiGLU 3072, bf16), a per-slot extent of at most 4096 positions, one workgroup per CU on a 256-CU part."""
        return (self.persistent and rows == 1 and self.fused_norms and self.dtype == torch.bfloat16
                and self.heads == 16 and self.kv_heads == 8
                and self.head_dim == 128 and self.inter == 3072 and self._extent <= 4096 and self._nwg == 256)

    def _run_args(self, b):
        """The persistent run's arguments for buffer set b (built once per buffer set; the spin limit refreshed)."""
        if self._run_table is None:
            rows = []
            for i, layer in enumerate(self.layers):
                a = layer.self_attn
                rows.append(ops.BackboneLayer(
                    self.pqkv[i].data.data_ptr(), self.po[i].data.data_ptr(), self.pgate[i].data.data_ptr(),
                    self.pup[i].data.data_ptr(), self.pdown[i].data.data_ptr(), a.q_norm.weight.data_ptr(),
                    a.k_norm.weight.data_ptr(), self._kfull[i].data_ptr(), self._vfull[i].data_ptr()))
            self._run_table = ops.backbone_layer_table(rows, self.device)
        a = b.__dict__.get('run')
        if a is None:
            a = b.run = ops.BackboneRunArgs()
            kc = self._kfull[0]
            # probe 1: a poll of more than one chunk per thread waits on its first chunk, then reads the rest
            a.layer, a.layers, a.cap, a.nwg, a.probe = self._run_table.data_ptr(), len(self.layers), self._extent, \
                self._nwg, 1
            a.eps, a.scale = self.eps, self.scaling
            a.x, a.h_out, a.slots, a.pos = b.x.data_ptr(), b.h.data_ptr(), b.slots.data_ptr(), b.pos.data_ptr()
            a.cos, a.sin, a.s_cos = self.cos.data_ptr(), self.sin.data_ptr(), self.cos.stride(0)
            a.w_in0 = self.layers[0].input_layernorm.weight.data_ptr()
            a.sk_s, a.sk_h, a.sk_t = kc.stride(0), kc.stride(1), kc.stride(2)
            a.xchg, a.sync = self._run_xchg.data_ptr(), self._run_sync.data_ptr()
            a.w_fin, a.y_out = self.norm.weight.data_ptr(), b.out.data_ptr()
            a.lengths, a.real = self.lengths.data_ptr(), b.real.data_ptr()
        a.spin_limit = int(self.spin_limit)
        return a

    def run_error(self):
        """True when a persistent run since construction (or the last clear) lost a step's input (its bounded waits
        ran out); that step's output rows are void. Synchronises with the device."""
        return bool(self._run_sync[2].item())

    @torch.inference_mode()
    def clear_run_error(self):
        """Reset the error word (stream-ordered)."""
        self._run_sync[2].zero_()
        self._watch.evt = None

    def forward(self, b):
        """One decode step over the rows of buffer set `b` (positions from lengths[slots] + offset); returns b.out."""
        H, KV, D, eps = self.heads, self.kv_heads, self.head_dim, self.eps
        ops.positions(self.lengths, b.slots, b.offset, b.pos)
        if self._persistent_ok(b.rows) and not b.mixed:
            # the 28 layers of the one-row step, its final norm and its length update in one launch
            ops.backbone_run(self._run_args(b))
            return b.out
        o3 = b.o.view(b.rows, H, D)
        fused = self.fused_norms
        rms = ops.NORM_RMS
        for i, layer in enumerate(self.layers):
            attn, kc, vc = layer.self_attn, self._kfull[i], self._vfull[i]
            w_in, w_post = layer.input_layernorm.weight, layer.post_attention_layernorm.weight
            qk = (b.qkv, b.q, kc, vc, b.slots, b.pos, self.cos, self.sin, attn.q_norm.weight, attn.k_norm.weight,
                  eps, H, KV)
            if i == 0:
                ops.add_rms(b.x, None, w_in, eps, y=b.y)
                ops.linear_qk_rope(b.y, self.pqkv[i], *qk)
            elif fused:  # the norm of the residual the previous down projection left, folded into the projection
                ops.linear_qk_rope(b.h, self.pqkv[i], *qk, part=b.part, eps_in=eps)
            else:
                ops.add_rms(b.h, b.pend, w_in, eps, h_out=b.h, y=b.y)
                ops.linear(b.y, self.pqkv[i], b.qkv)
                ops.qk_norm_rope_cache(*qk)
            ops.decode_attn(b.q, kc, vc, o3, b.slots, b.pos, self.scaling, b.ctx, b.chunk, b.attn_ws, H, KV,
                            items=b.items)
            if fused:
                ops.linear_resid(b.o, self.po[i], b.x if i == 0 else b.h, b.h, b.part, rms)
                ops.linear_normed(b.h, b.part, eps, rms, self.pgate[i], self.pup[i], ops.ACT_SWIGLU, y=b.act)
                ops.linear_resid(b.act, self.pdown[i], b.h, b.h, b.part, rms)
            else:
                ops.linear(b.o, self.po[i], b.a)
                ops.add_rms(b.x if i == 0 else b.h, b.a, w_post, eps, h_out=b.h, y=b.y)
                ops.linear_act(b.y, self.pgate[i], self.pup[i], ops.ACT_SWIGLU, b.act)
                ops.linear(b.act, self.pdown[i], b.pend)
        if fused:
            ops.add_rms(b.h, None, self.norm.weight, eps, y=b.out)
        else:
            ops.add_rms(b.h, b.pend, self.norm.weight, eps, h_out=b.h, y=b.out)
        ops.lengths_add(self.lengths, b.slots, b.real)
        return b.out

    # ---------------------------------------------------------------- graphs
    @torch.inference_mode()
    def _graph(self, rows, ctx, mixed=False, items=False):
        key = (rows, ctx, 'mixed') if mixed else ((rows, ctx, 'items') if items else (rows, ctx))
        g = self.graphs.get(key)
        if g is not None:
            return g
        g = _StepGraph(self.make_buffers(rows, ctx, mixed, items))
        if g.bufs.items is not None:
            g.items = Upload(g.bufs.items, ring=2)
        if self.use_graphs:
            if self.pool is None:
                self.pool = torch.cuda.graph_pool_handle()
            # warm-up and capture see all-dummy rows: only the dummy slot's cache rows and length are touched,
            # and the dummy's length is put back
            g.graph = capture(lambda: self.forward(g.bufs), self.pool, warm=2, keep=(self.lengths,))
        self.graphs[key] = g
        return g

    @torch.inference_mode()
    def warmup(self, batch_buckets=None, ctx_buckets=None, mixed=False):
        """Captures the decode graphs of the buckets, for buckets of at least ITEM_MIN_ROWS rows with both attention
        launches (with mixed=True also the graphs of steps with inline prefills; otherwise those are captured on
        first use)."""
        for rows in self._rows.largest_first(batch_buckets):
            for ctx in self._ctx.largest_first({min(int(c), self.capacity) for c in (ctx_buckets or self.ctx_buckets)}):
                self._graph(rows, ctx)
                if rows >= ITEM_MIN_ROWS and not self._persistent_ok(rows):
                    self._graph(rows, ctx, items=True)
                if mixed:
                    self._graph(rows, ctx, True)
        torch.cuda.synchronize()

    def _spread(self, rows, runs):
        """Whether a decode step of `rows` rows (runs as _rows_of gives them) takes the item launch: its longest
        context more than ITEM_SKEW times the mean."""
        if rows < ITEM_MIN_ROWS or self._persistent_ok(rows):
            return False
        ctxs = np.asarray(runs, dtype=np.int64).reshape(-1, 3)[:, 2] + 1
        return int(ctxs.max()) > ITEM_SKEW * (int(ctxs.sum()) / len(ctxs))

    def _rows_of(self, slots, prefills):
        """The step's rows: one per decoding seat, then T per prefill (same slot, offsets 0..T-1). Validates the
        slots and the context; returns (row slots, row offsets, runs for the attention items as int32 [runs, 3] of
        (first row, rows, first position), context needed). Built as arrays: a step with inline prefills has
        thousands of rows."""
        check_slots(list(slots) + [s for s, _ in prefills], self.max_slots)
        nd = len(slots)
        dec = np.fromiter((self.lengths_cpu[s] for s in slots), dtype=np.int64, count=nd)
        sizes = np.fromiter((t.shape[0] for _, t in prefills), dtype=np.int64, count=len(prefills))
        pstart = np.fromiter((self.lengths_cpu[s] for s, _ in prefills), dtype=np.int64, count=len(prefills))
        first = nd + np.concatenate(([0], np.cumsum(sizes)[:-1])) if len(prefills) else sizes
        runs = np.empty((nd + len(prefills), 3), dtype=np.int32)
        runs[:nd, 0] = np.arange(nd)
        runs[:nd, 1] = 1
        runs[:nd, 2] = dec
        runs[nd:, 0] = first
        runs[nd:, 1] = sizes
        runs[nd:, 2] = pstart
        total = nd + int(sizes.sum())
        row_slot = np.empty(total, dtype=np.int64)
        row_slot[:nd] = np.fromiter(slots, dtype=np.int64, count=nd)
        row_off = np.zeros(total, dtype=np.int64)
        if len(prefills):
            pslots = np.fromiter((s for s, _ in prefills), dtype=np.int64, count=len(prefills))
            row_slot[nd:] = np.repeat(pslots, sizes)
            row_off[nd:] = np.arange(total - nd) - np.repeat(first - nd, sizes)
        need = max(int(dec.max()) + 1 if nd else 0, int((pstart + sizes).max()) if len(prefills) else 0)
        if need > self.capacity:
            raise ValueError(f'context {need} exceeds capacity {self.capacity}')
        return row_slot, row_off, runs, need

    def _replay(self, slots, x, prefills):
        """Stage and run one step; returns the step's output rows (a view of the graph's buffer). Raises when an
        earlier persistent one-row step failed (the reference fails the engine on a GPU-side error,
        maya3/engine.py:375-385)."""
        self._watch.raise_if_set()
        row_slot, row_off, runs, need = self._rows_of(slots, prefills)
        n = len(row_slot)
        rows = self._rows.pick(n, 'batch')
        spread = not prefills and self._spread(rows, runs)
        g = self._graph(rows, self._ctx.pick(need, 'context'), bool(prefills), spread)
        b = g.bufs
        # a decode step keyed by its seats restages nothing when they repeat
        b.table.stage(dict(slot=row_slot, real=np.ones(n, dtype=np.int64), offset=row_off),
                      key=None if prefills else ('decode', tuple(slots)))
        if prefills or spread:
            # a decode step's list stays valid while every row keeps its number of splits (the kernels take each
            # split's keys and a row's split count from the positions at run time): it is rebuilt only when a row
            # crosses a split boundary or the seats change
            key = None if prefills else (tuple(slots), tuple(((runs[:, 2] + b.chunk) // b.chunk).tolist()))
            if key is None or key != g.items_key:
                if b.rows > n:  # padding rows on the dummy slot
                    pad = np.zeros((b.rows - n, 3), dtype=np.int32)
                    pad[:, 0] = np.arange(n, b.rows)
                    pad[:, 1] = 1
                    runs = np.concatenate([runs, pad])
                items = ops.attn_items(runs, self.heads, self.kv_heads, b.item_bins, b.chunk)
                g.items.buffer()[:len(items)] = items
                g.items.send(len(items))
            g.items_key = key
        parts = ([x] if slots else []) + [t for _, t in prefills]
        if len(parts) > 1 and all(p.dim() == 2 and p.dtype == b.x.dtype and p.device == b.x.device for p in parts):
            torch.cat(parts, out=b.x[:n])  # one copy kernel for the decode rows and every prefill
        else:
            at = 0
            for p in parts:
                b.x[at:at + p.shape[0]].copy_(p)
                at += p.shape[0]
        if g.graph is not None:
            g.graph.replay()
        else:
            self.forward(b)
        if self._persistent_ok(b.rows) and not b.mixed:
            self._watch.after()
        for s in slots:
            self.lengths_cpu[s] += 1
        for s, t in prefills:
            self.lengths_cpu[s] += t.shape[0]
        return b.out

    @torch.inference_mode()
    def step(self, slots, x):
        """Decode one token for each seat; x [B, hidden] -> the final-normed hidden states [B, hidden] (owned)."""
        B = len(slots)
        if B == 0:
            return x.new_zeros(0, self.hidden)
        if tuple(x.shape) != (B, self.hidden):
            check_slots(slots, self.max_slots)
            raise ValueError(f'x must be [{B}, {self.hidden}], got {tuple(x.shape)}')
        return self._replay(list(slots), x, ())[:B].clone()

    @torch.inference_mode()
    def step_mixed(self, slots, x, prefills):
        """One graphed step for decoding seats plus inline prefills.

        prefills: list of (slot, tokens [T, hidden]) for slots that already hold their prefix. A prefill's T rows
        sit at consecutive positions of its slot; every layer writes all rows' K/V before its attention and each
        row attends to keys up to its own position, so the rows form an exact causal prefill.
        Returns (decoding seats' hidden states [B, hidden], [last position's hidden state per prefill])
        (serve/fast_backbone.py:326-359)."""
        B = len(slots)
        if B + sum(t.shape[0] for _, t in prefills) == 0:
            return x.new_zeros(0, self.hidden), []
        out = self._replay(list(slots), x, list(prefills))
        ends, at = [], B
        for _, t in prefills:
            at += t.shape[0]
            ends.append(at - 1)
        return out[:B].clone(), [out[e].clone() for e in ends]

    def memory_bytes(self):
        return sum(t.numel() * t.element_size() for t in self._kfull + self._vfull)
