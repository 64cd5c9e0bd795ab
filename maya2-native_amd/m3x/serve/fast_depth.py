"""Whole-frame depth decoder on m3x gfx950 kernels, one hipGraph per batch bucket.

Drop-in for serve/fast_depth.py (FastDepth, :32-257): same constructor, `set_speaker`, `warmup`, `bucket_for`,
`__call__(slots, h, cb0) -> (codes [B,32] int64, feedback [B,d])`, the per-slot `row_seed`/`row_ctr` streams the
engine writes (maya3/engine.py:436-437), and `_fn(slots_idx, h, cb0)` for direct calls. One replay = 31 depth
levels with in-graph sampling + the backbone feedback embedding, following the fused body
(`_compute_fused`, :143-203):
  prefix[0] = in_proj(h) + level_emb[0]; prefix[1] = embed[0][cb0]
  level L: a group start recomputes positions 0..L causally (T = L+1, the last layer only at position L);
           a repeated group runs position L alone over the within-group K/V (T = 1);
           layers: y = n1(x); qkv; attention; x += o -> n2; FFN; x += f (+ speaker constant) -> next norm;
           logits = heads[L-1](norm(x_L)); code = top-k sample(logits / temp, u[L]); prefix[L+1] = embed[L][code]
  feedback = audio_in.norm(sum_l audio_in.table[code_l + 2048 l] / sqrt(32))
Sampling uses one uniform per (seat, level) from the slot's Philox stream (row_seed, row_ctr); the trunk may be
the reference's (LayerNorm, GELU, 16x64 heads, 11 weight groups, speaker cross constant: tts/model/depth_v2.py)
or the SwiGLU/RMSNorm single-trunk variant (m3x.synth.swiglu_depth).
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import torch

from .. import ops
from .._lib import lib

N_LEVELS = 32
REFERENCE_GROUP_OF_LEVEL = [None] + list(range(8)) + [8] * 8 + [9] * 8 + [10] * 7


def _w(mod, dtype, device):
    return mod.weight.detach().to(device=device, dtype=dtype).contiguous()


def _pw(mod, dtype, device):
    """The module's weight in MFMA fragment order for the projection kernels."""
    return ops.pack_weight(_w(mod, dtype, device))


def _norm(mod, dtype, device):
    """(kind, weight, bias, eps) of a LayerNorm- or RMSNorm-like module."""
    b = getattr(mod, 'bias', None)
    eps = getattr(mod, 'eps', None)
    w = _w(mod, dtype, device)
    if b is not None:
        return SimpleNamespace(kind=ops.NORM_LAYER, w=w, b=b.detach().to(device=device, dtype=dtype).contiguous(),
                               eps=1e-5 if eps is None else float(eps))
    return SimpleNamespace(kind=ops.NORM_RMS, w=w, b=None,
                           eps=float(torch.finfo(dtype).eps if eps is None else eps))


class FastDepth:
    def __init__(self, model, max_slots, dtype=torch.bfloat16, temp=0.7, top_k=64,
                 batch_buckets=(1, 2, 4, 8, 16, 24, 32, 48, 64, 80, 96), seed=1234, greedy=False, compile=False,
                 fused=False):
        if model.depth.n_q != N_LEVELS:
            raise ValueError('FastDepth expects the 32-codebook depth stack')
        lib()
        self.max_slots = int(max_slots)
        self.dtype = dtype
        self.temp = float(temp)
        self.top_k = int(top_k)
        self.greedy = bool(greedy)
        self.batch_buckets = tuple(sorted(set(int(b) for b in batch_buckets)))
        self.fused = bool(fused)
        with torch.inference_mode():
            d = model.depth
            self.device = d.in_proj.weight.device
            if self.device.type != 'cuda':
                raise ValueError('FastDepth runs on the GPU; the model is on ' + str(self.device))
            dev = self.device
            self.n_codes = d.n_codes
            self.D = d.in_proj.weight.shape[0]
            self.H = int(getattr(d, 'n_heads', 16))
            self.hd = self.D // self.H
            self.group_of_level = list(getattr(d, 'group_of_level', REFERENCE_GROUP_OF_LEVEL))
            self.in_proj = _pw(d.in_proj, dtype, dev)
            if hasattr(d, 'embed'):
                self.embed = d.embed.detach().to(device=dev, dtype=dtype).contiguous()
                self.level0 = d.level0.detach().to(device=dev, dtype=dtype).contiguous()
            else:
                # position k+1 of the prefix = code_up(code_lo[cb_k + k*n_codes]) + level_emb[k+1] (:48-51)
                table = (d.code_lo.weight.detach().to(dev, dtype) @ d.code_up.weight.detach().to(dev, dtype).t())
                table = table.view(N_LEVELS - 1, self.n_codes, self.D)
                lvl = d.level_emb.weight.detach().to(dev, dtype)
                self.embed = (table + lvl[1:N_LEVELS, None]).contiguous()
                self.level0 = lvl[0].clone().contiguous()
            self.trunks = []
            for blocks in d.groups:
                layers = []
                for blk in blocks:
                    L = SimpleNamespace(n1=_norm(blk.n1, dtype, dev), n2=_norm(blk.n2, dtype, dev),
                                        qkv=_pw(blk.qkv, dtype, dev), o=_pw(blk.o, dtype, dev))
                    if hasattr(blk, 'gate_up'):
                        w1 = _pw(blk.gate_up, dtype, dev)
                        L.act, L.ffn, L.w2 = ops.ACT_SWIGLU, w1.N // 2, _pw(blk.down, dtype, dev)
                        L.wg, L.wu = w1.rows(0, L.ffn), w1.rows(L.ffn, w1.N)
                    else:
                        L.act, L.wg, L.wu, L.w2 = ops.ACT_GELU, _pw(blk.f1, dtype, dev), None, _pw(blk.f2, dtype, dev)
                        L.ffn = L.wg.N
                    layers.append(L)
                self.trunks.append(layers)
            self.layers = len(self.trunks[0])
            self.final_norm = _norm(d.norm, dtype, dev)
            self.heads = [_pw(h, dtype, dev) for h in d.heads]  # 31 x [n_codes, D]
            self.cross = getattr(d, 'cross', None)
            self.cross_w = None
            if self.cross is not None:
                self.cross_w = [(_pw(c.kv, dtype, dev), _pw(c.o, dtype, dev)) for c in self.cross]
            self.audio_in = model.audio_in  # shared, read-only (engine dtype)
            self.fb_table = model.audio_in.table.weight
            if self.fb_table.dtype not in (torch.bfloat16, torch.float16):
                self.fb_table = self.fb_table.detach().to(torch.bfloat16).contiguous()  # serving keeps it in bf16
            self.fb_norm = _norm(model.audio_in.norm, self.fb_table.dtype, dev)
            self.feedback_scale = math.sqrt(N_LEVELS)
            self.cross_const = torch.zeros(self.max_slots + 1, self.layers, self.D, device=dev, dtype=dtype)
            torch.cuda.current_stream(dev).synchronize()  # packing ran on the current stream
        self.pool = None
        self.graphs = {}
        self.seed_t = torch.full((1,), int(seed) % (2 ** 31 - 1), device=self.device, dtype=torch.int32)
        self.row_seed = torch.zeros(self.max_slots + 1, device=self.device, dtype=torch.int32)
        self.row_ctr = torch.zeros(self.max_slots + 1, device=self.device, dtype=torch.int32)
        self.per_row = True
        self._fn = self._compute

    @torch.inference_mode()
    def set_speaker(self, slot, mem, ref_mask):
        """Per-slot speaker constant o(v(mem) * keep) per layer (single-token cross attention; :73-82)."""
        if mem.ndim != 3 or mem.shape[0] != 1 or mem.shape[1] != 1 or tuple(ref_mask.shape) != (1, 1):
            raise ValueError(f'FastDepth serves exactly one reference per slot; got mem {tuple(mem.shape)}')
        if not 0 <= slot < self.max_slots:
            raise IndexError(f'slot {slot} outside 0..{self.max_slots - 1}')
        if self.cross_w is None:
            return  # a trunk without speaker cross-attention: the constant stays zero
        mem = mem.to(self.device, self.dtype).reshape(1, self.D).contiguous()
        keep = ref_mask.to(self.device, self.dtype).reshape(1, 1)
        for layer, (wkv, wo) in enumerate(self.cross_w):
            kv = ops.linear(mem, wkv)
            v = (kv[:, self.D:] * keep).contiguous()
            self.cross_const[slot, layer].copy_(ops.linear(v, wo)[0])

    # ---------------------------------------------------------------- frame body
    def make_buffers(self, B, h=None, codes=None):
        """Static buffers of one batch bucket. `h`/`codes` may be shared with a caller (the frame step)."""
        dev, dt, D = self.device, self.dtype, self.D
        NP = N_LEVELS
        Fmax = max(L.ffn for t in self.trunks for L in t)
        b = SimpleNamespace(B=B)
        b.slots = torch.full((B,), self.max_slots, dtype=torch.long, device=dev)
        b.h = h if h is not None else torch.zeros(B, self.in_proj.K, dtype=dt, device=dev)
        b.codes = codes if codes is not None else torch.zeros(B, N_LEVELS, dtype=torch.int32, device=dev)
        b.u = torch.zeros(B, N_LEVELS - 1, dtype=torch.float32, device=dev)
        b.prefix = torch.zeros(B, NP, D, dtype=dt, device=dev)
        b.tmp = torch.empty(B, D, dtype=dt, device=dev)
        R = B * NP
        b.xw = torch.empty(R, D, dtype=dt, device=dev)
        b.xw2 = torch.empty(R, D, dtype=dt, device=dev)
        b.yw = torch.empty(R, D, dtype=dt, device=dev)
        b.y2 = torch.empty(R, D, dtype=dt, device=dev)
        b.qkv = torch.empty(R, 3 * D, dtype=dt, device=dev)
        b.att = torch.empty(R, D, dtype=dt, device=dev)
        b.a = torch.empty(R, D, dtype=dt, device=dev)
        b.ffn_act = torch.empty(R, Fmax, dtype=dt, device=dev)
        b.f = torch.empty(R, D, dtype=dt, device=dev)
        b.kd = [torch.zeros(B, self.H, NP, self.hd, dtype=dt, device=dev) for _ in range(self.layers)]
        b.vd = [torch.zeros(B, self.H, NP, self.hd, dtype=dt, device=dev) for _ in range(self.layers)]
        b.logits = torch.empty(B, self.n_codes, dtype=dt, device=dev)
        b.crossb = torch.zeros(B, self.layers * D, dtype=dt, device=dev) if self.cross_w is not None else None
        b.feedback = torch.empty(B, self.fb_table.shape[1], dtype=self.fb_table.dtype, device=dev)
        return b

    def run(self, b, uniforms=True, trace=None):
        """The frame body over buffer set `b` (inputs b.slots, b.h, b.codes[:, 0]); fills b.codes and b.feedback.
        uniforms=True draws b.u from the slots' Philox streams; False uses b.u as the caller filled it.
        trace: a list that receives a copy of each level's head logits (eager runs only)."""
        B, D, H, hd = b.B, self.D, self.H, self.hd
        if b.crossb is not None:
            ops.copy_rows(self.cross_const.view(self.max_slots + 1, self.layers * D), b.crossb, src_idx=b.slots)
        if uniforms:
            ops.philox_uniforms(self.row_seed, self.row_ctr, b.slots, b.u, 1)
        ops.linear(b.h, self.in_proj, b.tmp)
        ops.add_rows(b.tmp, self.level0, b.prefix[:, 0])
        ops.copy_rows(self.embed[0], b.prefix[:, 1], src_idx=b.codes[:, 0])
        scale = hd ** -0.5
        inv_temp = 1.0 / self.temp
        previous = None
        normed = False  # the previous sampler already wrote this level's input row and its norm
        for level in range(1, N_LEVELS):
            group = self.group_of_level[level]
            n = level + 1
            incremental = group == previous
            T, p0 = (1, level) if incremental else (n, 0)
            layers = self.trunks[group]
            R = B * T
            first = layers[0].n1
            if not normed:
                ops.add_norm(b.prefix[:, p0:p0 + T], None, None, b.xw[:R], b.yw[:R], first.w, first.b, first.eps, T,
                             first.kind)
            for li, L in enumerate(layers):
                last_only = li == self.layers - 1 and not incremental
                tq0 = T - 1 if last_only else 0
                Tq = T - tq0
                R2 = B * Tq
                ops.linear(b.yw[:R], L.qkv, b.qkv[:R])
                ops.depth_attn(b.qkv[:R], b.kd[li], b.vd[li], b.att[:R2], B, T, p0, tq0, H, hd, scale, True)
                ops.linear(b.att[:R2], L.o, b.a[:R2])
                x_res = b.xw[:R].view(B, T, D)[:, tq0:]
                ops.add_norm(x_res, b.a[:R2], None, b.xw2[:R2], b.y2[:R2], L.n2.w, L.n2.b, L.n2.eps, Tq, L.n2.kind)
                F = L.ffn
                ops.linear_act(b.y2[:R2], L.wg, L.wu, L.act, b.ffn_act[:R2, :F])
                ops.linear(b.ffn_act[:R2, :F], L.w2, b.f[:R2])
                nxt = layers[li + 1].n1 if li + 1 < self.layers else self.final_norm
                c = b.crossb[:, li * D:(li + 1) * D] if b.crossb is not None else None
                ops.add_norm(b.xw2[:R2], b.f[:R2], c, b.xw[:R2], b.yw[:R2], nxt.w, nxt.b, nxt.eps, Tq, nxt.kind)
                R, T, p0 = R2, Tq, p0 + tq0
            ops.linear(b.yw[:B], self.heads[level - 1], b.logits)
            if trace is not None:
                trace.append(b.logits.clone())
            u = b.u[:, level - 1]
            if n < N_LEVELS:
                # the sampler gathers the drawn code's prefix row; when the next level continues this group
                # incrementally, its input is that one row, so the sampler also writes its norm
                normed = self.group_of_level[n] == group
                if normed:
                    ops.topk_sample_embed(b.logits, u, inv_temp, self.top_k, self.greedy, b.codes[:, level],
                                          self.embed[level], b.prefix[:, n], x_out=b.xw[:B], y=b.yw[:B], w=first.w,
                                          b=first.b, eps=first.eps, kind=first.kind)
                else:
                    ops.topk_sample_embed(b.logits, u, inv_temp, self.top_k, self.greedy, b.codes[:, level],
                                          self.embed[level], b.prefix[:, n])
            else:
                ops.topk_sample(b.logits, u, inv_temp, self.top_k, self.greedy, b.codes[:, level])
            previous = group
        ops.ctr_add(self.row_ctr, b.slots)
        ops.feedback(self.fb_table, b.codes, b.feedback, self.fb_norm.w, self.fb_norm.eps, self.feedback_scale,
                     N_LEVELS, self.n_codes)
        return b.codes, b.feedback

    def _compute(self, slots_idx, h, cb0):
        """Eager frame body (the reference tests call `_fn(slots_idx, h, cb0)`, maya3/tests/test_depth_fused.py:35)."""
        B = h.shape[0]
        b = self.make_buffers(B)
        b.slots.copy_(slots_idx)
        b.h.copy_(h)
        b.codes[:, 0].copy_(cb0)
        codes, fb = self.run(b)
        return codes.long(), fb

    # ---------------------------------------------------------------- graphs
    @torch.inference_mode()
    def _capture(self, bucket):
        if bucket in self.graphs:
            return self.graphs[bucket]
        s = {'bufs': self.make_buffers(bucket), 'last_slots': None}
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        ctr = self.row_ctr.clone()
        with torch.cuda.stream(stream):
            for _ in range(3):
                self.run(s['bufs'])  # all-dummy rows: only the dummy slot's counter moves
        torch.cuda.current_stream().wait_stream(stream)
        self.row_ctr.copy_(ctr)
        if self.pool is None:
            self.pool = torch.cuda.graph_pool_handle()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.pool, stream=stream):
            self.run(s['bufs'])
        s['graph'] = graph
        self.graphs[bucket] = s
        return s

    def warmup(self, batch_buckets=None):
        # largest first so smaller captures reuse the shared pool's blocks
        for bucket in sorted(set(batch_buckets or self.batch_buckets), reverse=True):
            self._capture(int(bucket))

    def bucket_for(self, batch):
        for bucket in self.batch_buckets:
            if bucket >= batch:
                return bucket
        raise ValueError(f'batch {batch} exceeds the largest bucket {self.batch_buckets[-1]}')

    @torch.inference_mode()
    def __call__(self, slots, h, cb0):
        B = len(slots)
        if h.shape[0] != B or cb0.shape[0] != B:
            raise ValueError('slots, h and cb0 must have the same batch size')
        s = self._capture(self.bucket_for(B))
        b = s['bufs']
        key = tuple(slots)
        if key != s['last_slots']:
            if any(not 0 <= slot < self.max_slots for slot in key):
                raise IndexError(f'slot outside 0..{self.max_slots - 1}')
            padded = list(key) + [self.max_slots] * (b.slots.shape[0] - B)
            b.slots.copy_(torch.tensor(padded, dtype=torch.long))
            s['last_slots'] = key
        b.h[:B].copy_(h)
        b.codes[:B, 0].copy_(cb0)
        s['graph'].replay()
        return b.codes[:B].long(), b.feedback[:B].clone()
