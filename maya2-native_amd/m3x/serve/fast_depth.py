"""Whole-frame depth decoder on m3x gfx950 kernels, one hipGraph per batch bucket.

Drop-in for serve/fast_depth.py (FastDepth, :32-257). The surface is the reference's: constructor arguments,
`set_speaker`, `warmup`, `bucket_for`, `__call__(slots, h, cb0) -> (codes [B, 32] int64, feedback [B, d])`,
`_fn(slots_idx, h, cb0)` for direct calls (maya3/tests/test_depth_fused.py:35), and the per-slot sampling streams
`row_seed` / `row_ctr` the engine writes (maya3/engine.py:436-437).

One frame, for every seat (the fused body, serve/fast_depth.py:143-203):
  prefix[0] = in_proj(h) + level_emb[0]; prefix[1] = embed[0][cb0]
  level L = 1..31, trunk = the weight group of L:
    the first level of a group recomputes positions 0..L causally (the last layer only at position L); a level
    that continues its group runs position L alone against the group's cached K/V;
    per layer: y = n1(x); qkv; attention; x += o -> n2; FFN; x += f (+ speaker constant) -> next norm
    code_L = top-k sample(heads[L-1](norm(x_L)) / temp, u_L); prefix[L+1] = embed[L][code_L]
  feedback = audio_in.norm(sum_l audio_in.table[code_l + 2048 l] / sqrt(32))
u_L is one uniform per (seat, level) from the slot's Philox stream (row_seed, row_ctr). The trunk may be the
reference's DepthV2 (LayerNorm, GELU, 16 x 64 heads, 11 weight groups, speaker cross constant: tts/model/
depth_v2.py) or a SwiGLU/RMSNorm trunk shared by every level (m3x.synth.swiglu_depth).
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import torch

from .. import ops
from .._lib import lib
from ..staging import Buckets, ErrorWatch, RowTable, capture, check_slots

N_LEVELS = 32
REFERENCE_GROUP_OF_LEVEL = [None] + list(range(8)) + [8] * 8 + [9] * 8 + [10] * 7


def _dev_copy(t, dtype, device):
    return t.detach().to(device=device, dtype=dtype).contiguous()


def _packed(mod, dtype, device):
    """A Linear-like module's weight in MFMA fragment order for the projection kernels."""
    return ops.pack_weight(_dev_copy(mod.weight, dtype, device))


def _norm_spec(mod, dtype, device):
    """(kind, weight, bias, eps) of a LayerNorm-like (has a bias) or RMSNorm-like module; an RMSNorm without eps
    uses finfo(dtype).eps, as torch's nn.RMSNorm(eps=None) does."""
    bias = getattr(mod, 'bias', None)
    eps = getattr(mod, 'eps', None)
    if bias is not None:
        return SimpleNamespace(kind=ops.NORM_LAYER, w=_dev_copy(mod.weight, dtype, device),
                               b=_dev_copy(bias, dtype, device), eps=1e-5 if eps is None else float(eps))
    return SimpleNamespace(kind=ops.NORM_RMS, w=_dev_copy(mod.weight, dtype, device), b=None,
                           eps=float(torch.finfo(dtype).eps if eps is None else eps))


def _folded(mod, norm, dtype, device):
    """(packed, u, v) of a projection consuming rows normed by `norm`, the norm folded in (ops.fold_norm)."""
    return ops.fold_norm(_dev_copy(mod.weight, dtype, device), norm.w, norm.b)


def _block(blk, dtype, device, fold):
    """A trunk block's norms and packed weights. fold: also the copies with the norms folded in for the fused-norm
    launch path (fq: q|k|v after n1; fg, fu: gate and up (or f1) after n2, with their column vectors)."""
    L = SimpleNamespace(n1=_norm_spec(blk.n1, dtype, device), n2=_norm_spec(blk.n2, dtype, device),
                        qkv=_packed(blk.qkv, dtype, device), o=_packed(blk.o, dtype, device))
    if hasattr(blk, 'gate_up'):
        gu = _packed(blk.gate_up, dtype, device)
        L.act, L.ffn = ops.ACT_SWIGLU, gu.N // 2
        L.wg, L.wu, L.w2 = gu.rows(0, L.ffn), gu.rows(L.ffn, gu.N), _packed(blk.down, dtype, device)
    else:
        L.act, L.wg, L.wu, L.w2 = ops.ACT_GELU, _packed(blk.f1, dtype, device), None, _packed(blk.f2, dtype, device)
        L.ffn = L.wg.N
    if fold:
        L.fq = _folded(blk.qkv, L.n1, dtype, device)
        if L.act == ops.ACT_SWIGLU:
            p, u, v = _folded(blk.gate_up, L.n2, dtype, device)
            L.fg, L.fu, L.fuv = p.rows(0, L.ffn), p.rows(L.ffn, p.N), (u, v)
        else:
            p, u, v = _folded(blk.f1, L.n2, dtype, device)
            L.fg, L.fu, L.fuv = p, None, (u, v)
    return L


class FastDepth:
    def __init__(self, model, max_slots, dtype=torch.bfloat16, temp=0.7, top_k=64,
                 batch_buckets=(1, 2, 4, 8, 16, 24, 32, 48, 64, 80, 96), seed=1234, greedy=False, compile=False,
                 fused=False):
        if model.depth.n_q != N_LEVELS:
            raise ValueError('FastDepth expects the 32-codebook depth stack')
        if dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise ValueError(f'FastDepth computes in bfloat16, float16 or float32, got {dtype}')
        lib()
        self.max_slots, self.dtype = int(max_slots), dtype
        self.temp, self.top_k, self.greedy, self.fused = float(temp), int(top_k), bool(greedy), bool(fused)
        self._buckets = Buckets(batch_buckets)
        self.batch_buckets = self._buckets.sizes
        with torch.inference_mode():
            self._load(model)
        dev = self.device
        rows = self.max_slots + 1  # row max_slots: the dummy slot that pads a batch
        self.cross_const = torch.zeros(rows, self.layers, self.D, device=dev, dtype=dtype)
        self.seed_t = torch.full((1,), int(seed) % (2 ** 31 - 1), device=dev, dtype=torch.int32)
        self.row_seed = torch.zeros(rows, device=dev, dtype=torch.int32)
        self.row_ctr = torch.zeros(rows, device=dev, dtype=torch.int32)
        self.per_row = True
        self.graphs = {}
        self.pool = None
        self._fn = self._compute
        # the persistent run of continuing levels (m3x_depth_run): its exchange area, epoch/error words, and the
        # workgroup count (one per CU)
        self.persistent = True
        # polling rounds before a persistent run's wait gives up (0: the kernel's default); a run whose wait gives
        # up sets the error word, and its codes come back as -1 (run_error, clear_run_error)
        self.spin_limit = 0
        self._run_xchg = torch.zeros(ops.depth_run_xchg_bytes() // 8, dtype=torch.int64, device=dev)
        self._run_sync = torch.zeros(4, dtype=torch.int32, device=dev)
        self._nwg = torch.cuda.get_device_properties(dev).multi_processor_count
        self._watch = ErrorWatch(self._run_sync, 'FastDepth: a persistent depth run')

    def _load(self, model):
        d, dt = model.depth, self.dtype
        self.device = dev = d.in_proj.weight.device
        if dev.type != 'cuda':
            raise ValueError('FastDepth runs on the GPU; the model is on ' + str(dev))
        self.n_codes = d.n_codes
        self.D = d.in_proj.weight.shape[0]
        self.H = int(getattr(d, 'n_heads', 16))
        self.hd = self.D // self.H
        self.group_of_level = list(getattr(d, 'group_of_level', REFERENCE_GROUP_OF_LEVEL))
        self.in_proj = _packed(d.in_proj, dt, dev)
        if hasattr(d, 'embed'):  # per-codebook input tables with the level embedding folded in
            self.embed, self.level0 = _dev_copy(d.embed, dt, dev), _dev_copy(d.level0, dt, dev)
        else:
            # the reference's factorised tables: position k+1 of the prefix reads
            # code_up(code_lo[code + k * n_codes]) + level_emb[k+1] (serve/fast_depth.py:48-51), folded here
            lo, up = _dev_copy(d.code_lo.weight, dt, dev), _dev_copy(d.code_up.weight, dt, dev)
            lvl = _dev_copy(d.level_emb.weight, dt, dev)
            self.embed = ((lo @ up.t()).view(N_LEVELS - 1, self.n_codes, self.D) + lvl[1:N_LEVELS, None]).contiguous()
            self.level0 = lvl[0].clone()
        # 16-bit trunks of width 1024 take the fused-norm launch path: the o and down projections add into the
        # residual and leave its tile statistics; the next q|k|v, gate|up (f1) and the codebook head carry the norm
        # folded into their weights and apply each row's scale (and shift) in their epilogue
        self.fused_norms = dt != torch.float32 and self.D == 1024
        self.trunks = [[_block(blk, dt, dev, self.fused_norms) for blk in blocks] for blocks in d.groups]
        self.layers = len(self.trunks[0])
        self.final_norm = _norm_spec(d.norm, dt, dev)
        self.heads = [_packed(h, dt, dev) for h in d.heads]  # 31 x [n_codes, D]
        # the heads with the final norm folded in (fused-norm launch path)
        self.fheads = [_folded(h, self.final_norm, dt, dev) for h in d.heads] if self.fused_norms else None
        self.cross = getattr(d, 'cross', None)
        self.cross_w = None if self.cross is None else [(_packed(c.kv, dt, dev), _packed(c.o, dt, dev))
                                                       for c in self.cross]
        self.audio_in = model.audio_in  # shared and read-only, in the engine's dtype
        table = model.audio_in.table.weight
        if table.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            table = table.detach().to(torch.bfloat16).contiguous()  # the serving dtype of the feedback table
        self.fb_table = table
        self.fb_norm = _norm_spec(model.audio_in.norm, table.dtype, dev)
        self.feedback_scale = math.sqrt(N_LEVELS)
        torch.cuda.current_stream(dev).synchronize()  # packing ran on the current stream

    @torch.inference_mode()
    def set_speaker(self, slot, mem, ref_mask):
        """Per-slot speaker constant: the cross-attention of a single reference token has softmax weight 1, so
        each layer's cross output is o(v(mem) * keep) whatever the query (serve/fast_depth.py:73-82)."""
        if mem.ndim != 3 or mem.shape[:2] != (1, 1) or tuple(ref_mask.shape) != (1, 1):
            raise ValueError(f'FastDepth serves exactly one reference per slot; got mem {tuple(mem.shape)}')
        check_slots([slot], self.max_slots)
        if self.cross_w is None:
            return  # a trunk without speaker cross-attention: the constant stays zero
        v_in = mem.to(self.device, self.dtype).reshape(1, self.D).contiguous()
        keep = ref_mask.to(self.device, self.dtype).reshape(1, 1)
        for layer, (wkv, wo) in enumerate(self.cross_w):
            v = (ops.linear(v_in, wkv)[:, self.D:] * keep).contiguous()
            self.cross_const[slot, layer].copy_(ops.linear(v, wo)[0])

    # ---------------------------------------------------------------- frame body
    def make_buffers(self, B, h=None, codes=None):
        """Static buffers of one batch bucket. `h`/`codes` may be shared with a caller (the frame step); b.table's
        `slot` column (b.slots) holds the seats' slots, padded with the dummy slot."""
        dev, dt, D = self.device, self.dtype, self.D
        b = SimpleNamespace(B=B)
        b.table = RowTable(('slot',), B, dev, pad=dict(slot=self.max_slots))
        b.slots = b.table['slot']
        b.h = h if h is not None else torch.zeros(B, self.in_proj.K, dtype=dt, device=dev)
        b.codes = codes if codes is not None else torch.zeros(B, N_LEVELS, dtype=torch.int32, device=dev)
        b.u = torch.zeros(B, N_LEVELS - 1, dtype=torch.float32, device=dev)
        b.prefix = torch.zeros(B, N_LEVELS, D, dtype=dt, device=dev)
        b.tmp = torch.empty(B, D, dtype=dt, device=dev)
        R = B * N_LEVELS  # the most rows a level can hold (a group start at the last level)
        for name in ('xw', 'xw2', 'yw', 'y2', 'att', 'a', 'f'):
            setattr(b, name, torch.empty(R, D, dtype=dt, device=dev))
        b.qkv = torch.empty(R, 3 * D, dtype=dt, device=dev)
        b.part = torch.empty(ops.tile_stats_elems(R, D), dtype=torch.float32, device=dev)
        b.ffn_act = torch.empty(R, max(L.ffn for t in self.trunks for L in t), dtype=dt, device=dev)
        b.kd = [torch.zeros(B, self.H, N_LEVELS, self.hd, dtype=dt, device=dev) for _ in range(self.layers)]
        b.vd = [torch.zeros(B, self.H, N_LEVELS, self.hd, dtype=dt, device=dev) for _ in range(self.layers)]
        b.logits = torch.empty(B, self.n_codes, dtype=dt, device=dev)
        b.crossb = None if self.cross_w is None else torch.zeros(B, self.layers * D, dtype=dt, device=dev)
        b.feedback = torch.empty(B, self.fb_table.shape[1], dtype=self.fb_table.dtype, device=dev)
        return b

    def _trunk(self, b, layers, T, p0):
        """The trunk over T positions from p0 per seat (rows b.yw: the first layer's normed input, b.xw: the
        residual). On return b.xw[:B] holds the last position's residual; with fused norms (self.fused_norms)
        b.part holds its tile statistics for the final norm (applied by the head projection), else b.yw[:B] holds
        the final-normed row."""
        B, D = b.B, self.D
        R = B * T
        incremental = T == 1
        fused = self.fused_norms
        for li, L in enumerate(layers):
            # at a group start the last layer is evaluated at the last position only
            tq0 = T - 1 if (li == self.layers - 1 and not incremental) else 0
            Tq = T - tq0
            R2 = B * Tq
            if li > 0 and fused:  # the layer's input norm, from the residual's tile statistics
                w, u, v = L.fq
                ops.linear_normed(b.xw[:R], b.part, L.n1.eps, L.n1.kind, w, u=u, v=v, y=b.qkv[:R])
            else:
                ops.linear(b.yw[:R], L.qkv, b.qkv[:R])
            ops.depth_attn(b.qkv[:R], b.kd[li], b.vd[li], b.att[:R2], B, T, p0, tq0, self.H, self.hd,
                           self.hd ** -0.5, True)
            nxt = layers[li + 1].n1 if li + 1 < self.layers else self.final_norm
            c = None if b.crossb is None else b.crossb[:, li * D:(li + 1) * D]
            if fused:
                # residual rows of the attended positions: all rows, or each seat's last one (row stride T * D)
                res = b.xw[:R] if tq0 == 0 else b.xw[:R].view(B, T * D)[:, tq0 * D:]
                ops.linear_resid(b.att[:R2], L.o, res, b.xw2[:R2], b.part, L.n2.kind)
                ops.linear_normed(b.xw2[:R2], b.part, L.n2.eps, L.n2.kind, L.fg, L.fu, L.act, u=L.fuv[0], v=L.fuv[1],
                                  y=b.ffn_act[:R2, :L.ffn])
                ops.linear_resid(b.ffn_act[:R2, :L.ffn], L.w2, b.xw2[:R2], b.xw[:R2], b.part, nxt.kind, c=c, tc=Tq)
            else:
                ops.linear(b.att[:R2], L.o, b.a[:R2])
                ops.add_norm(b.xw[:R].view(B, T, D)[:, tq0:], b.a[:R2], None, b.xw2[:R2], b.y2[:R2], L.n2.w,
                             L.n2.b, L.n2.eps, Tq, L.n2.kind)
                ops.linear_act(b.y2[:R2], L.wg, L.wu, L.act, b.ffn_act[:R2, :L.ffn])
                ops.linear(b.ffn_act[:R2, :L.ffn], L.w2, b.f[:R2])
                ops.add_norm(b.xw2[:R2], b.f[:R2], c, b.xw[:R2], b.yw[:R2], nxt.w, nxt.b, nxt.eps, Tq, nxt.kind)
            R, T, p0 = R2, Tq, p0 + tq0

    def _head(self, b, level):
        """Logits of `level` from the trunk's last rows: the final norm and the codebook head."""
        fn = self.final_norm
        if self.fused_norms:
            w, u, v = self.fheads[level - 1]
            ops.linear_normed(b.xw[:b.B], b.part, fn.eps, fn.kind, w, u=u, v=v, y=b.logits)
        else:
            ops.linear(b.yw[:b.B], self.heads[level - 1], b.logits)

    def run(self, b, uniforms=True, trace=None):
        """The frame body over buffer set `b` (inputs b.slots, b.h, b.codes[:, 0]); fills b.codes and b.feedback.
        uniforms=True draws b.u from the slots' Philox streams; False uses b.u as the caller filled it.
        trace: a list that receives a copy of each level's head logits (eager runs only)."""
        B = b.B
        if b.crossb is not None:
            ops.copy_rows(self.cross_const.view(self.max_slots + 1, self.layers * self.D), b.crossb, src_idx=b.slots)
        if uniforms:
            ops.philox_uniforms(self.row_seed, self.row_ctr, b.slots, b.u, 1)
        ops.linear(b.h, self.in_proj, b.tmp)
        ops.add_rows(b.tmp, self.level0, b.prefix[:, 0])
        ops.copy_rows(self.embed[0], b.prefix[:, 1], src_idx=b.codes[:, 0])
        inv_temp = 1.0 / self.temp
        staged = False  # the previous sampler already wrote this level's input row and its norm
        level = 1
        while level < N_LEVELS:
            group = self.group_of_level[level]
            continues = level > 1 and self.group_of_level[level - 1] == group
            if continues and self._persistent_ok(B, group):
                # every level that continues this group, in one persistent kernel
                end = level
                while end < N_LEVELS and self.group_of_level[end] == group:
                    end += 1
                a = self._run_args(b, level, end, group)
                logits = None
                if trace is not None:
                    logits = torch.empty(N_LEVELS - 1, B, self.n_codes, dtype=self.dtype, device=self.device)
                    a.logits_out = logits.data_ptr()
                ops.depth_run(a)
                ops.depth_run_void(self._run_sync, b.codes, B, level, end)
                a.logits_out = None
                if trace is not None:
                    trace.extend(logits[lv - 1].clone() for lv in range(level, end))
                level, staged = end, False
                continue
            T, p0 = (1, level) if continues else (level + 1, 0)
            layers = self.trunks[group]
            n1 = layers[0].n1
            if not staged:
                ops.add_norm(b.prefix[:, p0:p0 + T], None, None, b.xw[:B * T], b.yw[:B * T], n1.w, n1.b, n1.eps, T,
                             n1.kind)
            self._trunk(b, layers, T, p0)
            self._head(b, level)
            if trace is not None:
                trace.append(b.logits.clone())
            u = b.u[:, level - 1]
            nxt = level + 1
            if nxt == N_LEVELS:
                ops.topk_sample(b.logits, u, inv_temp, self.top_k, self.greedy, b.codes[:, level])
                break
            # the sampler writes the drawn code's prefix row; when the next level continues this group its input
            # is exactly that one row, so the sampler also writes the row's first-layer norm
            staged = self.group_of_level[nxt] == group and not self._persistent_ok(B, group)
            norm_out = dict(x_out=b.xw[:B], y=b.yw[:B], w=n1.w, b=n1.b, eps=n1.eps, kind=n1.kind) if staged else {}
            ops.topk_sample_embed(b.logits, u, inv_temp, self.top_k, self.greedy, b.codes[:, level],
                                  self.embed[level], b.prefix[:, nxt], **norm_out)
            level = nxt
        ops.ctr_add(self.row_ctr, b.slots)
        ops.feedback(self.fb_table, b.codes, b.feedback, self.fb_norm.w, self.fb_norm.eps, self.feedback_scale,
                     N_LEVELS, self.n_codes)
        return b.codes, b.feedback

    # ---------------------------------------------------------------- persistent run
    # The kernel takes up to 16 seats; past 4 its handovers (every residual workgroup reads the whole rows of each
    # step's output) cost more than the launch path's kernels on MI355X (graph-timed 31-codebook frames: 2.70 vs
    # 2.74 ms at 4 seats, 2.90 vs 2.87 at 5, 3.04 vs 2.78 at 8), so larger batches take the launch path.
    PERSISTENT_SEATS = 4
    # a handover poll with more 16-byte chunks per thread than this first waits on one chunk per thread (0: every
    # poll does; measured best at 1-4 seats and within 1.5 % of the best at 8 and 16 on MI355X)
    POLL_PROBE = 0

    def _persistent_ok(self, B, group):
        """Whether levels continuing `group` run as one persistent kernel for B seats: at most PERSISTENT_SEATS and
        one (seat, head) pair per residual workgroup, one workgroup per CU on a 256-CU part, the trunk geometries the
        kernel implements (width 1024, 2048 codes, SwiGLU 2816 with 128-wide heads or GELU 3072 with 64-wide
        heads; RMSNorm with SwiGLU, LayerNorm with GELU) in bf16 or fp16."""
        if (not self.persistent or self.dtype == torch.float32 or B > self.PERSISTENT_SEATS or B * self.H > 192
                or self._nwg != 256):
            return False
        layers = self.trunks[group]
        kinds = {L.n1.kind for L in layers} | {L.n2.kind for L in layers} | {self.final_norm.kind}
        geo = {(L.act, L.ffn) for L in layers}
        swiglu = layers[0].act == ops.ACT_SWIGLU
        return (self.D == 1024 and self.n_codes == 2048 and len(layers) <= 4 and len(geo) == 1
                and geo.pop() in ((ops.ACT_SWIGLU, 2816), (ops.ACT_GELU, 3072))
                and kinds == {ops.NORM_RMS if swiglu else ops.NORM_LAYER} and self.hd == (128 if swiglu else 64))

    def _run_args(self, b, L0, L1, group):
        """The persistent run's arguments for buffer set b and levels L0 .. L1-1 (built once; the pointers are
        those of b's static buffers). The sampling settings and the spin limit are refreshed on every call, so a
        run follows the current temp / top_k / greedy like the launch path's levels of the same frame."""
        runs = b.__dict__.setdefault('runs', {})
        key = (L0, L1, group)
        a = runs.get(key)
        if a is None:
            a = runs[key] = self._new_run_args(b, L0, L1, group)
        a.inv_temp, a.top_k, a.greedy = 1.0 / self.temp, self.top_k, int(self.greedy)
        a.spin_limit = int(self.spin_limit)
        return a

    def _new_run_args(self, b, L0, L1, group):
        layers = self.trunks[group]
        a = ops.DepthRunArgs()
        a.B, a.L0, a.L1, a.layers, a.H, a.hd = b.B, L0, L1, len(layers), self.H, self.hd
        a.F, a.V, a.act, a.norm_kind = layers[0].ffn, self.n_codes, layers[0].act, layers[0].n1.kind
        a.dtype, a.nwg, a.probe = ops._DT[self.dtype], self._nwg, self.POLL_PROBE
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        for l, L in enumerate(layers):
            a.eps1[l], a.eps2[l] = L.n1.eps, L.n2.eps
            a.n1w[l], a.n1b[l], a.n2w[l], a.n2b[l] = p(L.n1.w), p(L.n1.b), p(L.n2.w), p(L.n2.b)
            a.wqkv[l], a.wo[l], a.wg[l], a.wd[l] = p(L.qkv.data), p(L.o.data), p(L.wg.data), p(L.w2.data)
            a.wu[l] = p(L.wu.data) if L.wu is not None else None
            a.kd[l], a.vd[l] = p(b.kd[l]), p(b.vd[l])
        a.eps_f, a.fw, a.fb = self.final_norm.eps, p(self.final_norm.w), p(self.final_norm.b)
        for i, hw in enumerate(self.heads):
            a.heads[i] = p(hw.data)
        a.embed = p(self.embed)
        if b.crossb is not None:
            a.cross, a.ld_cross = p(b.crossb), b.crossb.stride(0)
        a.prefix, a.ld_prefix = p(b.prefix), b.prefix.stride(0)
        a.codes, a.ld_codes = p(b.codes), b.codes.stride(0)
        a.u, a.ld_u = p(b.u), b.u.stride(0)
        a.kv_sb, a.kv_sh = b.kd[0].stride(0), b.kd[0].stride(1)
        a.xchg, a.sync = p(self._run_xchg), p(self._run_sync)
        return a

    def run_error(self):
        """True when a persistent run since construction (or the last clear) lost a step's input (its bounded waits
        ran out): that run's codes came back as -1 and the frame is void. Synchronises with the device."""
        return bool(self._run_sync[2].item())

    @torch.inference_mode()
    def clear_run_error(self):
        """Reset the error word (stream-ordered), e.g. after the caller has failed the frame's requests."""
        self._run_sync[2].zero_()
        self._watch.evt = None

    def _compute(self, slots_idx, h, cb0):
        """Eager frame body over fresh buffers (the reference's tests call `_fn(slots_idx, h, cb0)`)."""
        b = self.make_buffers(h.shape[0])
        b.slots.copy_(slots_idx)
        b.h.copy_(h)
        b.codes[:, 0].copy_(cb0)
        self._watch.raise_if_set()
        codes, fb = self.run(b)
        if b.__dict__.get('runs'):
            self._watch.after()
        return codes.long(), fb

    # ---------------------------------------------------------------- graphs
    @torch.inference_mode()
    def _graph(self, bucket):
        g = self.graphs.get(bucket)
        if g is None:
            bufs = self.make_buffers(bucket)
            if self.pool is None:
                self.pool = torch.cuda.graph_pool_handle()
            # warm-up and capture run all-dummy rows; the dummy slot's frame counter is put back
            graph = capture(lambda: self.run(bufs), self.pool, warm=3, keep=(self.row_ctr,))
            g = self.graphs[bucket] = SimpleNamespace(bufs=bufs, graph=graph)
        return g

    def warmup(self, batch_buckets=None):
        for bucket in self._buckets.largest_first(batch_buckets):
            self._graph(bucket)

    def bucket_for(self, batch):
        return self._buckets.pick(batch)

    @torch.inference_mode()
    def __call__(self, slots, h, cb0):
        B = len(slots)
        if h.shape[0] != B or cb0.shape[0] != B:
            raise ValueError('slots, h and cb0 must have the same batch size')
        g = self._graph(self.bucket_for(B))
        key = tuple(slots)
        if key != g.bufs.table.key:
            check_slots(key, self.max_slots, distinct=False)
            g.bufs.table.stage(dict(slot=key), key=key)
        self._watch.raise_if_set()
        g.bufs.h[:B].copy_(h)
        g.bufs.codes[:B, 0].copy_(cb0)
        g.graph.replay()
        if g.bufs.__dict__.get('runs'):
            self._watch.after()
        return g.bufs.codes[:B].long(), g.bufs.feedback[:B].clone()
