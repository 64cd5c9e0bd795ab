"""Tensor-level wrappers over the m3x C ABI (include/m3x.h).

Each wrapper checks devices, dtypes and shapes (ValueError, like the reference surfaces), passes raw pointers,
element strides and torch's current HIP stream, and raises RuntimeError on a non-zero status. Nothing here
allocates on the device except where a function documents that it returns a new tensor; graph-captured code
passes preallocated outputs and workspaces.
"""
from __future__ import annotations

import ctypes


import numpy as np

import torch

from ._lib import check, lib

NORM_LAYER, NORM_RMS = 0, 1
ACT_NONE, ACT_SWIGLU, ACT_GELU = -1, 0, 1
_DT = {torch.bfloat16: 0, torch.float16: 1}
_DT_ANY = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dt(t: torch.Tensor) -> int:
    if t.dtype not in _DT:
        raise ValueError(f"m3x kernels take bfloat16 or float16 tensors, got {t.dtype}")
    return _DT[t.dtype]


def _dt3(t: torch.Tensor) -> int:
    """dtype code for the entry points that also have an fp32 instance (projections, depth norms / attention /
    sampler / feedback, and the codec's kernels)."""
    if t.dtype not in _DT_ANY:
        raise ValueError(f"m3x kernels take bfloat16, float16 or float32 tensors, got {t.dtype}")
    return _DT_ANY[t.dtype]


def _dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("m3x kernels take device tensors")


def _rows2d(t: torch.Tensor, name: str):
    if t.dim() != 2 or t.stride(-1) != 1:
        raise ValueError(f"{name} must be a 2-D tensor with a contiguous last dimension, got {tuple(t.shape)}")


def _need(t: torch.Tensor, dtype, name: str):
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")


def _index(slots=None, pos=None):
    """The ABI's index types: slot tensors are int64, position tensors int32 (a wrong width would be read as
    out-of-range indices on the device)."""
    if slots is not None:
        _need(slots, torch.long, "slots")
    if pos is not None:
        _need(pos, torch.int32, "pos")


# ---------------------------------------------------------------- backbone step
def positions(lengths, slots, offset, pos):
    _dev(lengths, slots, offset, pos)
    _need(lengths, torch.long, "lengths")
    _need(slots, torch.long, "slots")
    _need(pos, torch.int32, "pos")
    if offset is not None:
        _need(offset, torch.long, "offset")
    check(lib().m3x_positions(_p(lengths), _p(slots), _p(offset), _p(pos), slots.numel(), _stream()), "positions")


def lengths_add(lengths, slots, real):
    _dev(lengths, slots, real)
    _index(slots=slots)
    check(lib().m3x_lengths_add(_p(lengths), _p(slots), _p(real), slots.numel(), _stream()), "lengths_add")


def add_rms(h, a, w, eps, h_out=None, y=None):
    """h_out = bf16(h + a); y = RMSNorm(h_out) (a None: y = RMSNorm(h), h_out unused). Returns (h_out, y)."""
    _dev(h, a, w, h_out, y)
    _rows2d(h, "h")
    if h.dtype != torch.bfloat16:
        raise ValueError("fused add+norm kernel is bf16-only")
    rows, n = h.shape
    if y is None:
        y = torch.empty_like(h)
    if a is not None:
        _rows2d(a, "a")
        if a.shape != h.shape:
            raise ValueError(f"add_rms: a {tuple(a.shape)} != h {tuple(h.shape)}")
        if h_out is None:
            h_out = torch.empty_like(h)
    check(lib().m3x_add_rms(_p(h), h.stride(0), _p(a), 0 if a is None else a.stride(0), _p(h_out),
                            0 if h_out is None else h_out.stride(0), _p(y), y.stride(0), _p(w), float(eps), rows, n,
                            _stream()), "add_rms")
    return h_out, y


def qk_norm_rope_cache(qkv, q_out, k_cache, v_cache, slots, pos, cos, sin, wq, wk, eps, heads, kv_heads):
    _dev(qkv, q_out, k_cache, v_cache, slots, pos, cos, sin, wq, wk)
    _index(slots=slots, pos=pos)
    D = k_cache.shape[-1]
    rows = qkv.shape[0]
    if qkv.shape[1] != (heads + 2 * kv_heads) * D:
        raise ValueError(f"qkv width {qkv.shape[1]} != (heads + 2*kv_heads)*head_dim")
    check(lib().m3x_qk_norm_rope_cache(
        _p(qkv), qkv.stride(0), _p(q_out), q_out.stride(0), q_out.stride(1), _p(k_cache), _p(v_cache),
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), _p(slots), _p(pos), _p(cos), _p(sin), cos.stride(0),
        _p(wq), _p(wk), float(eps), rows, heads, kv_heads, D, k_cache.shape[2], _stream()), "qk_norm_rope_cache")


def linear_qk_rope(x, w, qkv, q_out, k_cache, v_cache, slots, pos, cos, sin, wq, wk, eps, heads, kv_heads,
                   part=None, eps_in=0.0):
    """The q|k|v projection (x @ W.T, or with part given linear_normed's RMSNorm-folded product, W from fold_norm)
    followed by qk_norm_rope_cache on its output, in one launch when the row count's plan holds whole heads per
    workgroup (then qkv is not written), else two through qkv. Same bits as linear / linear_normed +
    qk_norm_rope_cache."""
    M, K, qkv = _lin_args(x, w, qkv, w.N)
    _dev(q_out, k_cache, v_cache, slots, pos, cos, sin, wq, wk, part)
    _index(slots=slots, pos=pos)
    D = k_cache.shape[-1]
    if w.N != (heads + 2 * kv_heads) * D:
        raise ValueError(f"linear_qk_rope: weight rows {w.N} != (heads + 2*kv_heads)*head_dim")
    if x.dtype != torch.bfloat16:
        raise ValueError("linear_qk_rope: bf16 only")
    if part is not None and (part.dtype != torch.float32 or not part.is_contiguous()
                             or part.numel() < tile_stats_elems(M, K)):
        raise ValueError("linear_qk_rope: part must hold the tile statistics of x")
    check(lib().m3x_linear_qk_rope(
        _p(x), x.stride(0), _p(part), float(eps_in), _p(w.data), _p(qkv), qkv.stride(0), _p(q_out), q_out.stride(0),
        q_out.stride(1), _p(k_cache), _p(v_cache), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), _p(slots),
        _p(pos), _p(cos), _p(sin), cos.stride(0), _p(wq), _p(wk), float(eps), M, K, heads, kv_heads, D,
        k_cache.shape[2], _stream()), "linear_qk_rope")


def decode_attn_workspace(rows, kv_heads, max_ctx, chunk) -> int:
    return int(lib().m3x_decode_attn_workspace(rows, kv_heads, max_ctx, chunk))


def decode_attn(q, k_cache, v_cache, out, slots, pos, scale, max_ctx, chunk, workspace, heads, kv_heads,
                items=None):
    """q, out: [rows, heads, D] (any row/head strides, contiguous D); caches [slots, kv_heads, cap, D].
    items (int32, optional): the step's work items (attn_items with attn_item_bins bins); the rows of an inline
    prefill then share one pass over their slot's keys per min(16, 2 * (16 // (heads // kv_heads))) rows."""
    _dev(q, k_cache, v_cache, out, slots, pos, workspace, items)
    _index(slots=slots, pos=pos)
    rows = q.shape[0]
    if items is not None:
        bins = attn_item_bins(rows, kv_heads, max_ctx, chunk)
        if items.dtype != torch.int32 or not items.is_contiguous() or items.numel() < 2 + bins:
            raise ValueError(f"decode_attn: items must be contiguous int32 with {bins} bins (attn_items)")
    ws = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib().m3x_decode_attn(
        _p(q), q.stride(0), q.stride(1), _p(k_cache), _p(v_cache), k_cache.stride(0), k_cache.stride(1),
        k_cache.stride(2), k_cache.shape[2], _p(out), out.stride(0), out.stride(1), _p(slots), _p(pos), _p(items),
        float(scale), rows, heads, kv_heads, k_cache.shape[-1], int(max_ctx), int(chunk), _p(workspace), ws,
        _stream()), "decode_attn")


def attn_item_bins(rows, kv_heads, max_ctx, chunk) -> int:
    return int(lib().m3x_decode_attn_item_bins(rows, kv_heads, max_ctx, chunk))


def attn_items(runs, heads, kv_heads, bins, chunk):
    """Work items of decode_attn for rows laid out as runs: (first row, rows, first position) per run, a decode
    row being a run of one row and an inline prefill of T tokens a run of T rows at consecutive positions of one
    slot. Each run is cut into blocks of up to min(16, 2 * (16 // (heads // kv_heads))) rows and each block's keys into splits of
    `chunk` keys; an item is one split of one block. The items are dealt into `bins` bins (attn_item_bins) longest
    processing time first: each goes to the least loaded bin, its cost its keys plus a fixed 64. Returns int32
    [bins, start[0..bins], codes bin by bin], code = 2048 * first_row + 32 * split + rows. Built on the host by the
    library (m3x_decode_attn_items)."""
    r = np.ascontiguousarray(np.asarray(runs, dtype=np.int32).reshape(-1, 3))
    qb = max(1, 16 // (heads // kv_heads))
    n, p0 = r[:, 1].astype(np.int64), r[:, 2].astype(np.int64)
    bound = int((-(-n // qb) * (-(-(p0 + n) // chunk))).sum())  # blocks x the run's most splits
    out = np.empty(2 + bins + bound, dtype=np.int32)
    cnt = lib().m3x_decode_attn_items(r.ctypes.data, r.shape[0], heads, kv_heads, bins, chunk, out.ctypes.data,
                                      out.size)
    if cnt < 0:
        raise ValueError(f"attn_items: m3x_decode_attn_items returned {cnt}")
    return out[:cnt]


class PackedWeight:
    """An [N, K] weight (bf16, fp16 or fp32) in MFMA fragment order (see m3x_pack_weight): `data` holds
    ceil(N/16)*16*K elements."""
    __slots__ = ("data", "N", "K")

    def __init__(self, data, N, K):
        self.data, self.N, self.K = data, N, K

    @property
    def dtype(self):
        return self.data.dtype

    @property
    def device(self):
        return self.data.device

    def rows(self, start, stop):
        """Rows [start, stop) as their own packed weight (start % 16 == 0); shares storage."""
        if start % 16 or not 0 <= start < stop <= self.N:
            raise ValueError(f"rows({start}, {stop}) of a packed [{self.N}, {self.K}] weight")
        return PackedWeight(self.data[start * self.K:-(-stop // 16) * 16 * self.K], stop - start, self.K)


def pack_weight(w):
    """Pack w [N, K] (row stride % 8 == 0, K % 32 == 0) into fragment order; one launch on the current stream."""
    _dev(w)
    _rows2d(w, "w")
    N, K = w.shape
    n = int(lib().m3x_packed_weight_elems(N, K))
    if n < 0:
        raise ValueError(f"pack_weight: K={K} must be a multiple of 32")
    out = torch.empty(n, dtype=w.dtype, device=w.device)
    check(lib().m3x_pack_weight(_p(w), w.stride(0), N, K, _p(out), _dt3(w), _stream()), "pack_weight")
    return PackedWeight(out, N, K)


def _lin_args(x, w, y, N):
    if not isinstance(w, PackedWeight):
        raise TypeError("linear: the weight must be packed with ops.pack_weight")
    _dev(x, w.data, y)
    _rows2d(x, "x")
    M, K = x.shape
    if w.K != K or w.dtype != x.dtype:
        raise ValueError(f"linear: x {tuple(x.shape)} {x.dtype} vs packed w [{w.N}, {w.K}] {w.dtype}")
    if y is None:
        y = torch.empty(M, N, dtype=x.dtype, device=x.device)
    _rows2d(y, "y")
    if y.shape != (M, N) or y.dtype != x.dtype:
        raise ValueError(f"linear: y {tuple(y.shape)} {y.dtype}, expected {(M, N)} {x.dtype}")
    return M, K, y


def linear(x, w, y=None):
    """y = x @ W.T with x [M, K] and W [N, K] packed by pack_weight (same dtype); returns y [M, N]."""
    M, K, y = _lin_args(x, w, y, w.N)
    check(lib().m3x_linear(_p(x), x.stride(0), _p(w.data), _p(y), y.stride(0), M, w.N, K, _dt3(x), _stream()),
          "linear")
    return y


def linear_act(x, w_gate, w_up, kind, y=None):
    """SWIGLU: y = bf16(silu(x @ Wg.T)) * (x @ Wu.T); GELU: y = gelu(x @ Wg.T) (w_up None); weights packed."""
    I = w_gate.N
    M, K, y = _lin_args(x, w_gate, y, I)
    if kind == ACT_SWIGLU:
        if not isinstance(w_up, PackedWeight) or (w_up.N, w_up.K) != (w_gate.N, w_gate.K):
            raise ValueError("linear_act: w_up must be a packed weight of w_gate's shape")
        _dev(w_up.data)
    check(lib().m3x_linear_act(_p(x), x.stride(0), _p(w_gate.data), _p(w_up.data if kind == ACT_SWIGLU else None),
                               _p(y), y.stride(0), M, I, K, kind, _dt3(x), _stream()), "linear_act")
    return y


def tile_stats_elems(rows, n):
    """float32 elements of the tile statistics linear_resid writes for `rows` rows of width n (2 per 16 columns)."""
    return rows * (n // 16) * 2


def linear_resid(x, w, h, h_out, part, kind, c=None, tc=1):
    """h_out = dt(h + dt(x @ W.T)) [then dt(h_out + c[m // tc])], and the 16-column tile statistics of h_out into
    `part` (float32, >= tile_stats_elems(M, N)) for a following norm of `kind` (NORM_RMS or NORM_LAYER).
    h may be a strided row view (row stride h.stride(0)); h_out may be h."""
    M, K, h_out = _lin_args(x, w, h_out, w.N)
    _dev(h, c, part)
    for t, name in ((h, "h"), (c, "c")):
        if t is not None and (t.dim() != 2 or t.stride(-1) != 1 or t.dtype != x.dtype or t.shape[1] < w.N):
            raise ValueError(f"linear_resid: {name} must be a row-strided [rows, >= {w.N}] {x.dtype} view")
    if h.shape[0] < M or (c is not None and c.shape[0] * tc < M):
        raise ValueError("linear_resid: h / c have too few rows")
    if part.dtype != torch.float32 or not part.is_contiguous() or part.numel() < tile_stats_elems(M, w.N):
        raise ValueError("linear_resid: part must be a contiguous float32 buffer of tile_stats_elems(M, N)")
    check(lib().m3x_linear_resid(_p(x), x.stride(0), _p(w.data), _p(h), h.stride(0), _p(c),
                                 0 if c is None else c.stride(0), tc, _p(h_out), h_out.stride(0), _p(part), M, w.N, K,
                                 kind, _dt(x), _stream()), "linear_resid")
    return h_out


def fold_norm(w, nw, nb=None):
    """Load-time preparation of a projection w [N, K] that consumes normed rows (linear_normed): the norm's weight
    nw [K] (and LayerNorm bias nb [K]) folded in. Returns (packed dt(w * nw), u, v): for LayerNorm the fp32 column
    vectors u[n] = sum_k dt(w * nw)[n, k] and v[n] = sum_k nb[k] w[n, k]; None for RMSNorm. A joined gate|up weight
    [2I, K] gives u, v in the same [gate | up] order that linear_normed takes with ACT_SWIGLU."""
    _dev(w, nw, nb)
    if w.dim() != 2 or nw.numel() != w.shape[1] or (nb is not None and nb.numel() != w.shape[1]):
        raise ValueError("fold_norm: w [N, K] with nw (and nb) of K elements")
    wf = (w.float() * nw.float()[None]).to(w.dtype).contiguous()
    packed = pack_weight(wf)
    if nb is None:
        return packed, None, None
    return packed, wf.float().sum(1).contiguous(), (w.float() @ nb.float()).contiguous()


def linear_normed(x, part, eps, kind, w_gate, w_up=None, act_kind=ACT_NONE, u=None, v=None, y=None):
    """y = act(norm(x) @ W.T) for rows x of width 1024 whose tile statistics linear_resid left in `part`, with the
    weights prepared by fold_norm (u, v: its column vectors, LayerNorm only; [2N] for ACT_SWIGLU). act_kind
    ACT_NONE (w_up None), ACT_SWIGLU (w_up) or ACT_GELU."""
    M, K, y = _lin_args(x, w_gate, y, w_gate.N)
    _dev(part, u, v)
    if act_kind == ACT_SWIGLU and (not isinstance(w_up, PackedWeight) or (w_up.N, w_up.K) != (w_gate.N, w_gate.K)):
        raise ValueError("linear_normed: w_up must be a packed weight of w_gate's shape")
    if part.dtype != torch.float32 or not part.is_contiguous() or part.numel() < tile_stats_elems(M, K):
        raise ValueError("linear_normed: part must hold the tile statistics of x")
    ncol = w_gate.N * (2 if act_kind == ACT_SWIGLU else 1)
    if kind == NORM_LAYER:
        for t, name in ((u, "u"), (v, "v")):
            if t is None or t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != ncol:
                raise ValueError(f"linear_normed: LayerNorm needs fold_norm's {name} ({ncol} float32)")
    check(lib().m3x_linear_normed(_p(x), x.stride(0), _p(part), _p(u), _p(v), eps, kind, _p(w_gate.data),
                                  _p(w_up.data if act_kind == ACT_SWIGLU else None), _p(y), y.stride(0), M,
                                  w_gate.N, K, act_kind, _dt(x), _stream()), "linear_normed")
    return y


def act(inp, out, kind):
    """SWIGLU: out[:, :I] = bf16(silu(g))*u for inp = [g | u]; GELU: out = gelu(inp[:, :I])."""
    _dev(inp, out)
    _rows2d(inp, "inp")
    _rows2d(out, "out")
    check(lib().m3x_act(_p(inp), inp.stride(0), _p(out), out.stride(0), inp.shape[0], out.shape[1], kind, _dt(inp),
                        _stream()), "act")
    return out


# ---------------------------------------------------------------- depth step
def _bt_strides(t, T):
    """(row-of-b stride, row-of-t stride) of a [B, T, N] view or a contiguous [B*T, N] tensor."""
    if t.dim() == 3:
        if t.stride(-1) != 1:
            raise ValueError("last dimension must be contiguous")
        return t.stride(0), t.stride(1)
    _rows2d(t, "x")
    return T * t.stride(0), t.stride(0)


def add_norm(x, a, c, x_out, y, w, b, eps, T, kind):
    """x, a: [B, T, N] views or [B*T, N]; c: [B, N] (row stride may be 0) or None; x_out/y contiguous [B*T, N]."""
    _dev(x, a, c, x_out, y, w, b)
    n = x.shape[-1]
    rows = y.shape[0]
    sxb, sxt = _bt_strides(x, T)
    sab, sat = _bt_strides(a, T) if a is not None else (0, 0)
    check(lib().m3x_add_norm(_p(x), sxb, sxt, _p(a), sab, sat, _p(c), 0 if c is None else c.stride(0), _p(x_out),
                             _p(y), _p(w), _p(b), float(eps), rows, T, n, kind, _dt3(y), _stream()), "add_norm")


def add_rows(x, bias, out):
    """out = x + bias (bias [N] broadcast, or [rows, N])."""
    _dev(x, bias, out)
    ldb = 0 if bias.dim() == 1 else bias.stride(0)
    check(lib().m3x_add_rows(_p(x), x.stride(0), _p(bias), ldb, _p(out), out.stride(0), x.shape[0], x.shape[-1],
                             _dt3(x), _stream()), "add_rows")


def depth_attn(qkv, kd, vd, out, B, T, p0, tq0, heads, head_dim, scale, write_kv=True):
    _dev(qkv, kd, vd, out)
    sqb, sqt = _bt_strides(qkv, T)
    sob, sot = _bt_strides(out, T - tq0)
    check(lib().m3x_depth_attn(_p(qkv), sqb, sqt, _p(kd), _p(vd), _p(out), sob, sot, B, T, p0, tq0, heads, head_dim,
                               kd.shape[2], float(scale), int(write_kv), _dt3(qkv), _stream()), "depth_attn")


def topk_sample(logits, u, inv_temp, top_k, greedy, out, out_i64=False):
    """logits [B, V] 16-bit; u [B] view (any stride) or None for greedy; out [B] view (int32/int64)."""
    _dev(logits, u, out)
    _rows2d(logits, "logits")
    B, V = logits.shape
    check(lib().m3x_topk_sample(_p(logits), logits.stride(0), V, _p(u), 0 if u is None else u.stride(0),
                                float(inv_temp), int(top_k), int(greedy), _p(out), out.stride(0), int(out_i64), B,
                                _dt3(logits), _stream()), "topk_sample")


def topk_sample_embed(logits, u, inv_temp, top_k, greedy, out, table, prefix, x_out=None, y=None, w=None, b=None,
                      eps=0.0, kind=NORM_RMS, out_i64=False):
    """topk_sample, then prefix[r] = table[code_r]; with y given also x_out[r] = table[code_r] and
    y[r] = norm(table[code_r]) (the add_norm arithmetic with no addend). prefix: [B, n] view (any row stride);
    x_out, y: contiguous [B, n]."""
    _dev(logits, u, out, table, prefix, x_out, y, w, b)
    _rows2d(logits, "logits")
    _rows2d(table, "table")
    B, V = logits.shape
    n = table.shape[-1]
    if prefix.shape[-1] != n or prefix.shape[0] != B:
        raise ValueError("topk_sample_embed: prefix must be [B, n]")
    if table.shape[0] < V:
        raise ValueError(f"topk_sample_embed: table has {table.shape[0]} rows for {V} codes")
    if any(t is not None and t.dtype != logits.dtype for t in (table, prefix, x_out, y, w, b)):
        raise ValueError("topk_sample_embed: logits, table, prefix, x_out, y, w and b share one dtype")
    for t, name in ((x_out, "x_out"), (y, "y")):
        if t is not None and (not t.is_contiguous() or tuple(t.shape) != (B, n)):
            raise ValueError(f"topk_sample_embed: {name} must be contiguous [B, n]")
    check(lib().m3x_topk_sample_embed(
        _p(logits), logits.stride(0), V, _p(u), 0 if u is None else u.stride(0), float(inv_temp), int(top_k),
        int(greedy), _p(out), out.stride(0), int(out_i64), B, _p(table), table.stride(0), table.shape[0], _p(prefix),
        prefix.stride(0), _p(x_out), _p(y), _p(w), _p(b), float(eps), int(kind), n, _dt3(logits), _stream()),
        "topk_sample_embed")


def cb0_sample(logits, aeos, slots, u, temp_t=None, temp=1.0, topk_t=None, top_k=50, aeos_bias=None, rep_t=None,
               hist_t=None, frames_t=None, min_t=None, hazard_t=None, ctr_t=None, cb0_out=None, cb0_i32=None,
               stop_out=None, topp_t=None, top_p=1.0):
    _dev(logits, slots, u, temp_t, topk_t, aeos_bias, rep_t, hist_t, frames_t, min_t, hazard_t, ctr_t, cb0_out,
         cb0_i32, stop_out, topp_t)
    _index(slots=slots)
    if topp_t is not None and topp_t.dtype != torch.float32:
        raise ValueError("topp_t must be float32")
    _rows2d(logits, "logits")
    if logits.dtype != torch.bfloat16:
        raise ValueError("cb0 logits must be bfloat16")
    B, V = logits.shape
    check(lib().m3x_cb0_sample(
        _p(logits), logits.stride(0), V, int(aeos), _p(slots), _p(u), u.stride(0), _p(temp_t), float(temp),
        _p(topk_t), int(top_k), _p(topp_t), float(top_p), _p(aeos_bias), _p(rep_t), _p(hist_t), 0 if hist_t is None else hist_t.shape[1],
        _p(frames_t), _p(min_t), _p(hazard_t), _p(ctr_t), _p(cb0_out), _p(cb0_i32),
        0 if cb0_i32 is None else cb0_i32.stride(0), _p(stop_out), B, _stream()), "cb0_sample")


def philox_uniforms(seeds, ctrs, slots, out, level0):
    """out [B, nlevels] (row stride free) = Philox uniforms for levels level0.. of each slot's stream."""
    _dev(seeds, ctrs, slots, out)
    _index(slots=slots)
    _need(seeds, torch.int32, "seeds")
    _need(ctrs, torch.int32, "ctrs")
    _need(out, torch.float32, "out")
    check(lib().m3x_philox_uniforms(_p(seeds), _p(ctrs), _p(slots), _p(out), out.stride(0), int(level0),
                                    out.shape[1], slots.numel(), _stream()), "philox_uniforms")


def philox_exponential(seeds, ctrs, out, level):
    """out [B, V] = Exp(1) noise of each row's (seed, counter) stream at `level`."""
    _dev(seeds, ctrs, out)
    _need(seeds, torch.int32, "seeds")
    _need(ctrs, torch.int32, "ctrs")
    _need(out, torch.float32, "out")
    check(lib().m3x_philox_exponential(_p(seeds), _p(ctrs), _p(out), out.stride(0), int(level), out.shape[1],
                                       out.shape[0], _stream()), "philox_exponential")


def philox_block(counter, key, out):
    check(lib().m3x_philox_block(_p(counter), _p(key), _p(out), _stream()), "philox_block")


def ctr_add(ctr, slots):
    _dev(ctr, slots)
    _index(slots=slots)
    check(lib().m3x_ctr_add(_p(ctr), _p(slots), slots.numel(), _stream()), "ctr_add")


def feedback(table, codes, out, w, eps, scale, n_q, n_codes):
    _dev(table, codes, out, w)
    _need(codes, torch.int32, "codes")
    check(lib().m3x_feedback(_p(table), _p(codes), codes.stride(0), _p(out), out.stride(0), _p(w), float(eps),
                             float(scale), out.shape[0], out.shape[1], int(n_q), int(n_codes), _dt3(table),
                             _stream()), "feedback")


def copy_rows(src, dst, src_idx=None, src_off=0, dst_idx=None, rows=None):
    """dst[dst_idx[r] or r] = src[src_idx[r] + src_off or r] for r < rows (rows of 16-bit elements with
    width % 8 == 0, or of fp32 elements with width % 4 == 0, moved as pairs of 16-bit halves)."""
    _dev(src, dst, src_idx, dst_idx)
    if src.dtype != dst.dtype or src.element_size() not in (2, 4):
        raise ValueError(f"copy_rows: {src.dtype} -> {dst.dtype}")
    w = src.element_size() // 2  # 16-bit units per element
    n = src.shape[-1] * w
    if dst.shape[-1] * w != n:
        raise ValueError("copy_rows: row widths differ")
    if rows is None:
        rows = src_idx.numel() if src_idx is not None else (dst_idx.numel() if dst_idx is not None else src.shape[0])
    idx_i32 = 0
    ld_idx = 1
    if src_idx is not None:
        if src_idx.dtype == torch.int32:
            idx_i32 = 1
        elif src_idx.dtype != torch.long:
            raise ValueError("indices must be int32 or int64")
        ld_idx = src_idx.stride(0)
    if dst_idx is not None:
        _need(dst_idx, torch.long, "dst_idx")
    check(lib().m3x_copy_rows(_p(src), src.stride(-2) * w, _p(src_idx), int(src_off), src.shape[-2], _p(dst),
                              dst.stride(-2) * w, _p(dst_idx), int(rows), n, idx_i32, ld_idx, _stream()), "copy_rows")


def cast_rows(src, dst):
    """dst = src converted to dst's dtype (bf16 / fp16 / fp32 rows with a contiguous last dimension)."""
    _dev(src, dst)
    _rows2d(src, "src")
    _rows2d(dst, "dst")
    if src.shape != dst.shape or src.dtype not in _DT_ANY or dst.dtype not in _DT_ANY:
        raise ValueError(f"cast_rows: {tuple(src.shape)} {src.dtype} -> {tuple(dst.shape)} {dst.dtype}")
    check(lib().m3x_cast_rows(_p(src), src.stride(0), _DT_ANY[src.dtype], _p(dst), dst.stride(0),
                              _DT_ANY[dst.dtype], src.shape[0], src.shape[1], _stream()), "cast_rows")
    return dst


def code_ring_write(codes, ring, head, B):
    _dev(codes, ring, head)
    check(lib().m3x_code_ring_write(_p(codes), codes.stride(0), _p(ring), _p(head), ring.shape[0], ring.shape[1],
                                    ring.shape[2], int(B), _stream()), "code_ring_write")


# ---------------------------------------------------------------- the depth frame as one persistent run
class DepthRunArgs(ctypes.Structure):
    """Mirror of M3xDepthRun (include/m3x.h); its size is checked against the library's."""
    _P4 = ctypes.c_void_p * 4
    _fields_ = [(n, ctypes.c_int) for n in ("B", "L0", "L1", "layers", "H", "hd", "F", "V", "act", "norm_kind",
                                            "dtype", "nwg")] + [
        ("inv_temp", ctypes.c_float), ("top_k", ctypes.c_int), ("greedy", ctypes.c_int),
        ("eps1", ctypes.c_float * 4), ("eps2", ctypes.c_float * 4), ("eps_f", ctypes.c_float),
        ("n1w", _P4), ("n1b", _P4), ("n2w", _P4), ("n2b", _P4), ("fw", ctypes.c_void_p), ("fb", ctypes.c_void_p),
        ("wqkv", _P4), ("wo", _P4), ("wg", _P4), ("wu", _P4), ("wd", _P4), ("heads", ctypes.c_void_p * 31),
        ("embed", ctypes.c_void_p), ("cross", ctypes.c_void_p), ("ld_cross", ctypes.c_long),
        ("prefix", ctypes.c_void_p), ("ld_prefix", ctypes.c_long), ("codes", ctypes.c_void_p),
        ("ld_codes", ctypes.c_long), ("u", ctypes.c_void_p), ("ld_u", ctypes.c_long), ("kd", _P4), ("vd", _P4),
        ("kv_sb", ctypes.c_long), ("kv_sh", ctypes.c_long), ("xchg", ctypes.c_void_p), ("sync", ctypes.c_void_p),
        ("logits_out", ctypes.c_void_p), ("prof", ctypes.c_void_p), ("probe", ctypes.c_int),
        ("spin_limit", ctypes.c_uint)]


def depth_run_xchg_bytes() -> int:
    return int(lib().m3x_depth_run_xchg_bytes())


def depth_run(args: DepthRunArgs):
    """Launch a persistent depth run on the current stream (args built by FastDepth)."""
    if ctypes.sizeof(DepthRunArgs) != int(lib().m3x_depth_run_args_bytes()):
        raise RuntimeError("DepthRunArgs does not match the library's M3xDepthRun: rebuild the library")
    check(lib().m3x_depth_run(ctypes.byref(args), _stream()), "depth_run")


def depth_run_void(sync, codes, B, L0, L1):
    """After a run (stream order): codes[:B, L0:L1] = -1 when the run's error word sync[2] is set."""
    _dev(sync, codes)
    check(lib().m3x_depth_run_void(_p(sync), _p(codes), codes.stride(0), B, L0, L1, _stream()), "depth_run_void")


# ---------------------------------------------------------------- one-row backbone run (serve/fast_backbone.py)
class BackboneLayer(ctypes.Structure):
    """Mirror of M3xBackboneLayer (include/m3x.h); rows of a device table, one per layer."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("wqkv", "wo", "wg", "wu", "wd", "wq", "wk", "kc", "vc")]


class BackboneRunArgs(ctypes.Structure):
    """Mirror of M3xBackboneRun (include/m3x.h); its size is checked against the library's."""
    _fields_ = [("layer", ctypes.c_void_p)] + [(n, ctypes.c_int) for n in ("layers", "cap", "nwg", "probe")] + [
        ("spin_limit", ctypes.c_uint), ("eps", ctypes.c_float), ("scale", ctypes.c_float),
        ("x", ctypes.c_void_p), ("h_out", ctypes.c_void_p), ("slots", ctypes.c_void_p), ("pos", ctypes.c_void_p),
        ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p), ("s_cos", ctypes.c_long), ("w_in0", ctypes.c_void_p),
        ("sk_s", ctypes.c_long), ("sk_h", ctypes.c_long), ("sk_t", ctypes.c_long), ("xchg", ctypes.c_void_p),
        ("sync", ctypes.c_void_p), ("prof", ctypes.c_void_p), ("w_fin", ctypes.c_void_p), ("y_out", ctypes.c_void_p),
        ("lengths", ctypes.c_void_p), ("real", ctypes.c_void_p)]


def backbone_run_xchg_bytes() -> int:
    return int(lib().m3x_backbone_run_xchg_bytes())


def backbone_layer_table(layers, device):
    """The device table of M3xBackboneLayer rows for `layers` (lists of BackboneLayer)."""
    if ctypes.sizeof(BackboneLayer) != int(lib().m3x_backbone_run_layer_bytes()):
        raise RuntimeError("BackboneLayer does not match the library's M3xBackboneLayer: rebuild the library")
    raw = (BackboneLayer * len(layers))(*layers)
    host = torch.frombuffer(bytearray(bytes(raw)), dtype=torch.int64).clone()
    return host.to(device)


def backbone_run(args: BackboneRunArgs):
    """Launch a one-row backbone run on the current stream (args built by StaticBackbone)."""
    if ctypes.sizeof(BackboneRunArgs) != int(lib().m3x_backbone_run_args_bytes()):
        raise RuntimeError("BackboneRunArgs does not match the library's M3xBackboneRun: rebuild the library")
    check(lib().m3x_backbone_run(ctypes.byref(args), _stream()), "backbone_run")


# ---------------------------------------------------------------- Mimi decode (serve/fast_codec.py)
def rvq_decode(codes, tables, out):
    """out[b] = [table_0[codes[b, 0]] | sum over q >= 1 of table_q[codes[b, q]]]; tables [nq, n_codes, dim]."""
    _dev(codes, tables, out)
    nq, n_codes, dim = tables.shape
    check(lib().m3x_rvq_decode(_p(codes), codes.stride(0), _p(tables), _p(out), out.stride(0), codes.shape[0], nq,
                               n_codes, dim, _dt3(tables), _stream()), "rvq_decode")


def dwconvt(x, w, tail, slots, out, k, s):
    """Depthwise transposed conv of one frame per seat with per-slot overlap tails; out [B * s, C]."""
    _dev(x, w, tail, slots, out)
    _index(slots=slots)
    check(lib().m3x_dwconvt(_p(x), x.stride(0), _p(w), _p(tail), tail.stride(0), _p(slots), _p(out), x.shape[0],
                            x.shape[1], k, s, _dt3(x), _stream()), "dwconvt")


def conv_gather(x, state, slots, cols, B, T, C, k, dil, use_elu, chunk):
    """GEMM rows of a causal conv with per-slot input history (state [slots, pad * C] or None when pad = 0);
    cols None only advances the history."""
    _dev(x, state, slots, cols)
    _index(slots=slots)
    check(lib().m3x_conv_gather(_p(x), x.stride(0), _p(state), 0 if state is None else state.stride(0), _p(slots),
                                _p(cols), 0 if cols is None else cols.stride(0), B, T, C, k, dil, int(use_elu), chunk,
                                _dt3(x), _stream()),
          "conv_gather")


def rows_op(g, out, bias=None, scale=None, res=None, use_elu=False):
    """out = act(res + scale * (g + bias)), act = ELU when use_elu; rows of g and out [rows, C]."""
    _dev(g, out, bias, scale, res)
    check(lib().m3x_rows_op(_p(g), g.stride(0), _p(bias), _p(scale), _p(res), 0 if res is None else res.stride(0),
                            _p(out), out.stride(0), out.shape[0], out.shape[1], int(use_elu), _dt3(g), _stream()),
          "rows_op")


def conv_gemm(x, w, y, bias=None, res=None, use_elu=False, gather=None):
    """y = act(res + (x @ W.T + bias)) for a packed W with N in {16, 32, 64, 128}; act = ELU when use_elu.
    gather = (state, slots, T, C, dil, pre_elu): x is the conv's input [B * T, C] and the product reads
    m3x_conv_gather's rows in place (the history is not advanced here)."""
    if not isinstance(w, PackedWeight):
        raise TypeError("conv_gemm: the weight must be packed with ops.pack_weight")
    st, slots, T, C, dil, pre = gather if gather is not None else (None, None, 0, 0, 1, False)
    _dev(x, w.data, y, bias, res, st, slots)
    _index(slots=slots)
    check(lib().m3x_conv_gemm(_p(x), x.stride(0), _p(w.data), _p(bias), _p(res), 0 if res is None else res.stride(0),
                              _p(y), y.stride(0), y.shape[0], w.N, w.K, int(use_elu), _p(st),
                              0 if st is None else st.stride(0), _p(slots), T, C, dil, int(pre), _dt3(x), _stream()),
          "conv_gemm")
    return y


def resid_ln(h, a, scale, w, b, eps, y):
    """h = h + scale * a in place (16-bit rounding once), then y = LayerNorm(h) with (w, b, eps); rows of 512."""
    _dev(h, a, scale, w, b, y)
    check(lib().m3x_resid_ln(_p(h), h.stride(0), _p(a), a.stride(0), _p(scale), _p(w), _p(b), _p(y), y.stride(0),
                             float(eps), h.shape[0], h.shape[1], _dt3(h), _stream()), "resid_ln")


def convt_overlap(cols, tail, slots, bias, out, B, Tin, C, k, s, chunk):
    """Overlap-add of a transposed conv's GEMM columns with per-slot tails; out [B * Tin * s, C]."""
    _dev(cols, tail, slots, bias, out)
    _index(slots=slots)
    check(lib().m3x_convt_overlap(_p(cols), cols.stride(0), _p(tail), tail.stride(0), _p(slots), _p(bias), _p(out),
                                  out.stride(0), B, Tin, C, k, s, chunk, _dt3(cols), _stream()), "convt_overlap")


def ring_attn(qkv, kring, vring, key_pos, tokens, slots, inv_freq, rope_scale, out, B, T, H, ring, window):
    """Sliding-window attention of T new tokens per seat over per-slot rings of post-RoPE keys."""
    _dev(qkv, kring, vring, key_pos, tokens, slots, inv_freq, out)
    _index(slots=slots)
    check(lib().m3x_ring_attn(_p(qkv), qkv.stride(0), _p(kring), _p(vring), _p(key_pos), _p(tokens), _p(slots),
                              _p(inv_freq), float(rope_scale), _p(out), out.stride(0), B, T, H, 64, ring, window,
                              _dt3(qkv), _stream()), "ring_attn")


def advance_tokens(tokens, slots, B, T, dummy):
    _dev(tokens, slots)
    _index(slots=slots)
    check(lib().m3x_advance_tokens(_p(tokens), _p(slots), B, T, dummy, _stream()), "advance_tokens")


def final_conv(x, state, slots, w, bias, pcm, B, T, C, k, chunk):
    """fp32 PCM of the last causal conv (C -> 1 channel) with per-slot history; pcm [B, >= T] float32."""
    _dev(x, state, slots, w, pcm)
    _index(slots=slots)
    check(lib().m3x_final_conv(_p(x), x.stride(0), _p(state), 0 if state is None else state.stride(0), _p(slots),
                               _p(w), float(bias), _p(pcm), pcm.stride(0), B, T, C, k, chunk, _dt3(x), _stream()),
          "final_conv")
