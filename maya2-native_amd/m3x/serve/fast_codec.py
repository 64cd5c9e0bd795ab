"""Slot-based, static-state, graphed one-frame Mimi decoder on m3x kernels.

Drop-in for serve/fast_codec.py StaticMimi (:32-277): same constructor arguments (plus an optional compute dtype;
by default the Mimi module's own dtype, as the reference computes, :47-49, i.e. float32 for the engine's codec,
maya3/engine.py:165,201), the same public calls (decode, reset, warmup, state_bytes_per_slot, samples_per_frame) and the same streaming
semantics: causal-conv input history, transposed-conv overlap tails stored without bias, sliding-window attention
at absolute RoPE positions (a query at position p sees keys with p - window < key_pos <= p), one row of every
state per slot plus the dummy row max_slots that pads a batch to its bucket.

The frame runs as m3x launches on time-major activations [seat * T + t, channels] in the compute dtype (fp32, or
16-bit with fp32 accumulation): the codebook sum (m3x_rvq_decode) and its 1x1 projections as one GEMM, the depthwise upsample with
its tail (m3x_dwconvt), per transformer layer q|k|v GEMM, ring attention (m3x_ring_attn), o GEMM, layer-scaled
residual fused with the next LayerNorm (m3x_resid_ln), fc1 GEMM + GELU, fc2 GEMM, layer-scaled residual fused with
the next layer's LayerNorm; every SEANet conv as
history gather (m3x_conv_gather, ELU fused) + GEMM + bias/residual/ELU row op (m3x_rows_op), every transposed
conv as GEMM + overlap-add with tail (m3x_convt_overlap), and the last conv to fp32 PCM (m3x_final_conv).
"""
from __future__ import annotations

from types import SimpleNamespace

import torch

from .. import ops
from ..staging import Buckets, RowTable, capture, check_slots

NEVER = -(1 << 40)  # key_pos of an empty ring entry; outside every window


def _thin(n, k, rows):
    """Convs that go to the fused conv GEMM (m3x_conv_gemm): up to 128 outputs over a short reduction, or a
    reduction of up to 768 over at least 4096 rows (a wave walks K alone, so a long K over few rows is faster on
    the tiled GEMM + row op; measured on the 96-row and 21504-row cases of the 128-output conv)."""
    return n in (16, 32, 64, 128) and (k <= 384 or (k <= 768 and rows >= 4096))


def _chunk(rows, B, depth, target=2048):
    """Rows per workgroup of a stateful kernel over `rows` rows per seat: about `target` workgroups for the batch,
    at least the state's depth (only the first chunk of a seat may read its state)."""
    return max(depth, 1, -(-rows * B // target))


class StaticMimi:
    def __init__(self, mimi, max_slots, batch_buckets=(1, 2, 4, 8, 16, 24, 32, 48, 64, 80, 96), ring=256,
                 dtype=None, use_graphs=True):
        from transformers.models.mimi.modeling_mimi import MimiConv1d, MimiConvTranspose1d, MimiResnetBlock
        dtype = next(mimi.parameters()).dtype if dtype is None else dtype
        _check_codec(mimi, dtype)
        cfg = mimi.config
        self.m = mimi
        self.device, self.dtype = next(mimi.parameters()).device, dtype
        self.max_slots = self.dummy = int(max_slots)
        self._sizes = Buckets(batch_buckets)
        self.batch_buckets = self._sizes.sizes
        self.window, self.ring = int(cfg.sliding_window), int(ring)
        self.frame_tokens = int(mimi.upsample.conv.stride[0])
        self.codebooks = int(cfg.num_quantizers)
        if not self.window + self.frame_tokens <= self.ring <= 256 or self.frame_tokens > 2:
            raise ValueError("the KV ring must hold sliding_window + frame_tokens entries and at most 256, with at "
                             "most 2 tokens per frame")
        self.use_graphs = use_graphs
        rows = self.max_slots + 1
        dt = dtype

        def cvt(t):
            return t.detach().to(self.device, dt).contiguous()

        with torch.inference_mode():
            # quantizer: tables [semantic rows | acoustic rows], output projections side by side
            q = mimi.quantizer
            sem, ac = q.semantic_residual_vector_quantizer, q.acoustic_residual_vector_quantizer
            if q.num_semantic_quantizers != 1 or sem.output_proj is None or ac.output_proj is None:
                raise ValueError("expected one semantic codebook and 1x1 output projections")
            if sem.output_proj.bias is not None or ac.output_proj.bias is not None:
                raise ValueError("quantizer output projections carry no bias")
            self.tables = cvt(torch.stack([l.codebook.embed for l in list(sem.layers) + list(ac.layers)]))
            self.n_codes, self.cb_dim = self.tables.shape[1], self.tables.shape[2]
            self.w_quant = ops.pack_weight(cvt(torch.cat([sem.output_proj.weight[:, :, 0],
                                                          ac.output_proj.weight[:, :, 0]], 1)))
            self.hidden = self.w_quant.N
            up = mimi.upsample.conv
            if up.groups != up.in_channels or up.bias is not None or up.dilation != (1,):
                raise ValueError("expected a depthwise bias-free upsample")
            self.up_k, self.up_s = up.kernel_size[0], up.stride[0]
            self.w_up = cvt(up.weight[:, 0, :])
            # transformer
            self.layers = []
            for L in mimi.decoder_transformer.layers:
                a = L.self_attn
                if any(p.bias is not None for p in (a.q_proj, a.k_proj, a.v_proj, a.o_proj, L.mlp.fc1, L.mlp.fc2)):
                    raise ValueError("expected bias-free attention and MLP projections")
                if a.num_key_value_groups != 1 or a.head_dim != 64:
                    raise ValueError("ring attention takes head_dim 64 and as many kv heads as heads")
                self.layers.append(dict(
                    ln1=(cvt(L.input_layernorm.weight), cvt(L.input_layernorm.bias), L.input_layernorm.eps),
                    qkv=ops.pack_weight(cvt(torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]))),
                    o=ops.pack_weight(cvt(a.o_proj.weight)), s1=cvt(L.self_attn_layer_scale.scale),
                    ln2=(cvt(L.post_attention_layernorm.weight), cvt(L.post_attention_layernorm.bias),
                         L.post_attention_layernorm.eps),
                    fc1=ops.pack_weight(cvt(L.mlp.fc1.weight)), fc2=ops.pack_weight(cvt(L.mlp.fc2.weight)),
                    s2=cvt(L.mlp_layer_scale.scale)))
            self.heads = mimi.decoder_transformer.layers[0].self_attn.num_heads
            rot = mimi.decoder_transformer.rotary_emb
            self.inv_freq = rot.inv_freq.detach().float().to(self.device).contiguous()
            self.rope_scale = float(rot.attention_scaling)
            # SEANet decoder: conv, (ELU, conv-T, resnet)*, ELU, conv
            mods = list(mimi.decoder.layers)
            self.plan = []
            state_sizes = [("upsample", (self.up_k - self.up_s) * self.hidden)]
            first = mods[0]
            if not isinstance(first, MimiConv1d):
                raise ValueError("decoder must start with a conv")
            self.plan.append(self._conv_step("decoder.0", first, pre_elu=False, post_elu=True))
            state_sizes.append(("decoder.0", self.plan[-1]["pad"] * self.plan[-1]["cin"]))
            i = 1
            while i < len(mods) - 2:
                elu, ct, res = mods[i], mods[i + 1], mods[i + 2]
                if not (isinstance(elu, torch.nn.ELU) and elu.alpha == 1.0 and isinstance(ct, MimiConvTranspose1d)
                        and isinstance(res, MimiResnetBlock) and isinstance(res.shortcut, torch.nn.Identity)):
                    raise ValueError(f"unexpected decoder layers at {i}")
                c = ct.conv
                if ct.padding_left != 0 or c.dilation != (1,) or c.groups != 1 or ct.padding_right != c.kernel_size[0] - c.stride[0]:
                    raise ValueError("unsupported transpose-convolution geometry")
                k, s, cin, cout = c.kernel_size[0], c.stride[0], c.in_channels, c.out_channels
                self.plan.append(dict(kind="convt", key=f"decoder.{i + 1}", k=k, s=s, cin=cin, cout=cout,
                                      w=ops.pack_weight(cvt(c.weight.permute(2, 1, 0).reshape(k * cout, cin))),
                                      bias=None if c.bias is None else cvt(c.bias)))
                state_sizes.append((f"decoder.{i + 1}", (k - s) * cout))
                blk = list(res.block)
                if len(blk) != 4 or not all(isinstance(b, torch.nn.ELU) and b.alpha == 1.0 for b in blk[::2]):
                    raise ValueError("resnet block must be ELU, conv, ELU, conv")
                ca = self._conv_step(f"decoder.{i + 2}.block.1", blk[1], pre_elu=True, post_elu=True)
                cb = self._conv_step(f"decoder.{i + 2}.block.3", blk[3], pre_elu=False, post_elu=True)
                if cb["pad"] or cb["k"] != 1:
                    raise ValueError("the resnet block's second conv must be 1x1")
                self.plan.append(dict(kind="resnet", a=ca, b=cb))
                state_sizes.append((ca["key"], ca["pad"] * ca["cin"]))
                i += 3
            elu, last = mods[i], mods[i + 1] if i + 1 < len(mods) else None
            if not (isinstance(elu, torch.nn.ELU) and isinstance(last, MimiConv1d) and last.conv.out_channels == 1):
                raise ValueError("decoder must end with ELU and a conv to one channel")
            lc = last.conv
            k = lc.kernel_size[0]
            if lc.dilation != (1,) or lc.stride != (1,):
                raise ValueError("the last conv must have stride and dilation 1")
            self.final = dict(key=f"decoder.{i + 1}", k=k, cin=lc.in_channels,
                              w=lc.weight[0].t().contiguous().reshape(-1).float().to(self.device),
                              bias=float(lc.bias[0]) if lc.bias is not None else 0.0)
            state_sizes.append((self.final["key"], (k - 1) * lc.in_channels))
            # per-slot state: one flat row per slot, one column range per stateful layer ([frames][channels])
            total = sum(n for _, n in state_sizes)
            self.conv_flat = torch.zeros(rows, total, device=self.device, dtype=dt)
            self.state, off = {}, 0
            for key, n in state_sizes:
                self.state[key] = self.conv_flat[:, off:off + n] if n else None
                off += n
            self.kv = torch.zeros(len(self.layers), 2, rows, self.ring, self.heads, 64, device=self.device, dtype=dt)
            self.key_pos = torch.full((rows, self.ring), NEVER, device=self.device, dtype=torch.long)
            self.tokens = torch.zeros(rows, device=self.device, dtype=torch.long)
            # samples per frame: the SEANet's strides times the upsample's tokens
            t = self.frame_tokens
            for st in self.plan:
                if st["kind"] == "convt":
                    t *= st["s"]
            self.samples_per_frame = t
        self._pool = None
        self._buckets = {}

    def _conv_step(self, key, mod, pre_elu, post_elu):
        c = mod.conv
        if c.stride != (1,) or c.groups != 1:
            raise ValueError("Only stride-one dense decoder convolutions are supported")
        k, dil = c.kernel_size[0], c.dilation[0]
        return dict(kind="conv", key=key, k=k, dil=dil, pad=(k - 1) * dil, cin=c.in_channels, cout=c.out_channels,
                    pre_elu=pre_elu, post_elu=post_elu,
                    w=ops.pack_weight(c.weight.detach().to(self.device, self.dtype).permute(0, 2, 1)
                                      .reshape(c.out_channels, k * c.in_channels).contiguous()),
                    bias=None if c.bias is None else c.bias.detach().to(self.device, self.dtype).contiguous())

    def state_bytes_per_slot(self):
        """Bytes of one slot's streaming state, by kind (the engine sizes its seat count from these)."""
        per_row = lambda t: t.stride(0) * t.element_size()  # noqa: E731  (one row of a [rows, ...] tensor)
        ring = self.kv.shape[0] * self.kv.shape[1] * per_row(self.kv[0, 0])
        return {"conv": per_row(self.conv_flat), "attention_kv": ring,
                "attention_index": per_row(self.key_pos) + per_row(self.tokens)}

    # ---- buffers and the frame body ---------------------------------------------------------------
    def _buffers(self, B):
        T0, D = self.frame_tokens, self.hidden
        act = cols = inner = B * T0 * 2 * D
        t = T0
        for st in self.plan:
            if st["kind"] == "conv":
                cols = max(cols, B * t * st["k"] * st["cin"])
                act = max(act, B * t * st["cout"])
            elif st["kind"] == "convt":
                cols = max(cols, B * t * st["k"] * st["cout"])
                t *= st["s"]
                act = max(act, B * t * st["cout"])
            elif st["kind"] == "resnet":
                a = st["a"]
                cols = max(cols, B * t * a["k"] * a["cin"])
                inner = max(inner, B * t * a["cout"])
        z = lambda n: torch.zeros(n, device=self.device, dtype=self.dtype)  # noqa: E731
        R = B * T0
        return dict(e=z(B * 2 * self.cb_dim).view(B, 2 * self.cb_dim), u=z(B * D).view(B, D), h=z(R * D).view(R, D),
                    y=z(R * D).view(R, D), qkv=z(R * 3 * D).view(R, 3 * D), o=z(R * D).view(R, D),
                    a=z(R * D).view(R, D), f=z(R * 4 * D).view(R, 4 * D), X=z(act), G=z(act), I=z(inner),
                    C=z(cols), pcm=torch.zeros(B, self.samples_per_frame, device=self.device, dtype=torch.float32))

    def _forward(self, slots, codes, bf, B):
        T0, D, H = self.frame_tokens, self.hidden, self.heads
        R = B * T0
        ops.rvq_decode(codes, self.tables, bf["e"])
        ops.linear(bf["e"], self.w_quant, bf["u"])
        h, y = bf["h"], bf["y"]
        ops.dwconvt(bf["u"], self.w_up, self.state["upsample"], slots, h, self.up_k, self.up_s)
        w, b, eps = self.layers[0]["ln1"]
        ops.add_norm(h, None, None, None, y, w, b, eps, 1, ops.NORM_LAYER)
        for li, L in enumerate(self.layers):
            # y = input_layernorm(h) here
            ops.linear(y, L["qkv"], bf["qkv"])
            ops.ring_attn(bf["qkv"], self.kv[li, 0], self.kv[li, 1], self.key_pos, self.tokens, slots, self.inv_freq,
                          self.rope_scale, bf["o"], B, T0, H, self.ring, self.window)
            ops.linear(bf["o"], L["o"], bf["a"])
            w, b, eps = L["ln2"]
            ops.resid_ln(h, bf["a"], L["s1"], w, b, eps, y)  # h += s1 * attn; y = post_attention_layernorm(h)
            ops.linear_act(y, L["fc1"], None, ops.ACT_GELU, bf["f"])
            ops.linear(bf["f"], L["fc2"], bf["a"])
            if li + 1 < len(self.layers):
                w, b, eps = self.layers[li + 1]["ln1"]
                ops.resid_ln(h, bf["a"], L["s2"], w, b, eps, y)  # h += s2 * mlp; y = next input_layernorm(h)
            else:
                ops.rows_op(bf["a"], h, scale=L["s2"], res=h)
        ops.advance_tokens(self.tokens, slots, B, T0, self.dummy)
        # SEANet: x is the current activation [B * t, C]
        x, t = h, T0
        for st in self.plan:
            if st["kind"] == "conv":
                x = self._conv(st, x, slots, B, t, out=bf["X"])
            elif st["kind"] == "convt":
                cols = bf["C"][:B * t * st["k"] * st["cout"]].view(B * t, st["k"] * st["cout"])
                ops.linear(x, st["w"], cols)
                out = bf["X"][:B * t * st["s"] * st["cout"]].view(B * t * st["s"], st["cout"])
                ops.convt_overlap(cols, self.state[st["key"]], slots, st["bias"], out, B, t, st["cout"], st["k"],
                                  st["s"], _chunk(t * st["s"], B, st["k"] - st["s"]))
                x, t = out, t * st["s"]
            else:
                a, b = st["a"], st["b"]
                inner = self._conv(a, x, slots, B, t, out=bf["I"])
                if _thin(b["cout"], b["cin"], B * t):  # shortcut + block, then the next ELU
                    ops.conv_gemm(inner, b["w"], x, bias=b["bias"], res=x, use_elu=True)
                else:
                    g = bf["G"][:B * t * b["cout"]].view(B * t, b["cout"])
                    ops.linear(inner, b["w"], g)
                    ops.rows_op(g, x, bias=b["bias"], res=x, use_elu=True)
        f = self.final
        ops.final_conv(x, self.state[f["key"]], slots, f["w"], f["bias"], bf["pcm"], B, t, f["cin"], f["k"],
                       max(f["k"] - 1, 256))  # one thread per sample
        return bf["pcm"]

    def _conv(self, st, x, slots, B, t, out):
        """Causal conv of x [B * t, cin] -> act(out) [B * t, cout] (bias, ELU when post_elu)."""
        k, cin, cout = st["k"], st["cin"], st["cout"]
        if _thin(cout, k * cin, B * t) and (k > 1 or st["pre_elu"]):
            # the conv GEMM reads the input and the slot's history in place, then the history advances
            y = out[:B * t * cout].view(B * t, cout)
            ops.conv_gemm(x, st["w"], y, bias=st["bias"], use_elu=st["post_elu"],
                          gather=(self.state[st["key"]], slots, t, cin, st["dil"], st["pre_elu"]))
            if st["pad"]:
                ops.conv_gather(x, self.state[st["key"]], slots, None, B, t, cin, k, st["dil"], st["pre_elu"], t)
            return y
        if k == 1 and not st["pre_elu"]:
            src = x
        else:
            src = self._bf["C"][:B * t * k * cin].view(B * t, k * cin)
            ops.conv_gather(x, self.state[st["key"]], slots, src, B, t, cin, k, st["dil"], st["pre_elu"],
                            _chunk(t, B, st["pad"]))
        y = out[:B * t * cout].view(B * t, cout)
        if _thin(cout, k * cin, B * t):
            ops.conv_gemm(src, st["w"], y, bias=st["bias"], use_elu=st["post_elu"])
            return y
        g = self._bf["G"][:B * t * cout].view(B * t, cout)
        ops.linear(src, st["w"], g)
        ops.rows_op(g, y, bias=st["bias"], use_elu=st["post_elu"])
        return y

    def _run(self, bk, B):
        self._bf = bk.bufs
        return self._forward(bk.slots, bk.codes, bk.bufs, B)

    # ---- graphs -----------------------------------------------------------------------------------
    def _bucket(self, size):
        bk = self._buckets.get(size)
        if bk is not None:
            return bk
        table = RowTable(("slot",), size, self.device, pad=dict(slot=self.dummy))
        bk = SimpleNamespace(table=table, slots=table["slot"], bufs=self._buffers(size), graph=None,
                             codes=torch.zeros(size, self.codebooks, device=self.device, dtype=torch.long))
        bk.out = bk.bufs["pcm"]
        if self.use_graphs:
            if self._pool is None:
                self._pool = torch.cuda.graph_pool_handle()
            # the warm-up and capture runs decode on the dummy row only; its state is cleared after
            bk.graph = capture(lambda: self._run(bk, size), self._pool, warm=1)
            self._clear_row(self.dummy)
        self._buckets[size] = bk
        return bk

    @torch.inference_mode()
    def warmup(self, batch_buckets=None):
        for size in self._sizes.largest_first(batch_buckets):
            self._bucket(size)
        if batch_buckets is not None:  # sizes warmed outside the constructor's list become buckets too
            self._sizes = Buckets(self._sizes.sizes + tuple(int(b) for b in batch_buckets))
            self.batch_buckets = self._sizes.sizes

    # ---- public -----------------------------------------------------------------------------------
    def _clear_row(self, row):
        """A row's streaming state back to an empty stream: no conv history or tails, no reachable ring entry."""
        self.conv_flat[row].zero_()
        self.key_pos[row].fill_(NEVER)
        self.tokens[row].zero_()

    @torch.inference_mode()
    def reset(self, slot, zero_kv=False):
        """Start a new stream on the slot with fill kernels only (no host sync). Ring entries are unreachable once
        their key position is NEVER; zero_kv=True also clears their values."""
        check_slots([slot], self.max_slots)
        self._clear_row(slot)
        if zero_kv:
            self.kv[:, :, slot].zero_()

    @torch.inference_mode()
    def decode(self, slots, codes):
        """One frame per seat. slots: distinct ints in [0, max_slots), or a device long tensor of them; codes:
        [B, num_quantizers] long on the device. Returns an owned float32 [B, samples_per_frame] tensor."""
        B = len(slots)
        if codes.dim() != 2 or tuple(codes.shape) != (B, self.codebooks):
            raise ValueError(f"codes must be [{B},{self.codebooks}], got {tuple(codes.shape)}")
        bk = self._bucket(self._sizes.pick(B))
        if torch.is_tensor(slots):  # already on the device: written in place, the staged key is void
            bk.slots[:B].copy_(slots)
            bk.slots[B:].fill_(self.dummy)
            bk.table.forget()
        else:
            seats = tuple(int(s) for s in slots)
            if len(set(seats)) != B or any(not 0 <= s < self.max_slots for s in seats):
                raise ValueError("slots must be distinct and inside [0,max_slots)")
            bk.table.stage(dict(slot=seats), key=seats)
        bk.codes[:B].copy_(codes)
        bk.codes[B:].zero_()
        if bk.graph is not None:
            bk.graph.replay()
        else:
            self._run(bk, bk.slots.shape[0])
        return bk.out[:B].clone()


def _check_codec(mimi, dtype):
    """The codec shapes this decoder implements: causal constant-padded convs without right trim, an upsample
    layer, fp32 / fp16 / bf16 compute, weights on the GPU."""
    cfg = mimi.config
    if not cfg.use_causal_conv or cfg.pad_mode != "constant" or cfg.trim_right_ratio != 1:
        raise ValueError("Static decoder requires causal constant padding and trim_right_ratio=1")
    if mimi.upsample is None:
        raise ValueError("Static decoder expects the Mimi upsample layer")
    if dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError("StaticMimi computes in float32, float16 or bfloat16")
    if not next(mimi.parameters()).is_cuda:
        raise ValueError("StaticMimi runs on the GPU: move the Mimi model to a cuda device first")
