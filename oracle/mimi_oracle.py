"""fp32 CPU restatement of the one-frame streaming Mimi decode (test infrastructure only: tests/ and bench.py's CPU
leg use it as the reference they compare with; the product package never imports it).

Follows serve/fast_codec.py StaticMimi._forward (:186-192) and the layers it walks:
  quantizer   sum of the semantic codebook row and of the 31 acoustic rows, each group through its 1x1 output
              projection (:134-149; transformers MimiSplitResidualVectorQuantizer.decode)
  causal conv the last (k - 1) * dilation input frames of the previous call joined in front (:104-111)
  conv-T      the previous call's overlap tail added to the first k - s outputs; the new tail, bias removed, kept
              for the next call (:112-130)
  transformer per layer x += s1 * o(attn(LN1(x))), x += s2 * fc2(gelu(fc1(LN2(x)))), RoPE at absolute positions,
              keys at positions in (p - window, p] (:151-184)
Pinned in tests/test_oracle_mimi.py: frames decoded one at a time equal transformers' MimiModel.decode of the
whole code sequence.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


class MimiStream:
    def __init__(self, mimi, batch):
        from transformers.models.mimi.modeling_mimi import MimiConv1d, MimiConvTranspose1d
        self.m = mimi
        self.B = batch
        self.state = {}
        self.conv_types = (MimiConv1d, MimiConvTranspose1d)
        cfg = mimi.config
        self.window = cfg.sliding_window
        self.heads, self.hd = cfg.num_attention_heads, cfg.head_dim
        self.kv = [None] * cfg.num_hidden_layers
        self.pos = 0
        self.inv_freq = 1.0 / (cfg.rope_parameters["rope_theta"] ** (torch.arange(0, self.hd, 2).float() / self.hd))

    def _conv(self, mod, x):
        c = mod.conv
        pad = (c.kernel_size[0] - 1) * c.dilation[0]
        if pad:
            st = self.state.get(id(mod))
            if st is None:
                st = x.new_zeros(x.shape[0], x.shape[1], pad)
            x = torch.cat([st, x], -1)
            self.state[id(mod)] = x[..., -pad:].clone()
        return F.conv1d(x, c.weight, c.bias, stride=1, dilation=c.dilation[0], groups=c.groups)

    def _convt(self, mod, x):
        c = mod.conv
        s, k = c.stride[0], c.kernel_size[0]
        y = F.conv_transpose1d(x, c.weight, c.bias, stride=s, groups=c.groups)
        n = x.shape[-1] * s
        prev = self.state.get(id(mod))
        tail = y[..., n:].clone()
        if c.bias is not None:
            tail = tail - c.bias[None, :, None]
        self.state[id(mod)] = tail
        y = y[..., :n].clone()
        if prev is not None:
            y[..., :k - s] += prev
        return y

    def _layer(self, mod, x):
        from transformers.models.mimi.modeling_mimi import MimiConv1d, MimiConvTranspose1d, MimiResnetBlock
        if isinstance(mod, MimiConv1d):
            return self._conv(mod, x)
        if isinstance(mod, MimiConvTranspose1d):
            return self._convt(mod, x)
        if isinstance(mod, MimiResnetBlock):
            h = x
            for sub in mod.block:
                h = self._layer(sub, h)
            return x + h  # the shortcut is the identity (use_conv_shortcut = False)
        return mod(x)

    def _rope(self, x, pos):
        f = pos[:, None].float() * self.inv_freq[None]
        emb = torch.cat([f, f], -1)
        cos, sin = emb.cos(), emb.sin()
        x1, x2 = x[..., :self.hd // 2], x[..., self.hd // 2:]
        return x * cos + torch.cat([-x2, x1], -1) * sin

    def _transformer(self, h):
        B, T, D = h.shape
        H, hd = self.heads, self.hd
        pos = torch.arange(self.pos, self.pos + T)
        for li, L in enumerate(self.m.decoder_transformer.layers):
            a = L.self_attn
            x = L.input_layernorm(h)
            q = self._rope(a.q_proj(x).view(B, T, H, hd).transpose(1, 2), pos)
            k = self._rope(a.k_proj(x).view(B, T, H, hd).transpose(1, 2), pos)
            v = a.v_proj(x).view(B, T, H, hd).transpose(1, 2)
            if self.kv[li] is None:
                K, V, kp = k, v, pos
            else:
                K0, V0, kp0 = self.kv[li]
                K, V, kp = torch.cat([K0, k], 2), torch.cat([V0, v], 2), torch.cat([kp0, pos])
            keep = kp > pos[-1] - self.window  # entries the next calls can still see
            self.kv[li] = (K[:, :, keep], V[:, :, keep], kp[keep])
            mask = (kp[None, :] <= pos[:, None]) & (kp[None, :] > pos[:, None] - self.window)
            s = (q @ K.transpose(-1, -2)) / math.sqrt(hd)
            s = s.masked_fill(~mask, float("-inf"))
            o = (s.softmax(-1) @ V).transpose(1, 2).reshape(B, T, H * hd)
            h = h + L.self_attn_layer_scale(a.o_proj(o))
            h = h + L.mlp_layer_scale(L.mlp(L.post_attention_layernorm(h)))
        self.pos += T
        return h

    @torch.no_grad()
    def decode_frame(self, codes):
        """codes [B, 32] (one frame per seat) -> PCM [B, samples per frame] (fp32)."""
        m = self.m
        x = m.quantizer.decode(codes[:, :, None])
        x = self._convt(m.upsample, x)
        x = self._transformer(x.transpose(1, 2)).transpose(1, 2)
        for mod in m.decoder.layers:
            x = self._layer(mod, x)
        return x[:, 0]
