"""Ragged-cache interop with HF DynamicCache (drop-in for serve/cache.py, :7-62).

The static decode cache itself is StaticBackbone.k/v ([slots, kv_heads, capacity, head_dim] per layer); these
helpers build, pack and split the per-request HF caches that admission copies into it (StaticBackbone.load_slot
reads `cache.layers[i].keys[0, :, :length]`). Host-side tensor bookkeeping, no kernels.
"""
from __future__ import annotations

import torch


def cache_from_owned_tensors(layers):
    """A DynamicCache holding the given per-layer (keys, values) [1, KV, T, D] tensors as they are (no copy)."""
    from transformers import DynamicCache
    from transformers.cache_utils import DynamicLayer
    cache = DynamicCache()
    for keys, values in layers:
        layer = DynamicLayer()
        layer.keys, layer.values = keys, values
        layer.dtype, layer.device = keys.dtype, keys.device
        layer.is_initialized = True
        cache.layers.append(layer)
    return cache


def pack_caches(caches, new_tokens, device):
    """Left-pad per-request caches into one batch cache. Returns (cache or None, attention mask [B, max+new],
    lengths). A request without a cache (None) contributes length 0."""
    lengths = [0 if c is None else c.layers[0].keys.shape[-2] for c in caches]
    longest = max(lengths)
    if longest == 0:
        return None, None, lengths
    ref = next(c for c in caches if c is not None)
    packed = []
    for li in range(len(ref.layers)):
        pair = []
        for attr in ('keys', 'values'):
            like = getattr(ref.layers[li], attr)
            buf = like.new_zeros(len(caches), like.shape[1], longest, like.shape[-1])
            for row, (c, n) in enumerate(zip(caches, lengths)):
                if n:
                    buf[row:row + 1, :, longest - n:] = getattr(c.layers[li], attr)
            pair.append(buf)
        packed.append(tuple(pair))
    starts = torch.tensor([longest - n for n in lengths], device=device)
    mask = torch.arange(longest + new_tokens, device=device)[None] >= starts[:, None]
    return cache_from_owned_tensors(packed), mask, lengths


def split_cache(cache, lengths, keep=None, *, copy=True):
    """Per-row caches of the last `length` positions of each row (at most `keep`). copy=False returns views that
    share the packed storage (only safe for append/crop use)."""
    out = []
    for row, n in enumerate(lengths):
        n = n if keep is None else min(n, keep)
        layers = []
        for layer in cache.layers:
            k = layer.keys[row:row + 1, :, layer.keys.shape[-2] - n:]
            v = layer.values[row:row + 1, :, layer.values.shape[-2] - n:]
            if copy:
                k, v = k.contiguous().clone(), v.contiguous().clone()
            layers.append((k, v))
        out.append(cache_from_owned_tensors(layers))
    return out
