"""Shared test helpers (bit views and the bf16 parity bar)."""


def bf16_bits(t):
    """torch bf16/fp16 tensor -> numpy uint16 bit patterns (CPU)."""
    import numpy as np
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a, dtype):
    import numpy as np
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype)


def close(a, b, atol=2e-2, min_cos=0.9995, rel_ulps=2):
    """The bf16 parity bar: max |a-b| <= atol + rel_ulps * ulp_bf16(|b|) elementwise and cosine >= min_cos.
    (A 2e-2 bound alone cannot hold for |values| > 4, where one bf16 ulp is 0.03.)"""
    import torch
    a = a.detach().float().cpu().flatten()
    b = b.detach().float().cpu().flatten()
    ulp = torch.exp2(torch.floor(torch.log2(b.abs().clamp_min(1e-30))) - 7)
    err = (a - b).abs()
    bound = atol + rel_ulps * ulp
    cos = torch.nn.functional.cosine_similarity(a[None], b[None]).item()
    worst = (err - bound).max().item()
    return worst <= 0 and cos >= min_cos, dict(max_abs=err.max().item(), cos=cos, worst_over_bound=worst)
