"""Algorithmic bytes / flops of the frame step and MI355X peaks (AMD public figures).

Decode attention of one layer reads, per attended key, K and V of every kv head (kv*D*2 bytes each) and per row
the query and writes the output (heads*D*2 bytes each); flops are 2*heads*D per key for QK and as many for PV.
"""
from __future__ import annotations

HBM_PEAK_GBS = 8000.0          # HBM3E, GB/s
MFMA_BF16_TFLOPS = 2500.0      # dense bf16
MFMA_FP16_TFLOPS = 2500.0
VALU_FP32_TFLOPS = 157.3


def decode_attn_bytes(attended, rows, heads=16, kv_heads=8, head_dim=128, elem=2):
    """attended: sum over rows of (pos + 1) keys."""
    return attended * kv_heads * head_dim * elem * 2 + rows * heads * head_dim * elem * 2


def add_norm_bytes(rows, hidden=1024, elem=2):
    """Fused residual add + RMSNorm: h and a in, h + a and y out, plus the norm weight."""
    return rows * hidden * elem * 4 + hidden * elem


def decode_attn_flops(attended, heads=16, head_dim=128):
    return attended * heads * head_dim * 2 * 2


def backbone_weight_bytes(layers=28, hidden=1024, heads=16, kv_heads=8, head_dim=128, inter=3072, elem=2):
    per = (heads + 2 * kv_heads) * head_dim * hidden + hidden * heads * head_dim + 3 * inter * hidden
    return layers * per * elem


def backbone_step_bytes(attended, rows, layers=28, hidden=1024, heads=16, kv_heads=8, head_dim=128, inter=3072,
                        v0=2048):
    kv = layers * kv_heads * head_dim * 2 * 2
    return (backbone_weight_bytes(layers, hidden, heads, kv_heads, head_dim, inter) + attended * kv + rows * kv +
            rows * hidden * 2 * 2 + v0 * hidden * 2)


def backbone_step_flops(attended, rows, layers=28, hidden=1024, heads=16, kv_heads=8, head_dim=128, inter=3072,
                        v0=2048):
    """Projections (2 flops per weight per row), the cb0 head, and QK + PV over every attended key of every layer."""
    params = backbone_weight_bytes(layers, hidden, heads, kv_heads, head_dim, inter) // 2
    return 2 * rows * params + 2 * rows * hidden * v0 + layers * decode_attn_flops(attended, heads, head_dim)


def depth_frame_bytes(d=1024, ffn=2816, layers=4, n_codes=2048, n_q=32, d_backbone=1024, seats=1, ffn_mats=3):
    """ffn_mats: 3 for a gated FFN (gate, up, down), 2 for a plain one (the reference's GELU f1, f2)."""
    trunk = layers * (3 * d * d + d * d + ffn_mats * ffn * d) * 2
    head = n_codes * d * 2
    return (n_q - 1) * (trunk + head) + d * d_backbone * 2 + seats * (n_q - 1) * d * 2


def depth_frame_flops(seats, d=1024, ffn=2816, layers=4, n_codes=2048, n_q=32, d_backbone=1024):
    per_pos = layers * (3 * d * d + d * d + 3 * ffn * d) * 2
    return seats * ((n_q - 1) * (per_pos + n_codes * d * 2) + per_pos + d * d_backbone * 2)
