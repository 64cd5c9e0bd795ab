"""The Mimi streaming restatement (oracle.mimi_oracle.MimiStream, serve/fast_codec.py StaticMimi) pinned against
transformers' MimiModel.decode of the whole code sequence: frames decoded one call at a time, carrying conv states,
conv-T tails and the sliding-window KV, give the same audio as the full decode (fp32, CPU)."""
import torch

from m3x import synth
from oracle.mimi_oracle import MimiStream


def test_stream_equals_full_decode():
    m = synth.mimi(seed=3)
    cfg = m.config
    m.config._attn_implementation = "eager"
    B, T = 2, 5
    codes = synth.mimi_codes(B, T, seed=4)
    with torch.no_grad():
        full = m.decode(codes).audio_values[:, 0]
    st = MimiStream(m, B)
    parts = [st.decode_frame(codes[:, :, t]) for t in range(T)]
    stream = torch.cat(parts, -1)
    assert stream.shape == full.shape == (B, T * 1920)
    scale = full.abs().max().item()
    assert 1e-3 < scale < 100, scale  # the random codec makes real signal, not zeros or an explosion
    err = (stream - full).abs().max().item()
    assert err <= 2e-5 * max(1.0, scale), (err, scale)


def test_stream_equals_full_decode_past_the_window():
    """With a 6-token window (HF's mask and the restatement's ring read the same config), 8 frames = 16 tokens
    exercise keys leaving the window."""
    m = synth.mimi(seed=5)
    m.config._attn_implementation = "eager"
    m.config.sliding_window = 6
    for L in m.decoder_transformer.layers:
        L.self_attn.sliding_window = 6
    B, T = 1, 8
    codes = synth.mimi_codes(B, T, seed=6)
    with torch.no_grad():
        full = m.decode(codes).audio_values[:, 0]
    st = MimiStream(m, B)
    stream = torch.cat([st.decode_frame(codes[:, :, t]) for t in range(T)], -1)
    scale = full.abs().max().item()
    assert (stream - full).abs().max().item() <= 2e-5 * max(1.0, scale)
    # and the window matters: with a wider window the restatement differs
    st2 = MimiStream(m, B)
    st2.window = 250
    wide = torch.cat([st2.decode_frame(codes[:, :, t]) for t in range(T)], -1)
    assert (wide - full).abs().max().item() > 1e-3 * max(1.0, scale)
