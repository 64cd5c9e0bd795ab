"""StaticMimi (drop-in of serve/fast_codec.py) on the GPU against the fp32 streaming oracle (oracle.mimi_oracle,
itself pinned against transformers' full-sequence MimiModel.decode): seats join, leave, reorder and reset between
frames, pad to buckets through the dummy slot, and pass keys out of a short window around a wrapping ring.

StaticMimi computes in the Mimi module's dtype by default, float32 as in the reference (serve/fast_codec.py:47-49;
the engine's codec is float32, maya3/engine.py:165,201); float16 is an opt-in.
Tolerance, float32: the product and the oracle evaluate the same fp32 math in different orders (MFMA blocks,
hardware-free expm1 / sin / cos against torch's CPU kernels), so every frame of every seat must have relative RMS
error <= 1e-5 and max abs error <= 2e-5 of the frame's peak (measured worst on MI355X: 2.1e-6 and 3.1e-6), two
and a half orders of magnitude under the float16 bar.
Tolerance, float16: activations stored in float16 with fp32 accumulation. Rounding every stage of the oracle
itself to float16 moves its PCM by 0.12% RMS, so every frame must have relative RMS error <= 5e-3 and max abs
error <= 1e-2 of the frame's peak (an attention that dropped a query lane's broadcast was 1.4% off and fails)."""
import numpy as np
import pytest
import torch

from m3x import synth
from oracle.mimi_oracle import MimiStream

pytestmark = pytest.mark.gpu


TOL = {torch.float32: (1e-5, 2e-5), torch.float16: (5e-3, 1e-2)}
DTYPES = [torch.float32, torch.float16]


def _pair(gpu, seed, window=None, **kw):
    from m3x.serve.fast_codec import StaticMimi
    mc, mg = synth.mimi(seed=seed), synth.mimi(seed=seed, device=gpu)
    if window is not None:
        for m in (mc, mg):
            m.config.sliding_window = window
    return mc, StaticMimi(mg, **kw)


def _check(got, ref, what, dtype=torch.float16):
    peak = ref.abs().max().item()
    rms = ref.pow(2).mean().sqrt().item()
    err_rms = (got - ref).pow(2).mean().sqrt().item()
    err_max = (got - ref).abs().max().item()
    print(f"{what} [{dtype}]: peak {peak:.3g} rms {rms:.3g} err_rms/rms {err_rms / rms:.3g} "
          f"err_max/peak {err_max / peak:.3g}", flush=True)
    assert peak > 1e-3, what
    t_rms, t_max = TOL[dtype]
    assert err_rms <= t_rms * rms and err_max <= t_max * peak, (what, err_rms / rms, err_max / peak)


def _run(mc, sm, schedule, codes, gpu):
    """schedule: per frame a list of slots (or ('reset', slot)); codes[slot] [32, frames] long. Checks every seat's
    PCM against its own oracle stream."""
    streams, used = {}, {}
    for f, step in enumerate(schedule):
        if step[0] == "reset":
            sm.reset(step[1])
            streams.pop(step[1], None)
            used[step[1]] = 0
            continue
        slots = step
        cc = torch.stack([codes[s][:, used.get(s, 0)] for s in slots])
        got = sm.decode(slots, cc.to(gpu)).cpu()
        assert got.shape == (len(slots), sm.samples_per_frame) and got.dtype == torch.float32
        for i, s in enumerate(slots):
            st = streams.setdefault(s, MimiStream(mc, 1))
            ref = st.decode_frame(cc[i:i + 1])
            _check(got[i:i + 1], ref, f"frame {f} slot {s}", sm.dtype)
            used[s] = used.get(s, 0) + 1


@pytest.mark.parametrize("dtype", DTYPES)
def test_decode_matches_streaming_oracle(gpu, dtype):
    mc, sm = _pair(gpu, 31, max_slots=6, batch_buckets=(1, 2, 4, 8), dtype=dtype)
    assert sm.dtype == dtype
    codes = {s: synth.mimi_codes(1, 8, seed=40 + s)[0] for s in range(6)}
    schedule = [[0, 3, 5], [3, 0], [5, 0, 3, 1], ("reset", 3), [3, 1, 0], [1], [0, 1, 2, 3, 4, 5]]
    with torch.inference_mode():
        _run(mc, sm, schedule, codes, gpu)
    assert sm.samples_per_frame == 1920


@pytest.mark.parametrize("dtype", DTYPES)
def test_decode_past_a_short_window_and_ring_wrap(gpu, dtype):
    """window 6, ring 8: from the fourth frame on keys leave the window, from the fifth the ring wraps."""
    mc, sm = _pair(gpu, 33, window=6, max_slots=3, batch_buckets=(2,), ring=8, dtype=dtype)
    codes = {s: synth.mimi_codes(1, 12, seed=50 + s)[0] for s in range(3)}
    with torch.inference_mode():
        _run(mc, sm, [[0, 2]] * 6 + [[2]] + [[0, 2]] * 5, codes, gpu)


@pytest.mark.parametrize("dtype", DTYPES)
def test_graph_replay_equals_eager(gpu, dtype):
    from m3x.serve.fast_codec import StaticMimi
    a = StaticMimi(synth.mimi(seed=35, device=gpu), 4, batch_buckets=(4,), dtype=dtype)
    b = StaticMimi(synth.mimi(seed=35, device=gpu), 4, batch_buckets=(4,), use_graphs=False, dtype=dtype)
    codes = synth.mimi_codes(4, 4, seed=36).to(gpu)
    with torch.inference_mode():
        a.warmup()
        for t, slots in enumerate([[0, 1, 2], [2, 0], [1, 2, 0, 3], [3]]):
            c = codes[:len(slots), :, t]
            assert torch.equal(a.decode(slots, c), b.decode(slots, c)), t
        assert torch.equal(a.tokens, b.tokens) and torch.equal(a.key_pos[:4], b.key_pos[:4])
        assert a.tokens[:4].tolist() == [6, 4, 6, 4] and a.tokens[4].item() == 0


def test_surface_errors(gpu):
    from m3x.serve.fast_codec import StaticMimi
    sm = StaticMimi(synth.mimi(seed=37, device=gpu), 2, batch_buckets=(2,), use_graphs=False)
    c = torch.zeros(2, 32, dtype=torch.long, device=gpu)
    with pytest.raises(ValueError):
        sm.decode([0, 0], c)
    with pytest.raises(ValueError):
        sm.decode([0, 2], c)
    with pytest.raises(ValueError):
        sm.decode([0], c)
    with pytest.raises(ValueError):
        sm.decode([0, 1, 2], torch.zeros(3, 32, dtype=torch.long, device=gpu))
    with pytest.raises(IndexError):
        sm.reset(2)
    with pytest.raises(ValueError):
        StaticMimi(synth.mimi(seed=37, device=gpu), 2, ring=200)
    b = sm.state_bytes_per_slot()
    assert sm.dtype == torch.float32  # the module's dtype, as the reference computes
    assert b["attention_kv"] == 8 * 2 * 256 * 512 * 4 and b["attention_index"] == 256 * 8 + 8
    b16 = StaticMimi(synth.mimi(seed=37, device=gpu), 2, batch_buckets=(2,), use_graphs=False,
                     dtype=torch.float16).state_bytes_per_slot()
    assert b16["attention_kv"] == 8 * 2 * 256 * 512 * 2


def test_tick_frame_codes_through_codec_to_readout(gpu):
    """The tick on the device: a frame graph's codes go to StaticMimi.decode, whose PCM (checked against the
    streaming oracle on the same codes) the tick readout packs beside the codes in one host copy."""
    from m3x.serve.fast_codec import StaticMimi
    from m3x.tick import TickReadout
    from test_gpu_frame import _frame
    fs = _frame(gpu, seed=93)
    mc = synth.mimi(seed=94)
    sm = StaticMimi(synth.mimi(seed=94, device=gpu), 8, batch_buckets=(4,))
    rd = TickReadout(4, frame=1920, nq=32, with_loop=False, device=gpu)
    seats = [1, 6]
    streams = {s: MimiStream(mc, 1) for s in seats}
    with torch.inference_mode():
        g = fs.capture(4, 256)
        fs.set_slots(g, seats)
        for frame in range(3):
            fs.replay(g)
            codes = fs.codes(g)[:2]
            pcm = sm.decode(seats, codes)
            fs.readout(g, rd, B=2, pcm=pcm)
            got = rd.wait()
            assert np.array_equal(got["codes"], codes.cpu().numpy())
            want16 = (pcm.cpu().clamp(-1, 1) * 32767).round().to(torch.int16).numpy()
            assert np.array_equal(got["pcm"], want16)
            for i, s in enumerate(seats):
                _check(pcm[i:i + 1].cpu(), streams[s].decode_frame(codes[i:i + 1].cpu().long()), f"tick {frame} {s}",
                       sm.dtype)
