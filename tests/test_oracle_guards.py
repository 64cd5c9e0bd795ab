"""The loop-guard restatement (oracle.torch_oracle.loop_detect_batch, maya3/guards.py:80-107) pinned on cases whose
answer the rules fix by construction: constant tails, exact periods, the frame thresholds, and a lag-p match count
placed exactly on either side of the 0.7 threshold. CPU only."""
import numpy as np

from oracle import torch_oracle as O


def _fresh(rng, avoid):
    while True:
        v = int(rng.integers(0, 2048))
        if v not in avoid:
            return v


def _lag_matches(rng, length, p, match_at):
    """A sequence whose lag-p matches (x[i] == x[i - p]) are exactly the positions in match_at (i >= p), with no
    accidental equality at any other lag below p_max."""
    x = []
    for i in range(length):
        if i >= p and i in match_at:
            x.append(x[i - p])
        else:
            x.append(_fresh(rng, set(x[max(0, i - 20):i])))
    return np.array(x)


def test_stall_and_frame_thresholds():
    rng = np.random.default_rng(0)
    base = rng.integers(0, 2048, 96)
    stalled = base.copy()
    stalled[-32:] = 7
    W = np.stack([stalled, stalled, stalled, np.full(96, -1)])
    n = np.array([32, 31, 500, 40])
    # the last 32 codes equal -> stall once 32 frames exist; an all-empty row counts as equal as well
    assert O.loop_detect_batch(W, n) == ["stall", None, "stall", "stall"]
    almost = stalled.copy()
    almost[-32] = 8  # the first of the tail differs
    assert O.loop_detect_batch(almost[None], np.array([100]))[0] != "stall"


def test_exact_periods_smallest_p_first():
    rng = np.random.default_rng(1)
    for p in (2, 3, 5, 8, 16):
        pat = [_fresh(rng, set()) for _ in range(p)]
        while len(set(pat)) < p:
            pat = [_fresh(rng, set()) for _ in range(p)]
        row = np.array((pat * (96 // p + 1))[:96])
        assert O.loop_detect_batch(row[None], np.array([64]))[0] == f"period:{p}"
        assert O.loop_detect_batch(row[None], np.array([63]))[0] is None  # the period rule needs 64 frames
    # period 4 also matches at lag 8: the smallest lag is reported
    pat = [1, 2, 3, 4]
    assert O.loop_detect_batch(np.array((pat * 24)[:96])[None], np.array([100]))[0] == "period:4"


def test_threshold_is_inclusive_float64_mean():
    rng = np.random.default_rng(2)
    # lag 2 over the last 64 codes: 62 comparisons; 0.7 * 62 = 43.4 -> 44 matches hit, 43 do not.
    # lag 4: 60 comparisons; exactly 42 = 0.7 * 60 hits (the float64 mean equals the literal 0.7).
    for p, m, want in ((2, 44, "period:2"), (2, 43, None), (4, 42, "period:4"), (4, 41, None)):
        cmp_pos = list(range(32 + p, 96))  # window positions 32..95, comparisons at i - 32 >= p
        chosen = set(rng.choice(cmp_pos, size=m, replace=False).tolist())
        row = _lag_matches(rng, 96, p, chosen)
        win = row[-64:]
        assert int((win[p:] == win[:-p]).sum()) == m
        for q in range(2, 17):
            if q != p:
                assert np.mean(win[q:] == win[:-q]) < 0.7
        assert O.loop_detect_batch(row[None], np.array([80]))[0] == want, (p, m)
