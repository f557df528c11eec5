"""The oracle's restatement of imi's voice-code pick (imi_talker::next, imi/core/talk.cpp:147-164), pinned by what
the mathematics fixes: inverse-CDF sampling over softmax(l / temp), the penalty applied once per distinct code, the
boundary draws, and the limits of the temperature."""
import numpy as np

import oracle


def test_boundary_draws_and_inverse_cdf():
    rng = np.random.default_rng(0)
    for trial in range(20):
        V = int(rng.integers(2, 200))
        l = rng.standard_normal((3, V)).astype(np.float32) * 3
        temp = float(np.float32(rng.uniform(0.2, 2.0)))   # imi keeps temp as a float
        u = np.array([0.0, rng.uniform(), 1.0 - 2.0 ** -40])
        picks, keep, _ = oracle.voice_sample(l, [0, 0, 0], np.zeros((0, 1), np.int32), u, temp, 1.2)
        assert picks[0] == 0   # r = 0: the first subtraction already reaches <= 0
        p = np.exp((l[1] - l[1].max()).astype(np.float64) / temp)
        c = np.cumsum(p)   # in code order
        want = int(np.searchsorted(c, u[1] * c[-1], side="left"))
        assert picks[1] == min(want, V - 1)
        p2 = np.exp((l[2] - l[2].max()).astype(np.float64) / temp)
        c2 = np.cumsum(p2)
        assert picks[2] == min(int(np.searchsorted(c2, u[2] * c2[-1], side="left")), V - 1)
        assert abs(keep[2] - (1.0 - p2[-1] / c2[-1])) <= 1e-12


def test_frequencies_follow_softmax():
    l = np.array([[0.5, -1.0, 2.0, 0.0, 1.0]], np.float32)
    temp = 0.7
    us = (np.arange(20000) + 0.5) / 20000.0
    counts = np.zeros(5)
    for u in us[::7]:
        pk, _, _ = oracle.voice_sample(l, [0], np.zeros((0, 1), np.int32), [u], temp, 1.0)
        counts[pk[0]] += 1
    p = np.exp((l[0] - l[0].max()) / temp)
    p /= p.sum()
    n = counts.sum()
    assert np.all(np.abs(counts / n - p) <= 1.5 / n + 1e-12)   # stratified draws: off by at most one step


def test_repeat_penalty_once_per_code():
    V = 8
    l = np.array([[2.0, -1.0, 0.5, 0.0, 3.0, -2.0, 1.0, 0.25]], np.float32)
    # codebook 1 of 2: codes 0 (twice), 1, 7 (out of range on the other codebook), -1 and V are skipped
    hist = np.array([[5, 0], [6, 1], [7, 0], [0, -1], [1, V]], np.int32)
    _, _, pen = oracle.voice_sample(l, [1], hist, [0.5], 1.0, 2.0)
    want = l[0].copy()
    want[0] = 2.0 / 2.0      # once, though it appears twice
    want[1] = -1.0 * 2.0
    assert np.array_equal(pen[0], want)
    _, _, pen0 = oracle.voice_sample(l, [0], hist, [0.5], 1.0, 2.0)
    want = l[0].copy()
    for c in (5, 6, 7, 0, 1):
        want[c] = want[c] / 2.0 if want[c] > 0 else want[c] * 2.0
    assert np.array_equal(pen0[0], want)


def test_temperature_limits():
    rng = np.random.default_rng(3)
    l = rng.standard_normal((4, 50)).astype(np.float32)
    l[3, -1] = 10.0   # end-of-audio far ahead
    picks, keep, _ = oracle.voice_sample(l, [0, 1, 2, 3], np.zeros((0, 1), np.int32), [0.3, 0.6, 0.9, 0.5], 1e-3, 1.0)
    assert np.array_equal(picks, np.argmax(l, axis=1))
    assert np.all(keep[:3] > 1.0 - 1e-12) and keep[3] < 1e-12
