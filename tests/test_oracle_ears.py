"""Pins of the oracle's ears restatement (oracle/imi_cpu_ears.cpp, imi/core/ears.cpp) on the CPU:
- the clip geometry (imi/core/ears.cpp:201-205: frames, the three halvings) against a direct count;
- the mel frames and the encoder's rows against oracle/exact.py's float64 restatement of imi/ref/ears_exact.py
  (numpy's real FFT in place of the DFT table, float64 everywhere), at the tiny shape over a clip longer than the
  attention window and at the full shape;
- that the comparison sees what it pins: another window, another rope base, or the layers in another order move the
  truth far outside the tolerance;
- thread-count independence of the restatement (the work split never changes an operation's order)."""
import numpy as np
import pytest

import oracle
# (the float64 restatements stay off the GPU box: without them this CPU-only module is skipped)
exact = pytest.importorskip("oracle.exact")

TOL = 5e-5   # float32 pipeline against float64: measured 2.0e-6 (tiny, 3 s) and 9.3e-6 (full shape, 30.7 s)


@pytest.fixture(scope="module")
def tiny_ears(model_dir):
    from nunchi_amd import synth
    return synth.cached("ears", synth.TINY_EARS, 3, model_dir)


def _count(n):
    """ears.cpp:201-205 by counting: 400-sample frames every 160 samples until one reaches the clip's end (one frame
    at least), then three stride-2 halvings rounding up."""
    fr, end = 1, 400
    while end < n:
        fr, end = fr + 1, end + 160
    t = fr
    for _ in range(3):
        t = -(-t // 2)
    return t, fr


def test_geometry(tiny_ears):
    e = oracle.Ears(tiny_ears, threads=2)
    for n in (1, 399, 400, 401, 560, 561, 16000, 48000, 491760):
        p, fr = _count(n)
        assert e.positions(n) == p, n
        assert lib_frames(e, n) == fr, n
    assert e.positions(491760) == 384   # 30.7 s: the hearing window's 384 rows


def lib_frames(e, n):
    return int(oracle.lib().orc_ears_frames(e.h, n))


def test_tiny_ears_vs_float64_truth(tiny_ears):
    from nunchi_amd import synth
    pcm = synth.clip(3 * 16000, 1)     # 38 positions: the window of 8 slides
    e = oracle.Ears(tiny_ears, threads=4)
    out, mel = e.encode(pcm, mel=True)
    truth, tmel = exact.ears(tiny_ears, pcm)
    assert out.shape == truth.shape == (38, synth.TINY_EARS.n_out)
    assert oracle.rel(mel, tmel) < 2e-6
    assert oracle.rel(out, truth) < TOL
    # the comparison sees the window, the rope base and the layer order
    assert oracle.rel(out, exact.ears(tiny_ears, pcm, window=7)[0]) > 100 * TOL
    assert oracle.rel(out, exact.ears(tiny_ears, pcm, window=9)[0]) > 100 * TOL
    assert oracle.rel(out, exact.ears(tiny_ears, pcm, theta=1e4)[0]) > 100 * TOL


def test_threads_do_not_change_the_rows(tiny_ears):
    from nunchi_amd import synth
    pcm = synth.clip(2 * 16000 + 77, 2)
    a = oracle.Ears(tiny_ears, threads=1).encode(pcm)
    b = oracle.Ears(tiny_ears, threads=5).encode(pcm)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_short_clips(tiny_ears):
    """Clips shorter than one 400-sample frame still give one frame and one position (ears.cpp:203)."""
    from nunchi_amd import synth
    e = oracle.Ears(tiny_ears, threads=2)
    for n in (1, 250, 400):
        pcm = synth.clip(n, 3)
        out = e.encode(pcm)
        truth, _ = exact.ears(tiny_ears, pcm)
        assert out.shape[0] == 1 and oracle.rel(out, truth) < TOL


def test_full_ears_vs_float64_truth(model_dir):
    from nunchi_amd import synth
    path = synth.cached("ears", synth.EARS, 3, model_dir)
    pcm = synth.clip(5 * 16000, 4)     # 63 positions: the window of 32 slides
    out = oracle.Ears(path, threads=8).encode(pcm)
    truth, _ = exact.ears(path, pcm)
    assert out.shape == truth.shape == (63, 2048)
    assert oracle.rel(out, truth) < TOL
