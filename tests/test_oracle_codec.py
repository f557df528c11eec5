"""Pins of the oracle's codec restatement (oracle/imi_cpu_codec.cpp, imi/core/codec.cpp) on the CPU:
- the inverse DFT against closed forms (a single bin is a complex exponential) and numpy's FFT on random spectra;
- frame-by-frame decoding (carried conv memory, the attention window over earlier frames, the overlap-add with its
  start padding and tail) against the float64 whole-sequence restatement of imi/ref/codec_exact.py (oracle/exact.py),
  at the tiny shape over 9 frames (54 positions: the window of 30 wraps) and at the full codec shape;
- that those comparisons see what they pin: a window of 29 or 31, another rope base, or a dropped frame move the
  truth far outside the tolerance;
- the sample counts of imi's stream: 1440 on the first frame, 1920 after, 480 at the flush."""
import numpy as np
import pytest

import oracle
# (the float64 restatements stay off the GPU box: without them this CPU-only module is skipped)
exact = pytest.importorskip("oracle.exact")

TOL = 5e-5   # float32 pipeline (fma chains, float sums) against float64: measured 4.9e-6 (tiny) and 1.1e-5 (full)


@pytest.fixture(scope="module")
def tiny_codec(model_dir):
    from nunchi_amd import synth
    return synth.cached("codec", synth.TINY_CODEC, 2, model_dir)


def _decode(path, codes):
    c = oracle.Codec(path)
    parts = [c.frame(cc) for cc in codes]
    return parts, c.flush()


def test_ifft_single_bins_are_exponentials():
    n = 1280
    j = np.arange(n)
    for k in (0, 1, 5, 256, 321, 640, 1279):
        x = np.zeros(n, np.complex64)
        x[k] = 1
        y = oracle.ifft(x)
        assert np.abs(y - np.exp(2j * np.pi * k * j / n)).max() < 2e-6, k


def test_ifft_matches_numpy_on_random_spectra():
    rng = np.random.default_rng(3)
    for n in (1280, 640, 10, 5):
        x = (rng.standard_normal(n) + 1j * rng.standard_normal(n)).astype(np.complex64)
        ref = np.fft.ifft(x.astype(np.complex128)) * n
        y = oracle.ifft(x)
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-6, n


def test_stream_lengths(tiny_codec):
    from nunchi_amd import synth
    assert oracle.Codec(tiny_codec).n_codes == synth.TINY_CODEC.n_codes
    parts, tail = _decode(tiny_codec, np.random.default_rng(0).integers(0, 64, (3, 12)))
    assert [len(p) for p in parts] == [1440, 1920, 1920] and len(tail) == 480


def test_tiny_codec_vs_float64_truth(tiny_codec):
    codes = np.random.default_rng(1).integers(0, 64, (9, 12))
    parts, tail = _decode(tiny_codec, codes)
    pcm = np.concatenate(parts + [tail])
    truth, _ = exact.codec(tiny_codec, codes)
    assert len(pcm) == len(truth) == 9 * 6 * 320
    assert oracle.rel(pcm, truth) < TOL
    # the comparison sees the window, the rope base and the frame order
    assert oracle.rel(pcm, exact.codec(tiny_codec, codes, win=29)[0]) > 100 * TOL
    assert oracle.rel(pcm, exact.codec(tiny_codec, codes, win=31)[0]) > 100 * TOL
    assert oracle.rel(pcm, exact.codec(tiny_codec, codes, theta=1e4)[0]) > 100 * TOL
    shifted = np.concatenate([codes[:1], codes[:-1]])
    assert oracle.rel(pcm, exact.codec(tiny_codec, shifted)[0]) > 100 * TOL


def test_full_codec_vs_float64_truth(model_dir):
    from nunchi_amd import synth
    path = synth.cached("codec", synth.CODEC, 2, model_dir)
    codes = np.random.default_rng(1).integers(0, synth.CODEC.n_codes, (3, 12))
    parts, tail = _decode(path, codes)
    truth, _ = exact.codec(path, codes)
    assert oracle.rel(np.concatenate(parts + [tail]), truth) < TOL


def test_reset_repeats(tiny_codec):
    codes = np.random.default_rng(2).integers(0, 64, (4, 12))
    c = oracle.Codec(tiny_codec)
    a = np.concatenate([c.frame(cc) for cc in codes] + [c.flush()])   # flush resets
    b = np.concatenate([c.frame(cc) for cc in codes] + [c.flush()])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
