"""The ears on the device (nunchi_amd.Ears, sh_ears_*) against the oracle restatement of imi's ears.

Every float table product, norm, conv, attention and the LayerNorm are the oracle's operations in the same order;
the device takes the double log10 of the mel sums and the erff of the projector's GELU from its own math library
where imi calls the C library, which may differ in the last place. So the mel frames and the rows are compared
within 1e-6 relative L2 (the oracle itself sits within 5e-5 of the float64 truth, tests/test_oracle_ears.py), and
the mel frames and rows before the first GELU difference are in practice equal bit for bit."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu
TOL = 1e-6


@pytest.fixture(scope="module")
def tiny_ears(model_dir):
    from nunchi_amd import synth
    return synth.cached("ears", synth.TINY_EARS, 3, model_dir)


@pytest.mark.parametrize("n", [1, 400, 401, 3 * 16000, 7 * 16000 + 123])
def test_tiny_ears_matches_oracle(tiny_ears, n):
    import nunchi_amd
    from nunchi_amd import synth
    pcm = synth.clip(n, 5)
    g = nunchi_amd.Ears(tiny_ears)
    out = g.encode(pcm)
    ref, mel = oracle.Ears(tiny_ears, threads=4).encode(pcm, mel=True)
    assert out.shape == ref.shape
    assert oracle.rel(g.mel(), mel) < TOL
    assert oracle.rel(out, ref) < TOL, oracle.rel(out, ref)


def test_encode_repeats_and_shrinks(tiny_ears):
    """A longer clip, a shorter one (the work buffers are kept), then the first again: bit for bit the same rows."""
    import nunchi_amd
    from nunchi_amd import synth
    g = nunchi_amd.Ears(tiny_ears)
    a, b = synth.clip(5 * 16000, 6), synth.clip(16000, 7)
    ra = g.encode(a)
    rb = g.encode(b)
    assert np.array_equal(ra.view(np.uint32), g.encode(a).view(np.uint32))
    assert np.array_equal(rb.view(np.uint32), g.encode(b).view(np.uint32))


def test_full_ears_hearing_window(model_dir):
    """The full ears shape on a 30.7 s clip: the 384 rows of the hearing window."""
    import nunchi_amd
    from nunchi_amd import synth
    path = synth.cached("ears", synth.EARS, 3, model_dir)
    pcm = synth.clip(491760, 1)
    out = nunchi_amd.Ears(path).encode(pcm)
    ref = oracle.Ears(path, threads=8).encode(pcm)
    assert out.shape == ref.shape == (384, 2048)
    assert oracle.rel(out, ref) < TOL, oracle.rel(out, ref)


def test_bad_arguments_are_refused(tiny_ears):
    import nunchi_amd
    g = nunchi_amd.Ears(tiny_ears)
    with pytest.raises(nunchi_amd.SeoulError):
        g.encode(np.zeros(0, np.float32))


def test_mel_buffer_capacity_is_checked(tiny_ears):
    """sh_ears_mel writes only into a buffer that holds the last encode's frames: after a long clip, a buffer sized
    for a short one is refused with nothing written, and the binding sizes its buffer from the last encode."""
    import ctypes as C
    import nunchi_amd
    from nunchi_amd import synth
    g = nunchi_amd.Ears(tiny_ears)
    long_n, short_n = 7 * 16000 + 123, 16000
    g.encode(synth.clip(long_n, 5))
    _, f_long = g.positions(long_n)
    _, f_short = g.positions(short_n)
    assert f_short < f_long
    lib = nunchi_amd.load_library()
    buf = np.full((f_short + 1, g.info.n_mel), 7.0, np.float32)   # one guard frame past the capacity
    n = C.c_int(-1)
    rc = lib.sh_ears_mel(g.h, buf.ctypes.data, f_short, C.byref(n))
    assert rc == nunchi_amd.SH_E_ARG
    assert n.value == f_long
    assert np.all(buf == 7.0)
    m = g.mel()
    assert m.shape == (f_long, g.info.n_mel)
