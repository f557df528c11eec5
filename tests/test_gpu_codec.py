"""The codec decoder on the device (nunchi_amd.Codec, sh_codec_*) against the oracle restatement of imi's codec.

The network part (FSQ levels, projections, Q8_0 tables in imi_q8g's order, conv and attention with their carried
state, post-norm residuals) is the oracle's arithmetic operation for operation; the inverse STFT takes each bin's
cosine and sine from the device's double-precision routines where imi calls the C library's cosf / sinf, which may
differ in the last place. The samples are compared within 2e-6 relative L2: 10x the measured gap, and the oracle
itself sits within 5e-5 of the float64 truth (tests/test_oracle_codec.py)."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu
TOL = 2e-6


def _run(c, codes):
    return [c.frame(cc) for cc in codes], c.flush()


@pytest.fixture(scope="module")
def tiny_codec(model_dir):
    from nunchi_amd import synth
    return synth.cached("codec", synth.TINY_CODEC, 2, model_dir)


def test_tiny_codec_matches_oracle(tiny_codec):
    import nunchi_amd
    codes = np.random.default_rng(1).integers(0, 64, (9, 12))   # 54 positions: the key ring (36 slots) wraps
    g_parts, g_tail = _run(nunchi_amd.Codec(tiny_codec), codes)
    o = oracle.Codec(tiny_codec)
    o_parts, o_tail = _run(o, codes)
    assert [len(p) for p in g_parts] == [len(p) for p in o_parts] == [1440] + [1920] * 8 and len(g_tail) == 480
    g, r = np.concatenate(g_parts + [g_tail]), np.concatenate(o_parts + [o_tail])
    assert oracle.rel(g, r) < TOL, oracle.rel(g, r)
    for gp, op in zip(g_parts, o_parts):   # frame by frame too
        assert oracle.rel(gp, op) < 10 * TOL


def test_full_codec_matches_oracle(model_dir):
    import nunchi_amd
    from nunchi_amd import synth
    path = synth.cached("codec", synth.CODEC, 2, model_dir)
    codes = np.random.default_rng(4).integers(0, synth.CODEC.n_codes, (7, 12))
    g_parts, g_tail = _run(nunchi_amd.Codec(path), codes)
    o_parts, o_tail = _run(oracle.Codec(path), codes)
    g, r = np.concatenate(g_parts + [g_tail]), np.concatenate(o_parts + [o_tail])
    assert oracle.rel(g, r) < TOL, oracle.rel(g, r)


def test_reset_and_flush_repeat_bit_for_bit(tiny_codec):
    import nunchi_amd
    c = nunchi_amd.Codec(tiny_codec)
    codes = np.random.default_rng(2).integers(0, 64, (5, 12))
    a_parts, _ = _run(c, codes)   # (the flush resets)
    a = np.concatenate(a_parts)
    c.frame(codes[0])
    c.reset()
    b_parts, _ = _run(c, codes)
    b = np.concatenate(b_parts)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_bad_codes_are_refused(tiny_codec):
    import nunchi_amd
    c = nunchi_amd.Codec(tiny_codec)
    with pytest.raises(nunchi_amd.SeoulError):
        c.frame(np.full(12, 64))
    with pytest.raises(nunchi_amd.SeoulError):
        c.frame(np.full(12, -1))
    assert len(c.frame(np.zeros(12))) == 1440   # the refused calls left the stream untouched
