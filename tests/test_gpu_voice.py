"""GPU parity of the Q8_0 voice generator (C ABI: sh_voice_*) against the oracle's imi_voice restatement
(imi/core/voice.cpp:90-206).

The HIP path keeps each fp32 operation order of imi_q8g_group (the generic order for most codebook counts, the
scaled order for 6 and 12, the single-input order for the input projection and the word scores), of the norms,
the position rope, the attention softmax and SiLU, so the frame base, every score of every pass and the feedback row
sum equal the oracle's bit for bit. Each test plays frames the way imi's talk loop does (imi/core/talk.cpp:127-187):
begin_frame from a brain hidden state, masked passes that each score a few codebooks and fix their codes (here the
first index of the maximum, in place of sampling), then the feedback row sum.
"""
import numpy as np
import pytest

from conftest import rel

pytestmark = pytest.mark.gpu


def same(a, b) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _shape(**kw):
    from nunchi_amd import synth
    base = dict(n_embd=256, n_layer=2, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=256, n_cb=8, n_in=256)
    base.update(kw)
    return synth.VoiceShape(**base)


def _play(path, seed, schedule, n_frames=2, threads=4):
    import nunchi_amd
    import oracle
    g = nunchi_amd.Voice(path)
    o = oracle.Voice(path, threads=threads)
    assert (g.n_embd, g.n_vocab, g.n_cb, g.n_in, g.n_head, g.n_head_kv, g.head_dim, g.n_ff, g.n_layer) == \
        (o.n_embd, o.n_vocab, o.n_cb, o.n_in, o.n_head, o.n_head_kv, o.head_dim, o.n_ff, o.n_layer)
    rng = np.random.default_rng(seed)
    for f in range(n_frames):
        h = rng.standard_normal(g.n_in).astype(np.float32)
        g.begin_frame(h)
        o.begin_frame(h)
        assert same(g.base(), o.base()), f"frame {f}: base differs (rel {rel(g.base(), o.base()):.2e})"
        codes = np.full(g.n_cb, -1, np.int32)
        start = 0
        for n in schedule:
            need = np.arange(start, start + n, dtype=np.int32)
            sg = g.pass_(codes, need)
            so = o.pass_(codes, need)
            assert np.isfinite(sg).all()
            assert same(sg, so), f"frame {f}, codebooks {need.tolist()}: scores differ (rel {rel(sg, so):.2e})"
            codes[need] = np.argmax(so, axis=1)
            start += n
        fg = g.feedback(codes)
        fo = o.feedback(codes)
        assert same(fg, fo), f"frame {f}: feedback differs (rel {rel(fg, fo):.2e})"
    return g, o


def test_tiny_voice_frames(tiny_voice):
    """8 codebooks: the generic order; passes of 4 + 4 codebooks."""
    _play(tiny_voice, 1, (4, 4))


@pytest.mark.parametrize("n_cb,schedule", [(12, (6, 6)), (6, (3, 3)), (5, (2, 3)), (2, (1, 1))])
def test_codebook_counts(model_dir, n_cb, schedule):
    """12 and 6 codebooks take the scaled order (imi's 12-codebook talk schedule is {6, 6}); 5 and 2 the generic one."""
    from nunchi_amd import synth
    path = synth.cached("voice", _shape(n_cb=n_cb), 3, model_dir)
    _play(path, n_cb, schedule, n_frames=1)


def test_narrow_heads_and_odd_groups(model_dir):
    """head_dim 32, 4 query heads per kv head, widths that are not powers of two, an odd number of qkvg row groups."""
    from nunchi_amd import synth
    path = synth.cached("voice", _shape(n_head=8, n_head_kv=2, head_dim=32, n_ff=288, n_embd=192, n_in=96), 5, model_dir)
    _play(path, 5, (3, 5), n_frames=1)


def test_wide_inputs(model_dir):
    """n_ff > 1024 and an input projection wider than one staged chunk: several input chunks per table."""
    from nunchi_amd import synth
    path = synth.cached("voice", _shape(n_ff=2112, n_in=2048, n_embd=320, n_vocab=96), 6, model_dir)
    _play(path, 6, (8,), n_frames=1)


def test_wide_tables_split(model_dir):
    """o and down tables over several 1024-column chunks (attention width 1280, n_ff 3104: the last chunk ragged),
    5 codebooks: the per-chunk block sums are folded by a second kernel in the same block order."""
    from nunchi_amd import synth
    path = synth.cached("voice", _shape(n_cb=5, n_head=20, n_head_kv=4, n_ff=3104, n_embd=288, n_vocab=80), 8,
                        model_dir)
    _play(path, 8, (2, 3), n_frames=1)


def test_pass_arguments(tiny_voice):
    """No codebooks needed: nothing is scored; a codebook twice: the same scores twice; bad codes are refused."""
    import nunchi_amd
    import oracle
    g = nunchi_amd.Voice(tiny_voice)
    o = oracle.Voice(tiny_voice, threads=2)
    h = np.random.default_rng(0).standard_normal(g.n_in).astype(np.float32)
    g.begin_frame(h)
    o.begin_frame(h)
    codes = np.full(g.n_cb, -1, np.int32)
    assert g.pass_(codes, []).shape == (0, g.n_vocab)
    sg = g.pass_(codes, [2, 2, 7])
    assert same(sg, o.pass_(codes, [2, 2, 7])) and same(sg[0], sg[1])
    bad = codes.copy()
    bad[1] = g.n_vocab
    with pytest.raises(nunchi_amd.SeoulError):
        g.pass_(bad, [0])
    with pytest.raises(nunchi_amd.SeoulError):
        g.pass_(codes, [g.n_cb])
    with pytest.raises(nunchi_amd.SeoulError):
        g.feedback(codes)   # masked codes have no feedback row
    # the generator still works after refused calls
    assert same(g.pass_(codes, [0]), o.pass_(codes, [0]))


def test_full_voice_frame(model_dir):
    """The live voice frame's generator (6 layers, hidden 1024, FFN 4096, 8 codebooks x 2048 codes, 16/4 heads x
    64), passes of 4 + 4 codebooks."""
    from nunchi_amd import synth
    path = synth.cached("voice", synth.VOICE, 1, model_dir)
    _play(path, 11, (4, 4), n_frames=1, threads=8)


def test_device_sampling(tiny_voice):
    """sh_voice_sample against the oracle's pick (imi/core/talk.cpp:147-164) on the same pass scores, in a talk loop:
    a shuffled codebook order per frame, passes of 4 + 4, the repeat-penalty window of the last 64 frames (seeded
    with 70 frames of codes that repeat and hold -1), temperatures 0.4 and 1.5, rep 1.2. Picks are equal; keep
    (1 - p[end-of-audio] / sum) agrees within 1e-12 (the device's double exp and the C library's may differ in the
    last place)."""
    import nunchi_amd
    import oracle
    g = nunchi_amd.Voice(tiny_voice)
    rng = np.random.default_rng(21)
    hist = [rng.integers(-1, 12, g.n_cb).astype(np.int32) for _ in range(70)]
    for f in range(6):
        temp = 0.4 if f % 2 == 0 else 1.5
        order = rng.permutation(g.n_cb).astype(np.int32)
        codes = np.full(g.n_cb, -1, np.int32)
        g.begin_frame(rng.standard_normal(g.n_in).astype(np.float32))
        window = np.array(hist[-64:], np.int32)
        for k in (0, 4):
            need = order[k:k + 4]
            sg = g.pass_(codes, need)
            if k:   # the same pass again, its scores left on the device and not waited for
                assert g.pass_(codes, need, scores=False) is None
            u = rng.uniform(size=4)
            picks, keep = g.sample(window, u, temp, 1.2)
            po, ko, _ = oracle.voice_sample(sg, need, window, u, temp, 1.2)
            assert np.array_equal(picks, po), f"frame {f}, codebooks {need.tolist()}: {picks} vs {po}"
            assert np.all(np.abs(keep - ko) <= 1e-12), f"frame {f}: keep {keep} vs {ko}"
            codes[need] = picks
        hist.append(codes.copy())
    # the draws must lie in [0, 1)
    g.pass_(codes, [0, 1])
    with pytest.raises(nunchi_amd.SeoulError):
        g.sample(np.zeros((0, g.n_cb), np.int32), [0.5, 1.0])
    assert g.sample(np.zeros((0, g.n_cb), np.int32), [0.0, 0.0])[0].tolist() == [0, 0]
    # a pass is sampled once: its score rows now hold the penalised scores
    with pytest.raises(nunchi_amd.SeoulError):
        g.sample(np.zeros((0, g.n_cb), np.int32), [0.0, 0.0])


def test_device_sampling_ragged_vocab(model_dir):
    """90 codes per codebook (not a multiple of the sampler's 16-code blocks): draws near 1 land in the last,
    partial block; picks equal the oracle's."""
    import nunchi_amd
    import oracle
    from nunchi_amd import synth
    path = synth.cached("voice", _shape(n_vocab=90), 9, model_dir)
    g = nunchi_amd.Voice(path)
    rng = np.random.default_rng(9)
    codes = np.full(g.n_cb, -1, np.int32)
    g.begin_frame(rng.standard_normal(g.n_in).astype(np.float32))
    hist = rng.integers(0, 90, (5, g.n_cb)).astype(np.int32)
    for u in ([0.999999, 0.99, 0.5, 0.0], [1.0 - 2.0 ** -30, 0.75, 0.25, 0.9999]):
        need = np.arange(4, dtype=np.int32)
        sg = g.pass_(codes, need)
        picks, keep = g.sample(hist, u, 3.0, 1.2)
        po, ko, _ = oracle.voice_sample(sg, need, hist, u, 3.0, 1.2)
        assert np.array_equal(picks, po), f"{picks} vs {po}"
        assert np.all(np.abs(keep - ko) <= 1e-12)
