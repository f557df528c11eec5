"""GPU parity on the shape of the released Seoul brain files (imi/core/seoul.cpp:93-142 reads it from their keys):
24 layers, 16 query / 4 key-value heads of 128, FFN 7680 (a 240-block down table), a 7-tap short conv, rope_freqs
divisors, sliding-window layers with a window of 256 taken from the pattern key, and a Q6_K tied word table of
97,496 rows. Hidden states and word scores are compared bit for bit with the oracle over a prefill longer than the
window, single steps and step2 past it, and 64 device-side greedy ids.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

N_CTX = 512


def same(a, b) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module")
def real_model(model_dir):
    from nunchi_amd import synth
    return synth.cached("brain", synth.REAL_SEOUL, 51, model_dir), synth.REAL_SEOUL


@pytest.fixture(scope="module")
def engines(real_model):
    import nunchi_amd
    import oracle
    path, shape = real_model
    g = nunchi_amd.Brain(path, n_ctx=N_CTX)
    o = oracle.Engine(path, threads=16, n_ctx=N_CTX)
    return g, o, shape


def _prompt(n, vocab, seed):
    return np.random.default_rng(seed).integers(0, vocab, size=n).astype(np.int32)


def test_real_shape_loads(engines):
    g, _, shape = engines
    assert (g.n_embd, g.n_head, g.n_head_kv, g.head_dim, g.n_vocab) == (2048, 16, 4, 128, 97496)
    assert g.info.n_ff == 7680 and g.info.d_conv == 6 and g.info.n_swa == 256 and g.n_attn == 8


def test_real_prefill_steps_greedy(engines):
    """A 300-token prefill (past the 256 window), 8 single steps behind it, 64 greedy ids, then one more step."""
    g, o, shape = engines
    toks = _prompt(300, shape.n_vocab, 52)
    hg, lg, bg, hall_g = g.step_batch(toks, hidden_all=True)
    ho, lo, hall_o = o.step_batch(toks, hidden_all=True)
    for p in range(len(toks)):
        assert same(hall_g[p], hall_o[p]), p
    assert same(lg, lo)
    for i, t in enumerate(_prompt(8, shape.n_vocab, 53)):
        hg, lg, bg = g.step(int(t))
        ho, lo = o.step(int(t))
        assert same(hg, ho) and same(lg, lo), i
    ids_g, _ = g.generate(bg, 64)
    ids_o, _ = o.greedy(bg, 64)
    assert np.array_equal(ids_g, ids_o), int(np.argmax(ids_g != ids_o))
    hg, lg, _ = g.step(int(ids_g[-1]))
    ho, lo = o.step(int(ids_o[-1]))
    assert same(hg, ho) and same(lg, lo)


def test_real_step2(engines):
    """Two conversations per step from position 0, word scores on both every other step."""
    g, o, shape = engines
    ga, gb = g.new_state(), g.new_state()
    ob = o.new_state()
    o.swap_state(o.new_state())   # the oracle's own conversation starts over at position 0 (as ga does)
    ta, tb = _prompt(12, shape.n_vocab, 54), _prompt(12, shape.n_vocab, 55)
    for i in range(12):
        (ha, la, _), (hb, lb, _) = g.step2(int(ta[i]), None, True, gb, int(tb[i]), None, i % 2 == 0, a=ga)
        hoa, loa, hob, lob = o.step2(int(ta[i]), None, True, ob, int(tb[i]), None, i % 2 == 0)
        assert same(ha, hoa) and same(hb, hob) and same(la, loa), i
        if i % 2 == 0:
            assert same(lb, lob), i


def test_real_shape_down_cut_in_its_own_prologue(real_model, monkeypatch):
    """SEOUL_HIP_PRECUT=0: the 240-block down table cuts its input in its own prologue (the 256-block cut body with the
    runtime block count) instead of taking gate|up's cut; the same numbers bit for bit."""
    import nunchi_amd
    import oracle
    path, shape = real_model
    monkeypatch.setenv("SEOUL_HIP_PRECUT", "0")   # read when the context is created
    g = nunchi_amd.Brain(path, n_ctx=64)
    o = oracle.Engine(path, threads=16, n_ctx=64)
    for i, t in enumerate(_prompt(6, shape.n_vocab, 56)):
        hg, lg, bg = g.step(int(t))
        ho, lo = o.step(int(t))
        assert same(hg, ho) and same(lg, lo), i
    ids_g, _ = g.generate(bg, 16)
    ids_o, _ = o.greedy(bg, 16)
    assert np.array_equal(ids_g, ids_o)
