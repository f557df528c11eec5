"""GPU parity with a Q6_K tied word table (imi's own format, imi/core/seoul.cpp:96): the input row of a word is
imi_q6k_dequant_row (seoul.cpp:363), the word scores cut the hidden state per 256 values and score each row with
imi_q6k_row (seoul.cpp:479-487, imi/core/tables.cpp:200-287). Hidden states and scores must be bitwise the oracle's
(its restatement is pinned in tests/test_oracle_kernels.py), for single steps, step2, device-side greedy ids and
the prefill.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def same(a, b) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module", params=["tiny", "mid"])
def q6_model(request, model_dir):
    from nunchi_amd import synth
    base = synth.TINY if request.param == "tiny" else synth.BrainShape(n_layer=4, attn_layers=(1, 3), n_vocab=4096)
    shape = synth.BrainShape(**{**base.__dict__, "vocab_type": "q6_k"})
    return synth.cached("brain", shape, 21, model_dir), shape


def _prompt(n, vocab, seed):
    return np.random.default_rng(seed).integers(0, vocab, size=n).astype(np.int32)


def test_q6k_steps(q6_model):
    import nunchi_amd
    import oracle
    path, shape = q6_model
    g = nunchi_amd.Brain(path, n_ctx=64)
    o = oracle.Engine(path, threads=4, n_ctx=64)
    toks = _prompt(12, shape.n_vocab, 22)
    emb = np.random.default_rng(23).standard_normal(shape.n_embd).astype(np.float32)
    for i, t in enumerate(toks):
        if i == 5:   # an embedding row instead of a word
            hg, lg, bg = g.step(-1, embd=emb)
            ho, lo = o.step(-1, embd=emb)
        else:
            hg, lg, bg = g.step(int(t))
            ho, lo = o.step(int(t))
        assert same(hg, ho), f"hidden differs at {i}"
        assert same(lg, lo), f"scores differ at {i}"
        assert bg == oracle.top(lo)


def test_q6k_step2_and_greedy(q6_model, monkeypatch):
    import nunchi_amd
    import oracle
    path, shape = q6_model
    g = nunchi_amd.Brain(path, n_ctx=128)
    o = oracle.Engine(path, threads=4, n_ctx=128)
    gb, ob = g.new_state(), o.new_state()
    ta, tb = _prompt(6, shape.n_vocab, 24), _prompt(6, shape.n_vocab, 25)
    for i in range(6):
        (ha, la, ba), (hb, lb, bb) = g.step2(int(ta[i]), None, True, gb, int(tb[i]), None, True)
        hoa, loa, hob, lob = o.step2(int(ta[i]), None, True, ob, int(tb[i]), None, True)
        assert same(ha, hoa) and same(hb, hob) and same(la, loa) and same(lb, lob)
    ids_g, _ = g.generate(ba, 48)
    ids_o, _ = o.greedy(ba, 48)
    assert np.array_equal(ids_g, ids_o)


def test_q6k_prefill(q6_model):
    import nunchi_amd
    import oracle
    path, shape = q6_model
    g = nunchi_amd.Brain(path, n_ctx=160)
    o = oracle.Engine(path, threads=4, n_ctx=160)
    toks = _prompt(70, shape.n_vocab, 26)
    hg, lg, bg, hall_g = g.step_batch(toks, hidden_all=True)
    ho, lo, hall_o = o.step_batch(toks, hidden_all=True)
    for p in range(len(toks)):
        assert same(hall_g[p], hall_o[p]), p
    assert same(lg, lo) and bg == oracle.top(lo)
