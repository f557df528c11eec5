"""GPU parity on model features the real Seoul files use beyond BASELINE's synthetic shape (imi/core/seoul.cpp:99-114,
136-142, 288-295, 428-431): rope_freqs angle divisors, sliding-window attention layers (window, pattern and their
own RoPE base, no divisors), and a 7-tap short conv (6 positions of conv memory). Every hidden state and score is
compared bit for bit with the oracle, on single steps past the window, step2, device-side greedy ids and a prefill
longer than the window, through the graph of per-table kernels.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def same(a, b) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module", params=["tiny", "mid"])
def feat_model(request, model_dir):
    from nunchi_amd import synth
    base = synth.TINY if request.param == "tiny" else synth.BrainShape(n_layer=4, attn_layers=(1, 3), n_vocab=4096)
    shape = synth.BrainShape(**{**base.__dict__, "n_layer": 5, "attn_layers": (1, 2, 4), "conv_kernel": 7,
                                "rope_freqs": True, "sliding_window": 16, "swa_layers": (1, 4)})
    return synth.cached("brain", shape, 31, model_dir), shape


def _prompt(n, vocab, seed):
    return np.random.default_rng(seed).integers(0, vocab, size=n).astype(np.int32)


def test_features_steps_and_greedy(feat_model):
    import nunchi_amd
    import oracle
    path, shape = feat_model
    g = nunchi_amd.Brain(path, n_ctx=128)
    o = oracle.Engine(path, threads=4, n_ctx=128)
    for i, t in enumerate(_prompt(40, shape.n_vocab, 32)):   # past the 16-position window
        hg, lg, bg = g.step(int(t))
        ho, lo = o.step(int(t))
        assert same(hg, ho) and same(lg, lo), i
    ids_g, _ = g.generate(bg, 48)
    ids_o, _ = o.greedy(bg, 48)
    assert np.array_equal(ids_g, ids_o)


def test_features_step2(feat_model):
    import nunchi_amd
    import oracle
    path, shape = feat_model
    g = nunchi_amd.Brain(path, n_ctx=64)
    o = oracle.Engine(path, threads=4, n_ctx=64)
    gb, ob = g.new_state(), o.new_state()
    ta, tb = _prompt(24, shape.n_vocab, 33), _prompt(24, shape.n_vocab, 34)
    for i in range(24):
        (ha, la, _), (hb, lb, _) = g.step2(int(ta[i]), None, True, gb, int(tb[i]), None, i % 3 == 0)
        hoa, loa, hob, lob = o.step2(int(ta[i]), None, True, ob, int(tb[i]), None, i % 3 == 0)
        assert same(ha, hoa) and same(hb, hob) and same(la, loa), i
        if i % 3 == 0:
            assert same(lb, lob), i


def test_features_prefill(feat_model):
    import nunchi_amd
    import oracle
    path, shape = feat_model
    g = nunchi_amd.Brain(path, n_ctx=160)
    o = oracle.Engine(path, threads=4, n_ctx=160)
    toks = _prompt(70, shape.n_vocab, 35)
    hg, lg, bg, hall_g = g.step_batch(toks, hidden_all=True)
    ho, lo, hall_o = o.step_batch(toks, hidden_all=True)
    for p in range(len(toks)):
        assert same(hall_g[p], hall_o[p]), p
    assert same(lg, lo) and bg == oracle.top(lo)
    hg, lg, _ = g.step(7)   # and a step after it reads the prefill's caches and conv memory
    ho, lo = o.step(7)
    assert same(hg, ho) and same(lg, lo)


@pytest.fixture(scope="module", params=["tiny", "mid"])
def wide_head_model(request, model_dir):
    """head_dim 128 (the reference loader's default key_length): 8/2 heads at width 1024, 16/4 heads at 2048 (the
    q|k|v|gate rows stay a multiple of 8, as imi's table build requires)."""
    from nunchi_amd import synth
    if request.param == "tiny":
        shape = synth.BrainShape(**{**synth.TINY.__dict__, "n_embd": 1024, "n_head": 8, "n_head_kv": 2, "head_dim": 128,
                                    "n_ff": 1024})
    else:
        shape = synth.BrainShape(n_layer=4, attn_layers=(1, 3), n_head=16, n_head_kv=4, head_dim=128, n_vocab=4096)
    return synth.cached("brain", shape, 36, model_dir), shape


def test_head_dim_128_long_context(wide_head_model):
    """Single steps, then 600 device-side greedy ids (several value tiles, key rows past one pass of the block),
    then one more step compared bit for bit."""
    import nunchi_amd
    import oracle
    path, shape = wide_head_model
    g = nunchi_amd.Brain(path, n_ctx=640)
    o = oracle.Engine(path, threads=8, n_ctx=640)
    for i, t in enumerate(_prompt(8, shape.n_vocab, 37)):
        hg, lg, bg = g.step(int(t))
        ho, lo = o.step(int(t))
        assert same(hg, ho) and same(lg, lo), i
    ids_g, _ = g.generate(bg, 600)
    ids_o, _ = o.greedy(bg, 600)
    assert np.array_equal(ids_g, ids_o), int(np.argmax(ids_g != ids_o))
    hg, lg, _ = g.step(int(ids_g[-1]))
    ho, lo = o.step(int(ids_o[-1]))
    assert same(hg, ho) and same(lg, lo)


def test_head_dim_128_step2_and_prefill(wide_head_model):
    import nunchi_amd
    import oracle
    path, shape = wide_head_model
    g = nunchi_amd.Brain(path, n_ctx=160)
    o = oracle.Engine(path, threads=4, n_ctx=160)
    toks = _prompt(70, shape.n_vocab, 38)
    hg, lg, bg, hall_g = g.step_batch(toks, hidden_all=True)
    ho, lo, hall_o = o.step_batch(toks, hidden_all=True)
    for p in range(len(toks)):
        assert same(hall_g[p], hall_o[p]), p
    assert same(lg, lo) and bg == oracle.top(lo)
    gb, ob = g.new_state(), o.new_state()
    for i in range(8):
        (ha, la, _), (hb, lb, _) = g.step2(int(toks[i]), None, True, gb, int(toks[-1 - i]), None, True)
        hoa, loa, hob, lob = o.step2(int(toks[i]), None, True, ob, int(toks[-1 - i]), None, True)
        assert same(ha, hoa) and same(hb, hob) and same(la, loa) and same(lb, lob), i


@pytest.fixture(scope="module", params=["tiny", "mid"])
def q4_1_model(request, model_dir):
    """Every layer table Q4_1 (weight = code * d + m; imi/core/tables.cpp:62, 78-83, 127-143 with HAS_M)."""
    from nunchi_amd import synth
    base = synth.TINY if request.param == "tiny" else synth.BrainShape(n_layer=4, attn_layers=(1, 3), n_vocab=4096)
    shape = synth.BrainShape(**{**base.__dict__, "layer_type": "q4_1"})
    return synth.cached("brain", shape, 42, model_dir), shape


def test_q4_1_tables_steps_greedy(q4_1_model):
    import nunchi_amd
    import oracle
    path, shape = q4_1_model
    g = nunchi_amd.Brain(path, n_ctx=96)
    o = oracle.Engine(path, threads=4, n_ctx=96)
    for i, t in enumerate(_prompt(10, shape.n_vocab, 43)):
        hg, lg, bg = g.step(int(t))
        ho, lo = o.step(int(t))
        assert same(hg, ho) and same(lg, lo), i
    ids_g, _ = g.generate(bg, 48)
    ids_o, _ = o.greedy(bg, 48)
    assert np.array_equal(ids_g, ids_o)


def test_q4_1_tables_step2_and_prefill(q4_1_model):
    import nunchi_amd
    import oracle
    path, shape = q4_1_model
    g = nunchi_amd.Brain(path, n_ctx=160)
    o = oracle.Engine(path, threads=4, n_ctx=160)
    toks = _prompt(70, shape.n_vocab, 44)
    hg, lg, bg, hall_g = g.step_batch(toks, hidden_all=True)
    ho, lo, hall_o = o.step_batch(toks, hidden_all=True)
    for p in range(len(toks)):
        assert same(hall_g[p], hall_o[p]), p
    assert same(lg, lo) and bg == oracle.top(lo)
    gb, ob = g.new_state(), o.new_state()
    for i in range(6):
        (ha, la, _), (hb, lb, _) = g.step2(int(toks[i]), None, True, gb, int(toks[-1 - i]), None, True)
        hoa, loa, hob, lob = o.step2(int(toks[i]), None, True, ob, int(toks[-1 - i]), None, True)
        assert same(ha, hoa) and same(hb, hob) and same(la, loa) and same(lb, lob), i
