"""GPU parity of the brain step (C ABI: sh_step / sh_step2 / sh_step_batch / sh_generate) against the oracle.

The oracle is the CPU restatement of imi's engine (imi/core/seoul.cpp). The HIP path keeps every fp32 operation of
imi's AVX2 arithmetic in the same order (per-row GEMV chains, the AVX2 reduction orders of the norms and dot
products, the C library's expf, the fp16 cache), so its hidden states and word scores are bit for bit the oracle's;
the tests hold it to that, which is stricter than the north star's 1e-3 relative L2 and same greedy ids. Bitwise
equality matters: imi cuts every table input to int8, so a one-ulp difference anywhere can flip a code and move the
scores by ~1e-3.
"""
import numpy as np
import pytest

from conftest import rel

pytestmark = pytest.mark.gpu

def same(a, b) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _prompt(n, vocab, seed):
    return np.random.default_rng(seed).integers(0, vocab, size=n).astype(np.int32)


def _compare_steps(path, tokens, n_ctx=256, threads=4):
    import nunchi_amd
    import oracle
    g = nunchi_amd.Brain(path, n_ctx=n_ctx)
    o = oracle.Engine(path, threads=threads, n_ctx=n_ctx)
    for i, t in enumerate(tokens):
        hg, lg, bg = g.step(int(t))
        ho, lo = o.step(int(t))
        assert same(hg, ho), f"hidden differs at position {i} (rel {rel(hg, ho):.2e})"
        assert same(lg, lo), f"word scores differ at position {i} (rel {rel(lg, lo):.2e})"
        assert bg == oracle.top(lo) == int(np.argmax(lg))


def test_tiny_model_steps(tiny_model):
    _compare_steps(tiny_model, _prompt(40, 1000, 1))


def test_seoul_width_steps(mid_model):
    _compare_steps(mid_model, _prompt(24, 4096, 2))


def test_embedding_input_and_no_logits(tiny_model):
    import nunchi_amd
    import oracle
    g = nunchi_amd.Brain(tiny_model, n_ctx=64)
    o = oracle.Engine(tiny_model, threads=2, n_ctx=64)
    rng = np.random.default_rng(4)
    for i in range(6):
        e = rng.standard_normal(g.n_embd).astype(np.float32)
        want = i % 2 == 0
        hg, lg, bg = g.step(-1, e, want_logits=want)
        ho, lo = o.step(-1, e, want_logits=want)
        assert same(hg, ho)
        if want:
            assert same(lg, lo) and bg == oracle.top(lo)
        else:
            assert lg is None and bg == -1


def test_step2_equals_two_steps(tiny_model):
    """imi/core/seoul.cpp:222-224: each conversation of step2 gets exactly its own step's numbers."""
    import nunchi_amd
    g = nunchi_amd.Brain(tiny_model, n_ctx=64)
    b = g.new_state()
    a1, b1 = g.new_state(), g.new_state()
    ta, tb = _prompt(12, 1000, 5), _prompt(12, 1000, 6)
    rng = np.random.default_rng(7)
    for i in range(12):
        eb = rng.standard_normal(g.n_embd).astype(np.float32) if i % 3 == 2 else None
        tok_b = -1 if eb is not None else int(tb[i])
        (ha, la, ba), (hb, lb, bb) = g.step2(int(ta[i]), None, True, b, tok_b, eb, i % 2 == 0)
        ha1, la1, ba1 = g.step(int(ta[i]), st=a1)
        hb1, lb1, bb1 = g.step(tok_b, eb, want_logits=i % 2 == 0, st=b1)
        assert np.array_equal(ha, ha1) and np.array_equal(la, la1) and ba == ba1
        assert np.array_equal(hb, hb1) and bb == bb1
        if i % 2 == 0:
            assert np.array_equal(lb, lb1)
    assert g.pos == 12 and b.pos == 12


def test_step2_matches_oracle(mid_model):
    import nunchi_amd
    import oracle
    g = nunchi_amd.Brain(mid_model, n_ctx=64)
    o = oracle.Engine(mid_model, threads=4, n_ctx=64)
    gb, ob = g.new_state(), o.new_state()
    ta, tb = _prompt(10, 4096, 8), _prompt(10, 4096, 9)
    for i in range(10):
        (ha, la, ba), (hb, lb, bb) = g.step2(int(ta[i]), None, True, gb, int(tb[i]), None, True)
        hoa, loa, hob, lob = o.step2(int(ta[i]), None, True, ob, int(tb[i]), None, True)
        assert same(ha, hoa) and same(hb, hob)
        assert same(la, loa) and same(lb, lob)
        assert ba == oracle.top(loa) and bb == oracle.top(lob)


def test_step_batch_matches_oracle(tiny_model):
    import nunchi_amd
    import oracle
    g = nunchi_amd.Brain(tiny_model, n_ctx=160)
    o = oracle.Engine(tiny_model, threads=4, n_ctx=160)
    toks = _prompt(70, 1000, 10)   # more than one 64-position chunk on the oracle side
    hg, lg, bg, hall_g = g.step_batch(toks, hidden_all=True)
    ho, lo, hall_o = o.step_batch(toks, hidden_all=True)
    for p in range(len(toks)):
        assert same(hall_g[p], hall_o[p]), p
    assert same(lg, lo) and bg == oracle.top(lo)
    assert np.array_equal(hg, hall_g[-1])
    assert g.pos == 70


def test_greedy_generation_matches_oracle(mid_model):
    import nunchi_amd
    import oracle
    g = nunchi_amd.Brain(mid_model, n_ctx=128)
    o = oracle.Engine(mid_model, threads=4, n_ctx=128)
    prompt = _prompt(8, 4096, 11)
    _, _, bg, _ = g.step_batch(prompt)
    _, lo, _ = o.step_batch(prompt)
    first = oracle.top(lo)
    assert bg == first
    ids_g, secs = g.generate(first, 48)
    ids_o, _ = o.greedy(first, 48)
    assert np.array_equal(ids_g, ids_o), (ids_g, ids_o)
    assert g.pos == 8 + 48 and secs > 0


def test_greedy_two_conversations(tiny_model):
    import nunchi_amd
    import oracle
    g = nunchi_amd.Brain(tiny_model, n_ctx=96)
    o = oracle.Engine(tiny_model, threads=4, n_ctx=96)
    gb, ob = g.new_state(), o.new_state()
    ia, ib, _ = g.generate(3, 40, b=gb, first_b=977)
    oa, obb, _ = o.greedy2(ob, 3, 977, 40)
    assert np.array_equal(ia, oa) and np.array_equal(ib, obb)


def _long_greedy(path, vocab, n_ctx, n_gen, seed):
    """Prompt, n_gen greedy ids on the device and on the oracle, then one more step compared bit for bit."""
    import nunchi_amd
    import oracle
    g = nunchi_amd.Brain(path, n_ctx=n_ctx)
    o = oracle.Engine(path, threads=8, n_ctx=n_ctx)
    prompt = _prompt(8, vocab, seed)
    for t in prompt[:-1]:
        g.step(int(t), want_logits=False)
        o.step(int(t), want_logits=False)
    hg, lg, bg = g.step(int(prompt[-1]))
    ho, lo = o.step(int(prompt[-1]))
    assert same(hg, ho) and same(lg, lo) and bg == oracle.top(lo)
    ids_g, _ = g.generate(bg, n_gen)
    ids_o, _ = o.greedy(bg, n_gen)
    assert np.array_equal(ids_g, ids_o), int(np.argmax(ids_g != ids_o))
    hg, lg, _ = g.step(int(ids_g[-1]))
    ho, lo = o.step(int(ids_o[-1]))
    assert same(hg, ho) and same(lg, lo)


def test_long_context_attention(mid_model):
    """Head width 64 over 1,200 positions: several value tiles and key rows per thread in the decode attention."""
    _long_greedy(mid_model, 4096, 1280, 1200, 13)


def test_long_context_attention_narrow_heads(tiny_model):
    """Head width 32 over 600 positions."""
    _long_greedy(tiny_model, 1000, 640, 600, 14)


@pytest.mark.parametrize("shape", ["tiny", "mid"])
def test_sharp_attention_in_order_sum(model_dir, shape):
    """q/k norm weights scaled by 6: scores spread over hundreds and most e_t = expf(s_t - max) fall far below the
    double sum's last bit, so the sum has rounding steps and the kernel adds it in position order (its exact-sum
    shortcut does not apply); the default models take the shortcut."""
    from nunchi_amd import synth
    base = synth.TINY if shape == "tiny" else synth.BrainShape(n_layer=4, attn_layers=(1, 3), n_vocab=4096)
    sharp = synth.BrainShape(**{**base.__dict__, "qk_norm_scale": 6.0})
    path = synth.cached("brain", sharp, 15, model_dir)
    _long_greedy(path, sharp.n_vocab, 640, 560, 16)


def test_state_semantics(tiny_model):
    """reset / rewind / swap_state / context full (imi/core/seoul.cpp:188-209, 353)."""
    import nunchi_amd
    g = nunchi_amd.Brain(tiny_model, n_ctx=8)
    toks = _prompt(8, 1000, 12)
    first = [g.step(int(t))[1] for t in toks]
    with pytest.raises(nunchi_amd.ContextFull):
        g.step(1)
    assert g.pos == 8
    g.reset()
    assert g.pos == 0
    again = [g.step(int(t))[1] for t in toks]
    assert all(np.array_equal(a, b) for a, b in zip(first, again))
    # rewind to position 4 and replay: the K/V cache is overwritten by position, conv memory must be restored by
    # replaying from a reset, so replay from 0 with the same prefix
    other = g.new_state()
    g.swap_state(other)
    assert g.pos == 0 and other.pos == 8
    h0 = g.step(int(toks[0]))[1]
    assert np.array_equal(h0, first[0])
    g.swap_state(other)
    assert g.pos == 8


def test_full_seoul_step_and_greedy(model_dir):
    """cfg 2: the full Seoul-shaped model, a 32-token prompt, then 256 greedy ids; every id and the final state agree."""
    import nunchi_amd
    import oracle
    from nunchi_amd import synth
    path = synth.cached("brain", synth.SEOUL, 0, model_dir)
    g = nunchi_amd.Brain(path, n_ctx=512)
    o = oracle.Engine(path, threads=8, n_ctx=512)
    prompt = _prompt(32, synth.SEOUL.n_vocab, 0)
    for t in prompt[:-1]:
        g.step(int(t), want_logits=False)
        o.step(int(t), want_logits=False)
    hg, lg, bg = g.step(int(prompt[-1]))
    ho, lo = o.step(int(prompt[-1]))
    assert same(hg, ho) and same(lg, lo) and bg == oracle.top(lo)
    ids_g, _ = g.generate(bg, 255)   # 256 generated ids with bg
    ids_o, _ = o.greedy(bg, 255)
    assert np.array_equal(ids_g, ids_o)
    # and the state after the loop is the same: one more step gives identical scores
    hg, lg, _ = g.step(int(ids_g[-1]))
    ho, lo = o.step(int(ids_o[-1]))
    assert same(hg, ho) and same(lg, lo)


@pytest.mark.parametrize("shape", ["tiny", "mid"])
def test_sharp_attention_prefill(model_dir, shape):
    """The prefill's softmax on the sharp model (q/k norm weights x 6): in-order double sums, bit for bit."""
    import nunchi_amd
    import oracle
    from nunchi_amd import synth
    base = synth.TINY if shape == "tiny" else synth.BrainShape(n_layer=4, attn_layers=(1, 3), n_vocab=4096)
    sharp = synth.BrainShape(**{**base.__dict__, "qk_norm_scale": 6.0})
    path = synth.cached("brain", sharp, 15, model_dir)
    g = nunchi_amd.Brain(path, n_ctx=320)
    o = oracle.Engine(path, threads=8, n_ctx=320)
    toks = _prompt(300, sharp.n_vocab, 17)
    hg, lg, bg, hall_g = g.step_batch(toks, hidden_all=True)
    ho, lo, hall_o = o.step_batch(toks, hidden_all=True)
    for p in range(len(toks)):
        assert same(hall_g[p], hall_o[p]), p
    assert same(lg, lo) and bg == oracle.top(lo)


def test_full_seoul_two_conversations_greedy(model_dir):
    """cfg 2 at B=2: the full Seoul-shaped model, two seeded 32-token prompts through step2 (one weight read for
    both conversations, imi/core/seoul.cpp:208-350), then 256 greedy ids each from the device loop; every id of both
    conversations agrees with the oracle's greedy2, and so do the scores of one more step2."""
    import nunchi_amd
    import oracle
    from nunchi_amd import synth
    path = synth.cached("brain", synth.SEOUL, 0, model_dir)
    g = nunchi_amd.Brain(path, n_ctx=512)
    o = oracle.Engine(path, threads=8, n_ctx=512)
    pa, pb = _prompt(32, synth.SEOUL.n_vocab, 0), _prompt(32, synth.SEOUL.n_vocab, 1)
    gb, ob = g.new_state(), o.new_state()
    for i in range(32):
        last = i == 31
        (hga, lga, bga), (hgb, lgb, bgb) = g.step2(int(pa[i]), None, last, gb, int(pb[i]), None, last)
        hoa, loa, hob, lob = o.step2(int(pa[i]), None, last, ob, int(pb[i]), None, last)
        assert same(hga, hoa) and same(hgb, hob), i
    assert same(lga, loa) and same(lgb, lob)
    assert bga == oracle.top(loa) and bgb == oracle.top(lob)
    ids_ga, ids_gb, _ = g.generate(bga, 256, b=gb, first_b=bgb)
    ids_oa, ids_ob, _ = o.greedy2(ob, bga, bgb, 256)
    assert np.array_equal(ids_ga, ids_oa) and np.array_equal(ids_gb, ids_ob)
    (hga, lga, _), (hgb, lgb, _) = g.step2(int(ids_ga[-1]), None, True, gb, int(ids_gb[-1]), None, True)
    hoa, loa, hob, lob = o.step2(int(ids_oa[-1]), None, True, ob, int(ids_ob[-1]), None, True)
    assert same(hga, hoa) and same(lga, loa) and same(hgb, hob) and same(lgb, lob)


def test_voice_frame_brain_half_long_context(model_dir):
    """cfg 4's brain half (imi/core/flow.cpp:118, imi/core/seoul.cpp:208-350): the full Seoul-shaped model with a
    4096-position context; slot A is prefilled to position 2048 with seeded words, slot B (the voice slot) with 24
    embedding rows; then frames of step2 with A a greedy text step with scores and B a brain step fed an input
    vector (the feedback row sum's place) without scores. Hidden states, A's scores and picks are bit for bit the
    oracle's at every frame."""
    import nunchi_amd
    import oracle
    from nunchi_amd import synth
    path = synth.cached("brain", synth.SEOUL, 0, model_dir)
    n_ctx = 4096
    g = nunchi_amd.Brain(path, n_ctx=n_ctx)
    o = oracle.Engine(path, threads=8, n_ctx=n_ctx)
    words = _prompt(2048, synth.SEOUL.n_vocab, 21)
    hg, lg, bg, _ = g.step_batch(words)
    ho, lo, _ = o.step_batch(words)
    assert same(hg, ho) and same(lg, lo) and bg == oracle.top(lo)
    rng = np.random.default_rng(22)
    vb = rng.standard_normal((24, synth.SEOUL.n_embd)).astype(np.float32)
    gb, ob = g.new_state(), o.new_state()
    g.swap_state(gb)
    o.swap_state(ob)
    g.step_batch(embd=vb, want_logits=False)
    o.step_batch(embd=vb, want_logits=False)
    g.swap_state(gb)
    o.swap_state(ob)
    assert g.pos == 2048 and gb.pos == 24
    ta = bg
    for frame in range(6):
        fb = rng.standard_normal(synth.SEOUL.n_embd).astype(np.float32)
        (hga, lga, bga), (hgb, _, _) = g.step2(int(ta), None, True, gb, -1, fb, False)
        hoa, loa, hob, _ = o.step2(int(ta), None, True, ob, -1, fb, False)
        assert same(hga, hoa) and same(lga, loa) and same(hgb, hob), frame
        assert bga == oracle.top(loa), frame
        ta = bga
    assert g.pos == 2054 and gb.pos == 30


def test_destroy_context_before_its_states_and_tables(tiny_model):
    """The C ABI's ownership rule (include/seoul_hip.h): sh_destroy releases the device memory of the context's
    remaining states and tables and detaches their handles; sh_state_free / sh_q4_free afterwards only free the
    handles. Called in that order through the raw C functions, every call returns SH_OK, and a fresh context then
    steps as before."""
    import ctypes as C
    import nunchi_amd
    L = nunchi_amd.load_library()
    ctx, st, tab = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert L.sh_create(0, C.byref(ctx)) == 0
    assert L.sh_load(ctx, tiny_model.encode(), 32) == 0
    assert L.sh_state_new(ctx, C.byref(st)) == 0
    q = np.ascontiguousarray(__import__("conftest").q4_random(64, 256, 3))
    assert L.sh_q4_create(ctx, q.ctypes.data_as(C.c_void_p), 64, 256, C.byref(tab)) == 0
    h = np.zeros(256, np.float32)
    assert L.sh_step(ctx, st, 5, None, 0, h.ctypes.data_as(C.c_void_p), None, None) == 0
    assert L.sh_destroy(ctx) == 0
    assert L.sh_state_free(st) == 0
    assert L.sh_q4_free(tab) == 0
    g = nunchi_amd.Brain(tiny_model, n_ctx=32)
    h2 = g.step(5, want_logits=False)[0]
    assert same(h, h2)
