"""Pins of the oracle's engine (imi/core/seoul.cpp, imi/core/voice.cpp restated) at the model level:

- against the float64 restatement of imi/ref/ref_exact.py with imi's int8 cuts and fp16 cache applied at the same
  points (exact.brain(cut=True)), the cuts teacher-forced: the float64 model takes the engine's own int8 codes and
  fp16 keys and values after checking each as a rounding of its own float64 value (so a code the two arithmetics
  round apart, an fp32 value within rounding of a boundary, cannot move the positions after it). What remains is
  fp32 rounding, ~1e-6, for any model seed; without the cuts the gap is the cut error itself (a few per cent on
  random weights), and the greedy choice agrees
- the voice generator against imi/ref/gen_exact.py restated (no input cut: ~1e-6)
- invariants the reference states: results independent of thread count (imi/core/team.h, seoul.cpp:370-379),
  step2 == two steps (seoul.cpp:222-224), step_batch == n steps, reset, context full (seoul.cpp:353)
"""
import numpy as np
import pytest

import oracle
from conftest import rel
# (the float64 restatements stay off the GPU box: without them this CPU-only module is skipped)
exact = pytest.importorskip("oracle.exact")


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def forced_run(path, tokens=None, embd=None, threads=3):
    """The oracle's single steps over a sequence with its cut trace on, and the float64 model teacher-forced with
    those cuts: (hidden [T][E], scores [T][V]) of each, and the number of forced codes that differ from the float64
    values' own rounding."""
    n = len(tokens) if tokens is not None else len(embd)
    e = oracle.Engine(path, threads=threads, n_ctx=max(32, n))
    e.trace_cuts(True)
    hs, ls = [], []
    for i in range(n):
        h, lg = e.step(int(tokens[i]) if tokens is not None else -1, None if embd is None else embd[i])
        hs.append(h)
        ls.append(lg)
    n_attn = sum(1 for il in range(e.n_layer) if _is_attn(path, il))
    forced = {"cuts": e.take_cuts(), "kv": {ai: e.kv_cache(ai) for ai in range(n_attn)}}
    hid_c, lg_c = exact.brain(path, tokens=tokens, embd=embd, cut=True, forced=forced)
    return np.array(hs), np.array(ls), hid_c, lg_c, forced["flips"]


def _is_attn(path, il):
    from nunchi_amd.gguf import GGUFFile
    return f"blk.{il}.attn_q.weight" in GGUFFile(path).tensors


def test_engine_vs_float64_truth(tiny_model):
    toks = [5, 17, 300, 999, 0, 42, 42, 7, 640, 77, 3, 500]
    hs, ls, hid_c, lg_c, _ = forced_run(tiny_model, tokens=toks)
    hid_x, lg_x = exact.brain(tiny_model, tokens=toks, cut=False)
    for i in range(len(toks)):
        assert rel(hs[i], hid_c[i]) < 5e-6 and rel(ls[i], lg_c[i]) < 5e-6, i
        assert rel(hs[i], hid_x[i]) < 0.15
        assert oracle.top(ls[i]) == int(np.argmax(lg_c[i]))


def test_engine_embedding_input_vs_truth(tiny_model):
    emb = np.random.default_rng(3).standard_normal((6, 256)).astype(np.float32)
    hs, ls, hid_c, lg_c, _ = forced_run(tiny_model, embd=emb)
    for i in range(len(emb)):
        assert rel(hs[i], hid_c[i]) < 5e-6 and rel(ls[i], lg_c[i]) < 5e-6, i


def test_forced_cuts_are_checked():
    """The teacher-forced cut takes only codes that round the float64 values: a code off by one away from a
    rounding boundary, or an fp16 key one ulp off, is refused."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, 64))
    d = np.abs(x.astype(np.float32)).reshape(3, 2, 32).max(-1, keepdims=True) / np.float32(127)
    own = np.rint(x.reshape(3, 2, 32) / d.astype(np.float64)).astype(np.int8).reshape(3, 64)
    out, flips = exact.forced_cut(x, own)
    assert flips == 0 and np.abs(out - x).max() <= 0.51 * float(d.max())
    r = (x.reshape(3, 2, 32) / d.astype(np.float64)).reshape(3, 64)
    j = int(np.argmax(np.abs(np.abs(r - np.rint(r)) - 0.5)))   # the value farthest from a boundary
    bad = own.copy()
    bad.flat[j] += 1 if bad.flat[j] < 127 else -1
    with pytest.raises(AssertionError):
        exact.forced_cut(x, bad)
    k = rng.standard_normal((2, 4, 64))
    h = k.astype(np.float16)
    assert np.array_equal(exact.forced_half(k, h.view(np.uint16)), h.astype(np.float64))
    off = h.copy()
    off[1, 2, 5] = np.nextafter(off[1, 2, 5], np.float16(np.inf))
    with pytest.raises(AssertionError):
        exact.forced_half(k, off.view(np.uint16))


def test_voice_pass_vs_truth(tiny_voice):
    v = oracle.Voice(tiny_voice, threads=3)
    h = np.random.default_rng(0).standard_normal(v.n_in).astype(np.float32)
    v.begin_frame(h)
    for codes, need in [([-1] * 8, list(range(8))), ([3, -1, 5, -1, 100, 200, -1, 7], [1, 3, 6])]:
        codes = np.array(codes, np.int32)
        out = v.pass_(codes, need)
        truth = exact.voice_pass(tiny_voice, h, codes)[need]
        assert rel(out, truth) < 1e-5
        assert all(oracle.top(out[j]) == int(np.argmax(truth[j])) for j in range(len(need)))


def test_voice_feedback_is_row_sum(tiny_voice):
    from nunchi_amd.gguf import GGUFFile
    v = oracle.Voice(tiny_voice, threads=1)
    codes = np.array([0, 5, 17, 255, 1, 2, 3, 4], np.int32)
    fb = v.feedback(codes)
    t = GGUFFile(tiny_voice).tensors["a.gen.code.out_embd.weight"]
    rows = exact.dequant_q8_0(t.data, t.rows, t.ne[0])
    want = np.zeros(v.n_in, np.float32)
    for c in range(v.n_cb):
        want += rows[codes[c] + c * v.n_vocab].astype(np.float32)
    assert np.array_equal(fb, want)


def test_thread_count_independent(tiny_model):
    a = oracle.Engine(tiny_model, threads=1, n_ctx=16)
    b = oracle.Engine(tiny_model, threads=7, n_ctx=16)
    for t in (1, 2, 3, 500, 999):
        ha, la = a.step(t)
        hb, lb = b.step(t)
        assert _same(ha, hb) and _same(la, lb)


def test_step2_equals_two_steps(tiny_model):
    e = oracle.Engine(tiny_model, threads=3, n_ctx=16)
    a1 = oracle.Engine(tiny_model, threads=3, n_ctx=16)
    b1 = oracle.Engine(tiny_model, threads=3, n_ctx=16)
    sb = e.new_state()
    rng = np.random.default_rng(5)
    for i in range(6):
        ta, tb = int(rng.integers(0, 1000)), int(rng.integers(0, 1000))
        ha, la, hb, lb = e.step2(ta, None, True, sb, tb, None, i % 2 == 0)
        ha1, la1 = a1.step(ta)
        hb1, lb1 = b1.step(tb, want_logits=i % 2 == 0)
        assert _same(ha, ha1) and _same(la, la1) and _same(hb, hb1)
        if i % 2 == 0:
            assert _same(lb, lb1)
    assert e.pos == 6 and sb.pos == 6


def test_step_batch_equals_steps(tiny_model):
    toks = np.random.default_rng(6).integers(0, 1000, size=70).astype(np.int32)
    a = oracle.Engine(tiny_model, threads=4, n_ctx=128)
    b = oracle.Engine(tiny_model, threads=4, n_ctx=128)
    hl, lg, hall = a.step_batch(toks, hidden_all=True)
    for p, t in enumerate(toks):
        h, l = b.step(int(t), want_logits=p == len(toks) - 1)
        assert _same(hall[p], h), p
    assert _same(lg, l) and _same(hl, hall[-1]) and a.pos == 70


def test_reset_and_context_full(tiny_model):
    e = oracle.Engine(tiny_model, threads=2, n_ctx=4)
    first = [e.step(t)[1] for t in (1, 2, 3, 4)]
    assert e.pos == 4
    e.step(5)          # context full: prints and does not step
    assert e.pos == 4
    e.reset()
    again = [e.step(t)[1] for t in (1, 2, 3, 4)]
    assert all(_same(x, y) for x, y in zip(first, again))


@pytest.mark.parametrize("seed", [41, 1, 2])
def test_engine_q4_1_tables_vs_float64_truth(model_dir, seed):
    """Every layer table Q4_1: the restatement against the float64 model with the cuts applied (teacher-forced); a
    wrong m term would show at the first position."""
    from nunchi_amd import synth
    shape = synth.BrainShape(**{**synth.TINY.__dict__, "layer_type": "q4_1"})
    path = synth.cached("brain", shape, seed, model_dir)
    hs, ls, hid_c, lg_c, _ = forced_run(path, tokens=FEATURE_TOKENS)
    for i in range(len(FEATURE_TOKENS)):
        assert rel(hs[i], hid_c[i]) < 5e-6 and rel(ls[i], lg_c[i]) < 5e-6, i


def _feature_shape(**kw):
    from nunchi_amd import synth
    return synth.BrainShape(**{**synth.TINY.__dict__, **kw})


FEATURES = {
    # rope_freqs angle divisors (imi/core/seoul.cpp:19-28 with ff, ref_exact.py:41-48)
    "rope_freqs": dict(rope_freqs=True),
    # a sliding window of 3 positions on attention layer 1, its own RoPE base and no divisors (seoul.cpp:99-114,
    # 288-295, 428-431); layer 3 stays global
    "sliding_window": dict(sliding_window=3, swa_layers=(1,), rope_freqs=True),
    # 7-tap short conv: 6 positions of conv memory (seoul.cpp:136-142, 407-423)
    "conv_7_taps": dict(conv_kernel=7),
    # head_dim 128: 8 query heads over 2 kv heads (a 1024-wide attention over n_embd 256; q|k|v|gate rows stay a
    # multiple of 8, as imi's table build requires)
    "head_dim_128": dict(n_head=8, n_head_kv=2, head_dim=128),
}
FEATURE_TOKENS = [5, 17, 300, 999, 0, 42, 640, 77, 3, 500, 12, 801]


@pytest.mark.parametrize("seed", [1, 2, 3])
@pytest.mark.parametrize("feature", sorted(FEATURES))
def test_engine_feature_paths_vs_float64_truth(model_dir, feature, seed):
    """The oracle's loader-feature paths against the float64 restatement with the cuts applied (teacher-forced),
    position by position past the window (12 positions, window 3), every position within 5e-6 for every model seed.
    A wrong score scale, rope pairing or head grouping would move every position from the second on (position 0
    attends to itself alone, at angle 0)."""
    from nunchi_amd import synth
    path = synth.cached("brain", _feature_shape(**FEATURES[feature]), seed, model_dir)
    hs, ls, hid_c, lg_c, _ = forced_run(path, tokens=FEATURE_TOKENS)
    errs = [max(rel(hs[i], hid_c[i]), rel(ls[i], lg_c[i])) for i in range(len(FEATURE_TOKENS))]
    assert max(errs) < 5e-6, errs


@pytest.mark.parametrize("dropped", ["sliding_window", "rope_freqs"])
def test_feature_pins_see_the_feature(model_dir, dropped):
    """The pins above discriminate: the oracle on the windowed model (or the one with angle divisors) against the
    float64 truth of the same weights without the window (or the divisors), teacher-forced with the oracle's own
    cuts, either refuses the cuts (a forced code or fp16 key is no rounding of the truth's value) or is far outside
    the bound once the window is passed (or from the second position)."""
    from nunchi_amd import synth
    kw = FEATURES["sliding_window"]
    path = synth.cached("brain", _feature_shape(**kw), 44, model_dir)
    other = dict(kw, sliding_window=0) if dropped == "sliding_window" else dict(kw, rope_freqs=False, swa_layers=())
    path_other = synth.cached("brain", _feature_shape(**other), 44, model_dir)
    e = oracle.Engine(path, threads=3, n_ctx=32)
    e.trace_cuts(True)
    hs = [e.step(t)[0] for t in FEATURE_TOKENS]
    forced = {"cuts": e.take_cuts(), "kv": {ai: e.kv_cache(ai) for ai in range(2)}}
    try:
        hid_o, _ = exact.brain(path_other, tokens=FEATURE_TOKENS, cut=True, forced=forced)
    except AssertionError:
        return
    worst = max(rel(h, hid_o[i]) for i, h in enumerate(hs))
    assert worst > 1e-3, (dropped, worst)
