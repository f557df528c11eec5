"""GPU greedy pick against imi's rule (imi/core/hear.cpp:67-68: best = 0, then v replaces it only if
logits[v] > logits[best]) on word tables (Q4_0 and Q6_K) edited to force the cases random scores never reach: an exact tie at the
maximum (rows copied, so their scores are bit-identical) between workgroups and inside one 8-row group, a NaN
score at index 0 (imi keeps 0), and a NaN at the maximum (imi skips it). The prompt never reads an edited row, so
the hidden states, and every score but the edited rows', are those of the unedited model. Steps run with sh_step /
sh_step2, whose pick is returned to the host and never fed back into a device read."""
import dataclasses

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

PROMPT = [101, 202, 303, 404, 505, 606]


def _shape(edits=(), vocab_type="q4_0"):
    from nunchi_amd import synth
    return synth.BrainShape(n_layer=4, attn_layers=(1, 3), n_vocab=4096, vocab_edits=tuple(edits), vocab_type=vocab_type)


@pytest.fixture(scope="module", params=["q4_0", "q6_k"])
def vocab_type(request):
    """The word table as BASELINE's synthetic model has it (Q4_0) and as imi's engine requires it (Q6_K)."""
    return request.param


def _oracle_scores(path):
    import oracle
    o = oracle.Engine(path, threads=4, n_ctx=64)
    for t in PROMPT[:-1]:
        o.step(t, want_logits=False)
    return o.step(PROMPT[-1])[1]


def _gpu_pick(path, two=False):
    import nunchi_amd
    g = nunchi_amd.Brain(path, n_ctx=64)
    if not two:
        for t in PROMPT[:-1]:
            g.step(t, want_logits=False)
        _, lg, best = g.step(PROMPT[-1])
        return lg, best
    b = g.new_state()
    for i, t in enumerate(PROMPT):
        last = i == len(PROMPT) - 1
        (_, la, ba), (_, lb, bb) = g.step2(t, None, last, b, t, None, last)
    return la, ba, lb, bb


def _same_scores(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb_ = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb_) and np.array_equal(a[~na].view(np.uint32), b[~nb_].view(np.uint32))


@pytest.fixture(scope="module")
def base_top(model_dir, vocab_type):
    from nunchi_amd import synth
    import oracle
    path = synth.cached("brain", _shape((), vocab_type), 11, model_dir)
    lg = _oracle_scores(path)
    r = oracle.top(lg)
    masked = lg.copy()
    masked[r] = -np.inf
    return r, oracle.top(masked)


def _cases(r, second):
    low = 7 if r > 7 else r + 9          # a row below the maximum (or just after it), read by no prompt token
    cases = [("tie across workgroups", (("copy", r, low),), min(low, r)),
             ("nan at index 0", (("nan", 0),), 0),
             ("nan at the maximum", (("nan", r),), second)]
    if r % 8 != 0 and r - 1 not in PROMPT:
        cases.append(("tie inside an 8-row group", (("copy", r, r - 1),), r - 1))
    return cases


def test_greedy_pick_ties_and_nan(model_dir, base_top, vocab_type):
    from nunchi_amd import synth
    import oracle
    r, second = base_top
    for name, edits, want in _cases(r, second):
        path = synth.cached("brain", _shape(edits, vocab_type), 11, model_dir)
        lo = _oracle_scores(path)
        assert oracle.top(lo) == want, name
        lg, best = _gpu_pick(path)
        assert _same_scores(lg, lo), name
        assert best == want, (name, best, want)


def test_greedy_pick_ties_two_conversations(model_dir, base_top, vocab_type):
    from nunchi_amd import synth
    r, second = base_top
    for name, edits, want in _cases(r, second)[:2]:
        path = synth.cached("brain", _shape(edits, vocab_type), 11, model_dir)
        la, ba, lb, bb = _gpu_pick(path, two=True)
        assert ba == want and bb == want, (name, ba, bb, want)
        assert _same_scores(la, lb)
