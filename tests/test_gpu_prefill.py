"""GPU parity of the prefill (C ABI: sh_step_batch for n >= 2, sh_q4_gemm) against the oracle.

The prefill sends all positions through each table together on the int8 matrix cores: one v_mfma_i32_16x16x32_i8
per 32-column block gives each block's integer sum exactly, and the fp32 chains over the blocks, the norms, the
short conv along positions and the causal attention keep imi's operation order per position. So the tests hold it
to bit equality: with the oracle's batch kernel and step_batch (imi/core/tables.cpp:419-454, seoul.cpp:490-655),
and with n single steps on the GPU (imi's own invariant: a batch gives each position its step's numbers).
"""
import numpy as np
import pytest

from conftest import q4_random, rel

pytestmark = pytest.mark.gpu


def same(a, b) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("rows,cols,n", [(256, 2048, 1), (256, 2048, 2), (392, 256, 17), (2048, 8192, 64),
                                         (512, 2048, 130), (64, 1024, 512), (2048, 7680, 448), (64, 4608, 17)])
def test_gemm_matches_batch_kernel(rows, cols, n):
    """Matrix-core product vs the oracle's batch kernel (64 inputs at a time) and vs the GPU's own GEMV."""
    import nunchi_amd
    import oracle
    raw = q4_random(rows, cols, rows + cols + n)
    x = np.random.default_rng(n).standard_normal((n, cols)).astype(np.float32)
    x[0, :32] = 0.0                     # an all-zero block: scale 0, codes 0
    x[-1, 32:64] *= 1e-30               # tiny (subnormal-range) inputs
    ctx = nunchi_amd.Context()
    t = nunchi_amd.Q4Table(ctx, raw, rows, cols)
    y = t.gemm(x)
    o = oracle.Q4Table(raw, rows, cols)
    want = np.concatenate([o.gemv_batch(x[i:i + 64]) for i in range(0, n, 64)])
    assert same(y, want), f"rel {rel(y, want):.2e}"
    for i in (0, n - 1):
        assert same(y[i], t.gemv(x[i]))


def _prompt(n, vocab, seed):
    return np.random.default_rng(seed).integers(0, vocab, size=n).astype(np.int32)


def _check_batch(path, tokens=None, embd=None, n_ctx=1024, pre=(), threads=4):
    """step_batch after `pre` single steps, vs the oracle's step_batch and vs single steps on the GPU."""
    import nunchi_amd
    import oracle
    n = len(tokens) if tokens is not None else embd.shape[0]
    g = nunchi_amd.Brain(path, n_ctx=n_ctx)
    o = oracle.Engine(path, threads=threads, n_ctx=n_ctx)
    for t in pre:
        g.step(int(t), want_logits=False)
        o.step(int(t), want_logits=False)
    hl, lg, best, ha = g.step_batch(tokens, embd, want_logits=True, hidden_all=True)
    ohl, olg, oha = o.step_batch(tokens, embd, want_logits=True, hidden_all=True)
    for p in range(n):
        assert same(ha[p], oha[p]), f"hidden of position {p} differs (rel {rel(ha[p], oha[p]):.2e})"
    assert same(hl, ohl) and same(lg, olg), f"last scores differ (rel {rel(lg, olg):.2e})"
    assert best == oracle.top(olg) and g.pos == len(pre) + n
    # the state after the batch (K/V caches, conv memory, position) continues exactly
    h2, l2, b2 = g.step(int(best))
    oh2, ol2 = o.step(int(best))
    assert same(h2, oh2) and same(l2, ol2)
    # and single steps on the GPU give the same hidden states
    s = g.new_state()
    for t in pre:
        g.step(int(t), want_logits=False, st=s)
    for p in range(min(n, 24)):
        hp, _, _ = g.step(int(tokens[p]) if tokens is not None else -1, None if embd is None else embd[p],
                          want_logits=False, st=s)
        assert same(hp, ha[p]), f"position {p}: batch and single step differ"


def test_tiny_prefill_tokens(tiny_model):
    _check_batch(tiny_model, tokens=_prompt(40, 1000, 3))


def test_tiny_prefill_after_steps_and_embeddings(tiny_model):
    """A batch that starts mid-conversation (conv memory and cache already hold positions) and mixes embedding
    rows (token < 0) with words."""
    rng = np.random.default_rng(9)
    toks = _prompt(29, 1000, 4)
    toks[::3] = -1
    embd = rng.standard_normal((29, 256)).astype(np.float32)
    _check_batch(tiny_model, tokens=toks, embd=embd, pre=_prompt(5, 1000, 5))


def test_tiny_prefill_two_positions(tiny_model):
    """n = 2 (shorter than the conv memory of 2 taps plus one)."""
    _check_batch(tiny_model, tokens=_prompt(2, 1000, 6), pre=_prompt(1, 1000, 7))


def test_prefill_chunks(tiny_model):
    """More positions than one device chunk (512): the chunks continue each other exactly."""
    _check_batch(tiny_model, tokens=_prompt(600, 1000, 8), n_ctx=700)


def test_seoul_width_prefill(mid_model):
    _check_batch(mid_model, tokens=_prompt(100, 4096, 10))


@pytest.mark.parametrize("E,heads,D,window", [(256, (8, 4), 32, 0), (256, (8, 1), 32, 0), (256, (8, 8), 32, 0),
                                              (512, (8, 4), 64, 3), (512, (8, 2), 64, 6)])
def test_prefill_head_groups_and_windows(model_dir, E, heads, D, window):
    """Query heads per kv head 2, 8 (past the matrix-core attention's 4: the VALU form) and 1, and windows shorter
    than the key ranges of a workgroup's 4 positions (their ranges then differ at both ends). The attention is as
    wide as n_embd, as in imi's files: imi's step_batch cuts the attention rows for the o table at the n_embd width it
    last set (imi/core/seoul.cpp:546-554, 623), so a narrower or wider attention would make imi's batch disagree with
    its own steps."""
    from nunchi_amd import synth
    shape = synth.BrainShape(n_embd=E, n_layer=3, attn_layers=(1, 2), n_head=heads[0], n_head_kv=heads[1],
                             head_dim=D, n_ff=512, n_vocab=1000, sliding_window=window,
                             swa_layers=(1,) if window else ())
    path = synth.cached("brain", shape, 21, model_dir)
    _check_batch(path, tokens=_prompt(45, 1000, 22), pre=_prompt(3, 1000, 23))


def test_prefill_attention_valu_form(tiny_model, monkeypatch):
    """The VALU attention (SEOUL_HIP_PF_ATTN_VALU=1, read per launch) gives the same numbers as the oracle too."""
    monkeypatch.setenv("SEOUL_HIP_PF_ATTN_VALU", "1")
    _check_batch(tiny_model, tokens=_prompt(40, 1000, 24))


def test_prefill_context_full(tiny_model):
    import nunchi_amd
    g = nunchi_amd.Brain(tiny_model, n_ctx=64)
    g.step_batch(_prompt(60, 1000, 1), want_logits=False)
    with pytest.raises(nunchi_amd.ContextFull):
        g.step_batch(_prompt(5, 1000, 2))
    assert g.pos == 60


def test_hearing_window(model_dir):
    """The hearing window on the Seoul-shaped model: 384 embedding rows (fp32 ~N(0,1)) then 64 words, one causal
    prefill of 448 positions; every hidden state and the last position's word scores vs the oracle."""
    from nunchi_amd import synth
    rng = np.random.default_rng(12)
    emb = rng.standard_normal((448, 2048)).astype(np.float32)
    toks = np.full(448, -1, np.int32)
    toks[384:] = _prompt(64, synth.SEOUL.n_vocab, 13)
    path = synth.cached("brain", synth.SEOUL, 0, model_dir)
    _check_batch(path, tokens=toks, embd=emb, n_ctx=512, threads=8)
