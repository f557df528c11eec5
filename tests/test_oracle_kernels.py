"""Pins of the oracle's kernel-level restatement (oracle/imi_cpu_kernels.cpp), each against something the restatement
does not share: numpy's IEEE conversions, integer brute force, float64 closed forms, or another code path of the
oracle whose op order the reference fixes. A dropped term, a wrong nibble or index, a transposed operand or a
wrong rounding mode fails one of these.
"""
import numpy as np
import pytest

import oracle
from conftest import q4_random
# (the float64 restatements stay off the GPU box: without them this CPU-only module is skipped)
exact = pytest.importorskip("oracle.exact")
dequant_q4_0, dequant_q8_0 = exact.dequant_q4_0, exact.dequant_q8_0

rng = np.random.default_rng(1234)


def test_h2f_exhaustive():
    """imi_h2f (imi/core/tables.cpp:20-29) over all 65,536 halves vs numpy's IEEE conversion."""
    L = oracle.lib()
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([L.orc_h2f(int(x)) for x in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f2h_round_to_nearest_even():
    L = oracle.lib()
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-8, 5, 20000),
                        np.array([0.0, -0.0, 65504.0, 65520.0, -65520.0, 1e-8, 5.9604645e-08, 2.9802322e-08,
                                  1.0009765625, 1.00048828125, np.inf, -np.inf], np.float32)]).astype(np.float32)
    got = np.array([L.orc_f2h(float(v)) for v in x], np.uint16)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_q4_0_dequant_closed_form():
    """Q4_0: value i of a block is (qs[i] & 15) - 8 for i < 16, (qs[i-16] >> 4) - 8 after, times the fp16 scale;
    checked against a per-value loop over every byte value and scale edge case."""
    from nunchi_amd.gguf import Q4_0_BLOCK
    blk = np.empty(512, dtype=Q4_0_BLOCK)
    blk["d"] = np.array([0.0, -0.0, 1.0, -2.5, 6.1e-5, 5.96e-8, 65504.0, -0.001], np.float16)[np.arange(512) % 8]
    blk["qs"] = (np.arange(512 * 16) % 256).astype(np.uint8).reshape(512, 16)
    got = dequant_q4_0(blk, 16, 1024)
    for b in range(0, 512, 37):
        d = float(blk["d"][b])
        for i in range(32):
            byte = int(blk["qs"][b][i % 16])
            code = (byte & 15) if i < 16 else (byte >> 4)
            assert got.reshape(-1, 32)[b][i] == (code - 8) * d


def _cut_numpy(x, half_away=False):
    x = x.astype(np.float32).reshape(-1, 32)
    amax = np.abs(x).max(1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    t = (x * idv[:, None]).astype(np.float32)
    q = np.sign(t) * np.floor(np.abs(t) + np.float32(0.5)) if half_away else np.rint(t)
    return q.astype(np.int32), d


def test_cut32_brute_force_and_ties():
    x = rng.standard_normal(32 * 500).astype(np.float32) * 10.0 ** rng.integers(-3, 3, 32 * 500)
    x[:32] = 0.0                                             # all-zero block: d = 0, every code 0
    x[32:64] = np.float32(127.0) * np.arange(-16, 16) / 16   # amax 127: id = 1, exact ties at .5
    x[64:96] = np.float32(0.5) * np.arange(32)               # ties 0.5, 1.5, ...
    q, d, s = oracle.cut(x)
    qn, dn = _cut_numpy(x)
    assert np.array_equal(q.astype(np.int32), qn.reshape(-1)) and np.array_equal(d, dn)
    assert np.array_equal(s, (dn * qn.sum(1).astype(np.float32)).astype(np.float32))
    assert (q[:32] == 0).all() and d[0] == 0
    assert np.abs(q.astype(int)).max() == 127


def test_q4x8_cut_rounds_half_away():
    x = np.float32(0.5) * np.arange(-32, 32, dtype=np.float32)
    x[0] = np.float32(127 * 0.5)   # amax makes id = 2, so x * id = odd integers: no ties; scale instead
    x = (np.arange(-16, 16, dtype=np.float32) + np.float32(0.5))
    x = np.concatenate([x, x * 3])
    q = np.zeros(64, np.int8); d = np.zeros(2, np.float32); corr = np.zeros(2, np.float32)
    oracle.lib().orc_q4x8_quant_in(np.ascontiguousarray(x), 64, q, d, corr)
    qn, dn = _cut_numpy(x, half_away=True)
    assert np.array_equal(q.astype(np.int32), qn.reshape(-1)) and np.array_equal(d, dn)
    assert np.array_equal(corr, (np.float32(8) * dn * qn.sum(1).astype(np.float32)).astype(np.float32))


@pytest.mark.parametrize("rows,cols", [(64, 2048), (16, 8192), (8, 32), (24, 7680)])
def test_q4_block_sums_exact(rows, cols):
    """Integer (row, block) sums of imi's 8-row layout equal an int64 brute force from the file's nibbles."""
    blk = q4_random(rows, cols, seed=rows + cols)
    x = rng.standard_normal(cols).astype(np.float32)
    t = oracle.Q4Table(blk, rows, cols)
    got = t.block_sums(x)
    q, _, _ = oracle.cut(x)
    qs = blk["qs"].reshape(rows, cols // 32, 16).astype(np.int64)
    codes = np.concatenate([qs & 15, qs >> 4], axis=-1)
    want = (codes * q.reshape(cols // 32, 32).astype(np.int64)[None]).sum(-1)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("rows,cols", [(256, 2048), (64, 8192), (24, 96)])
def test_q4_gemv_float64_and_scalar_and_two_inputs(rows, cols):
    blk = q4_random(rows, cols, seed=3 * rows + cols)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    t = oracle.Q4Table(blk, rows, cols, threads=3)
    y0, _ = t.gemv(x[0])
    ys, _ = t.gemv(x[0], scalar=True)
    assert np.array_equal(y0, ys), "AVX2 lane bookkeeping differs from the plain per-row chain"
    y2, _ = t.gemv(x)
    assert np.array_equal(y2[0], y0) and np.array_equal(y2[1], t.gemv(x[1])[0]), "group2 != 2 x group"
    yb = t.gemv_batch(x)
    assert np.array_equal(yb, y2), "group_batch != n x group"
    # the same formula in float64 on the same cut input: sum_j d_j * dx_j * (isum_j - 8 * sum q_j)
    from oracle.exact import cut_dequant
    ref = dequant_q4_0(blk, rows, cols) @ cut_dequant(x[0])
    assert np.abs(y0 - ref).max() <= 1e-5 * np.sqrt((ref ** 2).mean())


def test_q4x8_layout_and_gemv():
    rows, cols = 64, 512
    blk = q4_random(rows, cols, seed=9)
    t = oracle.Q4x8Table(blk, rows, cols)
    codes, scales = t.layout()
    qs = blk["qs"].reshape(rows, cols // 32, 16).astype(np.int64)
    file_codes = np.concatenate([qs & 15, qs >> 4], axis=-1)    # [rows][nb][32]
    c = codes.reshape(rows // 8, cols // 32, 4, 32)
    for g in range(rows // 8):
        for k in range(4):
            assert np.array_equal(c[g, :, k, :] & 15, file_codes[8 * g + 2 * k])
            assert np.array_equal(c[g, :, k, :] >> 4, file_codes[8 * g + 2 * k + 1])
    assert np.array_equal(scales.reshape(rows // 8, cols // 32, 8).transpose(0, 2, 1).reshape(rows, -1),
                          blk["d"].reshape(rows, -1).astype(np.float32))
    x = rng.standard_normal(cols).astype(np.float32)
    y, _ = t.gemv(x)
    qn, dn = _cut_numpy(x, half_away=True)
    ref = dequant_q4_0(blk, rows, cols) @ (qn * dn[:, None]).reshape(-1)
    assert np.abs(y - ref).max() <= 1e-5 * np.sqrt((ref ** 2).mean())


@pytest.mark.parametrize("C", [1, 6, 8, 12])
def test_q8g_gemm_float64(C):
    from nunchi_amd import synth
    rows, cols = 20, 256   # rows not a multiple of 8: padded group
    blk = synth.q8_0_random(np.random.default_rng(C), rows, cols)
    xt = rng.standard_normal((cols, C)).astype(np.float32)
    out = np.zeros((C, (rows + 7) // 8 * 8), np.float32)
    oracle.lib().orc_q8g_gemm(np.ascontiguousarray(blk).view(np.uint8).reshape(-1), rows, cols, np.ascontiguousarray(xt), C, out)
    ref = (dequant_q8_0(blk, rows, cols) @ xt.astype(np.float64)).T
    assert np.abs(out[:, :rows] - ref).max() <= 1e-5 * np.abs(ref).max()


def test_rms_scale_and_rope_float64():
    L = oracle.lib()
    for n in (32, 64, 2048):
        x = rng.standard_normal(n).astype(np.float32)
        got = L.orc_rms_scale(x, n, np.float32(1e-5))
        want = 1.0 / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-5)
        assert abs(got - want) <= 2e-6 * want
    D = 64
    v = rng.standard_normal(D).astype(np.float32)
    for pos in (0, 1, 17, 511):
        r = v.copy()
        L.orc_rope(r, D, pos, np.float32(1e6), None)
        ang = pos * (1e6 ** (-np.arange(D // 2) * 2.0 / D))
        c, s = np.cos(ang), np.sin(ang)
        x0, x1 = v[:D // 2].astype(np.float64), v[D // 2:].astype(np.float64)
        want = np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c])
        assert np.abs(r - want).max() <= 2e-5 * max(1.0, pos / 64)


# ---- Q6_K word table (imi/core/tables.cpp:200-287) ----

def _q6k_blocks(n, rng):
    from nunchi_amd.gguf import Q6_K_BLOCK
    b = np.zeros(n, Q6_K_BLOCK)
    b["ql"] = rng.integers(0, 256, (n, 128), dtype=np.uint8)
    b["qh"] = rng.integers(0, 256, (n, 64), dtype=np.uint8)
    b["scales"] = rng.integers(-128, 128, (n, 16), dtype=np.int8)
    b["d"] = (rng.standard_normal(n) * 1e-3).astype(np.float16)
    return b


def _q6k_values(b):
    """[n][256] 6-bit values by the GGML Q6_K layout: per 128-value half n and l < 32, the four values l, l+32,
    l+64, l+96 take ql[l] low, ql[l+32] low, ql[l] high, ql[l+32] high nibbles and bit pairs 0, 2, 4, 6 of qh[l]."""
    ql, qh = b["ql"].astype(np.int32), b["qh"].astype(np.int32)
    out = np.zeros((len(b), 256), np.int32)
    for h in range(2):
        lo, hi = ql[:, 64 * h:64 * h + 64], qh[:, 32 * h:32 * h + 32]
        base = 128 * h
        out[:, base:base + 32] = (lo[:, :32] & 15) | ((hi & 3) << 4)
        out[:, base + 32:base + 64] = (lo[:, 32:] & 15) | (((hi >> 2) & 3) << 4)
        out[:, base + 64:base + 96] = (lo[:, :32] >> 4) | (((hi >> 4) & 3) << 4)
        out[:, base + 96:base + 128] = (lo[:, 32:] >> 4) | (((hi >> 6) & 3) << 4)
    return out


def test_q6k_dequant_closed_form():
    """imi_q6k_dequant_row: y = (d * scale[e / 16]) * (value - 32) in fp32, values decoded from the format; scale
    edge cases (+-128/127, 0) and fp16 d edge cases (0, subnormal, max, negative)."""
    r = np.random.default_rng(61)
    b = _q6k_blocks(64, r)
    b["scales"][0] = np.array([-128, 127, 0, 1, -1] + [64] * 11, np.int8)
    b["d"][:6] = np.array([0.0, 6e-8, 65504.0, -2.0, 1.0, -0.0], np.float16)
    q = _q6k_values(b)
    d = b["d"].astype(np.float32)[:, None]
    sc = np.repeat(b["scales"].astype(np.float32), 16, axis=1)
    want = (d * sc) * (q - 32).astype(np.float32)
    row = b.view(np.uint8).reshape(4, -1)          # 4 rows of 16 blocks (n_embd 4096)
    got = np.concatenate([oracle.q6k_dequant(row[i], 4096) for i in range(4)]).reshape(64, 256)
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_q8k_cut_brute_force():
    """imi_q8k::from: per 256 values d = amax / 127 (fp32 division), id = d ? 1 / d : 0, codes rint(x * id)
    half-even, int16 code sums per 16; with an all-zero block and exact ties."""
    r = np.random.default_rng(62)
    x = (r.standard_normal(2048) * 3).astype(np.float32)
    x[256:512] = 0.0
    x[512] = 127.0
    x[513:520] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5], np.float32)   # d = 1 exactly: ties
    q, d, bs = oracle.q8k(x)
    xb = x.reshape(8, 256)
    amax = np.abs(xb).max(axis=1).astype(np.float32)
    dd = (amax / np.float32(127)).astype(np.float32)
    idv = np.where(dd != 0, np.float32(1) / np.where(dd != 0, dd, 1), 0).astype(np.float32)
    wq = np.rint((xb * idv[:, None]).astype(np.float32)).astype(np.int32)
    assert np.array_equal(d.view(np.uint32), dd.view(np.uint32))
    assert np.array_equal(q.reshape(8, 256).astype(np.int32), wq)
    assert np.array_equal(bs.astype(np.int32), wq.reshape(128, 16).sum(axis=1))
    assert list(q[513:520]) == [0, 2, 2, 0, -2, -2, 126]


def _avx2_lanes(blk, xq, bsums):
    """The int32 lanes of imi_q6k_row's AVX2 body (imi/core/tables.cpp:246-270), emulated instruction by instruction
    on 32-byte registers: 16-bit shifts and byte masks build the 6-bit values, maddubs (u8 x s8 pairs -> s16,
    saturating), a per-128-bit-lane byte shuffle broadcasts the scales, madd (s16 pairs -> s32), then - 32 * corr."""
    ql, qh = blk["ql"], blk["qh"]
    sc = blk["scales"].astype(np.int16)

    def srli16(v, n):
        return (v.view(np.uint16) >> n).astype(np.uint16).view(np.uint8)

    def slli16(v, n):
        return (v.view(np.uint16) << n).astype(np.uint16).view(np.uint8)

    def maddubs(a, b):
        p = a.astype(np.int32) * b.astype(np.int32)
        return np.clip(p[0::2] + p[1::2], -32768, 32767).astype(np.int16)

    def madd(a, b):
        p = a.astype(np.int32) * b.astype(np.int32)
        return (p[0::2] + p[1::2]).astype(np.int32)

    isum = np.zeros(8, np.int64)
    for n in range(2):
        a, a2, h = ql[64 * n:64 * n + 32], ql[64 * n + 32:64 * n + 64], qh[32 * n:32 * n + 32]
        q = [(a & 15) | (slli16(h, 4) & 0x30), (a2 & 15) | (slli16(h, 2) & 0x30),
             (srli16(a, 4) & 15) | (h & 0x30), (srli16(a2, 4) & 15) | (srli16(h, 2) & 0x30)]
        s8 = sc[8 * n:8 * n + 8]
        s2 = np.concatenate([s8, s8]).view(np.uint8)           # 32 bytes, both 128-bit lanes hold the 8 scales
        for k in range(4):
            ctl = np.array([2 * (2 * k) + (i & 1) for i in range(16)] + [2 * (2 * k + 1) + (i & 1) for i in range(16)])
            sh = np.concatenate([s2[:16][ctl[:16]], s2[16:][ctl[16:]]]).view(np.int16)
            p = maddubs(q[k], xq[128 * n + 32 * k:128 * n + 32 * k + 32])
            isum += madd(p, sh)
    corr = madd(sc, bsums)
    return (isum - 32 * corr.astype(np.int64)).astype(np.int32)


def test_q6k_lanes_and_row():
    """imi_q6k_row: the oracle's 8 int32 lanes per block equal an instruction-level emulation of the AVX2 body, and
    their total equals the closed form sum_e (value_e - 32) * scale_e * x_e exactly; the row result is
    sum_i d_i * X.d_i * lanes in float64 to 1e-5 relative."""
    r = np.random.default_rng(63)
    nb, n_rows = 8, 24
    b = _q6k_blocks(n_rows * nb, r)
    x = (r.standard_normal(256 * nb) * 2).astype(np.float32)
    out, lanes = oracle.q6k_rows(b.view(np.uint8).reshape(n_rows, -1), x, lanes=True)
    q, d, bs = oracle.q8k(x)
    vals = _q6k_values(b).reshape(n_rows, nb, 256) - 32
    sc = np.repeat(b["scales"].astype(np.int64), 16, axis=1).reshape(n_rows, nb, 256)
    xq = q.astype(np.int64).reshape(nb, 256)
    assert np.array_equal(lanes.sum(axis=2).astype(np.int64), (vals * sc * xq[None]).sum(axis=2))
    for rr in range(0, n_rows, 5):
        for i in range(nb):
            blk = b[rr * nb + i]
            assert np.array_equal(lanes[rr, i], _avx2_lanes(blk, q[256 * i:256 * i + 256], bs[16 * i:16 * i + 16]))
    dd = b["d"].astype(np.float64).reshape(n_rows, nb) * d.astype(np.float64)[None]
    want = (dd * lanes.sum(axis=2)).sum(axis=1)
    assert np.allclose(out, want, rtol=1e-5, atol=1e-6 * np.abs(want).max())


@pytest.mark.parametrize("rows,cols", [(64, 512), (24, 2048)])
def test_q4_1_gemv_float64_and_scalar_and_two_inputs(rows, cols):
    """Q4_1 tables (imi/core/tables.cpp:127-143 with HAS_M): cor = fma(m, s, cor) and out = acc + cor. The AVX2
    kernel equals the plain per-row chain, group2 equals two groups, group_batch equals n groups, and the result
    equals sum over blocks of (code * d + m) . (q * dx) in float64."""
    from nunchi_amd import synth
    from oracle.exact import cut_dequant, dequant_q4_1
    blk = synth.q4_1_random(np.random.default_rng(5 * rows + cols), rows, cols)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    t = oracle.Q4Table(blk, rows, cols, threads=3, q4_1=True)
    y0, _ = t.gemv(x[0])
    ys, _ = t.gemv(x[0], scalar=True)
    assert np.array_equal(y0, ys)
    y2, _ = t.gemv(x)
    assert np.array_equal(y2[0], y0) and np.array_equal(y2[1], t.gemv(x[1])[0])
    assert np.array_equal(t.gemv_batch(x), y2)
    ref = dequant_q4_1(blk, rows, cols) @ cut_dequant(x[0])
    assert np.abs(y0 - ref).max() <= 1e-5 * np.sqrt((ref ** 2).mean())
    # a Q4_0 reading of the same codes would differ: the m term is what the restatement adds
    q0 = np.zeros(blk.shape, dtype=[("d", "<f2"), ("qs", "u1", 16)])
    q0["d"], q0["qs"] = blk["d"], blk["qs"]
    assert not np.allclose(oracle.Q4Table(q0, rows, cols).gemv(x[0])[0], y0)


def _imi_pick(lg):
    """imi/core/hear.cpp:67-68 as written: best = 0; v replaces it only if logits[v] > logits[best]."""
    best = 0
    for v in range(1, len(lg)):
        if lg[v] > lg[best]:
            best = v
    return best


def test_top_follows_imi_loop_with_ties_and_nan():
    """oracle.top against imi's literal greedy loop on scores with forced ties, NaNs (at 0, at the maximum,
    everywhere) and infinities: the first maximum wins, a NaN never wins, a NaN at index 0 is never beaten."""
    import oracle
    rng = np.random.default_rng(5)
    cases = [np.array([1.0, 3.0, 3.0, 2.0], np.float32), np.array([np.nan, 5.0, 7.0], np.float32),
             np.array([1.0, np.nan, 3.0, np.nan, 3.0], np.float32), np.full(6, np.nan, np.float32),
             np.array([-np.inf, -np.inf, np.nan], np.float32), np.array([-np.inf, np.nan, 2.0, np.inf, np.inf], np.float32),
             np.array([0.0, -0.0, 0.0], np.float32)]
    for _ in range(300):
        a = rng.integers(-3, 4, size=int(rng.integers(1, 40))).astype(np.float32)   # many ties
        a[rng.random(a.size) < 0.15] = np.nan
        cases.append(a)
    for a in cases:
        assert oracle.top(a) == _imi_pick(a), a
