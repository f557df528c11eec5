"""Pins of the oracle's kernel-level restatement (oracle/imi_cpu_kernels.cpp), each against something the restatement
does not share: numpy's IEEE conversions, integer brute force, float64 closed forms, or another code path of the
oracle whose op order the reference fixes. A dropped term, a wrong nibble or index, a transposed operand or a
wrong rounding mode fails one of these.
"""
import numpy as np
import pytest

import oracle
from conftest import q4_random
from oracle.exact import dequant_q4_0, dequant_q8_0

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
