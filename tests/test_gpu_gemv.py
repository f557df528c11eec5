"""GPU parity of the Q4_0 table kernels (C ABI: sh_q4_create / sh_q4_gemv / sh_q4_rows) against the oracle.

- dequantized rows: bit-exact against the Q4_0 closed form, every code 0..15 with ordinary, subnormal, zero and
  negative scales
- GEMV in the exact regime (power-of-two scales and inputs whose int8 cut is exact): every fp32 operation is exact,
  so GPU, oracle and the float64 value must agree bit for bit; a wrong nibble, row, scale or correction term fails
- GEMV on the synthetic distribution (cfg 0 and the layer shapes of cfg 1): bit for bit equal to imi's AVX2
  arithmetic (oracle), since the kernel keeps imi's per-row fp32 chain order; and within fp32 accuracy of the
  float64 value of the same int8-cut input
- two inputs riding one read give each input exactly its one-input result (imi/core/tables.cpp:145-163)
- imi/kernels/q4x8.cpp's input cut (roundf, half away from zero) on cut_mode 1
- several tables in grouped launches (sh_q4_gemv_group) give each table exactly its own GEMV
"""
import numpy as np
import pytest

from conftest import q4_random, rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import nunchi_amd
    return nunchi_amd.Context(0)


def _exact_case(rows, cols, seed):
    """Q4_0 table with scales in {2^-6, 2^-7} and an input whose cut is exact: block amax = 127 * 2^-m."""
    from nunchi_amd.gguf import Q4_0_BLOCK
    rng = np.random.default_rng(seed)
    nb = cols // 32
    blk = np.empty(rows * nb, dtype=Q4_0_BLOCK)
    blk["d"] = rng.choice(np.array([2.0 ** -6, 2.0 ** -7], np.float16), size=rows * nb)
    blk["qs"] = rng.integers(0, 256, size=(rows * nb, 16), dtype=np.uint8)
    q = rng.integers(-127, 128, size=(nb, 32))
    q[np.arange(nb), rng.integers(0, 32, size=nb)] = rng.choice([-127, 127], size=nb)
    m = rng.integers(0, 3, size=nb)
    x = (q * (2.0 ** -m)[:, None]).astype(np.float32).reshape(-1)
    return blk, x


def _dequant(blk, rows, cols):
    qs = blk["qs"].reshape(rows, cols // 32, 16).astype(np.int64)
    codes = np.concatenate([qs & 15, qs >> 4], axis=-1) - 8
    return (codes * blk["d"].astype(np.float64).reshape(rows, cols // 32, 1)).reshape(rows, cols)


def test_rows_dequant_bit_exact(ctx):
    import nunchi_amd
    from nunchi_amd.gguf import Q4_0_BLOCK
    rows, cols = 64, 256
    rng = np.random.default_rng(3)
    blk = np.empty(rows * cols // 32, dtype=Q4_0_BLOCK)
    special = np.array([0.0, -0.0, 1.0, -2.5, 6.1e-5, 5.96e-8, 3.0e-7, -4.1e-6, 65504.0, -65504.0, 0.000123], np.float16)
    blk["d"] = rng.choice(special, size=blk.size)
    # every byte value, so every (low, high) code pair appears
    blk["qs"] = (np.arange(blk.size * 16) % 256).astype(np.uint8).reshape(-1, 16)
    t = nunchi_amd.Q4Table(ctx, blk, rows, cols)
    got = t.rows_dequant(np.arange(rows))
    want = _dequant(blk, rows, cols).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(8192, 2048), (2048, 8192), (3104, 2048), (8, 32), (24, 96), (64, 7680), (2048, 7680),
                                       (16, 4608)])
def test_gemv_exact_regime_bitwise(ctx, rows, cols):
    import nunchi_amd
    import oracle
    blk, x = _exact_case(rows, cols, seed=rows + cols)
    t = nunchi_amd.Q4Table(ctx, blk, rows, cols)
    got = t.gemv(x)
    want64 = _dequant(blk, rows, cols) @ x.astype(np.float64)
    orc, _ = oracle.Q4Table(blk, rows, cols, threads=4).gemv(x)
    assert np.array_equal(orc, want64.astype(np.float32)), "oracle not exact in the exact regime"
    assert np.array_equal(got, orc)


def _cut_dequant(x):
    """imi's input cut (imi/core/vec.h:47-75) as float64 values q * d: per 32 values d = amax / 127 and
    q = rint(x / d) in float32 arithmetic, as the engine computes them."""
    x32 = np.asarray(x, np.float32).reshape(-1, 32)
    d = (np.abs(x32).max(-1, keepdims=True) / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    q = np.rint((x32 * idv).astype(np.float32))
    return (q.astype(np.float64) * d.astype(np.float64)).reshape(np.shape(x))


@pytest.mark.parametrize("rows,cols", [(8192, 2048), (2048, 2048), (512, 2048), (2048, 8192), (3104, 2048), (64, 7680),
                                       (2048, 7680), (16, 4608), (16, 64)])
def test_gemv_matches_imi_arithmetic(ctx, rows, cols):
    import nunchi_amd
    import oracle
    blk = q4_random(rows, cols, seed=rows * 3 + cols)
    x = np.random.default_rng(cols).standard_normal(cols).astype(np.float32)
    got = nunchi_amd.Q4Table(ctx, blk, rows, cols).gemv(x)
    orc, _ = oracle.Q4Table(blk, rows, cols, threads=4).gemv(x)
    assert np.array_equal(got.view(np.uint32), orc.view(np.uint32))
    # float64 of the same int8-cut input: both approximate it to fp32 accuracy
    ref = _dequant(blk, rows, cols) @ _cut_dequant(x)
    scale = np.sqrt((ref ** 2).mean())
    assert np.abs(got - ref).max() < 1e-5 * scale + 1e-30
    assert np.abs(orc - ref).max() < 1e-5 * scale + 1e-30


@pytest.mark.parametrize("rows,cols", [(2048, 8192), (2048, 7680)])
def test_gemv_two_inputs_match_oracle_group2(ctx, rows, cols):
    """imi_q4_group2 (imi/core/tables.cpp:145-163) on the oracle side, the two-input kernel on the GPU."""
    import nunchi_amd
    import oracle
    blk = q4_random(rows, cols, seed=21)
    x = np.random.default_rng(22).standard_normal((2, cols)).astype(np.float32)
    got = nunchi_amd.Q4Table(ctx, blk, rows, cols).gemv(x)
    orc, _ = oracle.Q4Table(blk, rows, cols, threads=4).gemv(x)
    assert np.array_equal(got.view(np.uint32), orc.view(np.uint32))


def test_group_equals_each_table_alone(ctx):
    """sh_q4_gemv_group: a layer's seven linears (cfg 1 shapes, 2048- and 8192-wide), 4096-wide tables and more
    tables of one width than one launch takes (9 of 2048 columns), at one and two inputs and with q4x8's cut: every
    output equals the table's own sh_q4_gemv bit for bit; the first is also checked against the oracle."""
    import nunchi_amd
    import oracle
    shapes = [(2048, 2048), (512, 2048), (512, 2048), (2048, 2048), (8192, 2048), (8192, 2048), (2048, 8192),
              (1024, 4096), (8, 2048), (64, 2048), (264, 4096), (16, 2048)]
    tabs, blks = [], []
    for i, (r, c) in enumerate(shapes):
        blks.append(q4_random(r, c, seed=300 + i))
        tabs.append(nunchi_amd.Q4Table(ctx, blks[-1], r, c))
    rng = np.random.default_rng(301)
    for n_in, cut in ((1, 0), (2, 0), (1, 1)):
        xs = [rng.standard_normal((n_in, c)).astype(np.float32) for _, c in shapes]
        got = nunchi_amd.q4_gemv_group(ctx, tabs, xs, cut_mode=cut)
        for t, x, y in zip(tabs, xs, got):
            assert y.shape == (n_in, t.rows)
            assert np.array_equal(y.view(np.uint32), t.gemv(x, cut_mode=cut).reshape(n_in, -1).view(np.uint32))
        if cut == 0:
            orc, _ = oracle.Q4Table(blks[0], *shapes[0], threads=4).gemv(xs[0] if n_in == 2 else xs[0][0])
            assert np.array_equal(got[0].reshape(orc.shape).view(np.uint32), orc.view(np.uint32))
    with pytest.raises(nunchi_amd.SeoulError):   # q4x8's cut takes one input
        nunchi_amd.q4_gemv_group(ctx, tabs[:2], [np.zeros((2, 2048), np.float32)] * 2, cut_mode=1)
    with pytest.raises(nunchi_amd.SeoulError):   # 1024 columns: no kernel width
        nunchi_amd.q4_gemv_group(ctx, [nunchi_amd.Q4Table(ctx, q4_random(8, 1024, seed=1), 8, 1024)],
                                 [np.zeros(1024, np.float32)])


def test_expf_is_the_c_library(ctx):
    """The kernels' exponential equals the C library's expf bit for bit: every 61st float bit pattern (70 M inputs
    over the whole range, all exponents and signs), plus the special values."""
    import oracle
    u = np.arange(0, 1 << 32, 61, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 88.72283, 88.72284, -103.97208, -103.97207, -87.33655,
                        1e-45, -1e-45, 1.0, -1.0], np.float32)
    x = np.concatenate([x, special])
    g = ctx.expf(x)
    c = oracle.expf(x)
    same = (g.view(np.uint32) == c.view(np.uint32)) | (np.isnan(g) & np.isnan(c))
    assert same.all(), f"{(~same).sum()} differ, first at {x[~same][:4]}"


def test_gemv_two_inputs_one_read(ctx):
    import nunchi_amd
    rows, cols = 4096, 2048
    blk = q4_random(rows, cols, seed=11)
    x = np.random.default_rng(12).standard_normal((2, cols)).astype(np.float32)
    t = nunchi_amd.Q4Table(ctx, blk, rows, cols)
    both = t.gemv(x)
    assert np.array_equal(both[0], t.gemv(x[0]))
    assert np.array_equal(both[1], t.gemv(x[1]))


def test_gemv_cfg0_half_away_cut(ctx):
    """cfg 0: imi/kernels/q4x8.cpp semantics (roundf cut, correction 8*d*sum per block)."""
    import nunchi_amd
    import oracle
    rows, cols = 8192, 2048
    blk = q4_random(rows, cols, seed=0)
    x = np.random.default_rng(1).standard_normal(cols).astype(np.float32)
    # exact .5 ties in some blocks, where the two roundings differ
    x[:32] = np.float32(127.0) * np.linspace(-1, 1, 32, dtype=np.float32)
    x[5] = np.float32(2.5)
    x[6] = np.float32(-3.5)
    got = nunchi_amd.Q4Table(ctx, blk, rows, cols).gemv(x, cut_mode=1)
    orc, _ = oracle.Q4x8Table(blk, rows, cols, threads=4).gemv(x)
    assert np.array_equal(got.view(np.uint32), orc.view(np.uint32))
    got_even = nunchi_amd.Q4Table(ctx, blk, rows, cols).gemv(x, cut_mode=0)
    assert not np.array_equal(got, got_even)


def test_gemv_zero_and_tiny_inputs(ctx):
    import nunchi_amd
    rows, cols = 256, 2048
    blk = q4_random(rows, cols, seed=5)
    t = nunchi_amd.Q4Table(ctx, blk, rows, cols)
    assert np.array_equal(t.gemv(np.zeros(cols, np.float32)), np.zeros(rows, np.float32))
    x = np.zeros(cols, np.float32)
    x[37] = 1e-30   # one block with a tiny scale, every other block all zero (d = 0, id = 0)
    import oracle
    orc, _ = oracle.Q4Table(blk, rows, cols).gemv(x)
    got = t.gemv(x)
    assert np.array_equal(got.view(np.uint32), orc.view(np.uint32))


def test_bad_arguments_rejected(ctx):
    import nunchi_amd
    blk = q4_random(8, 64, seed=1)
    with pytest.raises(ValueError):
        nunchi_amd.Q4Table(ctx, blk, 16, 64)
    with pytest.raises(nunchi_amd.SeoulError):
        nunchi_amd.Q4Table(ctx, q4_random(12, 64, 1), 12, 64)   # rows not a multiple of 8
    t = nunchi_amd.Q4Table(ctx, blk, 8, 64)
    with pytest.raises(nunchi_amd.SeoulError):
        t.rows_dequant([8])


def test_calibration_launches():
    """The dispatch and pure-read calibration launches run and refuse bad sizes."""
    import nunchi_amd
    assert 0.0 < nunchi_amd.bench_empty(grid=64, reps=20) < 1e4
    assert 0.0 < nunchi_amd.bench_read(1 << 20, copies=2, grid=64, reps=8) < 1e5
    with pytest.raises(nunchi_amd.SeoulError):
        nunchi_amd.bench_read(1000, copies=2)   # not a multiple of 16
