"""sh_q4_gemm_noalloc (the batch product with its int8 input cut in the library's fixed per-device scratch, for
callers that cannot allocate) against sh_q4_gemm (the same product with a work buffer allocated per call), bit for
bit, on two calls in a row, the second with a smaller input, so the scratch holds the first call's contents when
the second runs; and the scratch limit refused with SH_E_ARG before anything is launched. Inputs and outputs are
device buffers the test allocates itself through the HIP runtime the library is linked against; the C ABI is called
directly."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _table(ctx, rows, cols, seed):
    import nunchi_amd
    from conftest import q4_random
    return nunchi_amd.Q4Table(ctx, q4_random(rows, cols, seed), rows, cols)


def _hip():
    import nunchi_amd
    nunchi_amd.load_library()
    H = C.CDLL("libamdhip64.so.7")   # the runtime libseoul_hip.so is linked against, already loaded
    H.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    H.hipFree.argtypes = [C.c_void_p]
    H.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    return H


def _noalloc(ctx, t, x):
    import nunchi_amd
    L, H = nunchi_amd.load_library(), _hip()
    n, cols = x.shape
    x = np.ascontiguousarray(x, np.float32)
    y = np.full((n, t.rows), np.nan, np.float32)
    xd, yd = C.c_void_p(), C.c_void_p()
    assert H.hipMalloc(C.byref(xd), x.nbytes) == 0 and H.hipMalloc(C.byref(yd), y.nbytes) == 0
    try:
        assert H.hipMemcpy(xd, x.ctypes.data_as(C.c_void_p), x.nbytes, 1) == 0          # host to device
        assert H.hipMemcpy(yd, y.ctypes.data_as(C.c_void_p), y.nbytes, 1) == 0
        rc = L.sh_q4_gemm_noalloc(ctx.h, t.h, xd, n, yd)
        if rc != 0:
            return rc, None
        assert L.sh_sync(ctx.h) == 0
        assert H.hipMemcpy(y.ctypes.data_as(C.c_void_p), yd, y.nbytes, 2) == 0          # device to host
        return rc, y
    finally:
        H.hipFree(xd)
        H.hipFree(yd)


def _same(a, b):
    return a.shape == b.shape and np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_noalloc_gemm_matches_allocating_gemm():
    import nunchi_amd
    ctx = nunchi_amd.Context(0)
    rng = np.random.default_rng(3)
    big = _table(ctx, 2048, 2048, 5)      # first call: 448 positions x 2048 columns (917,504 codes)
    small = _table(ctx, 512, 1024, 6)     # second call: 37 positions x 1024 columns
    for t, n in ((big, 448), (small, 37)):
        x = rng.standard_normal((n, t.cols)).astype(np.float32)
        rc, y = _noalloc(ctx, t, x)
        assert rc == 0, nunchi_amd.load_library().sh_last_error()
        ref = t.gemm(x)
        assert _same(y, ref), (t.rows, t.cols, n)
    # the smaller input again after the large one, and one position (the product clamps its position reads to n - 1)
    for n in (5, 1):
        x = rng.standard_normal((n, small.cols)).astype(np.float32)
        rc, y = _noalloc(ctx, small, x)
        assert rc == 0 and _same(y, small.gemm(x)), n


def test_noalloc_gemm_refuses_above_the_scratch():
    import nunchi_amd
    ctx = nunchi_amd.Context(0)
    t = _table(ctx, 64, 8192, 7)
    x = np.zeros((129, 8192), np.float32)   # 129 * 8192 codes > 1 Mi
    rc, _ = _noalloc(ctx, t, x)
    assert rc == nunchi_amd.SH_E_ARG
    assert b"scratch" in nunchi_amd.load_library().sh_last_error()
    rc, y = _noalloc(ctx, t, x[:128])   # exactly at the limit
    assert rc == 0 and _same(y, t.gemm(x[:128]))


def test_noalloc_two_contexts_on_one_device():
    """Two contexts on device 0 share the device's scratch: the second context's call, enqueued while the first one's
    may still run, waits for it, so both products equal their allocating counterparts bit for bit."""
    import nunchi_amd
    L, H = nunchi_amd.load_library(), _hip()
    ca, cb = nunchi_amd.Context(0), nunchi_amd.Context(0)
    ta, tb = _table(ca, 2048, 2048, 8), _table(cb, 1024, 2048, 9)
    rng = np.random.default_rng(11)
    xa = rng.standard_normal((448, 2048)).astype(np.float32)
    xb = rng.standard_normal((400, 2048)).astype(np.float32)
    bufs = []
    try:
        def dev(a):
            p = C.c_void_p()
            assert H.hipMalloc(C.byref(p), a.nbytes) == 0
            bufs.append(p)
            assert H.hipMemcpy(p, a.ctypes.data_as(C.c_void_p), a.nbytes, 1) == 0
            return p
        ya = np.full((448, ta.rows), np.nan, np.float32)
        yb = np.full((400, tb.rows), np.nan, np.float32)
        xad, xbd, yad, ybd = dev(xa), dev(xb), dev(ya), dev(yb)
        for _ in range(3):   # a, b, a, b, ... with no wait between the two contexts' calls
            assert L.sh_q4_gemm_noalloc(ca.h, ta.h, xad, 448, yad) == 0
            assert L.sh_q4_gemm_noalloc(cb.h, tb.h, xbd, 400, ybd) == 0
        assert L.sh_sync(ca.h) == 0 and L.sh_sync(cb.h) == 0
        assert H.hipMemcpy(ya.ctypes.data_as(C.c_void_p), yad, ya.nbytes, 2) == 0
        assert H.hipMemcpy(yb.ctypes.data_as(C.c_void_p), ybd, yb.nbytes, 2) == 0
        assert _same(ya, ta.gemm(xa))
        assert _same(yb, tb.gemm(xb))
    finally:
        for p in bufs:
            H.hipFree(p)
