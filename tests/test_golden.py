"""The committed golden fixtures (tests/golden/make_golden.py): the oracle reproduces them bit for bit (CPU), and so
does the HIP path through the C ABI (GPU)."""
import os

import numpy as np
import pytest

import oracle
from conftest import ROOT

G = os.path.join(ROOT, "tests", "golden")


def _load(name):
    return np.load(os.path.join(G, name), allow_pickle=False)


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_oracle_reproduces_golden():
    f = _load("cut32.npz")
    q, d, s = oracle.cut(f["x"])
    assert np.array_equal(q, f["q"]) and _same(d, f["d"]) and _same(s, f["s"])
    g = _load("gemv_64x512.npz")
    y, _ = oracle.Q4Table(g["q4_0"], 64, 512).gemv(g["x"])
    y8, _ = oracle.Q4x8Table(g["q4_0"], 64, 512).gemv(g["x"][0])
    assert _same(y, g["y"]) and _same(y8, g["y_q4x8"])


def test_oracle_tiny_steps_golden(tiny_model):
    t = _load("tiny_steps.npz")
    eng = oracle.Engine(tiny_model, threads=3, n_ctx=16)
    for i, tok in enumerate(t["tokens"]):
        h, lg = eng.step(int(tok))
        assert _same(h, t["hidden"][i]) and _same(lg, t["logits"][i]) and oracle.top(lg) == t["best"][i]


@pytest.mark.gpu
def test_gpu_reproduces_golden(tiny_model):
    import nunchi_amd
    ctx = nunchi_amd.Context(0)
    g = _load("gemv_64x512.npz")
    t = nunchi_amd.Q4Table(ctx, g["q4_0"], 64, 512)
    assert _same(t.gemv(g["x"]), g["y"]) and _same(t.gemv(g["x"][0], cut_mode=1), g["y_q4x8"])
    s = _load("tiny_steps.npz")
    b = nunchi_amd.Brain(tiny_model, n_ctx=16, ctx=ctx)
    for i, tok in enumerate(s["tokens"]):
        h, lg, best = b.step(int(tok))
        assert _same(h, s["hidden"][i]) and _same(lg, s["logits"][i]) and best == s["best"][i]


@pytest.mark.gpu
def test_cpp_engine_api_on_gpu(tiny_model, tiny_voice, tmp_path):
    """imi's API (include/seoul_gpu.hpp) compiled with g++ against libseoul_hip.so, driving the GPU like imi's callers;
    its greedy ids and one voice frame's codes equal the oracle's."""
    import subprocess
    exe = str(tmp_path / "seoul_gpu_check")
    lib_dir = os.path.join(ROOT, "nunchi_amd")
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "cpp", "seoul_gpu_check.cpp"),
                        "-L", lib_dir, "-lseoul_hip", f"-Wl,-rpath,{lib_dir}", "-o", exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    out = subprocess.run([exe, tiny_model, tiny_voice], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    ids = [int(v) for v in out.stdout.split("\n")[0].split(":")[1].split()]
    eng = oracle.Engine(tiny_model, threads=2, n_ctx=128)
    for i, tok in enumerate([3, 141, 59, 26]):
        _, lg = eng.step(tok, want_logits=i == 3)
    want = [oracle.top(lg)]
    for _ in range(7):
        _, lg = eng.step(want[-1])
        want.append(oracle.top(lg))
    assert ids == want, (ids, want, out.stderr[-2000:])
    assert "pos 13/1" in out.stdout and "swapped pos 1/13" in out.stdout
    # the voice frame: same hidden-like input, passes of half the codebooks each, first maximum
    v = oracle.Voice(tiny_voice, threads=2)
    h = ((np.arange(v.n_in) % 17 - 8) * 0.125).astype(np.float32)
    v.begin_frame(h)
    codes = np.full(v.n_cb, -1, np.int32)
    half = v.n_cb // 2
    for need in (list(range(half)), list(range(half, v.n_cb))):
        sc = v.pass_(codes, need)
        codes[need] = [oracle.top(r) for r in sc]
    got = [int(c) for c in out.stdout.split("codes:")[1].split("\n")[0].split()]
    assert got == codes.tolist(), (got, codes.tolist())
