"""Host-side checks that need no GPU: the C ABI library loads and exports every entry point include/seoul_hip.h
declares; the C++ engine header compiles against it; GGUF files round-trip; the synthetic model has the byte
counts the measurement is quoted on; bench.py refuses more than one GPU."""
import os
import re
import subprocess
import sys

import numpy as np

from conftest import ROOT


def _declared():
    src = open(os.path.join(ROOT, "include", "seoul_hip.h")).read()
    return sorted(set(re.findall(r"^(?:int|int64_t|float|const char\*)\s+(sh_\w+)\(", src, re.M)))


def test_library_exports_every_declared_symbol():
    import ctypes
    import nunchi_amd
    lib = ctypes.CDLL(nunchi_amd.LIB_PATH)
    names = _declared()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(nunchi_amd.EXPORTS) == names


def test_no_gpu_fails_loudly():
    """Without a device the product path raises; there is no CPU fallback."""
    import nunchi_amd
    if os.path.exists("/dev/kfd"):
        return
    try:
        nunchi_amd.Context(0)
    except nunchi_amd.SeoulError as e:
        assert e.code in (nunchi_amd.SH_E_ARG, nunchi_amd.SH_E_HIP)
    else:
        raise AssertionError("a context was created with no GPU")


def test_cpp_engine_header_compiles():
    out = os.path.join("/tmp", f"seoul_gpu_check_{os.getpid()}.o")
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                        os.path.join(ROOT, "tests", "cpp", "seoul_gpu_check.cpp")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_gguf_round_trip(tmp_path):
    from nunchi_amd.gguf import GGUFFile, GGUFWriter, T_F32, T_Q4_0
    from nunchi_amd import synth
    w = GGUFWriter()
    w.add_u32("a.b", 7)
    w.add_f32("c", 0.25)
    w.add_str("s", "seoul")
    w.add_bool_array("pat", [True, False, True])
    q = synth.q4_0_random(np.random.default_rng(0), 16, 64)
    f = np.arange(12, dtype=np.float32)
    w.add_tensor("t.q", T_Q4_0, (64, 16), q)
    w.add_tensor("t.f", T_F32, (4, 3), f)
    p = str(tmp_path / "x.gguf")
    w.write(p)
    r = GGUFFile(p)
    assert r.kv["a.b"] == 7 and r.kv["c"] == 0.25 and r.kv["s"] == "seoul" and r.kv["pat"] == [1, 0, 1]
    assert np.array_equal(np.asarray(r.tensors["t.q"].data), q.view(np.uint8).reshape(-1))
    assert np.array_equal(np.asarray(r.tensors["t.f"].data).view(np.float32), f)
    assert r.tensors["t.f"].ne == (4, 3)


def test_seoul_shape_bytes():
    """The algorithmic bytes of a step (file bytes of every table) as the measurement quotes them."""
    from nunchi_amd import synth
    s = synth.SEOUL
    E, D = s.n_embd, s.head_dim
    def q4(rows, cols):
        return rows * cols // 32 * 18
    per = []
    for il in range(s.n_layer):
        b = q4(s.n_ff, E) * 2 + q4(E, s.n_ff)
        if il in s.attn_layers:
            b += q4(s.n_head * D + 2 * s.n_head_kv * D + s.n_head, E) + q4(E, s.n_head * D)
        else:
            b += q4(3 * E, E) + q4(E, E)
        per.append(b)
    assert sum(per) == 582_967_296
    assert q4(s.n_vocab, E) == 112_315_392
    assert len(s.attn_layers) == 6 and s.n_layer - len(s.attn_layers) == 10


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr
