"""imi_ears and imi_codec (include/seoul_gpu.hpp) from a compiled C++ caller on the device: the rows and samples equal
the Python binding's bit for bit (the same library underneath), and the members the caller reads carry the file's
shape."""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _build(tmp_path):
    exe = str(tmp_path / "sound_check")
    lib_dir = os.path.join(ROOT, "nunchi_amd")
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-I", os.path.join(ROOT, "include"),
                        os.path.join(ROOT, "tests", "cpp", "sound_check.cpp"), "-L", lib_dir, "-lseoul_hip",
                        f"-Wl,-rpath,{lib_dir}", "-o", exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def test_cpp_ears_and_codec_callers(model_dir, tmp_path):
    import nunchi_amd
    from nunchi_amd import synth
    ears_path = synth.cached("ears", synth.TINY_EARS, 3, model_dir)
    codec_path = synth.cached("codec", synth.TINY_CODEC, 2, model_dir)
    pcm = synth.clip(2 * 16000 + 311, 9)
    codes = np.random.default_rng(8).integers(0, synth.TINY_CODEC.n_codes, (4, 12)).astype(np.int32)
    clip_f, codes_f = tmp_path / "clip.f32", tmp_path / "codes.i32"
    rows_f, pcm_f = tmp_path / "rows.out", tmp_path / "pcm.out"
    pcm.tofile(clip_f)
    codes.tofile(codes_f)
    out = subprocess.run([_build(tmp_path), ears_path, str(clip_f), str(rows_f), codec_path, str(codes_f), str(pcm_f)],
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    e = synth.TINY_EARS
    g = nunchi_amd.Ears(ears_path)
    want = g.encode(pcm)
    P = want.shape[0]
    n_fr = g.positions(len(pcm))[1]
    assert (f"ears n_pos {P} n_out {e.n_out} n_embd {e.n_embd} n_mel {e.n_mel} window {e.window} "
            f"mel_frames {n_fr}") in out.stdout, out.stdout
    rows = np.fromfile(rows_f, np.float32).reshape(P, e.n_out)
    assert np.array_equal(rows.view(np.uint32), want.view(np.uint32))
    c = nunchi_amd.Codec(codec_path)
    ref = np.concatenate([c.frame(cc) for cc in codes] + [c.flush()])
    assert f"codec frames 4 samples {len(ref)} n_embd {synth.TINY_CODEC.n_embd} n_bins 641" in out.stdout, out.stdout
    assert np.array_equal(np.fromfile(pcm_f, np.float32).view(np.uint32), ref.view(np.uint32))
