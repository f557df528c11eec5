"""imi_file's surface (imi/model.h:12-36) through the library: load, get, key_i, key_f, keep, drop_data and the
tensors' ggml fields, checked against a GGUF parse written here from the format's definition (header, key/value
pairs, tensor infos, aligned data block); and a compiled brain.h / model.h caller (tests/cpp/brain_file_check.cpp),
whose file part runs without a device and whose imi_brain greedy loop runs on the GPU against the oracle."""
import os
import struct
import subprocess

import numpy as np
import pytest

from conftest import ROOT

# (bytes per block, values per block) of the ggml types the files hold: F32, F16, Q4_0, Q4_1, Q8_0, Q6_K
BLOCK = {0: (4, 1), 1: (2, 1), 2: (18, 32), 3: (20, 32), 8: (34, 32), 14: (210, 256)}
SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


def parse_gguf(path):
    """keys -> (type, value), tensors -> (type, ne, bytes) from the file as the GGUF format lays it out."""
    raw = open(path, "rb").read()
    at = 0

    def take(fmt):
        nonlocal at
        v = struct.unpack_from(fmt, raw, at)[0]
        at += struct.calcsize(fmt)
        return v

    def string():
        nonlocal at
        n = take("<Q")
        s = raw[at:at + n].decode()
        at += n
        return s

    def value(t):
        if t == 8:
            return string()
        if t == 9:
            et, n = take("<I"), take("<Q")
            return [value(et) for _ in range(n)]
        return take(SCALAR[t])

    assert take("<I") == 0x46554747 and take("<I") >= 2
    n_t, n_kv = take("<Q"), take("<Q")
    keys = {}
    for _ in range(n_kv):
        k = string()
        t = take("<I")
        keys[k] = (t, value(t))
    infos = []
    for _ in range(n_t):
        name = string()
        nd = take("<I")
        ne = [take("<Q") for _ in range(nd)] + [1] * (4 - nd)
        t = take("<I")
        off = take("<Q")
        infos.append((name, t, ne, off))
    align = keys.get("general.alignment", (4, 32))[1]
    data0 = (at + align - 1) // align * align
    tensors = {}
    for name, t, ne, off in infos:
        bb, per = BLOCK[t]
        n = ne[0] // per * bb * ne[1] * ne[2] * ne[3]
        tensors[name] = (t, ne, raw[data0 + off:data0 + off + n])
    return keys, tensors, len(raw) - data0


def test_file_reader_matches_the_format(tiny_model):
    import nunchi_amd
    keys, tensors, block = parse_gguf(tiny_model)
    f = nunchi_amd.File(tiny_model)
    listed = f.tensors()
    assert [t["name"] for t in listed] == list(tensors)   # file order
    for t in listed:
        ty, ne, data = tensors[t["name"]]
        bb, per = BLOCK[ty]
        assert t["type"] == ty and t["ne"] == ne
        assert t["nb"] == [bb, ne[0] // per * bb, ne[0] // per * bb * ne[1], ne[0] // per * bb * ne[1] * ne[2]]
        assert f.bytes_of(t["name"]) == data
    assert f.block()[1] == block
    # key_i reads u32 / i32 / u64 keys only, key_f f32 keys only (imi/model.cpp:117-131); others give the default
    for k, (t, v) in keys.items():
        if t in (4, 5, 10):
            assert f.key_i(k, -7) == v and f.key_f(k, -7.0) == -7.0
        elif t == 6:
            assert f.key_f(k, -7.0) == np.float32(v) and f.key_i(k, -7) == -7
        else:
            assert f.key_i(k, -7) == -7 and f.key_f(k, -7.0) == -7.0
    assert f.key_i("no.such.key", 5) == 5 and f.get("no.such.tensor") is None


def test_keep_and_drop_data(tiny_model):
    import nunchi_amd
    _, tensors, _ = parse_gguf(tiny_model)
    f = nunchi_amd.File(tiny_model)
    kept = f.keep("output_norm.weight")
    assert kept["data"] % 64 == 0 and f.bytes_of("output_norm.weight") == tensors["output_norm.weight"][2]
    f.drop_data()
    assert f.block() == (None, 0)
    assert f.get("blk.0.ffn_up.weight")["data"] is None          # not kept: bytes gone, shape readable
    assert f.get("blk.0.ffn_up.weight")["ne"] == tensors["blk.0.ffn_up.weight"][1]
    assert f.bytes_of("output_norm.weight") == tensors["output_norm.weight"][2]
    with pytest.raises(nunchi_amd.SeoulError):
        f.keep("no.such.tensor")


def test_swa_pattern_key(model_dir):
    import nunchi_amd
    from nunchi_amd import synth
    shape = synth.BrainShape(n_embd=256, n_layer=4, attn_layers=(1, 3), n_head=8, n_head_kv=2, head_dim=32, n_ff=512,
                             n_vocab=300, sliding_window=16, swa_layers=(1,))
    f = nunchi_amd.File(synth.cached("brain", shape, 0, model_dir))
    assert f.key_arr("lfm3.attention.sliding_window_pattern") == [0, 1, 0, 0]
    assert f.key_arr("lfm3.block_count") == [] and f.key_arr("no.such.key") == []


def _build_caller(tmp_path):
    exe = str(tmp_path / "brain_file_check")
    lib_dir = os.path.join(ROOT, "nunchi_amd")
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-I", os.path.join(ROOT, "include"),
                        os.path.join(ROOT, "tests", "cpp", "brain_file_check.cpp"), "-L", lib_dir, "-lseoul_hip",
                        f"-Wl,-rpath,{lib_dir}", "-o", exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def test_cpp_file_caller(tiny_model, tmp_path):
    """A model.h-style caller compiled against include/seoul_gpu.hpp: keys, a tensor's fields, keep, drop_data."""
    from nunchi_amd import synth
    exe = _build_caller(tmp_path)
    out = subprocess.run([exe, tiny_model], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    s = synth.TINY
    assert (f"keys block_count {s.n_layer} head_count {s.n_head} key_length {s.head_dim} eps "
            f"{float(np.float32(s.eps)):.9g} missing -7") in out.stdout, out.stdout
    assert (f"token_embd token_embd.weight type 2 ne {s.n_embd} {s.n_vocab} nb 18 {s.n_embd // 32 * 18} "
            f"bytes {s.n_vocab * s.n_embd // 32 * 18}") in out.stdout, out.stdout
    assert "optional missing 1 block 1" in out.stdout
    assert "kept aligned 1 same 1" in out.stdout
    assert "dropped table 1 kept 1 same 1 block 1" in out.stdout


@pytest.mark.gpu
def test_cpp_brain_caller_on_gpu(tiny_model, tmp_path):
    """imi_brain (imi/brain.h:20-65) from a compiled caller: its shape members and a greedy loop equal to the
    oracle's, and reset() repeats it."""
    import oracle
    from nunchi_amd import synth
    exe = _build_caller(tmp_path)
    out = subprocess.run([exe, tiny_model, "--step"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    s = synth.TINY
    assert (f"brain n_embd {s.n_embd} n_vocab {s.n_vocab} n_head {s.n_head} n_head_kv {s.n_head_kv} head_dim "
            f"{s.head_dim} d_conv {s.conv_kernel - 1} layers {s.n_layer} attn {len(s.attn_layers)}") in out.stdout
    ids = [int(v) for v in out.stdout.split("ids:")[1].split("\n")[0].split()]
    eng = oracle.Engine(tiny_model, threads=2, n_ctx=64)
    for i, tok in enumerate([3, 141, 59, 26]):
        _, lg = eng.step(tok, want_logits=i == 3)
    want = [oracle.top(lg)]
    for _ in range(7):
        _, lg = eng.step(want[-1])
        want.append(oracle.top(lg))
    assert ids == want, (ids, want)
    assert "pos 12" in out.stdout and "reset repeats 1" in out.stdout


def _crafted_gguf(path, *, alignment=32, align_type=4, ne=(64, 2), gtype=0, offset=0, data_bytes=512):
    """One F32 (or other) tensor after a general.alignment key, every field written as given (not checked here)."""
    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    out = bytearray(struct.pack("<IIQQ", 0x46554747, 3, 1, 1))
    out += s("general.alignment") + struct.pack("<I", align_type)
    out += struct.pack("<I" if align_type == 4 else "<Q", alignment)
    out += s("t") + struct.pack("<I", len(ne))
    for d in ne:
        out += struct.pack("<Q", d & 0xFFFFFFFFFFFFFFFF)
    out += struct.pack("<IQ", gtype, offset & 0xFFFFFFFFFFFFFFFF)
    out += b"\0" * ((-len(out)) % 32) + b"\1" * data_bytes
    with open(path, "wb") as f:
        f.write(out)


@pytest.mark.parametrize("case", [
    dict(offset=1 << 63),                       # offset past the file
    dict(offset=(1 << 64) - 64),                # offset that wraps the data start + offset sum
    dict(offset=64, data_bytes=512),            # in range, but the tensor runs past the end
    dict(ne=(64, -2)),                          # negative dimension
    dict(ne=(1 << 40, 1 << 30)),                # byte size overflows 64 bits
    dict(ne=(32, 1 << 40, 1 << 30), gtype=2),   # Q4_0 row count times rows overflows
    dict(alignment=3),                          # not a power of two
    dict(alignment=0),                          # zero
    dict(alignment=1 << 40, align_type=10),     # larger than the file
    dict(ne=(), data_bytes=0),                  # no dimensions
    dict(ne=(1, 1, 1, 1, 1)),                   # more than 4 dimensions
])
def test_malformed_headers_are_refused(tmp_path, case):
    """imi loads through ggml's gguf reader, which refuses these headers; the build's reader returns SH_E_FILE for
    each (no pointer outside the mapping is ever formed)."""
    import nunchi_amd
    p = str(tmp_path / "bad.gguf")
    _crafted_gguf(p, **case)
    with pytest.raises(nunchi_amd.SeoulError) as e:
        nunchi_amd.File(p)
    assert e.value.code == nunchi_amd.SH_E_FILE


def test_crafted_header_control_loads(tmp_path):
    """The same writer with sane fields loads, so the refusals above are about the field each one breaks."""
    import nunchi_amd
    p = str(tmp_path / "ok.gguf")
    _crafted_gguf(p)
    f = nunchi_amd.File(p)
    t = f.get("t")
    assert t is not None and tuple(t["ne"][:2]) == (64, 2)
