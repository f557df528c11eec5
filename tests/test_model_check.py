"""Load-time shape checks on the host (sh_check_model, the check sh_load runs before uploading anything): a brain
file whose tables do not have the shapes the kernels read is refused with SH_E_SHAPE, so a malformed file can never
make a kernel read or write past its device buffers (imi/core/seoul.cpp:93-162 reads the same keys and tensors; imi's
load returns false on a file it cannot use). Runs without a GPU: the check reads the file only."""
import numpy as np
import pytest

from nunchi_amd import gguf, synth

SH_E_SHAPE, SH_E_FILE = -4, -3


def _rewrite(src, dst, replace=None, drop=(), keys=None):
    """Copy a GGUF file with some tensors replaced ({name: (gtype, ne, data)}), dropped, or keys overridden."""
    f = gguf.GGUFFile(src)
    w = gguf.GGUFWriter()
    kv = dict(f.kv)
    kv.update(keys or {})
    for k, v in kv.items():
        if k == "general.alignment":
            continue
        if isinstance(v, str):
            w.add_str(k, v)
        elif isinstance(v, float):
            w.add_f32(k, v)
        elif isinstance(v, list):
            w.add_bool_array(k, v)
        else:
            w.add_u32(k, v)
    for name, t in f.tensors.items():
        if name in drop:
            continue
        if replace and name in replace:
            w.add_tensor(name, *replace[name])
        else:
            w.add_tensor(name, t.gtype, t.ne, np.asarray(t.data))
    w.write(dst)
    return dst


def _q4(rows, cols, seed=3):
    return gguf.T_Q4_0, (cols, rows), synth.q4_0_random(np.random.default_rng(seed), rows, cols)


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    return synth.write_brain(str(tmp_path_factory.mktemp("chk") / "tiny.gguf"), synth.TINY, 0)


def _status(path, n_ctx=64):
    import nunchi_amd
    try:
        nunchi_amd.check_model(path, n_ctx)
        return 0, ""
    except nunchi_amd.SeoulError as e:
        return e.code, str(e)


def test_valid_file_passes(tiny):
    import nunchi_amd
    info = nunchi_amd.check_model(tiny, 64)
    s = synth.TINY
    assert (info.n_embd, info.n_vocab, info.n_head, info.n_head_kv, info.head_dim, info.n_ff, info.n_layer, info.n_attn) == \
           (s.n_embd, s.n_vocab, s.n_head, s.n_head_kv, s.head_dim, s.n_ff, s.n_layer, len(s.attn_layers))
    assert info.d_conv == s.conv_kernel - 1 and info.n_ctx == 64


# one malformed table per case; TINY: n_embd 256, 8 query heads / 2 kv heads x 32, n_ff 512, layers 1 and 3 attention
BAD = {
    "attn_k narrower than one head (no kv head)": {"blk.1.attn_k.weight": _q4(16, 256)},
    "attn_k rows not a multiple of head_dim": {"blk.1.attn_k.weight": _q4(48, 256)},
    "attn_v rows differ from attn_k": {"blk.1.attn_v.weight": _q4(32, 256)},
    "attn_q rows differ from the head count": {"blk.1.attn_q.weight": _q4(128, 256)},
    "attn_gate rows differ from the head count": {"blk.1.attn_gate.weight": _q4(16, 256)},
    "attn_output columns differ from the attention width": {"blk.1.attn_output.weight": _q4(256, 128)},
    "attn_q columns differ from n_embd": {"blk.1.attn_q.weight": _q4(256, 128)},
    "kv heads differ between layers": {"blk.3.attn_k.weight": _q4(32, 256), "blk.3.attn_v.weight": _q4(32, 256)},
    "in_proj columns differ from n_embd": {"blk.0.shortconv.in_proj.weight": _q4(768, 128)},
    "out_proj rows differ from n_embd": {"blk.0.shortconv.out_proj.weight": _q4(128, 256)},
    "ffn widths differ between layers": {"blk.2.ffn_gate.weight": _q4(256, 256), "blk.2.ffn_up.weight": _q4(256, 256),
                                         "blk.2.ffn_down.weight": _q4(256, 256)},
    "ffn_up rows differ from ffn_gate": {"blk.0.ffn_up.weight": _q4(256, 256)},
    "ffn_down columns differ from n_ff": {"blk.0.ffn_down.weight": _q4(256, 256)},
    "a layer table in Q8_0": {"blk.0.ffn_down.weight": (gguf.T_Q8_0, (512, 256), synth.q8_0_random(np.random.default_rng(1), 256, 512))},
    "q norm not head_dim wide": {"blk.1.attn_q_norm.weight": (gguf.T_F32, (16,), np.ones(16, np.float32))},
}


@pytest.mark.parametrize("case", sorted(BAD))
def test_malformed_table_is_refused(tiny, tmp_path, case):
    path = _rewrite(tiny, str(tmp_path / "bad.gguf"), replace=BAD[case])
    code, msg = _status(path)
    assert code == SH_E_SHAPE, (case, code, msg)


def test_missing_table_and_bad_keys(tiny, tmp_path):
    assert _status(_rewrite(tiny, str(tmp_path / "a.gguf"), drop=("blk.2.ffn_down.weight",)))[0] == SH_E_FILE
    assert _status(_rewrite(tiny, str(tmp_path / "b.gguf"), keys={"lfm3.attention.key_length": 48}))[0] == SH_E_SHAPE
    assert _status(_rewrite(tiny, str(tmp_path / "c.gguf"), keys={"lfm3.shortconv.l_cache": 5}))[0] == SH_E_SHAPE


def test_context_the_attention_kernels_cannot_hold(tiny):
    code, msg = _status(tiny, n_ctx=1 << 17)
    assert code == SH_E_SHAPE and "n_ctx" in msg
    assert _status(tiny, n_ctx=4096)[0] == 0
