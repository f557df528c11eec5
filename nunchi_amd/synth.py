"""Seeded synthetic models with Seoul's shapes, written as GGUF files the engine (and imi) read.

Brain ("lfm3" keys, tensor names as imi/core/seoul.cpp:93-165 reads them): gated short-conv blocks and GQA attention
blocks with q/k norms and a per-head sigmoid gate, SwiGLU FFN, post-norm residuals, tied Q4_0 word table.
Voice generator ("a.gen.code." names as imi/core/voice.cpp:78-139 reads them): Q8_0 depthformer layers, proj_in,
per-codebook code tables (also the score tables) and feedback rows.

Weights: Q4_0 blocks with scale fp16(|N(0, 0.02)| / 8) and uniform 4-bit codes 0..15 (random bytes are exactly two
uniform nibbles); Q8_0 blocks with the same scales and int8 codes uniform in [-127, 127]. Norm weights
1 + 0.05 N(0, 1), conv taps N(0, 0.3) (fp32). Every tensor has its own seed derived from the model seed and its
name, so a model is reproducible tensor by tensor.
"""
from __future__ import annotations

import hashlib
import os
from dataclasses import dataclass, field

import numpy as np

from .gguf import GGUFWriter, Q4_0_BLOCK, Q4_1_BLOCK, Q6_K_BLOCK, Q8_0_BLOCK, T_F16, T_F32, T_Q4_0, T_Q4_1, T_Q6_K, T_Q8_0


@dataclass
class BrainShape:
    n_embd: int = 2048
    n_layer: int = 16
    attn_layers: tuple = (2, 5, 8, 10, 12, 14)   # the other layers are short-conv blocks
    n_head: int = 32
    n_head_kv: int = 8
    head_dim: int = 64
    n_ff: int = 8192
    n_vocab: int = 97496
    conv_kernel: int = 3                          # lfm3.shortconv.l_cache (d_conv = kernel - 1 taps of memory)
    rope_base: float = 1e6
    eps: float = 1e-5
    qk_norm_scale: float = 1.0                    # > 1 sharpens attention (scores grow with its square)
    vocab_type: str = "q4_0"                      # tied word table: "q4_0", or "q6_k" (imi's own format)
    rope_freqs: bool = False                      # write rope_freqs.weight (angle divisors, head_dim / 2 of them)
    sliding_window: int = 0                       # window of the layers in swa_layers (0: none)
    swa_layers: tuple = ()                        # attention layers with the window and the swa RoPE base
    rope_base_swa: float = 1e4
    layer_type: str = "q4_0"                      # layer tables: "q4_0", or "q4_1" (code * d + m)
    vocab_edits: tuple = ()                       # word table edits after drawing: ("copy", src, dst) copies row src
                                                  # over row dst (equal scores), ("nan", row) sets that row's block
                                                  # scales (Q4_0 d, Q6_K super-block d) to fp16 NaN (a NaN score)


SEOUL = BrainShape()
# the shape of the released Seoul brain files as imi's loader reads their keys (imi/core/seoul.cpp:93-142): 24 layers,
# 16 query / 4 key-value heads of 128, FFN 7680, 7-tap short conv, rope_freqs divisors and a Q6_K tied word table.
# The files' layer pattern is not published in the reference: attention every third layer from 2, the window of 256
# on every other attention layer (the pattern key's "sliding" entries), the rest short-conv blocks
REAL_SEOUL = BrainShape(n_layer=24, attn_layers=(2, 5, 8, 11, 14, 17, 20, 23), n_head=16, n_head_kv=4, head_dim=128,
                        n_ff=7680, conv_kernel=7, vocab_type="q6_k", rope_freqs=True, sliding_window=256,
                        swa_layers=(2, 8, 14, 20))
# small model with every feature of the path, for tests that must finish in seconds on the CPU oracle
TINY = BrainShape(n_embd=256, n_layer=4, attn_layers=(1, 3), n_head=8, n_head_kv=2, head_dim=32, n_ff=512,
                  n_vocab=1000, conv_kernel=3)


@dataclass
class VoiceShape:
    n_embd: int = 1024
    n_layer: int = 6
    n_head: int = 16
    n_head_kv: int = 4
    head_dim: int = 64
    n_ff: int = 4096
    n_vocab: int = 2048      # codes per codebook
    n_cb: int = 8            # codebooks
    n_in: int = 2048         # brain hidden width
    eps: float = 1e-5
    rope_theta: float = 1e6


VOICE = VoiceShape()
TALK_VOICE = VoiceShape(n_layer=3, n_cb=12)   # the generator's own shape: 12 codebooks (the codec's), 3 layers
TINY_VOICE = VoiceShape(n_embd=256, n_layer=2, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=256, n_cb=8,
                        n_in=256)


def _rng(seed: int, name: str) -> np.random.Generator:
    h = hashlib.sha256(f"{seed}:{name}".encode()).digest()
    return np.random.default_rng(int.from_bytes(h[:8], "little"))


def q4_0_random(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """[rows][cols/32] Q4_0 blocks: d = fp16(|N(0,0.02)|/8), 16 random bytes = 32 uniform codes 0..15."""
    nb = rows * (cols // 32)
    blk = np.empty(nb, dtype=Q4_0_BLOCK)
    blk["d"] = (np.abs(rng.standard_normal(nb, dtype=np.float32) * np.float32(0.02)) / np.float32(8)).astype(np.float16)
    blk["qs"] = np.frombuffer(rng.bytes(nb * 16), dtype=np.uint8).reshape(nb, 16)
    return blk


def q4_1_random(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """[rows][cols/32] Q4_1 blocks: d = fp16(|N(0,0.02)|/8), m = fp16(-(8 + N(0,1)) d) (near Q4_0's centring),
    16 random bytes of codes."""
    nb = rows * (cols // 32)
    blk = np.empty(nb, dtype=Q4_1_BLOCK)
    d = (np.abs(rng.standard_normal(nb, dtype=np.float32) * np.float32(0.02)) / np.float32(8)).astype(np.float16)
    blk["d"] = d
    blk["m"] = (-(np.float32(8) + rng.standard_normal(nb, dtype=np.float32)) * d.astype(np.float32)).astype(np.float16)
    blk["qs"] = np.frombuffer(rng.bytes(nb * 16), dtype=np.uint8).reshape(nb, 16)
    return blk


def q6_k_random(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """[rows][cols/256] Q6_K blocks: random ql/qh bytes (uniform 6-bit values 0..63), int8 scales uniform in
    [-64, 63], d = fp16(|N(0, 0.02)| / 1024), so values d * scale * (q - 32) are of the Q4_0 tables' size."""
    nb = rows * (cols // 256)
    blk = np.empty(nb, dtype=Q6_K_BLOCK)
    blk["ql"] = np.frombuffer(rng.bytes(nb * 128), dtype=np.uint8).reshape(nb, 128)
    blk["qh"] = np.frombuffer(rng.bytes(nb * 64), dtype=np.uint8).reshape(nb, 64)
    blk["scales"] = rng.integers(-64, 64, size=(nb, 16), dtype=np.int8)
    blk["d"] = (np.abs(rng.standard_normal(nb, dtype=np.float32) * np.float32(0.02)) / np.float32(1024)).astype(np.float16)
    return blk


def q8_0_random(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    nb = rows * (cols // 32)
    blk = np.empty(nb, dtype=Q8_0_BLOCK)
    blk["d"] = (np.abs(rng.standard_normal(nb, dtype=np.float32) * np.float32(0.02)) / np.float32(8)).astype(np.float16)
    blk["qs"] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8)
    return blk


def _norm_w(rng, n):
    return (1.0 + 0.05 * rng.standard_normal(n)).astype(np.float32)


def write_brain(path: str, shape: BrainShape = SEOUL, seed: int = 0) -> str:
    s = shape
    E, D = s.n_embd, s.head_dim
    w = GGUFWriter()
    w.add_str("general.architecture", "lfm3")
    w.add_u32("lfm3.block_count", s.n_layer)
    w.add_u32("lfm3.attention.head_count", s.n_head)
    w.add_u32("lfm3.attention.head_count_kv", s.n_head_kv)
    w.add_u32("lfm3.attention.key_length", D)
    w.add_f32("lfm3.attention.layer_norm_rms_epsilon", s.eps)
    w.add_f32("lfm3.rope.freq_base", s.rope_base)
    w.add_u32("lfm3.attention.sliding_window", s.sliding_window)
    if s.swa_layers:
        w.add_bool_array("lfm3.attention.sliding_window_pattern", [il in s.swa_layers for il in range(s.n_layer)])
        w.add_f32("lfm3.rope.freq_base_swa", s.rope_base_swa)
    w.add_u32("lfm3.shortconv.l_cache", s.conv_kernel)
    w.add_u32("lfm3.feed_forward_length", s.n_ff)

    def q4(name, rows, cols):
        if s.layer_type == "q4_1" and name != "token_embd.weight":
            w.add_tensor(name, T_Q4_1, (cols, rows), q4_1_random(_rng(seed, name), rows, cols))
        else:
            w.add_tensor(name, T_Q4_0, (cols, rows), q4_0_random(_rng(seed, name), rows, cols))

    def f32(name, arr, ne):
        w.add_tensor(name, T_F32, ne, np.ascontiguousarray(arr, dtype=np.float32))

    if s.vocab_type == "q6_k":
        blk = q6_k_random(_rng(seed, "token_embd.weight"), s.n_vocab, E)
        nb = E // 256
    else:
        blk = q4_0_random(_rng(seed, "token_embd.weight"), s.n_vocab, E)
        nb = E // 32
    if s.vocab_edits:
        for ed in s.vocab_edits:
            if ed[0] == "copy":
                blk[ed[2] * nb:(ed[2] + 1) * nb] = blk[ed[1] * nb:(ed[1] + 1) * nb]
            elif ed[0] == "nan":
                blk["d"][ed[1] * nb:(ed[1] + 1) * nb] = np.float16(np.nan)
            else:
                raise ValueError(f"unknown word-table edit {ed!r}")
    w.add_tensor("token_embd.weight", T_Q6_K if s.vocab_type == "q6_k" else T_Q4_0, (E, s.n_vocab), blk)
    f32("output_norm.weight", _norm_w(_rng(seed, "output_norm.weight"), E), (E,))
    if s.rope_freqs:
        ff = (1.0 + 3.0 * _rng(seed, "rope_freqs.weight").random(D // 2)).astype(np.float32)
        f32("rope_freqs.weight", ff, (D // 2,))
    for il in range(s.n_layer):
        p = f"blk.{il}."
        for n in ("attn_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm"):
            f32(p + n + ".weight", _norm_w(_rng(seed, p + n), E), (E,))
        if il in s.attn_layers:
            q4(p + "attn_q.weight", s.n_head * D, E)
            q4(p + "attn_k.weight", s.n_head_kv * D, E)
            q4(p + "attn_v.weight", s.n_head_kv * D, E)
            q4(p + "attn_gate.weight", s.n_head, E)
            q4(p + "attn_output.weight", E, s.n_head * D)
            f32(p + "attn_q_norm.weight", s.qk_norm_scale * _norm_w(_rng(seed, p + "q_norm"), D), (D,))
            f32(p + "attn_k_norm.weight", s.qk_norm_scale * _norm_w(_rng(seed, p + "k_norm"), D), (D,))
        else:
            K = s.conv_kernel
            cw = (0.3 * _rng(seed, p + "conv").standard_normal((E, K))).astype(np.float32)   # [channel][tap]
            f32(p + "shortconv.conv.weight", cw, (K, E))
            q4(p + "shortconv.in_proj.weight", 3 * E, E)
            q4(p + "shortconv.out_proj.weight", E, E)
        q4(p + "ffn_gate.weight", s.n_ff, E)
        q4(p + "ffn_up.weight", s.n_ff, E)
        q4(p + "ffn_down.weight", E, s.n_ff)
    w.write(path)
    return path


def write_voice(path: str, shape: VoiceShape = VOICE, seed: int = 1) -> str:
    s = shape
    E, D = s.n_embd, s.head_dim
    w = GGUFWriter()
    w.add_str("general.architecture", "lfm3-gen")
    g = "a.gen.code."

    def q8(name, rows, cols, planes=1):
        ne = (cols, rows) if planes == 1 else (cols, rows, planes)
        w.add_tensor(g + name, T_Q8_0, ne, q8_0_random(_rng(seed, name), rows * planes, cols))

    def f32(name, arr, ne):
        w.add_tensor(g + name, T_F32, ne, np.ascontiguousarray(arr, dtype=np.float32))

    q8("embd.weight", s.n_vocab, E, planes=s.n_cb)          # [n_cb][n_vocab][E]: inputs and score tables
    q8("out_embd.weight", s.n_vocab * s.n_cb, s.n_in)       # feedback rows, n_in wide
    q8("proj_in.weight", s.n_cb * E, s.n_in)
    f32("proj_in.bias", (0.1 * _rng(seed, "proj_in.bias").standard_normal(s.n_cb * E)), (s.n_cb * E,))
    f32("mask_embd", (0.1 * _rng(seed, "mask_embd").standard_normal(E)), (E,))
    f32("output_norm.weight", _norm_w(_rng(seed, "output_norm"), E), (E,))
    f32("head_norm.weight", _norm_w(_rng(seed, "head_norm"), s.n_cb * E), (E, s.n_cb))
    for il in range(s.n_layer):
        p = f"blk.{il}."
        f32(p + "ln1.weight", _norm_w(_rng(seed, p + "ln1"), E), (E,))
        f32(p + "ln2.weight", _norm_w(_rng(seed, p + "ln2"), E), (E,))
        f32(p + "attn_q_norm.weight", _norm_w(_rng(seed, p + "qn"), D), (D,))
        f32(p + "attn_k_norm.weight", _norm_w(_rng(seed, p + "kn"), D), (D,))
        q8(p + "attn_q.weight", s.n_head * D, E)
        q8(p + "attn_k.weight", s.n_head_kv * D, E)
        q8(p + "attn_v.weight", s.n_head_kv * D, E)
        q8(p + "attn_gate.weight", s.n_head, E)
        q8(p + "attn_out.weight", E, s.n_head * D)
        q8(p + "ffn_gate.weight", s.n_ff, E)
        q8(p + "ffn_up.weight", s.n_ff, E)
        q8(p + "ffn_down.weight", E, s.n_ff)
    w.write(path)
    return path


@dataclass(frozen=True)
class CodecShape:
    """The codec decoder ("a.gen.wav." names as imi/core/codec.cpp:43-95 reads them). Fixed by imi: 12 codes per frame,
    6 positions per frame, window 30, n_fft 1280, hop 320, 641 bins (imi/core/codec.h:1-5,34). Chosen here, as the
    reference's files do not state them: the FSQ table's rows (2016, as imi/ref/codec_exact.py notes) and width (4),
    the projection width (256), the FFN width, heads and the conv taps."""
    n_embd: int = 512
    n_ff: int = 2048
    n_head: int = 8
    n_head_kv: int = 8
    head_dim: int = 64
    conv_k: int = 4                  # taps of the depthwise conv (d_conv = conv_k - 1 rows of memory)
    layers: str = "ccaccaca"         # per layer: c = short conv, a = gated attention over the window
    n_codes: int = 2016              # rows of the FSQ level table
    n_lvl: int = 4
    n_cb: int = 12
    n_q: int = 256                   # width of the quantizer's output projection
    n_bins: int = 641


CODEC = CodecShape()
TINY_CODEC = CodecShape(n_embd=128, n_ff=256, n_head=2, n_head_kv=1, head_dim=64, layers="cac", n_codes=64, n_q=64)


def write_codec(path: str, shape: CodecShape = CODEC, seed: int = 2) -> str:
    """Q8_0 tables (scales |N(0, 0.02)| / 8 and int8 codes as the other files), fp32 FSQ levels uniform in [-1, 1],
    projections and biases N(0, 0.1)-sized, norms 1 + 0.05 N(0, 1), conv taps N(0, 0.3), fp32 head gates N(0, 0.05);
    the output bias puts the log magnitudes near -3 and the phases near 0."""
    s = shape
    E, D = s.n_embd, s.head_dim
    w = GGUFWriter()
    w.add_str("general.architecture", "lfm3-wav")
    g = "a.gen.wav."

    def q8(name, rows, cols):
        w.add_tensor(g + name, T_Q8_0, (cols, rows), q8_0_random(_rng(seed, name), rows, cols))

    def f32(name, arr, ne):
        w.add_tensor(g + name, T_F32, ne, np.ascontiguousarray(arr, dtype=np.float32))

    nq = s.n_cb * s.n_lvl
    f32("quant.first.codebook.weight", _rng(seed, "lvl").uniform(-1.0, 1.0, (s.n_codes, s.n_lvl)), (s.n_lvl, s.n_codes))
    f32("quant.first.out_proj.weight", _rng(seed, "qo").standard_normal((s.n_q, nq)) / np.sqrt(nq), (nq, s.n_q))
    f32("quant.first.out_proj.bias", 0.1 * _rng(seed, "qob").standard_normal(s.n_q), (s.n_q,))
    q8("tfm.in_proj.weight", E, s.n_q)
    f32("tfm.in_proj.bias", 0.1 * _rng(seed, "inb").standard_normal(E), (E,))
    for il, kind in enumerate(s.layers):
        p = f"tfm.blk.{il}."
        for n in ("ln1", "ln2", "attn_post_norm", "ffn_post_norm"):
            f32(p + n + ".weight", _norm_w(_rng(seed, p + n), E), (E,))
        if kind == "c":
            f32(p + "conv_dw.weight", 0.3 * _rng(seed, p + "dw").standard_normal((E, s.conv_k)), (s.conv_k, E))
            q8(p + "conv_pw1.weight", 3 * E, E)
            q8(p + "conv_pw2.weight", E, E)
        else:
            f32(p + "attn_q_norm.weight", _norm_w(_rng(seed, p + "qn"), D), (D,))
            f32(p + "attn_k_norm.weight", _norm_w(_rng(seed, p + "kn"), D), (D,))
            q8(p + "attn_q.weight", s.n_head * D, E)
            q8(p + "attn_k.weight", s.n_head_kv * D, E)
            q8(p + "attn_v.weight", s.n_head_kv * D, E)
            q8(p + "attn_out.weight", E, s.n_head * D)
            f32(p + "attn_gate.weight", 0.05 * _rng(seed, p + "gate").standard_normal((s.n_head, E)), (E, s.n_head))
        q8(p + "ffn_gate.weight", s.n_ff, E)
        q8(p + "ffn_up.weight", s.n_ff, E)
        q8(p + "ffn_down.weight", E, s.n_ff)
    f32("tfm.output_norm.weight", _norm_w(_rng(seed, "onorm"), E), (E,))
    q8("tfm.out_proj.weight", 2 * s.n_bins, E)
    ob = np.concatenate([-3.0 + 0.5 * _rng(seed, "obm").standard_normal(s.n_bins),
                         0.5 * _rng(seed, "obp").standard_normal(s.n_bins)])
    f32("tfm.out_proj.bias", ob, (2 * s.n_bins,))
    w.write(path)
    return path


@dataclass
class EarsShape:
    n_mel: int = 128
    n_ch: int = 256                       # downsampler channels
    n_embd: int = 768
    n_ff: int = 2048
    n_head: int = 12
    n_head_kv: int = 12
    head_dim: int = 64
    d_conv: int = 3
    layers: str = "ccaccaccaccaccacc"     # 17 layers: c = short conv, a = attention over the window
    window: int = 32
    n_out: int = 2048                     # the brain's width


EARS = EarsShape()
TINY_EARS = EarsShape(n_mel=64, n_ch=16, n_embd=128, n_ff=256, n_head=4, n_head_kv=2, head_dim=32, layers="cac",
                      window=8, n_out=256)


def write_ears(path: str, shape: EarsShape = EARS, seed: int = 3) -> str:
    """The ears file's tensors as imi reads them (imi/core/ears.cpp:40-138): F32 downsampler convolutions
    (3x3 taps N(0, 0.5) for the first, N(0, 0.4) depthwise, pointwise N(0, 1/C)), F16 tables N(0, 1/cols), norms
    1 + 0.05 N(0, 1), conv taps N(0, 0.3), biases N(0, 0.05); keys for the mel count, window, heads and eps."""
    s = shape
    E, D, C = s.n_embd, s.head_dim, s.n_ch
    w = GGUFWriter()
    w.add_str("general.architecture", "clip")
    w.add_u32("clip.audio.num_mel_bins", s.n_mel)
    w.add_u32("clip.audio.window_size", s.window)
    w.add_u32("clip.audio.attention.head_count", s.n_head)
    w.add_f32("clip.audio.attention.layer_norm_epsilon", 1e-5)

    def f16(name, rows, cols):
        v = _rng(seed, name).standard_normal((rows, cols)) / np.sqrt(cols)
        w.add_tensor(name, T_F16, (cols, rows), v.astype(np.float16))

    def f32(name, arr, ne):
        w.add_tensor(name, T_F32, ne, np.ascontiguousarray(arr, dtype=np.float32))

    def bias(name, n):
        f32(name, 0.05 * _rng(seed, name).standard_normal(n), (n,))

    f32("a.conv1d.0.weight", 0.5 * _rng(seed, "c0").standard_normal((C, 1, 3, 3)), (3, 3, 1, C))
    bias("a.conv1d.0.bias", C)
    for i in (2, 5):
        f32(f"a.conv1d.{i}.weight", 0.4 * _rng(seed, f"c{i}").standard_normal((C, 1, 3, 3)), (3, 3, 1, C))
        bias(f"a.conv1d.{i}.bias", C)
    for i in (3, 6):
        f32(f"a.conv1d.{i}.weight", _rng(seed, f"c{i}").standard_normal((C, C, 1, 1)) / np.sqrt(C), (1, 1, C, C))
        bias(f"a.conv1d.{i}.bias", C)
    f16("a.pre_encode.out.weight", E, C * s.n_mel // 8)
    bias("a.pre_encode.out.bias", E)
    for il, kind in enumerate(s.layers):
        p = f"a.blk.{il}."
        for n in ("ln1", "ln2"):
            f32(p + n + ".weight", _norm_w(_rng(seed, p + n), E), (E,))
        if kind == "c":
            f32(p + "conv_dw.weight", 0.3 * _rng(seed, p + "dw").standard_normal((E, s.d_conv)), (s.d_conv, E))
            f16(p + "conv_pw1.weight", 3 * E, E)
            f16(p + "conv_pw2.weight", E, E)
        else:
            f32(p + "attn_q_norm.weight", _norm_w(_rng(seed, p + "qn"), D), (D,))
            f32(p + "attn_k_norm.weight", _norm_w(_rng(seed, p + "kn"), D), (D,))
            f16(p + "attn_q.weight", s.n_head * D, E)
            f16(p + "attn_k.weight", s.n_head_kv * D, E)
            f16(p + "attn_v.weight", s.n_head_kv * D, E)
            f16(p + "attn_out.weight", E, s.n_head * D)
        f16(p + "ffn_gate.weight", s.n_ff, E)
        f16(p + "ffn_up.weight", s.n_ff, E)
        f16(p + "ffn_down.weight", E, s.n_ff)
    f32("a.post_ln.weight", _norm_w(_rng(seed, "post_ln"), E), (E,))
    f32("mm.a.mlp.0.weight", _norm_w(_rng(seed, "ln_w"), E), (E,))
    bias("mm.a.mlp.0.bias", E)
    f16("mm.a.mlp.1.weight", s.n_out, E)
    bias("mm.a.mlp.1.bias", s.n_out)
    f16("mm.a.mlp.3.weight", s.n_out, s.n_out)
    bias("mm.a.mlp.3.bias", s.n_out)
    w.write(path)
    return path


def clip(n: int, seed: int = 0) -> np.ndarray:
    """n samples at 16 kHz of a seeded stand-in for speech: a few gliding partials with a syllable-rate envelope,
    plus low noise, within [-1, 1]."""
    rng = np.random.default_rng(seed)
    t = np.arange(n) / 16000.0
    y = np.zeros(n)
    for _ in range(6):
        f0, glide, amp = rng.uniform(100, 3000), rng.uniform(-200, 200), rng.uniform(0.05, 0.15)
        y += amp * np.sin(2 * np.pi * (f0 * t + 0.5 * glide * t * t / max(t[-1], 1e-9)) + rng.uniform(0, 2 * np.pi))
    y *= 0.6 + 0.4 * np.sin(2 * np.pi * 4.0 * t + rng.uniform(0, 2 * np.pi))
    y += 0.01 * rng.standard_normal(n)
    return np.clip(y, -1.0, 1.0).astype(np.float32)


def cached(kind: str, shape, seed: int, directory: str | None = None) -> str:
    """Write the model once per (kind, shape, seed) into a cache directory and return its path."""
    directory = directory or os.environ.get("NUNCHI_MODEL_DIR", "/tmp/nunchi_models")
    os.makedirs(directory, exist_ok=True)
    tag = hashlib.sha256(repr((kind, shape, seed)).encode()).hexdigest()[:16]
    path = os.path.join(directory, f"{kind}-{tag}.gguf")
    if not os.path.exists(path):
        tmp = f"{path}.{os.getpid()}.tmp"
        {"brain": write_brain, "voice": write_voice, "codec": write_codec, "ears": write_ears}[kind](tmp, shape, seed)
        os.replace(tmp, path)
    return path
