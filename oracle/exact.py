"""ORACLE — test infrastructure only. Float64 "truth key" of the brain, the voice generator, the codec and the ears.

Restates imi/ref/ref_exact.py:37-87 (brain), imi/ref/gen_exact.py:27-54 (voice generator),
imi/ref/codec_exact.py:23-72 (codec, whole-sequence form with numpy's inverse real FFT) and
imi/ref/ears_exact.py:16-102 (ears, the mel with numpy's real FFT): the file's own
dequantized weights, run in float64 with no input rounding. Used to pin the int8-cut restatement (liboracle) at the
model level: a dropped term, a wrong sign or a transposed table moves it far outside the cut's error.
Dequantization is written here from the GGUF block formats (closed forms), not shared with the product code.
"""
from __future__ import annotations

import numpy as np

from nunchi_amd.gguf import GGUFFile, Q4_0_BLOCK, Q4_1_BLOCK, Q8_0_BLOCK, T_F16, T_F32, T_Q4_0, T_Q4_1, T_Q8_0


def dequant_q4_0(raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Q4_0: weight i of a block = ((qs[i] & 15) if i < 16 else (qs[i-16] >> 4)) - 8, times the fp16 scale."""
    b = np.frombuffer(np.ascontiguousarray(raw).tobytes(), dtype=Q4_0_BLOCK).reshape(rows, cols // 32)
    qs = b["qs"].astype(np.int64)
    codes = np.concatenate([qs & 15, qs >> 4], axis=-1) - 8              # [rows][nb][32]
    return (codes * b["d"].astype(np.float64)[..., None]).reshape(rows, cols)


def dequant_q4_1(raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Q4_1: weight i of a block = code_i * d + m, codes 0..15 as in Q4_0 (imi/core/tables.cpp:62, 138-142)."""
    b = np.frombuffer(np.ascontiguousarray(raw).tobytes(), dtype=Q4_1_BLOCK).reshape(rows, cols // 32)
    qs = b["qs"].astype(np.int64)
    codes = np.concatenate([qs & 15, qs >> 4], axis=-1)
    return (codes * b["d"].astype(np.float64)[..., None] + b["m"].astype(np.float64)[..., None]).reshape(rows, cols)


def dequant_q8_0(raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    b = np.frombuffer(np.ascontiguousarray(raw).tobytes(), dtype=Q8_0_BLOCK).reshape(rows, cols // 32)
    return (b["qs"].astype(np.float64) * b["d"].astype(np.float64)[..., None]).reshape(rows, cols)


class Weights:
    def __init__(self, path: str, prefix: str = ""):
        self.f = GGUFFile(path)
        self.prefix = prefix
        self._cache = {}

    def has(self, name):
        return self.prefix + name in self.f.tensors

    def __call__(self, name) -> np.ndarray:
        name = self.prefix + name
        if name in self._cache:
            return self._cache[name]
        t = self.f.tensors[name]
        cols, rows = t.ne[0], t.rows
        if t.gtype == T_Q4_0:
            w = dequant_q4_0(t.data, rows, cols)
        elif t.gtype == T_Q4_1:
            w = dequant_q4_1(t.data, rows, cols)
        elif t.gtype == T_Q8_0:
            w = dequant_q8_0(t.data, rows, cols)
        elif t.gtype == T_F32:
            w = np.frombuffer(np.ascontiguousarray(t.data).tobytes(), np.float32).astype(np.float64).reshape(rows, cols)
        elif t.gtype == T_F16:
            w = np.frombuffer(np.ascontiguousarray(t.data).tobytes(), np.float16).astype(np.float64).reshape(rows, cols)
        else:
            raise ValueError(name)
        if rows == 1:
            w = w[0]
        self._cache[name] = w
        return w


def cut_dequant(x: np.ndarray) -> np.ndarray:
    """imi's input cut (imi/core/vec.h:47-75) applied in place of a table input, returned as float64 values
    q * d: per 32 values d = amax / 127 and q = rint(x / d) in float32 arithmetic, as the engine computes them."""
    x32 = np.asarray(x, np.float32).reshape(*np.shape(x)[:-1], -1, 32)
    amax = np.abs(x32).max(-1, keepdims=True)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    q = np.rint((x32 * idv).astype(np.float32))
    return (q.astype(np.float64) * d.astype(np.float64)).reshape(np.shape(x))


def forced_cut(x: np.ndarray, codes: np.ndarray, tol: float = 0.02):
    """A cut whose int8 codes are given (teacher forcing): the scale d = amax / 127 of the float64 values x as the
    cut computes it, the codes checked as a rounding of x / d (each within 0.5 + tol of it, so a code may differ from
    x's own rounding only where x / d lies within tol of a rounding boundary), returned as float64 codes * d and the
    number of codes that differ from x's own rounding."""
    x32 = np.asarray(x, np.float32).reshape(*np.shape(x)[:-1], -1, 32)
    q = np.asarray(codes, np.int8).reshape(x32.shape).astype(np.float64)
    d = (np.abs(x32).max(-1, keepdims=True) / np.float32(127)).astype(np.float32).astype(np.float64)
    x64 = np.asarray(x, np.float64).reshape(x32.shape)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(d != 0, x64 / d, 0.0)
    bad = np.abs(r - q) > 0.5 + tol
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"forced code {q[tuple(i)]:.0f} is no rounding of x / d = {r[tuple(i)]:.6f}")
    own = np.rint((x32 * np.where(d != 0, np.float32(1) / d.astype(np.float32), np.float32(0))).astype(np.float32))
    return (q * d).reshape(np.shape(x)), int((own != q).sum())


def forced_half(x: np.ndarray, half: np.ndarray, rtol: float = 1e-5) -> np.ndarray:
    """An fp16 rounding whose results are given (the engine's key / value cache): each checked within half an fp16
    ulp of the float64 value plus rtol times the largest magnitude of its head row (the last axis: the fp32 norm,
    RoPE angle and sums before the rounding err on the row's scale, not the element's), returned as float64."""
    h = np.asarray(half, np.uint16).view(np.float16).reshape(np.shape(x))
    x = np.asarray(x, np.float64)
    ulp = np.spacing(np.abs(h)).astype(np.float64)
    err = np.abs(h.astype(np.float64) - x)
    lim = 0.5 * ulp + rtol * np.abs(x).max(-1, keepdims=True)
    if (err > lim).any():
        i = tuple(np.argwhere(err > lim)[0])
        raise AssertionError(f"forced fp16 {float(h[i])!r} is no rounding of {float(x[i])!r}")
    return h.astype(np.float64)


def brain(path: str, tokens=None, embd=None, cut: bool = False, forced: dict | None = None):
    """Hidden states and logits for every position of one sequence, float64 (ref_exact.py:37-87).

    cut=True also cuts every table input to int8 per 32 exactly where imi's engine does (imi/core/seoul.cpp:405,
    415, 457, 465, 469, 480) and rounds keys and values through fp16 as its cache does, so what is left between
    this and the engine is fp32 rounding alone.

    forced (with cut=True): the engine's own int8 codes and fp16 keys and values, {"cuts": the codes of every cut of
    the steps at these positions in the order one step makes them (attention-norm input, conv or attention output,
    FFN-norm input and SwiGLU output per layer, then the hidden state for the word scores), "kv": {attention layer
    index: (keys, values) as fp16 bits [position][kv heads x D]}}. Each is checked as a rounding of the float64 value
    (forced_cut, forced_half) and then used in its place, so that a code the two arithmetics round apart (an fp32
    value within rounding of a boundary) does not move the positions after it; forced["flips"] returns the number
    of such codes."""
    C = cut_dequant if cut else (lambda v: v)
    W = Weights(path)
    kv = W.f.kv
    eps = float(kv.get("lfm3.attention.layer_norm_rms_epsilon", 1e-5))
    base, base_swa = float(kv.get("lfm3.rope.freq_base", 1e6)), float(kv.get("lfm3.rope.freq_base_swa", 1e4))
    n_swa = int(kv.get("lfm3.attention.sliding_window", 0))
    n_layer = int(kv["lfm3.block_count"])
    swa_pat = [bool(x) for x in kv.get("lfm3.attention.sliding_window_pattern", [False] * n_layer)]
    H, D = int(kv.get("lfm3.attention.head_count", 16)), int(kv.get("lfm3.attention.key_length", 128))
    ff = W("rope_freqs.weight") if W.has("rope_freqs.weight") else None
    emb = W("token_embd.weight")
    X = emb[np.asarray(tokens)] if tokens is not None else np.asarray(embd, np.float64)
    T = X.shape[0]
    site = None
    if forced is not None:
        assert cut, "forced cuts replace the cuts of cut=True"
        E, Hq, n_ff = X.shape[1], H * D, W("blk.0.ffn_gate.weight").shape[0]
        widths = []
        for il in range(n_layer):
            widths += [E, E if W.has(f"blk.{il}.shortconv.conv.weight") else Hq, E, n_ff]
        widths.append(E)
        flat = np.asarray(forced["cuts"], np.int8)
        assert flat.size == T * sum(widths), (flat.size, T, sum(widths))
        cols = np.cumsum([0] + widths)
        per = flat.reshape(T, -1)
        forced["flips"] = 0
        sites = iter(range(len(widths)))

        def site(v):
            j = next(sites)
            out, n = forced_cut(v, per[:, cols[j]:cols[j + 1]])
            forced["flips"] += n
            return out
        C = site
    ai = -1

    def norm(x, w):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w

    def rope(v, b, fr):
        half = D // 2
        inv = b ** (-np.arange(half) * 2.0 / D)
        if fr is not None:
            inv = inv / fr
        ang = np.arange(T)[:, None] * inv[None, :]
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        x0, x1 = v[..., :half], v[..., half:]
        return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], -1)

    for il in range(n_layer):
        p = f"blk.{il}."
        h = C(norm(X, W(p + "attn_norm.weight")))
        if W.has(p + "shortconv.conv.weight"):
            E = X.shape[1]
            bcx = h @ W(p + "shortconv.in_proj.weight").T
            b, c, xx = bcx[:, :E], bcx[:, E:2 * E], bcx[:, 2 * E:]
            cw = W(p + "shortconv.conv.weight")            # [E, K]
            K = cw.shape[1]
            bx = np.concatenate([np.zeros((K - 1, E)), b * xx], 0)
            co = np.stack([(bx[t:t + K] * cw.T).sum(0) for t in range(T)])
            y = C(c * co) @ W(p + "shortconv.out_proj.weight").T
        else:
            q = (h @ W(p + "attn_q.weight").T).reshape(T, H, D)
            k = h @ W(p + "attn_k.weight").T
            Hk = k.shape[1] // D
            k = k.reshape(T, Hk, D)
            v = (h @ W(p + "attn_v.weight").T).reshape(T, Hk, D)
            g = 1 / (1 + np.exp(-(h @ W(p + "attn_gate.weight").T)))
            q, k = norm(q, W(p + "attn_q_norm.weight")), norm(k, W(p + "attn_k_norm.weight"))
            sw = swa_pat[il] if il < len(swa_pat) else False
            q = rope(q, base_swa if sw else base, None if sw else ff)
            k = rope(k, base_swa if sw else base, None if sw else ff)
            ai += 1
            if forced is not None:
                kf, vf = forced["kv"][ai]
                k = forced_half(k, np.asarray(kf)[:T].reshape(k.shape))
                v = forced_half(v, np.asarray(vf)[:T].reshape(v.shape))
            elif cut:   # the engine keeps keys and values in an fp16 cache (imi/core/seoul.cpp:438)
                k = k.astype(np.float32).astype(np.float16).astype(np.float64)
                v = v.astype(np.float32).astype(np.float16).astype(np.float64)
            a = np.zeros((T, H, D))
            for t in range(T):
                s0 = max(0, t - n_swa + 1) if (sw and n_swa > 0) else 0
                for hh in range(H):
                    kv_h = hh // (H // Hk)
                    sc = k[s0:t + 1, kv_h] @ q[t, hh] / np.sqrt(D)
                    pr = np.exp(sc - sc.max())
                    pr /= pr.sum()
                    a[t, hh] = pr @ v[s0:t + 1, kv_h]
            a *= g[:, :, None]
            y = C(a.reshape(T, H * D)) @ W(p + "attn_output.weight").T
        X = X + norm(y, W(p + "post_attention_norm.weight"))
        h = C(norm(X, W(p + "ffn_norm.weight")))
        gg, uu = h @ W(p + "ffn_gate.weight").T, h @ W(p + "ffn_up.weight").T
        fo = C(gg / (1 + np.exp(-gg)) * uu) @ W(p + "ffn_down.weight").T
        X = X + norm(fo, W(p + "post_ffw_norm.weight"))
    hid = norm(X, W("output_norm.weight"))
    return hid, C(hid) @ emb.T


def voice_pass(path: str, hidden, codes, eps=1e-5, theta=1e6):
    """Scores of every codebook for one pass (gen_exact.py:27-54), float64: [n_cb][n_vocab]."""
    W = Weights(path, "a.gen.code.")
    embd_t = W.f.tensors["a.gen.code.embd.weight"]
    E, V, P = embd_t.ne[0], embd_t.ne[1], embd_t.ne[2]
    embd = dequant_q8_0(embd_t.data, V * P, E).reshape(P, V, E)
    mask, onorm = W("mask_embd"), W("output_norm.weight")
    hnorm = W("head_norm.weight").reshape(P, E)
    pw, pb = W("proj_in.weight"), W("proj_in.bias")
    layers = []
    i = 0
    while W.has(f"blk.{i}.ln1.weight"):
        p = f"blk.{i}."
        layers.append({k: W(p + k + ".weight") for k in ["ln1", "ln2", "attn_q", "attn_k", "attn_v", "attn_out", "attn_gate",
                                                           "attn_q_norm", "attn_k_norm", "ffn_gate", "ffn_up", "ffn_down"]})
        i += 1
    D = layers[0]["attn_q_norm"].shape[0]
    H = layers[0]["attn_q"].shape[0] // D
    Hk = layers[0]["attn_k"].shape[0] // D

    def norm(x, w):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w

    def rope(v):
        half = D // 2
        inv = theta ** (-np.arange(half) * 2.0 / D)
        ang = np.arange(P)[:, None] * inv[None]
        c, s = np.cos(ang)[:, None], np.sin(ang)[:, None]
        a, b = v[..., :half], v[..., half:]
        return np.concatenate([a * c - b * s, a * s + b * c], -1)

    base = (pw @ np.asarray(hidden, np.float64) + pb).reshape(P, -1)
    x = base + np.stack([embd[c, codes[c]] if codes[c] >= 0 else mask for c in range(P)])
    for l in layers:
        hh = norm(x, l["ln1"])
        q = norm((hh @ l["attn_q"].T).reshape(P, H, D), l["attn_q_norm"])
        k = norm((hh @ l["attn_k"].T).reshape(P, Hk, D), l["attn_k_norm"])
        v = (hh @ l["attn_v"].T).reshape(P, Hk, D)
        g = 1 / (1 + np.exp(-(hh @ l["attn_gate"].T)))
        q, k = rope(q), rope(k)
        k, v = np.repeat(k, H // Hk, 1), np.repeat(v, H // Hk, 1)
        s = np.einsum("phd,thd->hpt", q, k) / np.sqrt(D)
        s = np.exp(s - s.max(-1, keepdims=True))
        s /= s.sum(-1, keepdims=True)
        a = np.einsum("hpt,thd->phd", s, v) * g[:, :, None]
        x = x + a.reshape(P, -1) @ l["attn_out"].T
        hh = norm(x, l["ln2"])
        gg = hh @ l["ffn_gate"].T
        x = x + (gg / (1 + np.exp(-gg)) * (hh @ l["ffn_up"].T)) @ l["ffn_down"].T
    z = norm(norm(x, onorm), hnorm)
    return np.stack([embd[c] @ z[c] for c in range(P)])


def codec(path: str, codes, eps=1e-5, win=30, theta=1e6, n_fft=1280, hop=320):
    """PCM of a run of frames (codes [F][12]) in float64, as imi/ref/codec_exact.py:23-72 computes it: N = 6F
    positions, the causal windowed attention over positions 0.., the conv over zeros before position 0, the inverse
    real FFT (numpy), periodic Hann, overlap-add normalised by the summed squared window, (n_fft - hop) / 2 trimmed
    at both ends: N * hop samples."""
    W = Weights(path, "a.gen.wav.")
    codes = np.asarray(codes, np.int64)
    F, P = len(codes), 6
    lvl = W("quant.first.codebook.weight")
    x = lvl[codes].reshape(F, -1) @ W("quant.first.out_proj.weight").T + W("quant.first.out_proj.bias")
    x = x @ W("tfm.in_proj.weight").T + W("tfm.in_proj.bias")
    x = np.repeat(x, P, 0)
    N = len(x)

    def norm(v, w):
        return v / np.sqrt((v * v).mean(-1, keepdims=True) + eps) * w

    def rope(v, D):
        half = D // 2
        inv = theta ** (-np.arange(half) * 2.0 / D)
        ang = np.arange(N)[:, None] * inv[None]
        c, sn = np.cos(ang)[:, None], np.sin(ang)[:, None]
        a, b = v[..., :half], v[..., half:]
        return np.concatenate([a * c - b * sn, a * sn + b * c], -1)

    il = 0
    while W.has(f"tfm.blk.{il}.ln1.weight"):
        p = f"tfm.blk.{il}."
        h = norm(x, W(p + "ln1.weight"))
        if W.has(p + "conv_dw.weight"):
            bcx = h @ W(p + "conv_pw1.weight").T
            E = x.shape[1]
            b, c, xx = bcx[:, :E], bcx[:, E:2 * E], bcx[:, 2 * E:]
            cw = W(p + "conv_dw.weight")
            K = cw.shape[1]
            bx = np.concatenate([np.zeros((K - 1, E)), b * xx])
            co = np.stack([(bx[t:t + K] * cw.T).sum(0) for t in range(N)])
            y = (c * co) @ W(p + "conv_pw2.weight").T
        else:
            qn = W(p + "attn_q_norm.weight")
            D = qn.shape[0]
            q = (h @ W(p + "attn_q.weight").T).reshape(N, -1, D)
            k = (h @ W(p + "attn_k.weight").T).reshape(N, -1, D)
            v = (h @ W(p + "attn_v.weight").T).reshape(N, -1, D)
            H, Hk = q.shape[1], k.shape[1]
            q, k = rope(norm(q, qn), D), rope(norm(k, W(p + "attn_k_norm.weight")), D)
            g = 1 / (1 + np.exp(-(h @ W(p + "attn_gate.weight").T)))
            a = np.zeros((N, H, D))
            for t in range(N):
                s0 = max(0, t - win + 1)
                for hh in range(H):
                    kv = hh // (H // Hk)
                    sc = k[s0:t + 1, kv] @ q[t, hh] / np.sqrt(D)
                    pr = np.exp(sc - sc.max())
                    pr /= pr.sum()
                    a[t, hh] = pr @ v[s0:t + 1, kv]
            y = (a * g[:, :, None]).reshape(N, -1) @ W(p + "attn_out.weight").T
        x = x + norm(y, W(p + "attn_post_norm.weight"))
        h = norm(x, W(p + "ln2.weight"))
        gg = h @ W(p + "ffn_gate.weight").T
        x = x + norm((gg / (1 + np.exp(-gg)) * (h @ W(p + "ffn_up.weight").T)) @ W(p + "ffn_down.weight").T,
                     W(p + "ffn_post_norm.weight"))
        il += 1
    out = norm(x, W("tfm.output_norm.weight")) @ W("tfm.out_proj.weight").T + W("tfm.out_proj.bias")
    nb = out.shape[1] // 2
    spec = np.exp(out[:, :nb]) * np.exp(1j * out[:, nb:])
    hann = 0.5 * (1 - np.cos(2 * np.pi * np.arange(n_fft) / n_fft))
    frames = np.fft.irfft(spec, n_fft, axis=1) * hann
    total = (N - 1) * hop + n_fft
    ola, ws = np.zeros(total), np.zeros(total)
    for i in range(N):
        ola[i * hop:i * hop + n_fft] += frames[i]
        ws[i * hop:i * hop + n_fft] += hann ** 2
    pcm = np.where(ws > 1e-8, ola / np.maximum(ws, 1e-30), ola)
    pad = (n_fft - hop) // 2
    return pcm[pad:pad + N * hop], out


def ears(path: str, pcm, window: int | None = None, theta: float = 1e6, eps: float = 1e-5, mel_only: bool = False):
    """Rows [positions][n_out] for 16 kHz samples in float64, as imi/ref/ears_exact.py:16-102 computes them: 400-sample
    periodic Hann frames every 160 samples, |rfft|^2, Slaney mel filters, (log10 + 4) / 4; three stride-2 3x3
    convolutions over [time][freq] with zero edges (SiLU; pointwise tables after the two depthwise ones); the
    pre_encode projection of feature c * F8 + f; the causal layers (pre-norm short conv over b * x, or attention over
    the last `window` positions with q/k norms and rope); the last norm, LayerNorm, GELU (erf) projector. `window`
    and `theta` may be overridden to show what the comparison sees. Returns (rows, mel)."""
    import math
    f = GGUFFile(path)
    W = Weights(path)
    n_mel = int(f.key("clip.audio.num_mel_bins", 128))
    win_n, hop, sr = 400, 160, 16000
    y0 = np.asarray(pcm, np.float64)
    n = len(y0)
    n_pad = win_n if n <= win_n else n + (hop - (n - win_n) % hop) % hop
    y = np.zeros(n_pad)
    y[:n] = y0
    n_fr = (n_pad - win_n) // hop + 1
    hann = 0.5 * (1 - np.cos(2 * np.pi * np.arange(win_n) / win_n))
    frames = np.stack([y[i * hop:i * hop + win_n] * hann for i in range(n_fr)])
    spec = np.abs(np.fft.rfft(frames, win_n)) ** 2
    lin, min_log_mel, step = 3 / 200, 15.0, math.log(6.4) / 27

    def hz2mel(v):
        return v * lin if v < 1000 else min_log_mel + math.log(v / 1000) / step

    def mel2hz(m):
        return m / lin if m < min_log_mel else 1000 * math.exp((m - min_log_mel) * step)

    lo, hi = hz2mel(0.0), hz2mel(sr / 2)
    pts = [mel2hz(lo + (hi - lo) * i / (n_mel + 1)) for i in range(n_mel + 2)]
    freqs = np.arange(win_n // 2 + 1) * sr / win_n
    fb = np.zeros((n_mel, win_n // 2 + 1))
    for m in range(n_mel):
        fl, fc, fr = pts[m:m + 3]
        up = (freqs >= fl) & (freqs <= fc)
        down = (freqs > fc) & (freqs <= fr)
        fb[m, up] = (freqs[up] - fl) / (fc - fl)
        fb[m, down] = (fr - freqs[down]) / (fr - fc)
        fb[m] *= 2 / (fr - fl)
    mel = (np.log10(np.maximum(spec @ fb.T, 1e-12)) + 4) / 4
    if mel_only:
        return None, mel

    def conv_s2(a, w, b, depthwise):   # a [T][F][C]; w [oc][ic][kh][kw], kw along time
        t_n, f_n, c_n = a.shape
        to, fo = (t_n + 1) // 2, (f_n + 1) // 2
        p = np.zeros((t_n + 2, f_n + 2, c_n))
        p[1:t_n + 1, 1:f_n + 1] = a
        out = np.zeros((to, fo, w.shape[0]))
        for kh in range(3):
            for kw in range(3):
                patch = p[kw:kw + 2 * to:2, kh:kh + 2 * fo:2]
                out += patch * w[:, 0, kh, kw] if depthwise else patch[..., :1] * w[:, 0, kh, kw]
        return out + b.reshape(-1)

    def silu(v):
        return v / (1 + np.exp(-v))

    def cw(name):
        w = W(name)
        return w.reshape(-1, 1, 3, 3)

    def pw(a, name, bname):
        w = W(name)
        c = int(round(math.sqrt(w.size)))
        return a @ w.reshape(c, c).T + W(bname).reshape(-1)

    a = silu(conv_s2(mel[:, :, None], cw("a.conv1d.0.weight"), W("a.conv1d.0.bias"), False))
    a = silu(pw(conv_s2(a, cw("a.conv1d.2.weight"), W("a.conv1d.2.bias"), True), "a.conv1d.3.weight", "a.conv1d.3.bias"))
    a = silu(pw(conv_s2(a, cw("a.conv1d.5.weight"), W("a.conv1d.5.bias"), True), "a.conv1d.6.weight", "a.conv1d.6.bias"))
    N = a.shape[0]
    x = a.transpose(0, 2, 1).reshape(N, -1) @ W("a.pre_encode.out.weight").T + W("a.pre_encode.out.bias")
    window = int(f.key("clip.audio.window_size", 32)) if window is None else window

    def norm(v, w):
        return v / np.sqrt((v * v).mean(-1, keepdims=True) + eps) * w

    def rope(v, D):
        half = D // 2
        inv = theta ** (-np.arange(half) * 2.0 / D)
        ang = np.arange(N)[:, None] * inv[None]
        c, s_ = np.cos(ang)[:, None], np.sin(ang)[:, None]
        p0, p1 = v[..., :half], v[..., half:]
        return np.concatenate([p0 * c - p1 * s_, p0 * s_ + p1 * c], -1)

    il = 0
    while W.has(f"a.blk.{il}.ln1.weight"):
        p = f"a.blk.{il}."
        h = norm(x, W(p + "ln1.weight"))
        E = x.shape[1]
        if W.has(p + "conv_dw.weight"):
            bcx = h @ W(p + "conv_pw1.weight").T
            b, c, xx = bcx[:, :E], bcx[:, E:2 * E], bcx[:, 2 * E:]
            w_dw = W(p + "conv_dw.weight")
            K = w_dw.shape[1]
            bx = np.concatenate([np.zeros((K - 1, E)), b * xx])
            co = np.stack([(bx[t:t + K] * w_dw.T).sum(0) for t in range(N)])
            yv = (c * co) @ W(p + "conv_pw2.weight").T
        else:
            qn = W(p + "attn_q_norm.weight")
            D = qn.shape[0]
            q = (h @ W(p + "attn_q.weight").T).reshape(N, -1, D)
            k = (h @ W(p + "attn_k.weight").T).reshape(N, -1, D)
            v = (h @ W(p + "attn_v.weight").T).reshape(N, -1, D)
            H, Hk = q.shape[1], k.shape[1]
            q, k = rope(norm(q, qn), D), rope(norm(k, W(p + "attn_k_norm.weight")), D)
            att = np.zeros((N, H, D))
            grp = H // Hk
            for t in range(N):
                s0 = max(0, t - window + 1)
                for hh in range(H):
                    kv = hh // grp
                    sc = k[s0:t + 1, kv] @ q[t, hh] / np.sqrt(D)
                    pr = np.exp(sc - sc.max())
                    pr /= pr.sum()
                    att[t, hh] = pr @ v[s0:t + 1, kv]
            yv = att.reshape(N, -1) @ W(p + "attn_out.weight").T
        x = x + yv
        h = norm(x, W(p + "ln2.weight"))
        g = h @ W(p + "ffn_gate.weight").T
        x = x + (silu(g) * (h @ W(p + "ffn_up.weight").T)) @ W(p + "ffn_down.weight").T
        il += 1
    x = norm(x, W("a.post_ln.weight"))
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    x = (x - mu) / np.sqrt(var + 1e-5) * W("mm.a.mlp.0.weight") + W("mm.a.mlp.0.bias")
    x = x @ W("mm.a.mlp.1.weight").T + W("mm.a.mlp.1.bias")
    erf = np.vectorize(math.erf)
    x = 0.5 * x * (1 + erf(x / math.sqrt(2)))
    x = x @ W("mm.a.mlp.3.weight").T + W("mm.a.mlp.3.bias")
    return x, mel

