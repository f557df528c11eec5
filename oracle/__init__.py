"""ORACLE — test infrastructure only. Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
as the checker; the product package (nunchi_amd) never imports it.

Python handle on liboracle.so, the C++ restatement of imi's CPU arithmetic (imi_cpu.h), plus exact.py, a float64
restatement of imi/ref/ref_exact.py and imi/ref/gen_exact.py.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def build(force: bool = False) -> str:
    """Compile liboracle.so with the recipe in oracle/Makefile."""
    subprocess.run(["make", "-s", "-C", HERE] + (["-B"] if force else []), check=True)
    return LIB_PATH


NATIVE_PATH = os.path.join(HERE, "_native", "liboracle.so")


def use_native(timeout: float = 240.0) -> bool:
    """Build the oracle for this host's CPU (oracle/Makefile `native`: -O3 -march=native, the same sources and flags
    otherwise) and load that library from now on: for timing the CPU path (every fma is written out and no reduction
    is reordered, so its numbers are the portable build's). False, keeping the portable library, if the build fails or
    a library is already loaded."""
    global LIB_PATH
    if _lib is not None:
        return LIB_PATH == NATIVE_PATH
    try:
        subprocess.run(["make", "-s", "-C", HERE, "native"], check=True, timeout=timeout, capture_output=True)
    except (subprocess.SubprocessError, OSError):
        return False
    LIB_PATH = NATIVE_PATH
    return True


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = C.CDLL(LIB_PATH)
    vp, i, f, d = C.c_void_p, C.c_int, C.c_float, C.c_double
    sig = {
        "orc_engine_load": (vp, [C.c_char_p, i, i]),
        "orc_engine_free": (None, [vp]),
        "orc_engine_info": (None, [vp, _i32p]),
        "orc_engine_reset": (None, [vp]),
        "orc_engine_set_pos": (None, [vp, i]),
        "orc_engine_step": (None, [vp, i, vp, i, vp, vp]),
        "orc_state_new": (vp, [vp]),
        "orc_state_free": (None, [vp]),
        "orc_state_info": (None, [vp, _i32p]),
        "orc_swap_state": (None, [vp, vp]),
        "orc_engine_step2": (None, [vp, i, vp, i, vp, i, vp, i, vp, vp, vp, vp]),
        "orc_engine_step_batch": (None, [vp, vp, vp, i, i, vp, vp, vp]),
        "orc_engine_greedy": (d, [vp, i, i, _i32p]),
        "orc_engine_greedy2": (d, [vp, vp, i, i, i, _i32p, _i32p]),
        "orc_engine_cache": (None, [vp, i, _u16p, _u16p]),
        "orc_engine_conv_state": (None, [vp, i, _f32p]),
        "orc_engine_trace_cuts": (None, [vp, i]),
        "orc_engine_take_cuts": (C.c_size_t, [vp, vp, C.c_size_t]),
        "orc_h2f": (f, [C.c_uint16]),
        "orc_q8k_from": (None, [_f32p, i, _i8p, _f32p, C.POINTER(C.c_int16)]),
        "orc_q6k_dequant_row": (None, [_u8p, i, _f32p]),
        "orc_q6k_rows": (None, [_u8p, i, i, _f32p, _f32p, vp]),
        "orc_f2h": (C.c_uint16, [f]),
        "orc_cut32": (f, [_f32p, _i8p, C.POINTER(C.c_int)]),
        "orc_cut": (None, [_f32p, i, _i8p, _f32p, _f32p]),
        "orc_q4_layout": (None, [_u8p, i, i, _u8p, _u16p]),
        "orc_q4_create": (vp, [_u8p, i, i, i, i]),
        "orc_q4_free": (None, [vp]),
        "orc_q4_gemv": (d, [vp, _f32p, i, _f32p, i, i]),
        "orc_q4_gemv_batch": (None, [vp, _f32p, i, _f32p]),
        "orc_q4_block_sums": (None, [vp, _f32p, _i32p]),
        "orc_q4x8_create": (vp, [_u8p, i, i, i]),
        "orc_q4x8_free": (None, [vp]),
        "orc_q4x8_gemv": (d, [vp, _f32p, _f32p, i]),
        "orc_q4x8_layout": (None, [vp, _u8p, _f32p]),
        "orc_q4x8_quant_in": (None, [_f32p, i, _i8p, _f32p, _f32p]),
        "orc_q8g_gemm": (None, [_u8p, i, i, _f32p, i, _f32p]),
        "orc_rms_scale": (f, [_f32p, i, f]),
        "orc_expf": (None, [_f32p, C.c_longlong, _f32p]),
        "orc_rope": (None, [_f32p, i, i, f, vp]),
        "orc_voice_load": (vp, [C.c_char_p, i]),
        "orc_voice_free": (None, [vp]),
        "orc_voice_info": (None, [vp, _i32p]),
        "orc_voice_begin_frame": (None, [vp, _f32p]),
        "orc_voice_base": (None, [vp, _f32p]),
        "orc_voice_pass": (None, [vp, _i32p, _i32p, i, _f32p]),
        "orc_voice_feedback": (None, [vp, _i32p, _f32p]),
        "orc_voice_sample": (None, [_f32p, i, i, _i32p, _i32p, i, i, C.POINTER(C.c_double), f, f, _i32p,
                                    C.POINTER(C.c_double)]),
        "orc_codec_load": (vp, [C.c_char_p]),
        "orc_codec_free": (None, [vp]),
        "orc_codec_info": (None, [vp, _i32p]),
        "orc_codec_reset": (None, [vp]),
        "orc_codec_frame": (i, [vp, _i32p, _f32p, vp]),
        "orc_codec_flush": (i, [vp, _f32p]),
        "orc_ifft": (None, [_f32p, _f32p, i, _f32p, _f32p]),
        "orc_ears_load": (vp, [C.c_char_p, i]),
        "orc_ears_free": (None, [vp]),
        "orc_ears_info": (None, [vp, _i32p]),
        "orc_ears_positions": (i, [vp, i]),
        "orc_ears_frames": (i, [vp, i]),
        "orc_ears_encode": (i, [vp, _f32p, i, _f32p, vp, C.POINTER(C.c_double)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class Engine:
    """imi_seoul restated (imi/core/seoul.h:28-94): load / reset / step / step2 / step_batch / new_state / swap."""

    def __init__(self, path: str, threads: int = 4, n_ctx: int = 1024):
        self.h = lib().orc_engine_load(path.encode(), threads, n_ctx)
        if not self.h:
            raise RuntimeError(f"oracle: cannot load {path}")
        info = np.zeros(12, np.int32)
        lib().orc_engine_info(self.h, info)
        (self.n_embd, self.n_vocab, self.n_head, self.n_head_kv, self.head_dim, self.n_ff, self.d_conv, self.n_ctx,
         self.n_layer, self.n_swa, _, self.n_threads) = (int(v) for v in info)
        self.hidden = np.zeros(self.n_embd, np.float32)
        self.logits = np.zeros(self.n_vocab, np.float32)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_engine_free(self.h)
            self.h = None

    @property
    def pos(self) -> int:
        info = np.zeros(12, np.int32)
        lib().orc_engine_info(self.h, info)
        return int(info[10])

    def reset(self):
        lib().orc_engine_reset(self.h)

    def set_pos(self, pos: int):
        lib().orc_engine_set_pos(self.h, pos)

    def step(self, token: int, embd=None, want_logits: bool = True):
        e = None if embd is None else np.ascontiguousarray(embd, np.float32)
        lib().orc_engine_step(self.h, int(token), _ptr(e), int(want_logits), _ptr(self.hidden), _ptr(self.logits))
        return self.hidden.copy(), (self.logits.copy() if want_logits else None)

    def new_state(self):
        return State(self)

    def swap_state(self, st: "State"):
        lib().orc_swap_state(self.h, st.h)

    def step2(self, ta, ea, la, st: "State", tb, eb, lb):
        ea = None if ea is None else np.ascontiguousarray(ea, np.float32)
        eb = None if eb is None else np.ascontiguousarray(eb, np.float32)
        ha, hb = np.zeros(self.n_embd, np.float32), np.zeros(self.n_embd, np.float32)
        lga, lgb = np.zeros(self.n_vocab, np.float32), np.zeros(self.n_vocab, np.float32)
        lib().orc_engine_step2(self.h, int(ta), _ptr(ea), int(la), st.h, int(tb), _ptr(eb), int(lb),
                               _ptr(ha), _ptr(lga), _ptr(hb), _ptr(lgb))
        return ha, (lga if la else None), hb, (lgb if lb else None)

    def step_batch(self, tokens=None, embd=None, n=None, want_logits=True, hidden_all=False):
        t = None if tokens is None else np.ascontiguousarray(tokens, np.int32)
        e = None if embd is None else np.ascontiguousarray(embd, np.float32)
        n = n if n is not None else (len(t) if t is not None else e.shape[0])
        hl = np.zeros(self.n_embd, np.float32)
        lg = np.zeros(self.n_vocab, np.float32)
        ha = np.zeros((n, self.n_embd), np.float32) if hidden_all else None
        lib().orc_engine_step_batch(self.h, _ptr(t), _ptr(e), n, int(want_logits), _ptr(hl), _ptr(lg), _ptr(ha))
        return hl, (lg if want_logits else None), ha

    def greedy(self, first_token: int, n: int):
        out = np.zeros(n, np.int32)
        secs = lib().orc_engine_greedy(self.h, int(first_token), n, out)
        return out, secs

    def greedy2(self, st: "State", ta: int, tb: int, n: int):
        oa, ob = np.zeros(n, np.int32), np.zeros(n, np.int32)
        secs = lib().orc_engine_greedy2(self.h, st.h, int(ta), int(tb), n, oa, ob)
        return oa, ob, secs

    def kv_cache(self, ai: int):
        n = self.n_ctx * self.n_head_kv * self.head_dim
        k, v = np.zeros(n, np.uint16), np.zeros(n, np.uint16)
        lib().orc_engine_cache(self.h, ai, k, v)
        return k.reshape(self.n_ctx, -1), v.reshape(self.n_ctx, -1)

    def trace_cuts(self, on: bool = True):
        """Record the int8 codes of every input cut the following single steps make (cleared when started)."""
        lib().orc_engine_trace_cuts(self.h, int(on))

    def take_cuts(self) -> np.ndarray:
        """The codes recorded since the trace started or was last taken, in the order the steps cut them."""
        n = lib().orc_engine_take_cuts(self.h, None, 0)
        out = np.zeros(n, np.int8)
        lib().orc_engine_take_cuts(self.h, _ptr(out), n)
        return out

    def conv_state(self, il: int):
        out = np.zeros(self.d_conv * self.n_embd, np.float32)
        lib().orc_engine_conv_state(self.h, il, out)
        return out.reshape(self.d_conv, self.n_embd)


class State:
    def __init__(self, eng: Engine):
        self.eng = eng
        self.h = lib().orc_state_new(eng.h)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_state_free(self.h)
            self.h = None

    @property
    def pos(self) -> int:
        p = np.zeros(1, np.int32)
        lib().orc_state_info(self.h, p)
        return int(p[0])


class Q4Table:
    """A Q4_0 (or, with q4_1, Q4_1) matrix in imi's 8-row layout with imi's GEMV (cut + group / group2 / group_batch)."""

    def __init__(self, q4_0: np.ndarray, rows: int, cols: int, threads: int = 1, q4_1: bool = False):
        self.raw = np.ascontiguousarray(q4_0).view(np.uint8).reshape(-1)
        self.rows, self.cols = rows, cols
        self.h = lib().orc_q4_create(self.raw, rows, cols, threads, int(q4_1))

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_q4_free(self.h)
            self.h = None

    def gemv(self, x: np.ndarray, scalar: bool = False, reps: int = 1):
        x = np.ascontiguousarray(x, np.float32)
        n_in = 1 if x.ndim == 1 else x.shape[0]
        y = np.zeros((n_in, self.rows), np.float32)
        secs = lib().orc_q4_gemv(self.h, x.reshape(-1), n_in, y.reshape(-1), 1 if scalar else 0, reps)
        return (y[0] if x.ndim == 1 else y), secs

    def gemv_batch(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros((x.shape[0], self.rows), np.float32)
        lib().orc_q4_gemv_batch(self.h, x.reshape(-1), x.shape[0], y.reshape(-1))
        return y

    def block_sums(self, x: np.ndarray):
        s = np.zeros((self.rows, self.cols // 32), np.int32)
        lib().orc_q4_block_sums(self.h, np.ascontiguousarray(x, np.float32), s.reshape(-1))
        return s


class Q4x8Table:
    """The cfg-0 kernel's table (imi/kernels/q4x8.cpp): pair-packed codes, fp32 scales, roundf input cut."""

    def __init__(self, q4_0: np.ndarray, rows: int, cols: int, threads: int = 1):
        self.raw = np.ascontiguousarray(q4_0).view(np.uint8).reshape(-1)
        self.rows, self.cols = rows, cols
        self.h = lib().orc_q4x8_create(self.raw, rows, cols, threads)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_q4x8_free(self.h)
            self.h = None

    def gemv(self, x: np.ndarray, reps: int = 1):
        y = np.zeros(self.rows, np.float32)
        secs = lib().orc_q4x8_gemv(self.h, np.ascontiguousarray(x, np.float32), y, reps)
        return y, secs

    def layout(self):
        codes = np.zeros(self.rows // 8 * self.cols // 32 * 128, np.uint8)
        scales = np.zeros(self.rows // 8 * self.cols // 32 * 8, np.float32)
        lib().orc_q4x8_layout(self.h, codes, scales)
        return codes, scales


class Voice:
    """imi_voice restated (imi/core/voice.h:17-51)."""

    def __init__(self, path: str, threads: int = 4):
        self.h = lib().orc_voice_load(path.encode(), threads)
        if not self.h:
            raise RuntimeError(f"oracle: cannot load {path}")
        info = np.zeros(9, np.int32)
        lib().orc_voice_info(self.h, info)
        (self.n_embd, self.n_vocab, self.n_cb, self.n_in, self.n_head, self.n_head_kv, self.head_dim, self.n_ff,
         self.n_layer) = (int(v) for v in info)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_voice_free(self.h)
            self.h = None

    def begin_frame(self, hidden):
        lib().orc_voice_begin_frame(self.h, np.ascontiguousarray(hidden, np.float32))

    def base(self):
        out = np.zeros(self.n_cb * self.n_embd, np.float32)
        lib().orc_voice_base(self.h, out)
        return out

    def pass_(self, codes, need):
        codes = np.ascontiguousarray(codes, np.int32)
        need = np.ascontiguousarray(need, np.int32)
        out = np.zeros(len(need) * self.n_vocab, np.float32)
        lib().orc_voice_pass(self.h, codes, need, len(need), out)
        return out.reshape(len(need), self.n_vocab)

    def feedback(self, codes):
        out = np.zeros(self.n_in, np.float32)
        lib().orc_voice_feedback(self.h, np.ascontiguousarray(codes, np.int32), out)
        return out


def voice_sample(scores, cbs, hist, u, temp=0.4, rep=1.2):
    """imi_talker::next's picks (imi/core/talk.cpp:147-164) of score rows scores[j] (codebook cbs[j]) given the
    history window hist [n_frames][n_cb] (oldest first) and one uniform draw u[j] per pick. Returns (picks,
    keep = 1 - p[eos] / sum, the penalised scores)."""
    l = np.array(scores, np.float32, order="C", copy=True)
    n, V = l.shape
    hist = np.ascontiguousarray(hist, np.int32)
    n_cb = hist.shape[1] if hist.ndim == 2 and hist.size else 1
    n_frames = hist.shape[0] if hist.size else 0
    u = np.ascontiguousarray(u, np.float64)
    picks = np.zeros(max(n, 1), np.int32)
    keep = np.zeros(max(n, 1), np.float64)
    lib().orc_voice_sample(l, n, V, np.ascontiguousarray(cbs, np.int32), hist.reshape(-1) if hist.size else
                           np.zeros(1, np.int32), n_frames, n_cb, u.ctypes.data_as(C.POINTER(C.c_double)),
                           float(temp), float(rep), picks, keep.ctypes.data_as(C.POINTER(C.c_double)))
    return picks[:n], keep[:n], l


def cut(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(x.size, np.int8)
    d = np.zeros(x.size // 32, np.float32)
    s = np.zeros(x.size // 32, np.float32)
    lib().orc_cut(x, x.size, q, d, s)
    return q, d, s


def q8k(x: np.ndarray):
    """imi_q8k::from (imi/core/tables.cpp:200-213): codes, d per 256, code sums per 16."""
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(x.size, np.int8)
    d = np.zeros(x.size // 256, np.float32)
    bs = np.zeros(x.size // 16, np.int16)
    lib().orc_q8k_from(x, x.size, q, d, bs.ctypes.data_as(C.POINTER(C.c_int16)))
    return q, d, bs


def q6k_dequant(row: np.ndarray, n_embd: int) -> np.ndarray:
    """imi_q6k_dequant_row of one row of n_embd / 256 blocks (bytes)."""
    row = np.ascontiguousarray(row, np.uint8)
    y = np.zeros(n_embd, np.float32)
    lib().orc_q6k_dequant_row(row, n_embd // 256, y)
    return y


def q6k_rows(rows: np.ndarray, x: np.ndarray, lanes: bool = False):
    """imi_q6k_row for every row of a [n_rows][nblocks * 210] byte table against x cut by q8k; with lanes, also the
    [n_rows][nblocks][8] int32 lane sums."""
    rows = np.ascontiguousarray(rows, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    n_rows, nb = rows.shape[0], x.size // 256
    out = np.zeros(n_rows, np.float32)
    ln = np.zeros((n_rows, nb, 8), np.int32) if lanes else None
    lib().orc_q6k_rows(rows, n_rows, nb, x, out, _ptr(ln))
    return (out, ln) if lanes else out


def expf(x: np.ndarray) -> np.ndarray:
    """The C library's expf (what imi calls), elementwise."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_expf(x.reshape(-1), x.size, y.reshape(-1))
    return y


class Codec:
    """imi_codec restated (imi/core/codec.h:17-65): frame(12 codes) -> its PCM samples (and, with spec, the frame's
    [6][2 * n_bins] log magnitudes and phases); flush() -> the tail the overlap holds back; reset()."""

    HOP, N_FS = 320, 6

    def __init__(self, path: str):
        self.h = lib().orc_codec_load(path.encode())
        if not self.h:
            raise RuntimeError(f"oracle: cannot load {path}")
        info = np.zeros(12, np.int32)
        lib().orc_codec_info(self.h, info)
        (self.n_embd, self.n_ff, self.n_head, self.n_head_kv, self.head_dim, self.d_conv, self.n_layer, self.n_bins,
         self.n_lvl, self.n_q, _, self.n_codes) = (int(v) for v in info)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_codec_free(self.h)
            self.h = None

    def reset(self):
        lib().orc_codec_reset(self.h)

    def frame(self, codes, spec: bool = False):
        codes = np.ascontiguousarray(codes, np.int32)
        pcm = np.zeros(self.N_FS * self.HOP, np.float32)
        sp = np.zeros((self.N_FS, 2 * self.n_bins), np.float32) if spec else None
        n = lib().orc_codec_frame(self.h, codes, pcm, _ptr(sp))
        return (pcm[:n], sp) if spec else pcm[:n]

    def flush(self):
        pcm = np.zeros(1280, np.float32)
        n = lib().orc_codec_flush(self.h, pcm)
        return pcm[:n]


def ifft(x) -> np.ndarray:
    """The codec's inverse DFT (imi/core/codec.cpp:25-39) of a complex vector, unnormalised."""
    x = np.asarray(x, np.complex64)
    re, im = np.ascontiguousarray(x.real, np.float32), np.ascontiguousarray(x.imag, np.float32)
    ore, oim = np.zeros_like(re), np.zeros_like(im)
    lib().orc_ifft(re, im, len(re), ore, oim)
    return ore.astype(np.complex64) + 1j * oim


def rel(a, b) -> float:
    """imi/core/seoul_check.cpp:10-14: ||a - b|| / ||b|| in double."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.sqrt(((a - b) ** 2).sum() / (((b ** 2).sum()) + 1e-30)))


def top(a) -> int:
    """imi's greedy pick (imi/core/hear.cpp:67-68, imi/core/seoul_check.cpp:15): best = 0, and score v replaces it
    only if logits[v] > logits[best]. That is the first index of the maximum; a NaN score never wins, and a NaN at
    index 0 is never beaten (nothing compares greater than it), so the pick is then 0."""
    a = np.asarray(a)
    if a.size == 0 or np.isnan(a[0]):
        return 0
    return int(np.argmax(np.where(np.isnan(a), -np.inf, a)))


class Ears:
    """imi_ears restated (imi/core/ears.h:17-51): encode(16 kHz samples) -> [positions][n_out] rows for the brain's
    prefill (and, with mel=True, the [frames][n_mel] log-mel frames the encoder read)."""

    def __init__(self, path: str, threads: int = 4):
        self.h = lib().orc_ears_load(path.encode(), int(threads))
        if not self.h:
            raise RuntimeError(f"oracle: cannot load ears from {path}")
        info = np.zeros(11, np.int32)
        lib().orc_ears_info(self.h, info)
        (self.n_mel, self.n_ch, self.n_embd, self.n_ff, self.n_head, self.n_head_kv, self.head_dim, self.window,
         self.n_out, self.d_conv, self.n_layer) = (int(v) for v in info)
        self.secs = 0.0

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_ears_free(self.h)
            self.h = None

    def positions(self, n: int) -> int:
        return int(lib().orc_ears_positions(self.h, int(n)))

    def encode(self, pcm, mel: bool = False):
        pcm = np.ascontiguousarray(pcm, np.float32)
        out = np.zeros((self.positions(len(pcm)), self.n_out), np.float32)
        m = np.zeros((lib().orc_ears_frames(self.h, len(pcm)), self.n_mel), np.float32) if mel else None
        secs = C.c_double(0)
        P = lib().orc_ears_encode(self.h, pcm, len(pcm), out, _ptr(m), C.byref(secs))
        assert P == out.shape[0]
        self.secs = secs.value
        return (out, m) if mel else out

