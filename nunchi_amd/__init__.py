"""nunchi_amd: imi's brain step (the Seoul hybrid LM token loop) on one MI355X.

Python face of libseoul_hip.so (C ABI in include/seoul_hip.h), shaped like imi's engine API
(imi/core/seoul.h:28-94): Brain.load / reset / step / step2 / step_batch / new_state / swap_state, plus a
device-side greedy loop and the kernel-level Q4_0 table API (imi/kernels/q4x8.h:14-18). There is no CPU fallback:
if the HIP library is missing or no GPU is present, constructing a Brain or a Q4Table raises.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
import weakref

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libseoul_hip.so")

SH_OK, SH_E_ARG, SH_E_HIP, SH_E_FILE, SH_E_SHAPE, SH_E_CONTEXT_FULL, SH_E_STATE, SH_E_NOMEM = 0, -1, -2, -3, -4, -5, -6, -7
EXPORTS = [
    "sh_last_error", "sh_create", "sh_destroy", "sh_load", "sh_info", "sh_check_model", "sh_state_new", "sh_state_free", "sh_state_reset",
    "sh_state_pos", "sh_state_set_pos", "sh_step", "sh_step2", "sh_step_batch", "sh_generate", "sh_bench_tables",
    "sh_bench_kernel", "sh_bench_step_kernel",
    "sh_q4_create", "sh_q4_free", "sh_q4_rows", "sh_q4_gemv", "sh_q4_gemm", "sh_q4_gemm_noalloc", "sh_q4_gemv_dev", "sh_q4_bench", "sh_q4_bench_kernel", "sh_q4_bench_graph",
    "sh_q4_gemv_group", "sh_q4_gemv_group_dev", "sh_q4_group_bench", "sh_expf", "sh_sync",
    "sh_voice_load", "sh_voice_free", "sh_voice_info", "sh_voice_begin_frame", "sh_voice_base", "sh_voice_pass",
    "sh_voice_feedback", "sh_voice_sample",
    "sh_file_load", "sh_file_free", "sh_file_get", "sh_file_key_i", "sh_file_key_f", "sh_file_keep", "sh_file_drop_data",
    "sh_file_n_tensors", "sh_file_tensor", "sh_file_key_arr", "sh_file_block",
    "sh_codec_load", "sh_codec_free", "sh_codec_info", "sh_codec_reset", "sh_codec_frame", "sh_codec_flush",
    "sh_ears_load", "sh_ears_free", "sh_ears_info", "sh_ears_positions", "sh_ears_encode", "sh_ears_mel",
    "sh_bench_empty", "sh_bench_read", "sh_bench_xcc", "sh_bench_l2_reuse",
]


class SeoulError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (status {code})")
        self.code = code


class ContextFull(SeoulError):
    pass


class ModelInfo(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_embd", "n_vocab", "n_head", "n_head_kv", "head_dim", "n_ff", "d_conv", "n_ctx",
                                       "n_layer", "n_attn", "n_swa")] + [("table_bytes", C.c_longlong), ("vector_bytes", C.c_longlong)]


class VoiceShape(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_embd", "n_vocab", "n_cb", "n_in", "n_head", "n_head_kv", "head_dim", "n_ff",
                                       "n_layer")] + [("table_bytes", C.c_longlong), ("feedback_bytes", C.c_longlong)]


class CodecShape(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "d_conv", "n_layer", "n_bins",
                                       "n_lvl", "n_q", "n_codes")] + [("table_bytes", C.c_longlong)]


class EarsShape(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_mel", "n_ch", "n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "window",
                                       "n_out", "d_conv", "n_layer", "n_attn", "n_mid")] + [("table_bytes", C.c_longlong)]


class Tensor(C.Structure):
    """sh_tensor: the ggml tensor fields imi reads (type, n_dims, ne, nb, data, name)."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("n_dims", C.c_int), ("ne", C.c_int64 * 4),
                ("nb", C.c_size_t * 4), ("data", C.c_void_p)]


_lib = None


def load_library(path: str = LIB_PATH):
    """Load libseoul_hip.so and declare its C ABI. Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is not built: run `python -m nunchi_amd.build` (hipcc, gfx950)")
    L = C.CDLL(path)
    vp, i, f, d = C.c_void_p, C.c_int, C.c_float, C.c_double
    P = C.POINTER
    sig = {
        "sh_last_error": (C.c_char_p, []),
        "sh_create": (i, [i, P(vp)]),
        "sh_destroy": (i, [vp]),
        "sh_load": (i, [vp, C.c_char_p, i]),
        "sh_info": (i, [vp, P(ModelInfo)]),
        "sh_check_model": (i, [C.c_char_p, i, P(ModelInfo)]),
        "sh_state_new": (i, [vp, P(vp)]),
        "sh_state_free": (i, [vp]),
        "sh_state_reset": (i, [vp]),
        "sh_state_pos": (i, [vp, P(i)]),
        "sh_state_set_pos": (i, [vp, i]),
        "sh_step": (i, [vp, vp, C.c_int32, vp, i, vp, vp, vp]),
        "sh_step2": (i, [vp, vp, C.c_int32, vp, i, vp, C.c_int32, vp, i, vp, vp, vp, vp, vp, vp]),
        "sh_step_batch": (i, [vp, vp, vp, vp, i, i, vp, vp, vp, vp]),
        "sh_generate": (i, [vp, vp, vp, C.c_int32, C.c_int32, i, vp, vp, P(d)]),
        "sh_bench_tables": (i, [vp, i, i, P(d), P(d), P(d), P(i)]),
        "sh_bench_kernel": (i, [vp, i, i, i, P(d), P(d)]),
        "sh_bench_step_kernel": (i, [vp, i, i, i, P(d), P(d), P(i)]),
        "sh_q4_create": (i, [vp, vp, i, i, P(vp)]),
        "sh_q4_free": (i, [vp]),
        "sh_q4_rows": (i, [vp, vp, vp, i, vp]),
        "sh_q4_gemv": (i, [vp, vp, vp, i, vp, i]),
        "sh_q4_gemv_dev": (i, [vp, vp, vp, i, vp, i]),
        "sh_q4_gemm": (i, [vp, vp, vp, i, vp]),
        "sh_q4_gemm_noalloc": (i, [vp, vp, vp, i, vp]),
        "sh_q4_bench": (i, [vp, vp, i, i, i, i, P(d)]),
        "sh_q4_bench_kernel": (i, [vp, vp, i, i, i, i, P(d)]),
        "sh_q4_bench_graph": (i, [vp, vp, i, i, i, i, P(d)]),
        "sh_q4_gemv_group": (i, [vp, i, vp, vp, vp, i, i]),
        "sh_q4_gemv_group_dev": (i, [vp, i, vp, vp, vp, i, i]),
        "sh_q4_group_bench": (i, [vp, i, i, vp, i, i, i, P(d)]),
        "sh_expf": (i, [vp, vp, C.c_longlong, vp]),
        "sh_sync": (i, [vp]),
        "sh_voice_load": (i, [i, C.c_char_p, P(vp)]),
        "sh_voice_free": (i, [vp]),
        "sh_voice_info": (i, [vp, P(VoiceShape)]),
        "sh_voice_begin_frame": (i, [vp, vp]),
        "sh_voice_base": (i, [vp, vp]),
        "sh_voice_pass": (i, [vp, vp, vp, i, vp]),
        "sh_voice_feedback": (i, [vp, vp, vp]),
        "sh_voice_sample": (i, [vp, vp, i, vp, f, f, vp, vp]),
        "sh_file_load": (i, [C.c_char_p, P(vp)]),
        "sh_file_free": (i, [vp]),
        "sh_file_get": (i, [vp, C.c_char_p, P(Tensor)]),
        "sh_file_key_i": (C.c_int64, [vp, C.c_char_p, C.c_int64]),
        "sh_file_key_f": (f, [vp, C.c_char_p, f]),
        "sh_file_keep": (i, [vp, C.c_char_p, P(Tensor)]),
        "sh_file_drop_data": (i, [vp]),
        "sh_file_n_tensors": (i, [vp]),
        "sh_file_tensor": (i, [vp, i, P(Tensor)]),
        "sh_file_key_arr": (i, [vp, C.c_char_p, P(C.c_int64), i]),
        "sh_file_block": (i, [vp, P(vp), P(C.c_size_t)]),
        "sh_codec_load": (i, [i, C.c_char_p, P(vp)]),
        "sh_codec_free": (i, [vp]),
        "sh_codec_info": (i, [vp, P(CodecShape)]),
        "sh_codec_reset": (i, [vp]),
        "sh_codec_frame": (i, [vp, vp, vp, P(i)]),
        "sh_codec_flush": (i, [vp, vp, P(i)]),
        "sh_bench_empty": (i, [i, i, i, P(d)]),
        "sh_bench_read": (i, [i, C.c_longlong, i, i, i, P(d), vp]),
        "sh_bench_xcc": (i, [i, i, i, vp]),
        "sh_bench_l2_reuse": (i, [i, i, P(d), P(d), P(i)]),
        "sh_ears_load": (i, [i, C.c_char_p, P(vp)]),
        "sh_ears_free": (i, [vp]),
        "sh_ears_info": (i, [vp, P(EarsShape)]),
        "sh_ears_positions": (i, [vp, i, P(i), P(i)]),
        "sh_ears_encode": (i, [vp, vp, i, vp, P(i)]),
        "sh_ears_mel": (i, [vp, vp, i, P(i)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc: int):
    if rc != SH_OK:
        msg = _lib.sh_last_error().decode()
        raise (ContextFull if rc == SH_E_CONTEXT_FULL else SeoulError)(rc, msg)


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def check_model(path: str, n_ctx: int = 1024) -> ModelInfo:
    """sh_check_model: the file's keys and table shapes against what the kernels take, on the host (no device).
    Raises SeoulError (status SH_E_SHAPE or SH_E_FILE) naming the first problem."""
    L = load_library()
    info = ModelInfo()
    _check(L.sh_check_model(path.encode(), int(n_ctx), C.byref(info)))
    return info


class File:
    """A GGUF file read into host memory through the library (imi_file, imi/model.h:12-36): get / key_i / key_f /
    keep / drop_data. No device is involved."""

    def __init__(self, path: str):
        L = load_library()
        self.h = C.c_void_p()
        _check(L.sh_file_load(path.encode(), C.byref(self.h)))

    def close(self):
        if getattr(self, "h", None) and self.h.value:
            _lib.sh_file_free(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        self.close()

    @staticmethod
    def _desc(t: Tensor) -> dict:
        return {"name": t.name.decode(), "type": t.type, "n_dims": t.n_dims, "ne": list(t.ne), "nb": list(t.nb),
                "data": t.data}

    def get(self, name: str) -> dict | None:
        t = Tensor()
        return self._desc(t) if _lib.sh_file_get(self.h, name.encode(), C.byref(t)) == SH_OK else None

    def bytes_of(self, name: str) -> bytes | None:
        """The tensor's bytes as the host holds them now (None once dropped and not kept)."""
        d = self.get(name)
        if d is None or not d["data"]:
            return None
        return C.string_at(d["data"], d["nb"][3] * d["ne"][3])

    def key_i(self, key: str, default: int) -> int:
        return int(_lib.sh_file_key_i(self.h, key.encode(), int(default)))

    def key_f(self, key: str, default: float) -> float:
        return float(_lib.sh_file_key_f(self.h, key.encode(), float(default)))

    def key_arr(self, key: str) -> list:
        n = _lib.sh_file_key_arr(self.h, key.encode(), None, 0)
        out = (C.c_int64 * max(n, 1))()
        _lib.sh_file_key_arr(self.h, key.encode(), out, n)
        return list(out)[:n]

    def keep(self, name: str) -> dict:
        t = Tensor()
        _check(_lib.sh_file_keep(self.h, name.encode(), C.byref(t)))
        return self._desc(t)

    def drop_data(self):
        _check(_lib.sh_file_drop_data(self.h))

    def block(self):
        d, n = C.c_void_p(), C.c_size_t()
        _check(_lib.sh_file_block(self.h, C.byref(d), C.byref(n)))
        return d.value, n.value

    def tensors(self) -> list:
        out = []
        for k in range(_lib.sh_file_n_tensors(self.h)):
            t = Tensor()
            _check(_lib.sh_file_tensor(self.h, k, C.byref(t)))
            out.append(self._desc(t))
        return out


_live_contexts = weakref.WeakSet()


class Context:
    """One device and its stream (sh_create). States and tables made on it are freed before it is destroyed (the
    C ABI requires it), whatever order the garbage collector finalizes them in."""

    def __init__(self, device: int = 0):
        load_library()
        self.h = C.c_void_p()
        self._children = weakref.WeakSet()
        _check(_lib.sh_create(device, C.byref(self.h)))
        _live_contexts.add(self)

    def _adopt(self, obj):
        self._children.add(obj)

    def close(self):
        if getattr(self, "h", None) and self.h.value:
            for ch in list(self._children):
                ch._free()
            _lib.sh_destroy(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        self.close()

    def sync(self):
        _check(_lib.sh_sync(self.h))

    def expf(self, x: np.ndarray) -> np.ndarray:
        """The kernels' exponential (glibc's expf, bit for bit) on the device."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        _check(_lib.sh_expf(self.h, _p(x), int(x.size), _p(y)))
        return y


class State:
    """One conversation's memory (imi_seoul_state, imi/core/seoul.h:21-26)."""

    def __init__(self, brain: "Brain"):
        self.brain = brain
        self.h = C.c_void_p()
        _check(_lib.sh_state_new(brain.ctx.h, C.byref(self.h)))
        self.hidden = np.zeros(brain.n_embd, np.float32)
        self.logits = np.zeros(brain.n_vocab, np.float32)
        brain.ctx._adopt(self)

    def _free(self):
        if getattr(self, "h", None) and self.h.value:
            _lib.sh_state_free(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        self._free()

    @property
    def pos(self) -> int:
        p = C.c_int()
        _check(_lib.sh_state_pos(self.h, C.byref(p)))
        return p.value

    @pos.setter
    def pos(self, v: int):
        _check(_lib.sh_state_set_pos(self.h, int(v)))

    def reset(self):
        _check(_lib.sh_state_reset(self.h))


class Brain:
    """imi_seoul on the GPU: load(path, ctx_len) then step / step2 / step_batch on its own state."""

    def __init__(self, path: str, n_ctx: int = 1024, device: int = 0, ctx: Context | None = None):
        self.ctx = ctx or Context(device)
        _check(_lib.sh_load(self.ctx.h, path.encode(), int(n_ctx)))
        info = ModelInfo()
        _check(_lib.sh_info(self.ctx.h, C.byref(info)))
        self.info = info
        for n, _ in ModelInfo._fields_:
            setattr(self, n, getattr(info, n))
        self.state = State(self)

    # the brain's own conversation (imi_seoul::hidden / logits / pos)
    @property
    def hidden(self):
        return self.state.hidden

    @property
    def logits(self):
        return self.state.logits

    @property
    def pos(self) -> int:
        return self.state.pos

    def new_state(self) -> State:
        return State(self)

    def swap_state(self, other: State):
        """imi_seoul::swap_state (imi/core/seoul.cpp:203-206): trade the brain's own memory for other's, O(1)."""
        mine = self.state
        mine.h, other.h = other.h, mine.h
        mine.hidden, other.hidden = other.hidden, mine.hidden
        mine.logits, other.logits = other.logits, mine.logits

    def reset(self):
        self.state.reset()

    def step(self, token: int, embd=None, want_logits: bool = True, st: State | None = None):
        st = st or self.state
        e = None if embd is None else np.ascontiguousarray(embd, np.float32)
        best = C.c_int32(-1)
        _check(_lib.sh_step(self.ctx.h, st.h, int(token), _p(e), int(bool(want_logits)), _p(st.hidden),
                            _p(st.logits) if want_logits else None, C.byref(best)))
        return st.hidden.copy(), (st.logits.copy() if want_logits else None), best.value

    def step2(self, token_a, embd_a, logits_a, b: State, token_b, embd_b, logits_b, a: State | None = None):
        a = a or self.state
        ea = None if embd_a is None else np.ascontiguousarray(embd_a, np.float32)
        eb = None if embd_b is None else np.ascontiguousarray(embd_b, np.float32)
        ba, bb = C.c_int32(-1), C.c_int32(-1)
        _check(_lib.sh_step2(self.ctx.h, a.h, int(token_a), _p(ea), int(bool(logits_a)), b.h, int(token_b), _p(eb),
                             int(bool(logits_b)), _p(a.hidden), _p(a.logits), C.byref(ba), _p(b.hidden), _p(b.logits),
                             C.byref(bb)))
        return ((a.hidden.copy(), a.logits.copy() if logits_a else None, ba.value),
                (b.hidden.copy(), b.logits.copy() if logits_b else None, bb.value))

    def step_batch(self, tokens=None, embd=None, want_logits: bool = True, hidden_all: bool = False, st: State | None = None):
        st = st or self.state
        t = None if tokens is None else np.ascontiguousarray(tokens, np.int32)
        e = None if embd is None else np.ascontiguousarray(embd, np.float32)
        n = len(t) if t is not None else e.shape[0]
        ha = np.zeros((n, self.n_embd), np.float32) if hidden_all else None
        best = C.c_int32(-1)
        _check(_lib.sh_step_batch(self.ctx.h, st.h, _p(t), _p(e), n, int(bool(want_logits)), _p(st.hidden),
                                  _p(st.logits) if want_logits else None, _p(ha), C.byref(best)))
        return st.hidden.copy(), (st.logits.copy() if want_logits else None), best.value, ha

    def generate(self, first: int, n: int, b: State | None = None, first_b: int = 0, a: State | None = None):
        """Greedy decode on the device (device-side argmax feedback). Returns ids (and b's ids) and device seconds."""
        a = a or self.state
        oa = np.zeros(n, np.int32)
        ob = np.zeros(n, np.int32) if b is not None else None
        secs = C.c_double(0)
        _check(_lib.sh_generate(self.ctx.h, a.h, b.h if b is not None else None, int(first), int(first_b), int(n),
                                _p(oa), _p(ob), C.byref(secs)))
        return (oa, ob, secs.value) if b is not None else (oa, secs.value)

    def bench_tables(self, ncol: int = 1, reps: int = 10):
        ms, us, by, nl = C.c_double(), C.c_double(), C.c_double(), C.c_int()
        _check(_lib.sh_bench_tables(self.ctx.h, int(ncol), int(reps), C.byref(ms), C.byref(us), C.byref(by), C.byref(nl)))
        return {"ms_per_pass": ms.value, "avg_launch_us": us.value, "bytes_per_pass": by.value, "launches": nl.value}

    KERNELS = {"ffn_gate_up": 0, "ffn_down": 1, "word_scores": 2}

    def bench_kernel(self, kind: str, n_in: int = 1, reps: int = 64):
        """Mean duration (us) and bytes per launch of the step's GEMV for one table kind."""
        us, by = C.c_double(), C.c_double()
        _check(_lib.sh_bench_kernel(self.ctx.h, self.KERNELS[kind], int(n_in), int(reps), C.byref(us), C.byref(by)))
        return {"avg_us": us.value, "bytes_per_launch": by.value}

    def bench_step_kernel(self, kind: str, n_in: int = 1, steps: int = 32):
        """Mean duration (us) of one table kind's GEMV kernel inside whole steps (its inputs just written by the
        step's previous kernel, its table read from HBM), bytes per launch and the number of launches timed."""
        us, by, n = C.c_double(), C.c_double(), C.c_int()
        _check(_lib.sh_bench_step_kernel(self.ctx.h, self.KERNELS[kind], int(n_in), int(steps), C.byref(us), C.byref(by),
                                         C.byref(n)))
        return {"avg_us": us.value, "bytes_per_launch": by.value, "launches": n.value}


class Q4Table:
    """One Q4_0 table on the device (kernel-level API): gemv(x) with imi's int8 input cut."""

    def __init__(self, ctx: Context, q4_0: np.ndarray, rows: int, cols: int):
        self.ctx = ctx
        self.rows, self.cols = rows, cols
        raw = np.ascontiguousarray(q4_0).view(np.uint8).reshape(-1)
        if raw.size != rows * cols // 32 * 18:
            raise ValueError("q4_0 buffer size does not match rows x cols")
        self.h = C.c_void_p()
        _check(_lib.sh_q4_create(ctx.h, _p(raw), rows, cols, C.byref(self.h)))
        ctx._adopt(self)

    def _free(self):
        if getattr(self, "h", None) and self.h.value:
            _lib.sh_q4_free(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        self._free()

    def rows_dequant(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.zeros((ids.size, self.cols), np.float32)
        _check(_lib.sh_q4_rows(self.ctx.h, self.h, _p(ids), int(ids.size), _p(out)))
        return out

    def gemv(self, x: np.ndarray, cut_mode: int = 0) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        n_in = 1 if x.ndim == 1 else x.shape[0]
        y = np.zeros((n_in, self.rows), np.float32)
        _check(_lib.sh_q4_gemv(self.ctx.h, self.h, _p(x.reshape(-1)), n_in, _p(y.reshape(-1)), int(cut_mode)))
        return y[0] if x.ndim == 1 else y


    def gemm(self, x: np.ndarray) -> np.ndarray:
        """n inputs through the prefill's matrix-core product (imi_q4_group_batch arithmetic)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.cols)
        y = np.zeros((x.shape[0], self.rows), np.float32)
        _check(_lib.sh_q4_gemm(self.ctx.h, self.h, _p(x), int(x.shape[0]), _p(y)))
        return y


def bench_empty(device: int = 0, grid: int = 1024, reps: int = 1000) -> float:
    """Microseconds per launch of an empty grid x 256 kernel, back to back on one stream."""
    L = load_library()
    us = C.c_double()
    _check(L.sh_bench_empty(int(device), int(grid), int(reps), C.byref(us)))
    return us.value


def bench_read(nbytes: int, copies: int = 64, grid: int = 1152, reps: int = 256, device: int = 0, stamps: bool = False):
    """Microseconds per launch of a pure read of nbytes (copies distinct buffers in rotation), back to back; with
    stamps, also one launch's (last workgroup start, median first loads back, last workgroup end) in microseconds after
    the first workgroup started."""
    L = load_library()
    us = C.c_double()
    st = np.zeros(3, np.float64)
    _check(L.sh_bench_read(int(device), int(nbytes), int(copies), int(grid), int(reps), C.byref(us),
                           st.ctypes.data if stamps else None))
    return (us.value, tuple(float(v) for v in st)) if stamps else us.value


def bench_xcc(grid: int = 256, launches: int = 4, device: int = 0) -> np.ndarray:
    """XCD of each workgroup over `launches` launches back to back: array [launches][grid]."""
    L = load_library()
    out = np.zeros((int(launches), int(grid)), np.int32)
    _check(L.sh_bench_xcc(int(device), int(grid), int(launches), out.ctypes.data))
    return out


def bench_l2_reuse(pairs: int = 8, device: int = 0) -> dict:
    """A launch reading what the launch before it read (same 72 KB slot per workgroup) against one reading fresh
    slots: event microseconds of each, and how many workgroups ran on the same XCD as their counterpart."""
    L = load_library()
    a, b, same = C.c_double(), C.c_double(), C.c_int()
    _check(L.sh_bench_l2_reuse(int(device), int(pairs), C.byref(a), C.byref(b), C.byref(same)))
    return {"second_read_us": a.value, "fresh_read_us": b.value, "same_xcd": same.value, "workgroups": 256 * int(pairs)}


def q4_bench(ctx: Context, tables, n_in: int = 1, cut_mode: int = 0, reps: int = 200) -> float:
    """Mean launch duration (us) of the GEMV over `tables` in rotation, inputs resident on the device."""
    arr = (C.c_void_p * len(tables))(*[t.h.value for t in tables])
    us = C.c_double()
    _check(_lib.sh_q4_bench(ctx.h, arr, len(tables), int(n_in), int(cut_mode), int(reps), C.byref(us)))
    return us.value


def q4_bench_graph(ctx: Context, tables, n_in: int = 1, cut_mode: int = 0, passes: int = 10) -> float:
    """Mean launch time (us) of the GEMV over `tables` when one pass over them (a launch per table) is captured into a
    HIP graph and replayed `passes` times back to back; after q4_bench on the same tables."""
    arr = (C.c_void_p * len(tables))(*[t.h.value for t in tables])
    us = C.c_double()
    _check(_lib.sh_q4_bench_graph(ctx.h, arr, len(tables), int(n_in), int(cut_mode), int(passes), C.byref(us)))
    return us.value


def q4_bench_kernel(ctx: Context, tables, n_in: int = 1, cut_mode: int = 0, reps: int = 200) -> float:
    """Mean duration (us) of the GEMV kernel itself (events around each launch), after q4_bench on the same tables."""
    arr = (C.c_void_p * len(tables))(*[t.h.value for t in tables])
    us = C.c_double()
    _check(_lib.sh_q4_bench_kernel(ctx.h, arr, len(tables), int(n_in), int(cut_mode), int(reps), C.byref(us)))
    return us.value


def q4_gemv_group(ctx: Context, tables, xs, cut_mode: int = 0):
    """Every table's GEMV in grouped launches (tables of one width share a launch): xs[i] is [n_in][cols_i] (or one
    vector); returns the outputs [n_in][rows_i] (or vectors), each bit for bit Q4Table.gemv's."""
    one = np.asarray(xs[0]).ndim == 1
    xs = [np.ascontiguousarray(x, np.float32).reshape(-1, t.cols) for x, t in zip(xs, tables)]
    n_in = xs[0].shape[0]
    ys = [np.zeros((n_in, t.rows), np.float32) for t in tables]
    n = len(tables)
    th = (C.c_void_p * n)(*[t.h.value for t in tables])
    xp = (C.c_void_p * n)(*[x.ctypes.data for x in xs])
    yp = (C.c_void_p * n)(*[y.ctypes.data for y in ys])
    _check(_lib.sh_q4_gemv_group(ctx.h, n, th, xp, yp, int(n_in), int(cut_mode)))
    return [y[0] for y in ys] if one else ys


def q4_group_bench(ctx: Context, sets, n_in: int = 1, cut_mode: int = 0, reps: int = 200) -> float:
    """Mean time (us) of one grouped call over a set of tables (sets: equal-length lists, in rotation), inputs
    resident on the device."""
    n = len(sets[0])
    flat = [t.h.value for s in sets for t in s]
    arr = (C.c_void_p * len(flat))(*flat)
    us = C.c_double()
    _check(_lib.sh_q4_group_bench(ctx.h, len(sets), n, arr, int(n_in), int(cut_mode), int(reps), C.byref(us)))
    return us.value


class Codec:
    """The codec decoder on the device, shaped like imi_codec (imi/core/codec.h:17-65): frame(12 codes) -> the
    frame's 24 kHz samples (1920, less the start padding after a reset), flush() -> the 480 held back, reset()."""

    FRAME, TAIL = 1920, 480

    def __init__(self, path: str, device: int = 0):
        L = load_library()
        self.h = C.c_void_p()
        _check(L.sh_codec_load(int(device), path.encode(), C.byref(self.h)))
        self.info = CodecShape()
        _check(L.sh_codec_info(self.h, C.byref(self.info)))

    def close(self):
        if getattr(self, "h", None) and self.h.value:
            _lib.sh_codec_free(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        self.close()

    def reset(self):
        _check(_lib.sh_codec_reset(self.h))

    def frame(self, codes) -> np.ndarray:
        codes = np.ascontiguousarray(codes, np.int32)
        if codes.size != 12:
            raise ValueError("a codec frame takes 12 codes")
        out = np.zeros(self.FRAME, np.float32)
        n = C.c_int()
        _check(_lib.sh_codec_frame(self.h, _p(codes), _p(out), C.byref(n)))
        return out[:n.value]

    def flush(self) -> np.ndarray:
        out = np.zeros(self.TAIL, np.float32)
        n = C.c_int()
        _check(_lib.sh_codec_flush(self.h, _p(out), C.byref(n)))
        return out[:n.value]


class Ears:
    """The ears (audio encoder) on the device, shaped like imi_ears (imi/core/ears.h:17-51): encode(16 kHz samples)
    -> [positions][n_out] rows for the brain's prefill; mel() -> the last encode's [frames][n_mel] log-mel frames."""

    def __init__(self, path: str, device: int = 0):
        L = load_library()
        self.h = C.c_void_p()
        _check(L.sh_ears_load(int(device), path.encode(), C.byref(self.h)))
        self.info = EarsShape()
        _check(L.sh_ears_info(self.h, C.byref(self.info)))

    def close(self):
        if getattr(self, "h", None) and self.h.value:
            _lib.sh_ears_free(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        self.close()

    def positions(self, n: int):
        p, f = C.c_int(), C.c_int()
        _check(_lib.sh_ears_positions(self.h, int(n), C.byref(p), C.byref(f)))
        return p.value, f.value

    def encode(self, pcm) -> np.ndarray:
        pcm = np.ascontiguousarray(pcm, np.float32)
        P, _ = self.positions(len(pcm))
        out = np.zeros((P, self.info.n_out), np.float32)
        n = C.c_int()
        _check(_lib.sh_ears_encode(self.h, _p(pcm), len(pcm), _p(out), C.byref(n)))
        assert n.value == P
        return out

    def mel(self) -> np.ndarray:
        """The last encode's mel frames [n_frames][n_mel], sized from that encode's frame count."""
        n = C.c_int()
        _check(_lib.sh_ears_mel(self.h, None, 0, C.byref(n)))
        m = np.zeros((n.value, self.info.n_mel), np.float32)
        _check(_lib.sh_ears_mel(self.h, _p(m), int(n.value), C.byref(n)))
        return m


_live_voices = weakref.WeakSet()


class Voice:
    """The Q8_0 voice generator on the device, shaped like imi_voice (imi/core/voice.h:17-51): begin_frame(hidden)
    once per frame, pass_(codes, need) per masked pass, feedback(codes) for the brain's next input."""

    def __init__(self, path: str, device: int = 0):
        load_library()
        self.h = C.c_void_p()
        _check(_lib.sh_voice_load(int(device), path.encode(), C.byref(self.h)))
        _live_voices.add(self)
        sh = VoiceShape()
        _check(_lib.sh_voice_info(self.h, C.byref(sh)))
        for n, _ in VoiceShape._fields_:
            setattr(self, n, getattr(sh, n))

    def close(self):
        if getattr(self, "h", None) and self.h.value:
            _lib.sh_voice_free(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        self.close()

    def begin_frame(self, hidden):
        hidden = np.ascontiguousarray(hidden, np.float32)
        if hidden.size != self.n_in:
            raise ValueError("hidden must have n_in values")
        _check(_lib.sh_voice_begin_frame(self.h, _p(hidden)))

    def base(self) -> np.ndarray:
        out = np.zeros(self.n_cb * self.n_embd, np.float32)
        _check(_lib.sh_voice_base(self.h, _p(out)))
        return out

    def pass_(self, codes, need, scores: bool = True):
        """One masked pass; returns the scores [len(need)][n_vocab], or None with scores=False (they stay on the
        device for sample(), and the call does not wait for the pass)."""
        codes = np.ascontiguousarray(codes, np.int32)
        need = np.ascontiguousarray(need, np.int32)
        if codes.size != self.n_cb:
            raise ValueError("codes must have n_cb entries")
        out = np.zeros((need.size, self.n_vocab), np.float32) if scores else None
        _check(_lib.sh_voice_pass(self.h, _p(codes), _p(need), int(need.size), _p(out)))
        self._scored = int(need.size)
        return out

    def feedback(self, codes) -> np.ndarray:
        codes = np.ascontiguousarray(codes, np.int32)
        if codes.size != self.n_cb:
            raise ValueError("codes must have n_cb entries")
        out = np.zeros(self.n_in, np.float32)
        self._scored = -1
        _check(_lib.sh_voice_feedback(self.h, _p(codes), _p(out)))
        return out

    def sample(self, hist, u, temp: float = 0.4, rep: float = 1.2):
        """Temperature sampling with a repeat penalty of the codebooks the last pass_ scored, on the device
        (imi_talker::next, imi/core/talk.cpp:147-164): hist [n_frames][n_cb] codes of the previous frames (oldest
        first; imi passes its last min(frames, rep_win = 64)), u [n_need] uniform draws in [0, 1), one per pick.
        Returns (picks [n_need] int32, keep [n_need] float64: 1 - p[end-of-audio] / sum)."""
        hist = np.ascontiguousarray(np.asarray(hist, np.int32).reshape(-1, self.n_cb))
        u = np.ascontiguousarray(u, np.float64)
        if u.size != getattr(self, "_scored", -1):
            raise ValueError("u must hold one draw per codebook the last pass scored")
        picks = np.zeros(max(u.size, 1), np.int32)
        keep = np.zeros(max(u.size, 1), np.float64)
        _check(_lib.sh_voice_sample(self.h, _p(hist), hist.shape[0], _p(u), float(temp), float(rep), _p(picks),
                                    _p(keep)))
        return picks[:u.size], keep[:u.size]


@atexit.register
def _close_all():
    """Destroy every live context (and its states and tables) and voice generator while the HIP runtime is up."""
    for v in list(_live_voices):
        v.close()
    for c in list(_live_contexts):
        c.close()
