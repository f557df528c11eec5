"""GGUF v3 reading and writing with numpy, for the model files the engine loads.

The layout is the public GGUF v3 format that imi reads through ggml (imi/model.cpp:48-106): a header, key/value
pairs, tensor infos (name, dims with ne[0] innermost, ggml type, offset), then tensor data aligned to
``general.alignment`` (default 32). Only the types on the brain-step path are handled: F32, F16, Q4_0, Q8_0.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = 0x46554747  # "GGUF" little-endian
T_F32, T_F16, T_Q4_0, T_Q4_1, T_Q8_0, T_Q6_K = 0, 1, 2, 3, 8, 14

# value types of GGUF key/value pairs
V_U8, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STR, V_ARR, V_U64, V_I64, V_F64 = range(13)
_SCALAR = {V_U8: "<B", V_I8: "<b", V_U16: "<H", V_I16: "<h", V_U32: "<I", V_I32: "<i", V_F32: "<f", V_BOOL: "<B",
           V_U64: "<Q", V_I64: "<q", V_F64: "<d"}

Q4_0_BLOCK = np.dtype([("d", "<f2"), ("qs", "u1", 16)])   # 18 bytes per 32 weights
Q4_1_BLOCK = np.dtype([("d", "<f2"), ("m", "<f2"), ("qs", "u1", 16)])   # 20 bytes: weight = code * d + m
Q8_0_BLOCK = np.dtype([("d", "<f2"), ("qs", "i1", 32)])   # 34 bytes per 32 weights
# 210 bytes per 256 weights: low 4 bits, high 2 bits, 16 int8 scales (one per 16 values), fp16 d
Q6_K_BLOCK = np.dtype([("ql", "u1", 128), ("qh", "u1", 64), ("scales", "i1", 16), ("d", "<f2")])


def row_bytes(gtype: int, ne0: int) -> int:
    if gtype == T_F32:
        return 4 * ne0
    if gtype == T_F16:
        return 2 * ne0
    if gtype == T_Q4_0:
        return ne0 // 32 * 18
    if gtype == T_Q4_1:
        return ne0 // 32 * 20
    if gtype == T_Q8_0:
        return ne0 // 32 * 34
    if gtype == T_Q6_K:
        return ne0 // 256 * 210
    raise ValueError(f"unsupported ggml type {gtype}")


@dataclass
class Tensor:
    name: str
    gtype: int
    ne: tuple            # ne[0] innermost (columns), as in ggml
    data: np.ndarray     # raw bytes (uint8) for quantized types, typed array otherwise

    @property
    def rows(self) -> int:
        n = 1
        for d in self.ne[1:]:
            n *= d
        return n


@dataclass
class GGUFWriter:
    kv: list = field(default_factory=list)
    tensors: list = field(default_factory=list)
    alignment: int = 32

    def add_u32(self, key, v): self.kv.append((key, V_U32, int(v)))
    def add_f32(self, key, v): self.kv.append((key, V_F32, float(v)))
    def add_str(self, key, v): self.kv.append((key, V_STR, str(v)))
    def add_bool_array(self, key, vals): self.kv.append((key, V_ARR, (V_BOOL, [int(bool(x)) for x in vals])))

    def add_tensor(self, name: str, gtype: int, ne: tuple, data: np.ndarray):
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        need = row_bytes(gtype, ne[0])
        for d in ne[1:]:
            need *= d
        if raw.size != need:
            raise ValueError(f"{name}: {raw.size} bytes, shape {ne} needs {need}")
        self.tensors.append(Tensor(name, gtype, tuple(int(x) for x in ne), raw))

    def write(self, path: str):
        def s(x: str) -> bytes:
            b = x.encode()
            return struct.pack("<Q", len(b)) + b
        out = bytearray()
        out += struct.pack("<IIQQ", GGUF_MAGIC, 3, len(self.tensors), len(self.kv) + 1)
        out += s("general.alignment") + struct.pack("<I", V_U32) + struct.pack("<I", self.alignment)
        for key, vt, v in self.kv:
            out += s(key) + struct.pack("<I", vt)
            if vt == V_STR:
                out += s(v)
            elif vt == V_ARR:
                et, vals = v
                out += struct.pack("<IQ", et, len(vals))
                for x in vals:
                    out += struct.pack(_SCALAR[et], x)
            else:
                out += struct.pack(_SCALAR[vt], v)
        offsets, off = [], 0
        for t in self.tensors:
            offsets.append(off)
            off += (t.data.size + self.alignment - 1) // self.alignment * self.alignment
        for t, o in zip(self.tensors, offsets):
            out += s(t.name) + struct.pack("<I", len(t.ne))
            for d in t.ne:
                out += struct.pack("<Q", d)
            out += struct.pack("<IQ", t.gtype, o)
        pad = (-len(out)) % self.alignment
        with open(path, "wb") as f:
            f.write(out)
            f.write(b"\0" * pad)
            for t, o in zip(self.tensors, offsets):
                f.write(t.data.tobytes())
                f.write(b"\0" * ((-t.data.size) % self.alignment))


class GGUFFile:
    """Memory-mapped GGUF reader: keys in ``.kv``, tensors by name in ``.tensors`` (raw bytes views)."""

    def __init__(self, path: str):
        self.path = path
        self.buf = np.memmap(path, dtype=np.uint8, mode="r")
        b = self.buf
        o = 0

        def take(fmt):
            nonlocal o
            n = struct.calcsize(fmt)
            v = struct.unpack_from(fmt, b, o)
            o += n
            return v[0] if len(v) == 1 else v

        def string():
            nonlocal o
            n = take("<Q")
            v = bytes(b[o:o + n]).decode()
            o += n
            return v

        magic, ver, nt, nkv = take("<IIQQ")
        if magic != GGUF_MAGIC or ver < 2:
            raise ValueError(f"{path}: not a GGUF v2/v3 file")
        self.kv = {}
        for _ in range(nkv):
            key = string()
            vt = take("<I")
            if vt == V_STR:
                self.kv[key] = string()
            elif vt == V_ARR:
                et, cnt = take("<IQ")
                if et == V_STR:
                    self.kv[key] = [string() for _ in range(cnt)]
                else:
                    self.kv[key] = [take(_SCALAR[et]) for _ in range(cnt)]
            else:
                self.kv[key] = take(_SCALAR[vt])
        align = int(self.kv.get("general.alignment", 32))
        infos = []
        for _ in range(nt):
            name = string()
            nd = take("<I")
            ne = tuple(take("<Q") for _ in range(nd))
            gtype, off = take("<IQ")
            infos.append((name, ne, gtype, off))
        data0 = (o + align - 1) // align * align
        self.tensors = {}
        for name, ne, gtype, off in infos:
            n = row_bytes(gtype, ne[0])
            for d in ne[1:]:
                n *= d
            start = data0 + off
            self.tensors[name] = Tensor(name, gtype, ne, b[start:start + n])

    def key(self, name, default=None):
        return self.kv.get(name, default)
