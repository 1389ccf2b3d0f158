"""Minimal GGUF writer for the tests (test infrastructure only), from the
published GGUF layout: magic "GGUF", u32 version, u64 tensor count, u64
metadata count; metadata entries (u64-length key, u32 type tag, value);
tensor infos (name, u32 rank, u64 dims innermost first, u32 GGML type, u64
offset into the data section); zero padding to the alignment; tensor data,
each tensor at an aligned offset.  Written independently of the C++ reader so
that the two check each other."""
import struct

import numpy as np

T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
           T_BOOL: "<B", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}

GGML = {"f32": 0, "f16": 1, "q4_0": 2, "q4_1": 3, "q5_0": 6, "q5_1": 7, "q8_0": 8, "q8_1": 9,
        "q2_k": 10, "q3_k": 11, "q4_k": 12, "q5_k": 13, "q6_k": 14}


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def encode_value(t, v):
    if t == T_STR:
        return _str(v)
    if t == T_ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(encode_value(et, x) for x in items)
    return struct.pack(_SCALAR[t], int(v) if t == T_BOOL else v)


class GGUFWriter:
    def __init__(self, version=3, alignment=32, magic=b"GGUF"):
        self.version, self.alignment, self.magic = version, alignment, magic
        self.kv = []
        self.tensors = []  # (name, dims, ggml_type, bytes)

    def add(self, key, t, value):
        self.kv.append((key, t, value))
        return self

    def add_tensor(self, name, dims, ggml_type, data):
        data = np.ascontiguousarray(data).view(np.uint8).tobytes() if not isinstance(data, bytes) else data
        self.tensors.append((name, list(dims), GGML[ggml_type] if isinstance(ggml_type, str) else ggml_type, data))
        return self

    def tobytes(self):
        out = bytearray(self.magic + struct.pack("<IQQ", self.version, len(self.tensors), len(self.kv)))
        for key, t, v in self.kv:
            out += _str(key) + struct.pack("<I", t) + encode_value(t, v)
        offsets, off = [], 0
        for _, _, _, data in self.tensors:
            offsets.append(off)
            off = (off + len(data) + self.alignment - 1) // self.alignment * self.alignment
        for (name, dims, gt, _), o in zip(self.tensors, offsets):
            out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            out += struct.pack("<IQ", gt, o)
        out += b"\0" * ((-len(out)) % self.alignment)
        self.data_start = len(out)
        for (_, _, _, data), o in zip(self.tensors, offsets):
            out += b"\0" * (self.data_start + o - len(out)) + data
        self.offsets = offsets
        return bytes(out)

    def write(self, path):
        b = self.tobytes()
        with open(path, "wb") as f:
            f.write(b)
        return b
