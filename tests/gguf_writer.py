"""Minimal GGUF v2/v3 writer for test fixtures (test infrastructure).

Writes the public GGUF layout: magic "GGUF", version, tensor count, KV count,
the KV pairs (key string, value type, value), the tensor infos (name,
n_dims, dims, ggml type, offset) and then the data section, aligned to
``general.alignment`` (32 unless set), each tensor at an aligned offset.
Strings are a u64 length and raw bytes.  Used to build the synthetic files
the reader tests open, including split shards and malformed variants.
"""
from __future__ import annotations

import struct

import numpy as np

# GGUF value type ids
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}

# ggml type ids
GGML_F32, GGML_F16, GGML_Q5_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 6, 8, 12, 14
GGML_IQ2_XXS, GGML_IQ3_XXS = 16, 18
GGML_BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q5_0: (32, 22), GGML_Q8_0: (32, 34),
              GGML_Q4_K: (256, 144), GGML_Q6_K: (256, 210), GGML_IQ2_XXS: (256, 66),
              GGML_IQ3_XXS: (256, 98)}


def gstr(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value(vtype: int, v) -> bytes:
    """Encodes one value of type vtype (no type tag).  Arrays are given as
    (element_type, [elements])."""
    if vtype == STR:
        return gstr(v)
    if vtype == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(value(et, x) for x in items)
    return struct.pack(_SCALAR[vtype], v)


def payload_bytes(ggml_type: int, ne) -> int:
    e, b = GGML_BLOCK[ggml_type]
    outer = 1
    for d in ne[1:]:
        outer *= d
    return (ne[0] // e) * b * outer


class GgufFile:
    def __init__(self, version: int = 3, alignment: int | None = None):
        self.version = version
        self.kv = []          # (key, type, value)
        self.tensors = []     # (name, ggml_type, dims, payload bytes)
        self.alignment = 32
        if alignment is not None:
            self.add_kv("general.alignment", U32, alignment)

    def add_kv(self, key, vtype, v):
        self.kv.append((key, vtype, v))
        if key == "general.alignment" and vtype in (U8, U16, U32, U64) and v > 0:
            self.alignment = v
        return self

    def add_tensor(self, name, ggml_type, dims, payload: bytes | np.ndarray | None = None):
        if payload is None:
            payload = b""
        payload = np.ascontiguousarray(payload).view(np.uint8).tobytes() \
            if isinstance(payload, np.ndarray) else bytes(payload)
        self.tensors.append((name, ggml_type, tuple(dims), payload))
        return self

    def header_and_offsets(self):
        a = self.alignment
        out = struct.pack("<IIQQ", 0x46554747, self.version, len(self.tensors), len(self.kv))
        for k, t, v in self.kv:
            out += gstr(k) + struct.pack("<I", t) + value(t, v)
        off, offs = 0, []
        for name, gt, dims, payload in self.tensors:
            off = (off + a - 1) // a * a
            offs.append(off)
            out += gstr(name) + struct.pack("<I", len(dims))
            out += b"".join(struct.pack("<Q", d) for d in dims)
            out += struct.pack("<IQ", gt, off)
            off += len(payload)
        return out, offs

    def to_bytes(self) -> bytes:
        a = self.alignment
        hdr, offs = self.header_and_offsets()
        data = bytearray()
        for (name, gt, dims, payload), off in zip(self.tensors, offs):
            data += b"\0" * (off - len(data))
            data += payload
        pad = (-len(hdr)) % a
        return hdr + b"\0" * pad + bytes(data)

    def write(self, path: str) -> bytes:
        b = self.to_bytes()
        with open(path, "wb") as f:
            f.write(b)
        return b
