"""In-memory GGUF v3 images for the tests: valid, boundary and malformed (no model data).

The same construction as the reference's test builder (runtime/tests/synthetic.rs:8-87): metadata
pairs as raw typed bytes, tensor descriptors with explicit offsets, the header padded to 32 bytes,
then a data section of the given length (byte i = i mod 251) or of given bytes.
"""
from __future__ import annotations

import struct

import numpy as np


def gstr(v) -> bytes:
    b = v.encode() if isinstance(v, str) else bytes(v)
    return struct.pack("<Q", len(b)) + b


class Builder:
    def __init__(self):
        self.kv: list[tuple[str, bytes]] = []
        self.tensors: list[tuple[str, list[int], int, int]] = []
        self.data_len = 0
        self.payload: bytes | None = None
        self.version = 3

    def raw_kv(self, key: str, type_and_value: bytes) -> "Builder":
        self.kv.append((key, type_and_value))
        return self

    def kv_str(self, key: str, v: str) -> "Builder":
        return self.raw_kv(key, struct.pack("<I", 8) + gstr(v))

    def kv_u32(self, key: str, v: int) -> "Builder":
        return self.raw_kv(key, struct.pack("<II", 4, v))

    def tensor(self, name: str, shape, ty: int, offset: int) -> "Builder":
        self.tensors.append((name, list(shape), ty, offset))
        return self

    def data(self, n: int) -> "Builder":
        self.data_len, self.payload = n, None
        return self

    def data_bytes(self, b: bytes) -> "Builder":
        self.payload = bytes(b)
        return self

    def build(self) -> bytes:
        out = bytearray(b"GGUF")
        out += struct.pack("<IQQ", self.version, len(self.tensors), len(self.kv))
        for k, v in self.kv:
            out += gstr(k) + v
        for name, shape, ty, off in self.tensors:
            out += gstr(name) + struct.pack("<I", len(shape))
            for dim in shape:
                out += struct.pack("<Q", dim)
            out += struct.pack("<IQ", ty, off)
        while len(out) % 32:
            out.append(0)
        if self.payload is not None:
            out += self.payload
        else:
            out += (np.arange(self.data_len, dtype=np.int64) % 251).astype(np.uint8).tobytes()
        return bytes(out)

    def copy(self) -> "Builder":
        b = Builder()
        b.kv, b.tensors = list(self.kv), list(self.tensors)
        b.data_len, b.payload, b.version = self.data_len, self.payload, self.version
        return b


def valid() -> Builder:
    """One F32 [8] tensor at 0 and one Q4_0 [32, 2] tensor at 32: 32 + 36 bytes of data."""
    return (Builder().kv_str("general.architecture", "test").kv_u32("general.alignment", 32)
            .tensor("a", [8], 0, 0).tensor("b", [32, 2], 2, 32).data(68))


def moe_layer_image(layers: dict, extra_f32: dict | None = None, align: int = 32) -> bytes:
    """An image holding, for each layer index L, the tensors of layers[L]: gate_up (Q4_0 rows of
    [n_exp][2ff][d]), down (Q4_0 rows of [n_exp][d][ff]), router (f32 [n_exp][d]) and down_scale
    (f32 [n_exp]) under the reference's names and ggml shapes (runtime/src/contract.rs:66-70), plus
    extra F32 tensors {name: array}."""
    b = Builder().kv_str("general.architecture", "gemma4").kv_u32("general.alignment", align)
    blobs, off = [], 0

    def add(name, shape, ty, arr):
        nonlocal off
        raw = np.ascontiguousarray(arr).tobytes()
        b.tensor(name, shape, ty, off)
        blobs.append(raw + bytes((-len(raw)) % align))
        off += len(blobs[-1])

    for L, t in layers.items():
        n_exp, d, ff = t["n_exp"], t["d"], t["ff"]
        add(f"blk.{L}.ffn_gate_up_exps.weight", [d, 2 * ff, n_exp], 2, t["gate_up"])
        add(f"blk.{L}.ffn_down_exps.weight", [ff, d, n_exp], 2, t["down"])
        add(f"blk.{L}.ffn_gate_inp.weight", [d, n_exp], 0, np.asarray(t["router"], np.float32))
        if t.get("down_scale") is not None:
            add(f"blk.{L}.ffn_down_exps.scale", [n_exp], 0, np.asarray(t["down_scale"], np.float32))
    for name, arr in (extra_f32 or {}).items():
        arr = np.asarray(arr, np.float32)
        add(name, list(arr.shape[::-1]), 0, arr)
    return b.data_bytes(b"".join(blobs)).build()
