"""GGUF v3 images and the device binding of a layer's MoE tensors (rvm_gguf_* of include/rvmoe.h).

Mirrors the reference's artifact path for the expert tensors: a read-only mapping of the file
(runtime/src/mmap.rs), the bounded zero-copy parser (runtime/src/gguf.rs:217-340) and the binding
of blk.L.ffn_gate_up_exps / ffn_down_exps / ffn_gate_inp (runtime/src/model.rs:33-40, shapes of
runtime/src/contract.rs:66-70), here followed by the device repack into the kernels' layout. The
parsing is the library's C++ code; this module keeps the image alive and checks ranges.
"""
from __future__ import annotations

import ctypes as C
import mmap
import os

import numpy as np

from . import hip
from .hip import DevBuf, lib
from .moe import MoeLayer

F32, Q4_0 = 0, 2


class GgufError(ValueError):
    """A malformed image or a binding mismatch, with the reference's message."""


def _check(code: int) -> None:
    if code != 0:
        if code == 1:  # hipErrorInvalidValue: the parser's or the binder's refusal
            raise GgufError(lib().rvm_gguf_last_error().decode())
        raise hip.DeviceError(code)


class Gguf:
    """A parsed image. `data` is bytes-like (kept alive here) or a path (mapped read-only)."""

    def __init__(self, data):
        self._map = None
        if isinstance(data, (str, os.PathLike)):
            if os.path.exists(data) and not os.path.isfile(data):
                raise GgufError("not a regular file")
            with open(data, "rb") as f:
                if os.fstat(f.fileno()).st_size == 0:
                    raise GgufError("empty file")
                self._map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
            self._buf = np.frombuffer(self._map, dtype=np.uint8)
        else:
            self._buf = np.frombuffer(bytes(data) if not isinstance(data, (bytes, bytearray, memoryview, np.ndarray))
                                      else data, dtype=np.uint8)
        h = C.c_void_p()
        ptr = self._buf.ctypes.data if self._buf.size else None
        _check(lib().rvm_gguf_open(ptr, self._buf.size, C.byref(h)))
        self.handle = h.value

    def close(self) -> None:
        """Releases the handle and the mapping; tensor views taken earlier must be dropped first."""
        if getattr(self, "handle", None):
            lib().rvm_gguf_close(self.handle)
            self.handle = None
        self._buf = None
        if getattr(self, "_map", None) is not None:
            self._map.close()
            self._map = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self) -> dict:
        v, a, off, n = C.c_uint32(), C.c_uint32(), C.c_uint64(), C.c_uint64()
        _check(lib().rvm_gguf_info(self.handle, C.byref(v), C.byref(a), C.byref(off), C.byref(n)))
        return {"version": v.value, "alignment": a.value, "data_offset": off.value, "n_tensors": n.value}

    def meta_str(self, key: str) -> str:
        out = C.c_char_p()
        _check(lib().rvm_gguf_meta_str(self.handle, key.encode(), C.byref(out)))
        return out.value.decode()

    def tensor(self, name: str):
        """(type, shape in ggml order, byte offset of the data in the image, the bytes as a view)."""
        t, nd, shape = C.c_uint32(), C.c_uint32(), (C.c_uint64 * 4)()
        p, n = C.c_void_p(), C.c_size_t()
        _check(lib().rvm_gguf_tensor(self.handle, name.encode(), C.byref(t), C.byref(nd), shape, C.byref(p),
                                     C.byref(n)))
        off = (p.value or 0) - self._buf.ctypes.data
        if off < 0 or off + n.value > self._buf.size:
            raise GgufError("tensor view outside the image")
        return t.value, [shape[i] for i in range(nd.value)], off, self._buf[off:off + n.value]

    def bind_layer(self, layer: int, n_exp: int, top_k: int, d: int, ff: int, down_scale: bool = True,
                   bias: np.ndarray | None = None) -> MoeLayer:
        """A device MoeLayer from blk.<layer>'s expert tensors, router and (optionally) down scales."""
        L = MoeLayer(n_exp, top_k, d, ff, None, bias, True if down_scale else None)
        staging = DevBuf(max(L.gu_bytes, L.dn_bytes))
        try:
            _check(lib().rvm_gguf_bind_moe(self.handle, layer, L.ptr(), staging.ptr, staging.nbytes))
        finally:
            staging.close()
        return L
