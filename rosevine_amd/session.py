"""A stack of MoE layers evaluated on the device (rvm_session_* of include/rvmoe.h).

The executor side of the reference's MoE path (runtime/src/hip_exec.rs:780-843) with placement
all-device and no host round trip: per layer the session issues only the kernels of one rvm_moe_*
call, reading the previous layer's output from device memory. Between layers it applies the
synthetic stack's RMSNorm, or each layer's block norms (the reference's router and expert norms).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import hip
from .hip import DevBuf, RvmBlockNorms, RvmLayer, check, lib
from .moe import BlockNorms, MoeLayer


class Session:
    def __init__(self, layers: list[MoeLayer], max_tokens: int, eps: float = 1e-6,
                 norms: list[BlockNorms] | None = None):
        if not layers:
            raise ValueError("a session needs at least one layer")
        if norms is not None and len(norms) != len(layers):
            raise ValueError("one block norm set per layer")
        self.layers, self.norms, self.max_tokens = list(layers), norms, max_tokens
        self._larr = (RvmLayer * len(layers))(*[L.struct for L in layers])
        self._narr = None if norms is None else (RvmBlockNorms * len(norms))(*[n.struct for n in norms])
        h = C.c_void_p()
        check(lib().rvm_session_create(C.addressof(self._larr), len(layers),
                                       None if self._narr is None else C.addressof(self._narr), max_tokens, eps,
                                       C.byref(h)))
        self.handle = h.value
        self.d = layers[0].d

    def eval(self, x: DevBuf, out: DevBuf, n_tok: int, flags: int = 0, x_off: int = 0, out_off: int = 0) -> None:
        """n_tok rows of x through every layer into out (rvm_session_eval)."""
        if n_tok > self.max_tokens:
            raise hip.BoundsError("session sized for fewer tokens")
        nb = n_tok * self.d * 4
        check(lib().rvm_session_eval(self.handle, x.at(x_off, nb), out.at(out_off, nb), n_tok, flags))
        self._next = 0

    def eval_range(self, x: DevBuf | None, out: DevBuf | None, n_tok: int, l0: int, l1: int, flags: int = 0,
                   x_off: int = 0, out_off: int = 0) -> None:
        """Layers [l0, l1) of one evaluation (rvm_session_eval_range): a caller polls its cancel flag
        between ranges, as the reference's HipSession::eval does before every layer
        (runtime/src/hip_exec.rs:645-655). The range checks are the library's, made here first."""
        n = len(self.layers)
        if not (0 <= l0 < l1 <= n):
            raise hip.BoundsError(f"layer range [{l0}, {l1}) outside a {n}-layer session")
        if not 0 < n_tok <= self.max_tokens:
            raise hip.BoundsError("session sized for fewer tokens")
        if l0 > 0 and (l0 != getattr(self, "_next", 0) or n_tok != getattr(self, "_ntok", 0)):
            raise hip.BoundsError(f"range from layer {l0} does not continue the evaluation in progress")
        nb = n_tok * self.d * 4
        if l0 == 0 and x is None:
            raise hip.BoundsError("a range from layer 0 reads x")
        if l1 == n and out is None:
            raise hip.BoundsError("the range that ends at the last layer writes out")
        xp = x.at(x_off, nb) if l0 == 0 else None
        op = out.at(out_off, nb) if l1 == n else None
        check(lib().rvm_session_eval_range(self.handle, xp, op, n_tok, flags, l0, l1))
        self._next, self._ntok = (0 if l1 == n else l1), n_tok

    def probe(self, events: list | None) -> None:
        """Span events (rvm_session_probe): 2 per layer and one at the end, or None to stop."""
        if events is None:
            check(lib().rvm_session_probe(self.handle, None, 0))
            self._probe = None
            return
        arr = (C.c_void_p * len(events))(*[e.ptr for e in events])
        check(lib().rvm_session_probe(self.handle, arr, len(events)))
        self._probe = (arr, events)  # kept alive while the library holds them

    def fallbacks(self) -> int:
        """Router selections of all layers so far whose certificate failed (rvm_workspace_fallbacks;
        synchronises)."""
        ws = C.c_void_p()
        check(lib().rvm_session_workspace(self.handle, C.byref(ws)))
        n = C.c_uint32()
        check(lib().rvm_workspace_fallbacks(ws.value, C.byref(n)))
        return n.value

    def selection(self, n_tok: int):
        """ids and weights of the last layer of the last evaluation (synchronises)."""
        ws = C.c_void_p()
        check(lib().rvm_session_workspace(self.handle, C.byref(ws)))
        L = self.layers[-1]
        ids = np.empty((n_tok, L.top_k), np.int32)
        w = np.empty((n_tok, L.top_k), np.float32)
        check(lib().rvm_workspace_selection(L.ptr(), n_tok, ws.value, ids.ctypes.data, w.ctypes.data))
        return ids, w

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().rvm_session_destroy(self.handle)
            self.handle = None

    def __del__(self):
        if hip._exiting:
            return
        try:
            self.close()
        except Exception:
            pass
