"""Host-side MoE layer: HBM-resident expert weights and the device dispatch.

Mirrors the MoE section of the reference's HipSession::layer (runtime/src/hip_exec.rs:780-843)
with placement fixed to all-device (the reference's cpu_expert_layers = 0, hip_exec.rs:429-433):
router, selection, grouping, experts and combine all run on the GPU, with no host round trip
between them. Weights arrive in the reference's Q4_0 row layout (the GGUF expert tensors
[2816,1408,128] and [704,2816,128], runtime/src/contract.rs:66-70) and are repacked once into
the kernels' planar layout.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import hip
from .hip import DevBuf, RvmLayer, check, lib


# RVM_FOLD_MIN_TOKENS: from this many tokens the router folds every logit in the reference's order
# (exact logits, ids and weights); decode and smaller batches use the certified estimates.
FOLD_MIN_TOKENS = 256


class MoeLayer:
    """One layer's device weights (`rvm_layer`)."""

    def __init__(self, n_exp: int, top_k: int, d: int, ff: int, router: np.ndarray | None,
                 bias: np.ndarray | None = None, down_scale: np.ndarray | bool | None = None):
        """router None leaves the router buffer to be filled later (a GGUF binding); down_scale True
        allocates the down-scale buffer likewise."""
        self.n_exp, self.top_k, self.d, self.ff = n_exp, top_k, d, ff
        if router is None:
            self.router = DevBuf(n_exp * d * 4)
        else:
            router = np.ascontiguousarray(router, dtype=np.float32)
            if router.shape != (n_exp, d):
                raise ValueError(f"router must be [{n_exp}, {d}]")
            self.router = DevBuf.from_array(router)
        self.bias = None if bias is None else DevBuf.from_array(np.asarray(bias, np.float32).reshape(n_exp))
        if down_scale is None or down_scale is False:
            self.down_scale = None
        elif down_scale is True:
            self.down_scale = DevBuf(n_exp * 4)
        else:
            self.down_scale = DevBuf.from_array(np.asarray(down_scale, np.float32).reshape(n_exp))
        self.gu_bytes = hip.q4_packed_bytes(n_exp, 2 * ff, d, hip.PACK_GATE_UP)
        self.dn_bytes = hip.q4_packed_bytes(n_exp, d, ff, hip.PACK_ROWS32)
        self.gate_up = DevBuf(self.gu_bytes)
        self.down = DevBuf(self.dn_bytes)
        self.struct = RvmLayer(n_exp, top_k, d, ff, self.router.ptr, self.bias.ptr if self.bias else None,
                               self.gate_up.ptr, self.down.ptr, self.down_scale.ptr if self.down_scale else None)

    @property
    def weight_bytes(self) -> int:
        return self.gu_bytes + self.dn_bytes

    def load_q4(self, gate_up: np.ndarray | DevBuf, down: np.ndarray | DevBuf) -> None:
        """Repack reference-layout Q4_0 expert stacks (host arrays or device buffers)."""
        for src, dst, n_out, k, fmt in ((gate_up, self.gate_up, 2 * self.ff, self.d, hip.PACK_GATE_UP),
                                        (down, self.down, self.d, self.ff, hip.PACK_ROWS32)):
            tmp = src if isinstance(src, DevBuf) else DevBuf.from_array(np.asarray(src, np.uint8))
            hip.pack_q4(tmp, dst, self.n_exp, n_out, k, fmt)
            if tmp is not src:
                hip.sync()
                tmp.close()

    def synth_weights(self, seed: int, gate_up_stream: int, down_stream: int, scratch: DevBuf | None = None) -> None:
        """Generate the seeded synthetic Q4_0 experts on the device, then repack them."""
        need = max(self.gu_bytes, self.dn_bytes)
        tmp = scratch if scratch is not None and scratch.nbytes >= need else DevBuf(need)
        hip.synth_q4(tmp, self.n_exp, 2 * self.ff, self.d, seed, gate_up_stream)
        hip.pack_q4(tmp, self.gate_up, self.n_exp, 2 * self.ff, self.d, hip.PACK_GATE_UP)
        hip.synth_q4(tmp, self.n_exp, self.d, self.ff, seed, down_stream)
        hip.pack_q4(tmp, self.down, self.n_exp, self.d, self.ff, hip.PACK_ROWS32)
        if tmp is not scratch:
            hip.sync()
            tmp.close()

    def ptr(self):
        return C.byref(self.struct)


class Workspace:
    """Device scratch for up to n_tok tokens through a layer of this shape (zeroed once)."""

    def __init__(self, layer: MoeLayer, n_tok: int):
        n = C.c_size_t()
        check(lib().rvm_moe_workspace_bytes(layer.ptr(), n_tok, C.byref(n)))
        self.nbytes = n.value
        self.n_tok = n_tok
        self.buf = DevBuf(self.nbytes)
        check(lib().rvm_workspace_init(self.buf.ptr, self.nbytes))

    def fallbacks(self) -> int:
        c = C.c_uint32()
        check(lib().rvm_workspace_fallbacks(self.buf.ptr, C.byref(c)))
        return c.value

    def selection(self, layer: MoeLayer, n_tok: int):
        """ids and weights [n_tok, top_k] of the last decode/forward call of n_tok tokens."""
        if n_tok > self.n_tok:
            raise hip.BoundsError("workspace sized for fewer tokens")
        ids = np.empty((n_tok, layer.top_k), np.int32)
        w = np.empty((n_tok, layer.top_k), np.float32)
        check(lib().rvm_workspace_selection(layer.ptr(), n_tok, self.buf.ptr, ids.ctypes.data, w.ctypes.data))
        return ids, w


def decode(layer: MoeLayer, x: DevBuf, out: DevBuf, ws: Workspace, flags: int = 0, eps: float = 1e-6,
           x_off: int = 0, out_off: int = 0) -> None:
    """One token: x[d] -> out[d] (rvm_moe_decode)."""
    nb = layer.d * 4
    check(lib().rvm_moe_decode(layer.ptr(), x.at(x_off, nb), out.at(out_off, nb), flags, eps, ws.buf.ptr,
                               ws.nbytes))


def decode_static(layer: MoeLayer, x: DevBuf, out: DevBuf, flags: int = 0, eps: float = 1e-6, x_off: int = 0,
                  out_off: int = 0) -> None:
    """One token with the library's static scratch instead of a workspace (rvm_moe_decode_static):
    the call allocates nothing; calls that overlap on one GPU race."""
    nb = layer.d * 4
    check(lib().rvm_moe_decode_static(layer.ptr(), x.at(x_off, nb), out.at(out_off, nb), flags, eps))


def forward(layer: MoeLayer, x: DevBuf, out: DevBuf, n_tok: int, ws: Workspace, flags: int = 0,
            eps: float = 1e-6) -> None:
    """n_tok tokens with device grouping (rvm_moe_forward)."""
    if n_tok > ws.n_tok:
        raise hip.BoundsError("workspace sized for fewer tokens")
    nb = n_tok * layer.d * 4
    check(lib().rvm_moe_forward(layer.ptr(), x.at(0, nb), out.at(0, nb), n_tok, flags, eps, ws.buf.ptr,
                                ws.nbytes))


class BlockNorms:
    """The MoE block's input norms (`rvm_block_norms`): the router input
    ((o * s) * router_post) * router_scale and the expert input (o * s) * expert_scale, with the
    reference's gate_inp_scale, 1/sqrt(d) and pre_ffw_norm_2 (runtime/src/hip_exec.rs:784-796)."""

    def __init__(self, d: int, router_scale: np.ndarray | None, expert_scale: np.ndarray | None, eps: float = 1e-6,
                 router_post: float | None = None):
        if router_post is None:  # the reference's 1.0 / (n_embd as f32).sqrt(), in f32
            router_post = float(np.float32(1.0) / np.sqrt(np.float32(d)))
        self.router_scale = None if router_scale is None else DevBuf.from_array(
            np.asarray(router_scale, np.float32).reshape(d))
        self.expert_scale = None if expert_scale is None else DevBuf.from_array(
            np.asarray(expert_scale, np.float32).reshape(d))
        self.struct = hip.RvmBlockNorms(eps, router_post, self.router_scale.ptr if self.router_scale else None,
                                        self.expert_scale.ptr if self.expert_scale else None)

    def ptr(self):
        return C.byref(self.struct)


def block_decode(layer: MoeLayer, norms: BlockNorms, o: DevBuf, out: DevBuf, ws: Workspace, flags: int = 0,
                 o_off: int = 0, out_off: int = 0) -> None:
    """The MoE block for one token from the hidden row o (rvm_moe_block_decode)."""
    nb = layer.d * 4
    check(lib().rvm_moe_block_decode(layer.ptr(), norms.ptr(), o.at(o_off, nb), out.at(out_off, nb), flags,
                                     ws.buf.ptr, ws.nbytes))


def block_forward(layer: MoeLayer, norms: BlockNorms, o: DevBuf, out: DevBuf, n_tok: int, ws: Workspace,
                  flags: int = 0) -> None:
    """The MoE block for n_tok tokens (rvm_moe_block_forward)."""
    if n_tok > ws.n_tok:
        raise hip.BoundsError("workspace sized for fewer tokens")
    nb = n_tok * layer.d * 4
    check(lib().rvm_moe_block_forward(layer.ptr(), norms.ptr(), o.at(0, nb), out.at(0, nb), n_tok, flags,
                                      ws.buf.ptr, ws.nbytes))


def router_select(layer: MoeLayer, x: DevBuf, n_tok: int, ws: Workspace, flags: int = 0, eps: float = 1e-6,
                  with_logits: bool = False):
    """ids[n_tok, top_k], weights[n_tok, top_k] (and logits) as host arrays."""
    if n_tok > ws.n_tok:
        raise hip.BoundsError("workspace sized for fewer tokens")
    k = layer.top_k
    ids, wts = DevBuf(n_tok * k * 4), DevBuf(n_tok * k * 4)
    lg = DevBuf(n_tok * layer.n_exp * 4) if with_logits else None
    check(lib().rvm_router_select(layer.ptr(), x.at(0, n_tok * layer.d * 4), n_tok, flags, eps, ids.ptr, wts.ptr,
                                  lg.ptr if lg else None, ws.buf.ptr, ws.nbytes))
    res = (ids.download(np.int32, n_tok * k).reshape(n_tok, k), wts.download(np.float32, n_tok * k).reshape(n_tok, k))
    if with_logits:
        res = res + (lg.download(np.float32, n_tok * layer.n_exp).reshape(n_tok, layer.n_exp),)
    return res
