"""Safe host view of the C ABI in include/rvmoe.h (librvmoe.so).

Mirrors the reference's Rust wrapper runtime/src/hip.rs: device memory is owned by `DevBuf`
and freed when it is closed or collected (hip.rs:240-310); every wrapper checks the byte range a
kernel reads or writes against the owning allocation before calling it, because the C side
validates only scalars (hip.rs:1-6, 258-263, 362-586); a non-zero return code becomes
`DeviceError(code)` (hip.rs:120-122, error.rs `Error::Device`).

There is no CPU fallback: if the HIP library is missing the import of this module's `lib()`
raises, naming the build step.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# RVM_LIB names another build of the same library (for side-by-side timing of two builds)
LIB_PATH = os.environ.get("RVM_LIB", os.path.join(HERE, "librvmoe.so"))

QK, Q4_BLOCK, Q8_BLOCK = 32, 18, 34
PACK_GATE_UP, PACK_ROWS32 = 1, 2
PRE_NORM, EXACT_SELECT = 1, 2


class DeviceError(RuntimeError):
    """A HIP error code returned through the ABI."""

    def __init__(self, code: int):
        self.code = code
        msg = lib().rvh_error_string(code)
        super().__init__(f"device error {code}: {msg.decode() if msg else '?'}")


class BoundsError(ValueError):
    """A kernel's byte range does not fit its buffer (refused before any launch)."""


class RvmLayer(C.Structure):
    """`rvm_layer` of include/rvmoe.h."""

    _fields_ = [
        ("n_exp", C.c_int),
        ("top_k", C.c_int),
        ("d", C.c_int),
        ("ff", C.c_int),
        ("router", C.c_void_p),
        ("router_bias", C.c_void_p),
        ("gate_up", C.c_void_p),
        ("down", C.c_void_p),
        ("down_scale", C.c_void_p),
    ]


class RvmBlockNorms(C.Structure):
    """`rvm_block_norms` of include/rvmoe.h: the MoE block's router and expert input norms."""

    _fields_ = [
        ("eps", C.c_float),
        ("router_post", C.c_float),
        ("router_scale", C.c_void_p),
        ("expert_scale", C.c_void_p),
    ]


_lib = None

# name -> (restype, argtypes); every symbol of include/rvmoe.h.
_vp, _sz, _i, _f, _u64 = C.c_void_p, C.c_size_t, C.c_int, C.c_float, C.c_uint64
_PL = C.POINTER(RvmLayer)
_PN = C.POINTER(RvmBlockNorms)
SIGNATURES = {
    "rvh_init": (_i, [_i]),
    "rvh_mem_info": (_i, [C.POINTER(_sz), C.POINTER(_sz)]),
    "rvh_alloc": (_i, [_sz, C.POINTER(_vp)]),
    "rvh_free": (_i, [_vp]),
    "rvh_upload": (_i, [_vp, _vp, _sz]),
    "rvh_download": (_i, [_vp, _vp, _sz]),
    "rvh_copy": (_i, [_vp, _vp, _sz]),
    "rvh_sync": (_i, []),
    "rvh_error_string": (C.c_char_p, [_i]),
    "rvh_event_create": (_i, [C.POINTER(_vp)]),
    "rvh_event_destroy": (_i, [_vp]),
    "rvh_event_record": (_i, [_vp]),
    "rvh_event_sync": (_i, [_vp]),
    "rvh_event_elapsed": (_i, [_vp, _vp, C.POINTER(_f)]),
    "rvh_rms_norm": (_i, [_vp, _vp, _vp, _i, _i, _f, _f]),
    "rvh_f32_mm": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "rvh_q4_mm": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "rvh_q4_mv": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "rvm_q4_mm_n": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i]),
    "rvh_geglu_split": (_i, [_vp, _vp, _i, _i]),
    "rvh_gather_rows": (_i, [_vp, _vp, _vp, _i, _i]),
    "rvh_moe_combine": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "rvh_kv_store": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "rvh_attention": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i]),
    "rvh_attn_split": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i]),
    "rvh_attn_combine": (_i, [_vp, _vp, _i, _i, _i]),
    "rvm_attn_decode": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i]),
    "rvm_set_stream": (_i, [_vp]),
    "rvm_stream_create": (_i, [C.POINTER(_vp)]),
    "rvm_stream_destroy": (_i, [_vp]),
    "rvm_graph_begin": (_i, []),
    "rvm_graph_end": (_i, [C.POINTER(_vp)]),
    "rvm_graph_launch": (_i, [_vp]),
    "rvm_graph_destroy": (_i, [_vp]),
    "rvm_q4_packed_bytes": (_i, [_i, _i, _i, _i, C.POINTER(_sz)]),
    "rvm_pack_q4": (_i, [_vp, _vp, _i, _i, _i, _i]),
    "rvm_synth_q4": (_i, [_vp, _i, _i, _i, _u64, _u64]),
    "rvm_synth_q4_host": (_i, [_vp, _i, _i, _i, _u64, _u64]),
    "rvm_quantize_q8_0": (_i, [_vp, _vp, _i, _i]),
    "rvm_q4q8_mm": (_i, [_vp, _i, _vp, _vp, _i, _i, _i]),
    "rvm_q4q8_block_sums": (_i, [_vp, _i, _vp, _vp, _i, _i]),
    "rvm_geglu_q8_0": (_i, [_vp, _vp, _i, _i]),
    "rvm_moe_workspace_bytes": (_i, [_PL, _i, C.POINTER(_sz)]),
    "rvm_workspace_init": (_i, [_vp, _sz]),
    "rvm_workspace_fallbacks": (_i, [_vp, C.POINTER(C.c_uint32)]),
    "rvm_workspace_selection": (_i, [_PL, _i, _vp, _vp, _vp]),
    "rvm_router_select": (_i, [_PL, _vp, _i, _i, _f, _vp, _vp, _vp, _vp, _sz]),
    "rvm_moe_plan": (_i, [_vp, _i, _i, _vp, _vp, _vp]),
    "rvm_moe_decode": (_i, [_PL, _vp, _vp, _i, _f, _vp, _sz]),
    "rvm_moe_decode_static": (_i, [_PL, _vp, _vp, _i, _f]),
    "rvm_moe_block_decode": (_i, [_PL, _PN, _vp, _vp, _i, _vp, _sz]),
    "rvm_moe_block_forward": (_i, [_PL, _PN, _vp, _vp, _i, _i, _vp, _sz]),
    "rvm_moe_forward": (_i, [_PL, _vp, _vp, _i, _i, _f, _vp, _sz]),
    "rvm_counters_get": (_i, [_vp]),
    "rvm_counters_reset": (_i, []),
    "rvm_phase_trace": (_i, [_vp, _sz]),
    "rvm_session_create": (_i, [_vp, _i, _vp, _i, _f, C.POINTER(_vp)]),
    "rvm_session_destroy": (_i, [_vp]),
    "rvm_session_eval": (_i, [_vp, _vp, _vp, _i, _i]),
    "rvm_session_eval_range": (_i, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "rvm_session_probe": (_i, [_vp, _vp, _i]),
    "rvm_session_workspace": (_i, [_vp, C.POINTER(_vp)]),
    "rvm_gguf_open": (_i, [_vp, _sz, C.POINTER(_vp)]),
    "rvm_gguf_close": (_i, [_vp]),
    "rvm_gguf_last_error": (C.c_char_p, []),
    "rvm_gguf_info": (_i, [_vp, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(_u64), C.POINTER(_u64)]),
    "rvm_gguf_meta_str": (_i, [_vp, C.c_char_p, C.POINTER(C.c_char_p)]),
    "rvm_gguf_tensor": (_i, [_vp, C.c_char_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(_u64),
                             C.POINTER(_vp), C.POINTER(_sz)]),
    "rvm_gguf_bind_moe": (_i, [_vp, _i, _PL, _vp, _sz]),
}


def lib() -> C.CDLL:
    """The HIP library. Raises if it has not been built (there is no CPU fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m rosevine_amd.build` "
                              "(or __graft_entry__.build()); the MoE path has no CPU fallback")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class Counters(C.Structure):
    """`rvm_counters`: device calls issued by this thread through the library."""

    _fields_ = [(n, C.c_uint64) for n in ("launches", "h2d", "d2h", "d2d", "syncs", "graphs")]

    def as_dict(self) -> dict:
        return {n: getattr(self, n) for n, _ in self._fields_}


def counters() -> dict:
    c = Counters()
    check(lib().rvm_counters_get(C.addressof(c)))
    return c.as_dict()


def reset_counters() -> None:
    check(lib().rvm_counters_reset())


def check(code: int) -> None:
    if code != 0:
        raise DeviceError(code)


def init(device: int = 0) -> None:
    check(lib().rvh_init(device))


def copy(dst: DevBuf, src: DevBuf, nbytes: int, dst_off: int = 0, src_off: int = 0) -> None:
    """rvh_copy: device-to-device, ordered on the current stream."""
    check(lib().rvh_copy(_need(dst, nbytes, dst_off), _need(src, nbytes, src_off), nbytes))


def sync() -> None:
    check(lib().rvh_sync())


def mem_info() -> tuple[int, int]:
    free, total = C.c_size_t(), C.c_size_t()
    check(lib().rvh_mem_info(C.byref(free), C.byref(total)))
    return free.value, total.value


# Set while the interpreter shuts down: finalizers then leave device memory to the process exit
# instead of calling into a HIP runtime whose own exit handlers may already have run.
_exiting = False


def _at_exit() -> None:
    global _exiting
    _exiting = True


atexit.register(_at_exit)


class DevBuf:
    """An owned device allocation (hip.rs `DevBuf`)."""

    def __init__(self, nbytes: int):
        if nbytes < 0:
            raise BoundsError("negative size")
        p = C.c_void_p()
        check(lib().rvh_alloc(nbytes, C.byref(p)))
        self.ptr = p.value
        self.nbytes = nbytes

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DevBuf":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def close(self) -> None:
        if getattr(self, "ptr", None):
            lib().rvh_free(self.ptr)
            self.ptr = None

    def __del__(self):
        if _exiting:
            return
        try:
            self.close()
        except Exception:
            pass

    def at(self, offset: int = 0, length: int = 0) -> int:
        """Device address of [offset, offset + length), checked against the allocation."""
        if not self.ptr:
            raise BoundsError("buffer is closed")
        if offset < 0 or length < 0 or offset + length > self.nbytes:
            raise BoundsError(f"range [{offset}, {offset + length}) outside a {self.nbytes}-byte buffer")
        return self.ptr + offset

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        check(lib().rvh_upload(self.at(offset, a.nbytes), a.ctypes.data, a.nbytes))

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype)
        check(lib().rvh_download(out.ctypes.data, self.at(offset, out.nbytes), out.nbytes))
        return out


def _need(buf: DevBuf, nbytes: int, offset: int = 0) -> int:
    return buf.at(offset, nbytes)


class Event:
    def __init__(self):
        p = C.c_void_p()
        check(lib().rvh_event_create(C.byref(p)))
        self.ptr = p.value

    def record(self) -> None:
        check(lib().rvh_event_record(self.ptr))

    def synchronize(self) -> None:
        check(lib().rvh_event_sync(self.ptr))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib().rvh_event_elapsed(self.ptr, end.ptr, C.byref(ms)))
        return ms.value

    def __del__(self):
        if _exiting:
            return
        try:
            if self.ptr:
                lib().rvh_event_destroy(self.ptr)
        except Exception:
            pass


class Stream:
    """A non-blocking stream at the default priority; `use()` routes later launches to it."""

    def __init__(self):
        p = C.c_void_p()
        check(lib().rvm_stream_create(C.byref(p)))
        self.ptr = p.value

    def use(self) -> None:
        check(lib().rvm_set_stream(self.ptr))

    @staticmethod
    def use_default() -> None:
        check(lib().rvm_set_stream(None))

    def close(self) -> None:
        if self.ptr:
            lib().rvm_stream_destroy(self.ptr)
            self.ptr = None


class Graph:
    """Launches captured on the current stream, instantiated once and replayed."""

    def __init__(self, ptr: int):
        self.ptr = ptr

    @staticmethod
    def begin() -> None:
        check(lib().rvm_graph_begin())

    @classmethod
    def end(cls) -> "Graph":
        p = C.c_void_p()
        check(lib().rvm_graph_end(C.byref(p)))
        return cls(p.value)

    def launch(self) -> None:
        check(lib().rvm_graph_launch(self.ptr))

    def close(self) -> None:
        if self.ptr:
            lib().rvm_graph_destroy(self.ptr)
            self.ptr = None


# ---- kernel wrappers: ranges checked here, scalars in C ----

def q4_packed_bytes(n_mat: int, n_out: int, k: int, fmt: int) -> int:
    n = C.c_size_t()
    check(lib().rvm_q4_packed_bytes(n_mat, n_out, k, fmt, C.byref(n)))
    return n.value


def pack_q4(src: DevBuf, dst: DevBuf, n_mat: int, n_out: int, k: int, fmt: int) -> None:
    nbytes = q4_packed_bytes(n_mat, n_out, k, fmt)
    check(lib().rvm_pack_q4(_need(src, nbytes), _need(dst, nbytes), n_mat, n_out, k, fmt))


def synth_q4(dst: DevBuf, n_mat: int, n_out: int, k: int, seed: int, stream0: int) -> None:
    nbytes = n_mat * n_out * (k // QK) * Q4_BLOCK
    check(lib().rvm_synth_q4(_need(dst, nbytes), n_mat, n_out, k, seed, stream0))


def synth_q4_host(n_mat: int, n_out: int, k: int, seed: int, stream0: int) -> np.ndarray:
    out = np.empty(n_mat * n_out * (k // QK) * Q4_BLOCK, np.uint8)
    check(lib().rvm_synth_q4_host(out.ctypes.data, n_mat, n_out, k, seed, stream0))
    return out


def quantize_q8_0(x: DevBuf, xq: DevBuf, rows: int, k: int) -> None:
    check(lib().rvm_quantize_q8_0(_need(x, rows * k * 4), _need(xq, rows * (k // QK) * Q8_BLOCK), rows, k))


def q4q8_mm(w: DevBuf, fmt: int, xq: DevBuf, y: DevBuf, n_out: int, k: int, n_in: int) -> None:
    wb = q4_packed_bytes(1, n_out, k, fmt)
    check(lib().rvm_q4q8_mm(_need(w, wb), fmt, _need(xq, n_in * (k // QK) * Q8_BLOCK), _need(y, n_in * n_out * 4),
                            n_out, k, n_in))


def q4q8_block_sums(w: DevBuf, fmt: int, xq: DevBuf, sums: DevBuf, n_out: int, k: int) -> None:
    wb = q4_packed_bytes(1, n_out, k, fmt)
    check(lib().rvm_q4q8_block_sums(_need(w, wb), fmt, _need(xq, (k // QK) * Q8_BLOCK),
                                    _need(sums, n_out * (k // QK) * 4), n_out, k))


def geglu_q8_0(gu: DevBuf, hq: DevBuf, rows: int, ff: int) -> None:
    check(lib().rvm_geglu_q8_0(_need(gu, rows * 2 * ff * 4), _need(hq, rows * (ff // QK) * Q8_BLOCK), rows, ff))


def rms_norm(x: DevBuf, out: DevBuf, weight: DevBuf | None, rows: int, width: int, eps: float, post: float) -> None:
    w = None if weight is None else _need(weight, width * 4)
    check(lib().rvh_rms_norm(_need(x, rows * width * 4), _need(out, rows * width * 4), w, rows, width, eps, post))


def f32_mm(w: DevBuf, x: DevBuf, y: DevBuf, n_out: int, k: int, n_in: int) -> None:
    check(lib().rvh_f32_mm(_need(w, n_out * k * 4), _need(x, n_in * k * 4), _need(y, n_in * n_out * 4), n_out, k,
                           n_in))


def q4_mm(w: DevBuf, x: DevBuf, y: DevBuf, n_out: int, k: int, n_in: int) -> None:
    check(lib().rvh_q4_mm(_need(w, n_out * (k // QK) * Q4_BLOCK), _need(x, n_in * k * 4),
                          _need(y, n_in * n_out * 4), n_out, k, n_in))


def q4_mm_n(ws: list, x: DevBuf, ys: list, n_outs: list, k: int, n_in: int) -> None:
    """rvm_q4_mm_n: up to four rvh_q4_mm products on one input in one launch (a matrix of 16384
    rows or more, k <= 8192, in a launch of its own)."""
    n = len(ws)
    if not (len(ys) == n and len(n_outs) == n):
        raise ValueError("one output and one row count per matrix")
    wp = (C.c_void_p * max(n, 1))(*[_need(w, r * (k // QK) * Q4_BLOCK) for w, r in zip(ws, n_outs)])
    yp = (C.c_void_p * max(n, 1))(*[_need(y, n_in * r * 4) for y, r in zip(ys, n_outs)])
    rp = (C.c_int * max(n, 1))(*n_outs)
    check(lib().rvm_q4_mm_n(n, wp, rp, yp, _need(x, n_in * k * 4), k, n_in))


def q4_mv(w: DevBuf, x: DevBuf, y: DevBuf, n_out: int, k: int, n_in: int) -> None:
    """rvh_q4_mv; like the reference wrapper (runtime/src/hip.rs:384-392) it takes rvh_q4_mm for
    activations that are not 16-byte aligned."""
    wp, xp = _need(w, n_out * (k // QK) * Q4_BLOCK), _need(x, n_in * k * 4)
    fn = lib().rvh_q4_mv if xp % 16 == 0 and wp % 2 == 0 else lib().rvh_q4_mm
    check(fn(wp, xp, _need(y, n_in * n_out * 4), n_out, k, n_in))


def geglu_split(gu: DevBuf, out: DevBuf, rows: int, ff: int) -> None:
    check(lib().rvh_geglu_split(_need(gu, rows * 2 * ff * 4), _need(out, rows * ff * 4), rows, ff))


def gather_rows(src: DevBuf, src_rows: int, idx: DevBuf, dst: DevBuf, n: int, width: int) -> None:
    check(lib().rvh_gather_rows(_need(src, src_rows * width * 4), _need(idx, n * 4), _need(dst, n * width * 4), n,
                                width))


def moe_combine(y: DevBuf, y_rows: int, pos: DevBuf, scale: DevBuf, weight: DevBuf, out: DevBuf, n_tok: int,
                used: int, width: int) -> None:
    pairs = n_tok * used
    check(lib().rvh_moe_combine(_need(y, y_rows * width * 4), _need(pos, pairs * 4), _need(scale, pairs * 4),
                                _need(weight, pairs * 4), _need(out, n_tok * width * 4), n_tok, used, width))


# ---- decode attention over a Q8_0 key/value ring (runtime/src/hip.rs:423-530) ----

ATTN_TARGET_BLOCKS = 1024  # runtime/src/hip.rs:481
ATTN_MIN_CHUNK = 64  # runtime/src/hip.rs:483
# The same policy with twice the query-head x chunk target: on MI355X, 16 query heads at depth
# 16384-32768 run 17-23% faster with 128 chunks than with 64, and 8 tokens at depth 16384 36%
# faster with 16 than with 8; shorter contexts keep ceil(keys / 64) chunks. Scratch doubles.
ATTN_TARGET_BLOCKS_MI355X = 2048


def q8_row_bytes(hd: int) -> int:
    return hd // QK * Q8_BLOCK


def attention_chunks(n_tok: int, n_head: int, longest: int, target_blocks: int = ATTN_TARGET_BLOCKS,
                     min_chunk: int = ATTN_MIN_CHUNK) -> int:
    """Key chunks per query head (runtime/src/hip.rs:486-490): ceil(keys / min_chunk) (64 there), at
    most target_blocks / (tokens * heads) so that decode fills the device and prefill takes one chunk."""
    by_keys = max(-(-longest // min_chunk), 1)
    by_blocks = max(target_blocks // max(n_tok * n_head, 1), 1)
    return min(by_keys, by_blocks)


def attention_split_scratch(n_tok: int, n_head: int, hd: int, target_blocks: int = ATTN_TARGET_BLOCKS) -> int:
    """f32 elements of partial scratch for attention_split at up to n_tok tokens, any context
    (runtime/src/hip.rs:495-497)."""
    return max(n_tok * n_head, target_blocks) * (hd + 2)


def _attn_longest(n_tok: int, p0: int, window: int) -> int:
    return min(p0 + n_tok, window) if window > 0 else p0 + n_tok


def kv_store(k: DevBuf, v: DevBuf, kc: DevBuf, vc: DevBuf, n_tok: int, n_kv: int, hd: int, p0: int, cap: int,
             k_off: int = 0, v_off: int = 0) -> None:
    """rvh_kv_store (runtime/src/hip.rs:423-438): Q8_0 of n_tok tokens' keys and values into slots
    (p0 + t) % cap."""
    n, c = n_tok * n_kv * hd * 4, cap * n_kv * q8_row_bytes(hd)
    check(lib().rvh_kv_store(_need(k, n, k_off), _need(v, n, v_off), _need(kc, c), _need(vc, c), n_tok, n_kv, hd,
                             p0, cap))


def attention(q: DevBuf, kc: DevBuf, vc: DevBuf, out: DevBuf, scores: DevBuf, n_tok: int, n_head: int, n_kv: int,
              hd: int, p0: int, cap: int, window: int, max_keys: int) -> None:
    """rvh_attention (runtime/src/hip.rs:440-478); scores must hold n_tok * n_head * max_keys floats."""
    nq, c = n_tok * n_head * hd * 4, cap * n_kv * q8_row_bytes(hd)
    check(lib().rvh_attention(_need(q, nq), _need(kc, c), _need(vc, c), _need(out, nq),
                              _need(scores, n_tok * n_head * max_keys * 4), n_tok, n_head, n_kv, hd, p0, cap,
                              window, max_keys))


def attn_split(q: DevBuf, kc: DevBuf, vc: DevBuf, out: DevBuf, part: DevBuf | None, n_tok: int, n_head: int,
               n_kv: int, hd: int, p0: int, cap: int, window: int, n_chunks: int) -> None:
    """rvh_attn_split with an explicit chunk count."""
    nq, c = n_tok * n_head * hd * 4, cap * n_kv * q8_row_bytes(hd)
    pp = _need(part, n_tok * n_head * n_chunks * (hd + 2) * 4) if n_chunks > 1 else (part.at() if part else None)
    check(lib().rvh_attn_split(_need(q, nq), _need(kc, c), _need(vc, c), _need(out, nq), pp, n_tok, n_head, n_kv,
                               hd, p0, cap, window, n_chunks))


def attn_combine(part: DevBuf, out: DevBuf, rows: int, hd: int, n_chunks: int) -> None:
    check(lib().rvh_attn_combine(_need(part, rows * n_chunks * (hd + 2) * 4), _need(out, rows * hd * 4), rows, hd,
                                 n_chunks))


def attn_decode(q: DevBuf, k: DevBuf, v: DevBuf, kc: DevBuf, vc: DevBuf, out: DevBuf, part: DevBuf | None,
                n_head: int, n_kv: int, hd: int, pos: int, cap: int, window: int, n_chunks: int, k_off: int = 0,
                v_off: int = 0) -> None:
    """rvm_attn_decode: one decode token's key/value store and split-K attention (with the merge)."""
    nq, nk, c = n_head * hd * 4, n_kv * hd * 4, cap * n_kv * q8_row_bytes(hd)
    pp = _need(part, n_head * n_chunks * (hd + 2) * 4) if n_chunks > 1 else (part.at() if part else None)
    check(lib().rvm_attn_decode(_need(q, nq), k.at(k_off, nk), v.at(v_off, nk), _need(kc, c), _need(vc, c),
                                _need(out, nq), pp, n_head, n_kv, hd, pos, cap, window, n_chunks))


def attention_split(q: DevBuf, kc: DevBuf, vc: DevBuf, out: DevBuf, part: DevBuf, n_tok: int, n_head: int, n_kv: int,
                    hd: int, p0: int, cap: int, window: int, target_blocks: int = ATTN_TARGET_BLOCKS,
                    min_chunk: int = ATTN_MIN_CHUNK) -> int:
    """Split-K attention as runtime/src/hip.rs:503-530: attention_chunks chunks per query head, the
    partials merged by rvh_attn_combine when there is more than one. part holds
    attention_split_scratch(..., target_blocks) floats. Returns the chunk count."""
    chunks = attention_chunks(n_tok, n_head, _attn_longest(n_tok, p0, window), target_blocks, min_chunk)
    attn_split(q, kc, vc, out, part, n_tok, n_head, n_kv, hd, p0, cap, window, chunks)
    if chunks > 1:
        attn_combine(part, out, n_tok * n_head, hd, chunks)
    return chunks


def moe_plan(ids: DevBuf, n_pairs: int, n_exp: int, order: DevBuf, pos_of: DevBuf, group_start: DevBuf) -> None:
    check(lib().rvm_moe_plan(_need(ids, n_pairs * 4), n_pairs, n_exp, _need(order, n_pairs * 4),
                             _need(pos_of, n_pairs * 4), _need(group_start, (n_exp + 1) * 4)))
