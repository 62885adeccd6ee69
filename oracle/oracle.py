"""ctypes view of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: what the HIP path is compared with. Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import this module; the product (rosevine_amd) never does.
Each wrapper names the reference function its C routine restates (moe_oracle.h).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

QK, Q4_BLOCK, Q8_BLOCK = 32, 18, 34

_lib = None


REF_SRC = "/root/reference/runtime/hip/rvhip.hip"
REF_LIB_PATH = os.path.join(HERE, "_ref", "librvhip_ref.so")


def build() -> None:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off), and the reference's own HIP
    kernels into _ref/ when the reference tree is present (where it is absent, a library built
    earlier is used)."""
    subprocess.run(["make", "-s", "-B", "-C", HERE, "liboracle.so"], check=True)
    if os.path.exists(REF_SRC):
        subprocess.run(["make", "-s", "-B", "-C", HERE, "_ref/librvhip_ref.so"], check=True)


def ref_lib():
    """The reference's HIP kernels (runtime/hip/rvhip.hip) built by oracle/Makefile, or None when
    they were not built. Loaded with local symbol binding: the product library exports the same
    rvh_* names, and each handle resolves to its own."""
    if not os.path.exists(REF_LIB_PATH):
        return None
    L = C.CDLL(REF_LIB_PATH, mode=os.RTLD_LOCAL | os.RTLD_NOW)
    vp, i, f = C.c_void_p, C.c_int, C.c_float
    sig = {
        "rvh_init": [i],
        "rvh_sync": [],
        "rvh_kv_store": [vp, vp, vp, vp, i, i, i, i, i],
        "rvh_attention": [vp, vp, vp, vp, vp, i, i, i, i, i, i, i, i],
        "rvh_attn_split": [vp, vp, vp, vp, vp, i, i, i, i, i, i, i, i],
        "rvh_attn_combine": [vp, vp, i, i, i],
        "rvh_q4_mm": [vp, vp, vp, i, i, i],
        "rvh_rms_norm": [vp, vp, vp, i, i, f, f],
        "rvh_f32_mm": [vp, vp, vp, i, i, i],
        "rvh_geglu_split": [vp, vp, i, i],
        "rvh_gather_rows": [vp, vp, vp, i, i],
        "rvh_moe_combine": [vp, vp, vp, vp, vp, i, i, i],
    }
    for name, args in sig.items():
        fn = getattr(L, name)
        fn.restype = i
        fn.argtypes = args
    return L


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _declare(L):
    vp, sz, f32, i32, u16 = C.c_void_p, C.c_size_t, C.c_float, C.c_int, C.c_uint16
    sig = {
        "orc_f16_to_f32": (f32, [u16]),
        "orc_f32_to_f16": (u16, [f32]),
        "orc_dequant_q4_0": (None, [vp, vp, sz]),
        "orc_dot_q4_0": (f32, [vp, vp, sz]),
        "orc_matmul_q4_0": (None, [vp, sz, vp, sz, vp, sz]),
        "orc_quantize_q8_0": (None, [vp, vp, sz]),
        "orc_dot_q8_scalar": (f32, [vp, vp, sz]),
        "orc_q4q8_block_sums": (None, [vp, vp, sz, vp]),
        "orc_dot_q8_avx2_order": (f32, [vp, vp, sz]),
        "orc_matvec_f32": (None, [vp, sz, vp, vp, sz]),
        "orc_rms_norm": (None, [vp, vp, sz, f32, f32]),
        "orc_gelu": (f32, [f32]),
        "orc_softmax": (None, [vp, sz]),
        "orc_dot_q8_0": (f32, [vp, vp, sz]),
        "orc_axpy_q8_0": (None, [vp, f32, vp, sz]),
        "orc_attention": (None, [vp, vp, vp, sz, sz, sz, sz, sz, sz, sz, vp]),
        "orc_test_rng_vec": (None, [C.POINTER(C.c_uint64), sz, f32, vp]),
        "orc_geglu_split": (None, [vp, vp, sz, sz]),
        "orc_top_k": (None, [vp, sz, sz, vp]),
        "orc_router_logits": (None, [vp, vp, vp, sz, sz, sz, vp]),
        "orc_select_experts": (None, [vp, sz, sz, sz, vp, vp]),
        "orc_moe_plan": (None, [vp, sz, sz, vp, vp, vp]),
        "orc_experts_q8": (i32, [vp, vp, vp, vp, sz, sz, sz, sz, vp, vp, vp, vp, vp, vp]),
        "orc_moe_layer": (i32, [vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, i32, f32, vp, vp, vp]),
        "cpb_create": (vp, [i32]),
        "cpb_destroy": (None, [vp]),
        "cpb_threads": (i32, [vp]),
        "cpb_uses_avx2": (i32, []),
        "cpb_expert_ns": (C.c_uint64, [vp]),
        "cpb_moe_layer": (i32, [vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, vp, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().orc_f32_to_f16(f)


def dequant_q4_0(row: np.ndarray, k: int) -> np.ndarray:
    out = np.empty(k, np.float32)
    row = _u8(row)
    lib().orc_dequant_q4_0(_p(row), _p(out), k)
    return out


def dot_q4_0(row, x) -> float:
    row, x = _u8(row), _f32(x)
    return lib().orc_dot_q4_0(_p(row), _p(x), x.size)


def matmul_q4_0(w, k, x, n_in, n_out) -> np.ndarray:
    w, x = _u8(w), _f32(x)
    y = np.empty(n_in * n_out, np.float32)
    lib().orc_matmul_q4_0(_p(w), k, _p(x), n_in, _p(y), n_out)
    return y.reshape(n_in, n_out)


def quantize_q8_0(x) -> np.ndarray:
    x = _f32(x).reshape(-1)
    out = np.empty(x.size // QK * Q8_BLOCK, np.uint8)
    lib().orc_quantize_q8_0(_p(x), _p(out), x.size)
    return out


class TestRng:
    """The reference tests' xorshift64 generator (runtime/tests/hip_ops.rs:9-22)."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed)

    def vec(self, n: int, scale: float) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().orc_test_rng_vec(C.byref(self.state), n, scale, _p(out))
        return out


def test_q8_caches(rng: TestRng, total: int, cap: int, nkv: int, hd: int):
    """runtime/tests/hip_ops.rs:229-241: positions 0..total-1, each kv head's key row then value row
    drawn from rng and quantised into ring slot p % cap (later positions overwrite)."""
    rows = rng.vec(total * nkv * 2 * hd, 1.0).reshape(total, nkv, 2, hd)
    row = hd // QK * Q8_BLOCK
    kc, vc = np.zeros((cap, nkv * row), np.uint8), np.zeros((cap, nkv * row), np.uint8)
    first = max(0, total - cap)  # older positions are overwritten
    slots = np.arange(first, total) % cap
    kc[slots] = quantize_q8_0(rows[first:, :, 0]).reshape(-1, nkv * row)
    vc[slots] = quantize_q8_0(rows[first:, :, 1]).reshape(-1, nkv * row)
    return kc.reshape(-1), vc.reshape(-1)


def dot_q8_0(row, x) -> float:
    """runtime/src/ops.rs:107-118: a Q8_0 row times f32 x."""
    row, x = _u8(row), _f32(x)
    return lib().orc_dot_q8_0(_p(row), _p(x), x.size)


def axpy_q8_0(row, w: float, out) -> np.ndarray:
    """runtime/src/ops.rs:120-128: out += w * row, in place on a float32 array."""
    row = _u8(row)
    assert out.dtype == np.float32 and out.flags.c_contiguous
    lib().orc_axpy_q8_0(_p(row), w, _p(out), out.size)
    return out


def attention(q, kc, vc, n_head, n_kv, hd, cap, window, p0, n_tok) -> np.ndarray:
    """runtime/tests/hip_ops.rs:245-271: CPU attention of n_tok queries at p0.. over a Q8_0 ring."""
    q, kc, vc = _f32(q).reshape(-1), _u8(kc).reshape(-1), _u8(vc).reshape(-1)
    row = hd // QK * Q8_BLOCK
    assert q.size == n_tok * n_head * hd and kc.size >= cap * n_kv * row and vc.size >= cap * n_kv * row
    longest = min(p0 + n_tok, window) if window > 0 else p0 + n_tok
    assert longest <= cap and n_head % n_kv == 0 and hd % QK == 0
    out = np.empty(n_tok * n_head * hd, np.float32)
    lib().orc_attention(_p(q), _p(kc), _p(vc), n_head, n_kv, hd, cap, window, p0, n_tok, _p(out))
    return out.reshape(n_tok, n_head, hd)


def dot_q8_scalar(row, xq, k) -> float:
    row, xq = _u8(row), _u8(xq)
    return lib().orc_dot_q8_scalar(_p(row), _p(xq), k)


def dot_q8_avx2_order(row, xq, k) -> float:
    row, xq = _u8(row), _u8(xq)
    return lib().orc_dot_q8_avx2_order(_p(row), _p(xq), k)


def q4q8_block_sums(row, xq, k) -> np.ndarray:
    row, xq = _u8(row), _u8(xq)
    out = np.empty(k // QK, np.int32)
    lib().orc_q4q8_block_sums(_p(row), _p(xq), k, _p(out))
    return out


def matvec_f32(w, x) -> np.ndarray:
    w, x = _f32(w), _f32(x)
    n_out = w.size // x.size
    y = np.empty(n_out, np.float32)
    lib().orc_matvec_f32(_p(w), x.size, _p(x), _p(y), n_out)
    return y


def rms_norm(x, weight=None, eps=1e-6, post=1.0) -> np.ndarray:
    x = _f32(x).copy()
    w = None if weight is None else _f32(weight)
    lib().orc_rms_norm(_p(x), None if w is None else _p(w), x.size, eps, post)
    return x


def gelu(x: float) -> float:
    return lib().orc_gelu(x)


def geglu_split(gu, ff) -> np.ndarray:
    gu = _f32(gu).reshape(-1, 2 * ff)
    out = np.empty((gu.shape[0], ff), np.float32)
    lib().orc_geglu_split(_p(gu), _p(out), gu.shape[0], ff)
    return out


def softmax(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().orc_softmax(_p(x), x.size)
    return x


def top_k(x, k) -> list:
    x = _f32(x)
    out = np.empty(k, np.uint32)
    lib().orc_top_k(_p(x), x.size, k, _p(out))
    return [int(v) for v in out]


def router_logits(w_r, bias, x, n_exp, d) -> np.ndarray:
    x = _f32(x).reshape(-1, d)
    w_r = _f32(w_r)
    b = None if bias is None else _f32(bias)
    out = np.empty((x.shape[0], n_exp), np.float32)
    lib().orc_router_logits(_p(w_r), None if b is None else _p(b), _p(x), x.shape[0], n_exp, d, _p(out))
    return out


def select_experts(logits, used):
    lg = _f32(logits).copy()
    n_tok, n_exp = lg.shape
    ids = np.empty((n_tok, used), np.uint32)
    w = np.empty((n_tok, used), np.float32)
    lib().orc_select_experts(_p(lg), n_tok, n_exp, used, _p(ids), _p(w))
    return ids, w, lg


def moe_plan(ids, n_exp):
    ids = np.ascontiguousarray(ids, dtype=np.uint32).reshape(-1)
    order = np.empty(ids.size, np.uint32)
    pos_of = np.empty(ids.size, np.uint32)
    gs = np.empty(n_exp + 1, np.uint32)
    lib().orc_moe_plan(_p(ids), ids.size, n_exp, _p(order), _p(pos_of), _p(gs))
    return order, pos_of, gs


def _ptr_array(mats, n_exp):
    """Array of n_exp row pointers (NULL where an expert is absent); keeps the arrays alive."""
    arr = (C.c_void_p * n_exp)()
    keep = []
    for e in range(n_exp):
        m = mats.get(e) if isinstance(mats, dict) else mats[e]
        if m is not None:
            m = _u8(m)
            keep.append(m)
            arr[e] = m.ctypes.data
    return arr, keep


def experts_q8(gate_up: dict, down: dict, down_scale, moe_in, d, ff, ids, weights, n_exp, intermediates=False):
    moe_in = _f32(moe_in).reshape(-1, d)
    n_tok = moe_in.shape[0]
    ids = np.ascontiguousarray(ids, dtype=np.uint32).reshape(n_tok, -1)
    used = ids.shape[1]
    weights = _f32(weights).reshape(n_tok, used)
    gu_p, k1 = _ptr_array(gate_up, n_exp)
    dn_p, k2 = _ptr_array(down, n_exp)
    ds = None if down_scale is None else _f32(down_scale)
    out = np.empty((n_tok, d), np.float32)
    pairs = n_tok * used
    gu = np.empty((pairs, 2 * ff), np.float32) if intermediates else None
    h = np.empty((pairs, ff), np.float32) if intermediates else None
    y = np.empty((pairs, d), np.float32) if intermediates else None
    rc = lib().orc_experts_q8(gu_p, dn_p, None if ds is None else _p(ds), _p(moe_in), n_tok, d, ff, used, _p(ids),
                              _p(weights), _p(out), None if gu is None else _p(gu), None if h is None else _p(h),
                              None if y is None else _p(y))
    if rc != 0:
        raise ValueError("a selected expert has no weights")
    del k1, k2
    if intermediates:
        return out, gu, h, y
    return out


def moe_layer(w_r, bias, gate_up: dict, down: dict, down_scale, x, n_exp, d, ff, used, pre_norm=False, eps=1e-6):
    x = _f32(x).reshape(-1, d)
    n_tok = x.shape[0]
    gu_p, k1 = _ptr_array(gate_up, n_exp)
    dn_p, k2 = _ptr_array(down, n_exp)
    w_r = _f32(w_r)
    b = None if bias is None else _f32(bias)
    ds = None if down_scale is None else _f32(down_scale)
    ids = np.empty((n_tok, used), np.uint32)
    w = np.empty((n_tok, used), np.float32)
    out = np.empty((n_tok, d), np.float32)
    rc = lib().orc_moe_layer(_p(w_r), None if b is None else _p(b), gu_p, dn_p, None if ds is None else _p(ds),
                             _p(x), n_tok, n_exp, d, ff, used, 1 if pre_norm else 0, eps, _p(ids), _p(w), _p(out))
    if rc != 0:
        raise ValueError("a selected expert has no weights")
    del k1, k2
    return ids, w, out


class CpuBaseline:
    """The reference CPU expert path on a persistent pool (cpu_baseline.c)."""

    def __init__(self, threads: int):
        self.pool = lib().cpb_create(threads)
        if not self.pool:
            raise ValueError("bad thread count")
        self.threads = threads

    @staticmethod
    def uses_avx2() -> bool:
        return bool(lib().cpb_uses_avx2())

    def close(self):
        if self.pool:
            lib().cpb_destroy(self.pool)
            self.pool = None

    def __del__(self):
        self.close()

    def expert_seconds(self) -> float:
        """Wall time of the expert part (after router and selection) of every layer call so far."""
        return lib().cpb_expert_ns(self.pool) * 1e-9

    def prepare(self, gate_up, down, n_exp):
        """Bind expert weight pointers once (they stay alive with this object)."""
        self._gu, self._k1 = _ptr_array(gate_up, n_exp)
        self._dn, self._k2 = _ptr_array(down, n_exp)
        self.n_exp = n_exp

    def layer(self, w_r, bias, down_scale, x, d, ff, used, out=None, ids=None, weights=None):
        x = _f32(x).reshape(-1, d)
        n_tok = x.shape[0]
        ids = np.empty((n_tok, used), np.uint32) if ids is None else ids
        weights = np.empty((n_tok, used), np.float32) if weights is None else weights
        out = np.empty((n_tok, d), np.float32) if out is None else out
        rc = lib().cpb_moe_layer(self.pool, _p(w_r), None if bias is None else _p(bias), self._gu, self._dn,
                                 None if down_scale is None else _p(down_scale), _p(x), n_tok, self.n_exp, d, ff,
                                 used, _p(ids), _p(weights), _p(out))
        if rc != 0:
            raise ValueError("a selected expert has no weights")
        return ids, weights, out
