"""The reference's own HIP kernels (runtime/hip/rvhip.hip, built into oracle/_ref by
oracle/Makefile) as a second reference, on the same device buffers and the reference tests' inputs.

For each operator whose reference is a HIP kernel, the library's entry point is compared with the
reference's at the bar the reference sets between its own implementations: bit for bit where it
asserts that (the key/value store, gather, the slot-order combine), relative L2 < 1e-5 where it
compares kernels of different summation order (attention: runtime/tests/hip_ops.rs:273-310; the
Q4_0 GEMV: hip_ops.rs:56-81), and 1e-6 for the elementwise and f32 helpers (hip_ops.rs:402-420).
Skipped when the reference kernels were not built (no reference tree at build time).
"""

import numpy as np
import pytest

from rosevine_amd import hip
from rosevine_amd.hip import DevBuf

pytestmark = pytest.mark.gpu

QK, Q8B, Q4B = 32, 34, 18


@pytest.fixture(scope="module")
def ref(gpu):
    from oracle import oracle
    L = oracle.ref_lib()
    if L is None:
        pytest.skip("the reference's HIP kernels were not built (oracle/Makefile _ref/librvhip_ref.so)")
    assert L.rvh_init(0) == 0
    return L


def dev(a):
    return DevBuf.from_array(np.ascontiguousarray(a))


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(np.sqrt(((a - b) ** 2).sum() / max((b ** 2).sum(), 1e-300)))


def ok(code):
    assert code == 0, f"reference kernel returned {code}"


def test_kv_store_bit_for_bit_with_the_reference_kernel(gpu, ref, orc):
    # the ring case of runtime/tests/hip_ops.rs:328-372, its generator and seed
    r = orc.TestRng(3)
    nkv, hd, cap, total, n = 8, 256, 1028, 1030, 4
    row = hd // QK * Q8B
    kv = dev(r.vec(total * nkv * hd, 1.0))
    vv = dev(r.vec(total * nkv * hd, 1.0))
    ours = [dev(np.zeros(cap * nkv * row, np.uint8)) for _ in range(2)]
    theirs = [dev(np.zeros(cap * nkv * row, np.uint8)) for _ in range(2)]
    for p0 in range(0, total, n):
        m = min(n, total - p0)
        off = p0 * nkv * hd * 4
        hip.kv_store(kv, vv, ours[0], ours[1], m, nkv, hd, p0, cap, k_off=off, v_off=off)
        ok(ref.rvh_kv_store(kv.at(off), vv.at(off), theirs[0].at(), theirs[1].at(), m, nkv, hd, p0, cap))
    ok(ref.rvh_sync())
    for a, b in zip(ours, theirs):
        assert np.array_equal(a.download(np.uint8, cap * nkv * row), b.download(np.uint8, cap * nkv * row))


def test_attention_against_the_reference_kernels(gpu, ref, orc):
    # runtime/tests/hip_ops.rs:273-310 with its inputs: the library's split attention (with the
    # reference's chunk policy) against the reference's split kernel at the same chunk count and
    # against its one-pass kernel
    r = orc.TestRng(5)
    cases = [
        ("local ring wrap", 16, 8, 256, 1024, 1028, 1030, 4),
        ("global decode", 16, 2, 512, 0, 5000, 5000, 1),
        ("global batch of 8", 16, 2, 512, 0, 5000, 5000, 8),
        ("global prefill microbatch", 16, 2, 512, 0, 5000, 5000, 64),
        ("short context", 16, 2, 512, 0, 100, 3, 1),
        ("ragged chunks", 16, 2, 512, 0, 200, 129, 1),
    ]
    for name, nh, nkv, hd, win, cap, total, n in cases:
        print(f"[ref attn] {name}", flush=True)
        kc, vc = orc.test_q8_caches(r, total, cap, nkv, hd)
        q = r.vec(n * nh * hd, 0.2)
        p0 = total - n
        dq, dk, dv = dev(q), dev(kc), dev(vc)
        nq = n * nh * hd
        ours = DevBuf(nq * 4)
        part = DevBuf(hip.attention_split_scratch(n, nh, hd) * 4)
        chunks = hip.attention_split(dq, dk, dv, ours, part, n, nh, nkv, hd, p0, cap, win)
        theirs_split, theirs_one = DevBuf(nq * 4), DevBuf(nq * 4)
        rpart = DevBuf(hip.attention_split_scratch(n, nh, hd) * 4)
        ok(ref.rvh_attn_split(dq.at(), dk.at(), dv.at(), theirs_split.at(), rpart.at() if chunks > 1 else None, n, nh,
                              nkv, hd, p0, cap, win, chunks))
        if chunks > 1:
            ok(ref.rvh_attn_combine(rpart.at(), theirs_split.at(), n * nh, hd, chunks))
        scores = DevBuf(n * nh * cap * 4)
        ok(ref.rvh_attention(dq.at(), dk.at(), dv.at(), theirs_one.at(), scores.at(), n, nh, nkv, hd, p0, cap, win,
                             cap))
        ok(ref.rvh_sync())
        got = ours.download(np.float32, nq)
        assert rel(got, theirs_split.download(np.float32, nq)) < 1e-5, name
        assert rel(got, theirs_one.download(np.float32, nq)) < 1e-5, name


def test_q4_mm_against_the_reference_kernel(gpu, ref):
    # rvh_q4_mm at the reference model's projection shapes (contract.rs:41-62), 1 and 7 tokens
    rng = np.random.default_rng(51)
    for n_out, k in [(4096, 2816), (2048, 2816), (2816, 4096), (2112, 2816), (2816, 2112)]:
        for n_in in (1, 7):
            nb = k // QK
            w = np.empty((n_out, nb, Q4B), np.uint8)
            w[:, :, :2] = rng.uniform(0.01, 0.03, (n_out, nb)).astype(np.float16).view(np.uint8).reshape(n_out, nb, 2)
            w[:, :, 2:] = rng.integers(0, 256, (n_out, nb, 16), dtype=np.uint8)
            x = rng.uniform(-1, 1, (n_in, k)).astype(np.float32)
            dw, dx = dev(w.reshape(-1)), dev(x)
            ours, theirs = DevBuf(n_in * n_out * 4), DevBuf(n_in * n_out * 4)
            hip.q4_mm(dw, dx, ours, n_out, k, n_in)
            ok(ref.rvh_q4_mm(dw.at(), dx.at(), theirs.at(), n_out, k, n_in))
            ok(ref.rvh_sync())
            assert rel(ours.download(np.float32, n_in * n_out), theirs.download(np.float32, n_in * n_out)) < 1e-5


def test_expert_path_helpers_against_the_reference_kernels(gpu, ref):
    rng = np.random.default_rng(52)
    # rvh_rms_norm, rows of 2816 with a weight and a post factor
    rows, width = 5, 2816
    x = rng.standard_normal((rows, width)).astype(np.float32)
    wgt = rng.uniform(0.5, 1.5, width).astype(np.float32)
    dx, dw = dev(x), dev(wgt)
    ours, theirs = DevBuf(x.nbytes), DevBuf(x.nbytes)
    hip.rms_norm(dx, ours, dw, rows, width, 1e-6, 0.5)
    ok(ref.rvh_rms_norm(dx.at(), theirs.at(), dw.at(), rows, width, 1e-6, 0.5))
    ok(ref.rvh_sync())
    assert rel(ours.download(np.float32, x.size), theirs.download(np.float32, x.size)) < 1e-6
    # rvh_f32_mm, the router shape
    W = (rng.standard_normal((128, 2816)) * 0.02).astype(np.float32)
    xs = rng.standard_normal((3, 2816)).astype(np.float32)
    dW, dxs = dev(W), dev(xs)
    ours, theirs = DevBuf(3 * 128 * 4), DevBuf(3 * 128 * 4)
    hip.f32_mm(dW, dxs, ours, 128, 2816, 3)
    ok(ref.rvh_f32_mm(dW.at(), dxs.at(), theirs.at(), 128, 2816, 3))
    ok(ref.rvh_sync())
    assert rel(ours.download(np.float32, 384), theirs.download(np.float32, 384)) < 1e-6
    # rvh_geglu_split, 24 rows of 2 x 704 (hip_ops.rs:402-420: rel < 1e-6)
    prs, fe = 24, 704
    gu = rng.uniform(-2, 2, (prs, 2 * fe)).astype(np.float32)
    dgu = dev(gu)
    ours, theirs = DevBuf(prs * fe * 4), DevBuf(prs * fe * 4)
    hip.geglu_split(dgu, ours, prs, fe)
    ok(ref.rvh_geglu_split(dgu.at(), theirs.at(), prs, fe))
    ok(ref.rvh_sync())
    assert rel(ours.download(np.float32, prs * fe), theirs.download(np.float32, prs * fe)) < 1e-6
    # rvh_gather_rows and rvh_moe_combine, bit for bit (hip_ops.rs:421-439)
    src = rng.standard_normal((40, 2816)).astype(np.float32)
    idx = rng.integers(0, 40, 24).astype(np.int32)
    dsrc, didx = dev(src), dev(idx)
    ours, theirs = DevBuf(24 * 2816 * 4), DevBuf(24 * 2816 * 4)
    hip.gather_rows(dsrc, 40, didx, ours, 24, 2816)
    ok(ref.rvh_gather_rows(dsrc.at(), didx.at(), theirs.at(), 24, 2816))
    ok(ref.rvh_sync())
    assert np.array_equal(ours.download(np.float32, 24 * 2816), theirs.download(np.float32, 24 * 2816))
    n_tok, used = 3, 8
    pairs = n_tok * used
    y = rng.standard_normal((pairs, 2816)).astype(np.float32)
    pos = rng.permutation(pairs).astype(np.int32)
    scale = rng.uniform(-1, 1, pairs).astype(np.float32)
    weight = rng.uniform(0, 1, pairs).astype(np.float32)
    dy, dpos, dsc, dwt = dev(y), dev(pos), dev(scale), dev(weight)
    ours, theirs = DevBuf(n_tok * 2816 * 4), DevBuf(n_tok * 2816 * 4)
    hip.moe_combine(dy, pairs, dpos, dsc, dwt, ours, n_tok, used, 2816)
    ok(ref.rvh_moe_combine(dy.at(), dpos.at(), dsc.at(), dwt.at(), theirs.at(), n_tok, used, 2816))
    ok(ref.rvh_sync())
    assert np.array_equal(ours.download(np.float32, n_tok * 2816), theirs.download(np.float32, n_tok * 2816))
