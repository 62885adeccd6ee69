"""Layer shapes other than the reference model's, through every dispatch of the C ABI, against the
oracle.

The kernels are compiled for d / 256 and ff / 64 in {1, 2, 4, 8, 11, 16} and up to 256 experts
with top-k up to 8 (include/rvmoe.h). Each shape below runs single-token decode, a small batch
(4-pair tiles), a batch of 8+ pairs per expert (16-pair MFMA tiles) and a batch from
RVM_FOLD_MIN_TOKENS (exact router folds), with a router bias and down scales, and is compared
with the oracle's selection (ids exact) and outputs (the layer tolerance). Below
RVM_FOLD_MIN_TOKENS every row also equals its single-token decode bit for bit; on the fold path
the outputs are the oracle's bits.
"""
import numpy as np
import pytest

from layer_util import assert_close, dev
from rosevine_amd import hip, moe, synth
from rosevine_amd.hip import DevBuf

pytestmark = pytest.mark.gpu

SHAPES = [  # n_exp, top_k, d, ff
    (64, 4, 1024, 256),
    (256, 8, 1024, 256),  # the most experts
    (16, 2, 4096, 1024),  # the longest rows (16 steps per lane)
    (8, 8, 256, 64),      # top_k = n_exp, the shortest rows (1 step per lane)
]


def build(shape, seed):
    n_exp, top_k, d, ff = shape
    rng = np.random.default_rng([seed, n_exp, d, 7])
    router = synth.router_weights(seed, 0, n_exp, d)
    bias = rng.standard_normal(n_exp).astype(np.float32) * np.float32(0.5)
    dsc = rng.uniform(0.5, 1.5, n_exp).astype(np.float32)
    gu = hip.synth_q4_host(n_exp, 2 * ff, d, seed, 1 << 40)
    dn = hip.synth_q4_host(n_exp, d, ff, seed, 3 << 40)
    L = moe.MoeLayer(n_exp, top_k, d, ff, router, bias, dsc)
    L.load_q4(gu, dn)
    rows = lambda raw, n_out, k: {e: r for e, r in enumerate(raw.reshape(n_exp, n_out * (k // 32) * 18))}
    return L, router, bias, dsc, rows(gu, 2 * ff, d), rows(dn, d, ff)


def oracle(orc, parts, x):
    L, router, bias, dsc, gu, dn = parts
    lg = orc.router_logits(router, bias, x, L.n_exp, L.d)
    ids, w, _ = orc.select_experts(lg, L.top_k)
    return ids, orc.experts_q8(gu, dn, dsc, x, L.d, L.ff, ids, w, L.n_exp)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_shape_through_every_path(gpu, orc, shape):
    n_exp, top_k, d, ff = shape
    parts = build(shape, 11)
    L = parts[0]
    mfma_n = max(16, -(-8 * n_exp // top_k))  # 8+ pairs per expert on average
    if mfma_n >= 256:  # only reachable from RVM_FOLD_MIN_TOKENS, where the fold path takes over
        mfma_n = 3
    sizes = sorted({1, 3, mfma_n, 300})
    print(f"[shapes] {shape}: batches {sizes}", flush=True)
    x = synth.tokens(12, max(sizes), d=d)
    want_ids, want = oracle(orc, parts, x)
    ws = moe.Workspace(L, max(sizes))
    xd = dev(x)
    rows = {}
    for n in sizes:
        out = DevBuf(n * d * 4)
        if n == 1:
            moe.decode(L, xd, out, ws)
        else:
            moe.forward(L, xd, out, n, ws)
        ids, _ = ws.selection(L, n)
        assert np.array_equal(ids, want_ids[:n].astype(np.int32)), (shape, n)
        got = out.download(np.float32, n * d).reshape(n, d)
        for t in range(n):
            assert_close(got[t], want[t], f"{shape} batch {n} token {t}")
        rows[n] = got
    # below the fold path a token's row does not depend on its batch
    o1 = DevBuf(d * 4)
    for t in (0, 2):
        moe.decode(L, xd, o1, ws, x_off=t * d * 4)
        row = o1.download(np.float32, d)
        assert np.array_equal(row, rows[3][t]) and np.array_equal(row, rows[mfma_n][t]), (shape, t)
        assert np.array_equal(row, rows[1][0]) or t > 0
    # the fold path: the oracle's bits
    assert np.array_equal(rows[300], want[:300]), shape
