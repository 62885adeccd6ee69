"""Writes the small golden fixtures of this directory from the CPU oracle.

    python tests/golden/make_golden.py

Each fixture is an .npz of plain arrays (no pickled objects): seeded inputs and the oracle's
outputs for them, at sizes small enough to read by eye (k = 32 to 96, 2 to 4 experts). They
freeze the oracle's results, so that a later change to the oracle that alters any bit shows up
as a failing test, and give the GPU tests fixed vectors that need no oracle at run time.

The oracle follows runtime/src/ops.rs, runtime/src/expert_kernel.rs and runtime/src/exec.rs of
the reference; the literal known answers of the reference's own tests are kept in
test_oracle.py.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as orc  # noqa: E402

QK, Q4B = 32, 18


def q4_rows(rng, n, k):
    """Reference-layout Q4_0 rows: f16 scales in [0.005, 0.02), uniform nibble bytes."""
    rows = np.empty((n, k // QK, Q4B), np.uint8)
    d = rng.uniform(0.005, 0.02, (n, k // QK)).astype(np.float16)
    rows[:, :, :2] = d.view(np.uint8).reshape(n, k // QK, 2)
    rows[:, :, 2:] = rng.integers(0, 256, (n, k // QK, 16), dtype=np.uint8)
    return rows.reshape(n, -1)


def codecs(rng):
    """Q8_0 quantisation of 4 rows of 96 with edge values; Q4_0 decode of 3 rows."""
    x = (rng.standard_normal((4, 96)) * rng.uniform(0.01, 100, (4, 1))).astype(np.float32)
    x[0, :32] = 0.0                          # all-zero block: d = 0, id = 0
    x[1, 5] = np.float32(np.nan)             # NaN is ignored by the block maximum and maps to 0
    x[2, 32:64] = np.linspace(-2.5, 2.5, 32)  # ties of the half-away rounding
    xq = np.stack([orc.quantize_q8_0(r) for r in x])
    w = q4_rows(rng, 3, 96)
    deq = np.stack([orc.dequant_q4_0(r, 96) for r in w])
    return dict(x=x, xq=xq, w=w, deq=deq)


def q4q8(rng):
    """Packed-path GEMV shapes: 64 rows of k = 64 against 2 activation rows."""
    n_out, k = 64, 64
    w = q4_rows(rng, n_out, k)
    x = rng.standard_normal((2, k)).astype(np.float32)
    xq = np.stack([orc.quantize_q8_0(r) for r in x])
    y = np.array([[orc.dot_q8_scalar(w[r], xq[t], k) for r in range(n_out)] for t in range(2)], np.float32)
    sums = np.stack([orc.q4q8_block_sums(w[r], xq[0], k) for r in range(n_out)])
    return dict(w=w, x=x, xq=xq, y=y, sums=sums, n_out=np.int32(n_out), k=np.int32(k))


def layer(rng):
    """A 4-expert, top-2 layer of width 256 and expert width 64, 3 tokens, router bias and
    down scales: ids, weights, logits and the layer output."""
    n_exp, top_k, d, ff, n_tok = 4, 2, 256, 64, 3
    router = (rng.standard_normal((n_exp, d)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(n_exp).astype(np.float32) * np.float32(0.1)
    ds = rng.uniform(0.5, 1.5, n_exp).astype(np.float32)
    gu = np.stack([q4_rows(rng, 2 * ff, d) for _ in range(n_exp)])
    dn = np.stack([q4_rows(rng, d, ff) for _ in range(n_exp)])
    x = rng.standard_normal((n_tok, d)).astype(np.float32)
    logits = orc.router_logits(router, bias, x, n_exp, d)
    ids, w, out = orc.moe_layer(router, bias, {e: gu[e] for e in range(n_exp)}, {e: dn[e] for e in range(n_exp)},
                                ds, x, n_exp, d, ff, top_k)
    return dict(router=router, bias=bias, down_scale=ds, gate_up=gu, down=dn, x=x, logits=logits,
                ids=ids.astype(np.int32), weights=w, out=out,
                shape=np.array([n_exp, top_k, d, ff, n_tok], np.int32))


FIXTURES = {"codecs": (codecs, 101), "q4q8": (q4q8, 102), "layer": (layer, 103)}


def make(name):
    fn, seed = FIXTURES[name]
    return fn(np.random.default_rng(seed))


def main():
    for name in FIXTURES:
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **make(name))
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
