"""Pins the oracle's attention functions (orc_dot_q8_0, orc_axpy_q8_0, orc_attention) and the
reference tests' input generator (orc_test_rng_vec).

The checks come from outside the oracle's formulas: the reference's own known answers
(runtime/src/ops.rs:370-391), exact f64 attention over the numpy-dequantised cache, cases that
the mathematics fixes (one key gives its value row exactly, a zero query averages the values),
and invariances of the definition (keys outside the window or of another kv head do not matter;
the ring slot of a position does not matter); the generator against Marsaglia's xorshift64 stated
again with Python integers. Planted mistakes in the oracle's source fail these
tests in test_oracle_mutations.py.
"""
import numpy as np

QK, Q8B = 32, 34


def deq_rows(cache, n_rows, hd):
    """numpy dequantisation of Q8_0 rows: d (numpy's IEEE half) times the int8 quants, in f64."""
    blk = cache.reshape(n_rows, hd // QK, Q8B)
    d = blk[:, :, :2].copy().view(np.float16).astype(np.float64)  # [rows][blocks][1]
    q = blk[:, :, 2:].view(np.int8).astype(np.float64)
    return (q * d).reshape(n_rows, hd)


def ring(orc, rng, total, cap, nkv, hd, scale=1.0):
    """K and V rings holding positions 0..total-1 at slots p % cap (later positions overwrite)."""
    row = hd // QK * Q8B
    kc, vc = np.zeros(cap * nkv * row, np.uint8), np.zeros(cap * nkv * row, np.uint8)
    for p in range(total):
        for g in range(nkv):
            o = ((p % cap) * nkv + g) * row
            kc[o:o + row] = orc.quantize_q8_0(rng.standard_normal(hd).astype(np.float32) * scale)
            vc[o:o + row] = orc.quantize_q8_0(rng.standard_normal(hd).astype(np.float32) * scale)
    return kc, vc


def attention_f64(q, kc, vc, nh, nkv, hd, cap, win, p0, n):
    K, V = deq_rows(kc, cap * nkv, hd), deq_rows(vc, cap * nkv, hd)
    q = q.reshape(n, nh, hd).astype(np.float64)
    out = np.zeros((n, nh, hd))
    for t in range(n):
        pos = p0 + t
        lo = max(0, pos + 1 - win) if win > 0 else 0
        keys = np.arange(lo, pos + 1)
        for h in range(nh):
            g = h // (nh // nkv)
            rows = (keys % cap) * nkv + g
            s = K[rows] @ q[t, h]
            e = np.exp(s - s.max())
            out[t, h] = (e / e.sum()) @ V[rows]
    return out


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(np.sqrt(((a - b) ** 2).sum() / max((b ** 2).sum(), 1e-300)))


def test_q8_dot_and_axpy_reference_known_answers(orc):
    # runtime/src/ops.rs:370-391: x_i = sin(0.37 i), 64 values
    x = np.sin(np.arange(64, dtype=np.float32) * np.float32(0.37)).astype(np.float32)
    q8 = orc.quantize_q8_0(x)
    assert abs(orc.dot_q8_0(q8, np.ones(64, np.float32)) - float(x.sum())) < 0.05
    acc = orc.axpy_q8_0(q8, 2.0, np.zeros(64, np.float32))
    assert np.all(np.abs(acc - 2.0 * x) < 0.02)


def test_q8_dot_exact_cases(orc):
    # d = 0.5 and quants -16..15 against ones: 0.5 * (-16) = -8; d = 2, quants 1 against 0..31:
    # 2 * 496 = 992. Every partial sum is an integer, so the f32 result is exact.
    row = np.zeros(2 * Q8B, np.uint8)
    row[0:2] = np.array([0.5], np.float16).view(np.uint8)
    row[2:34] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    row[34:36] = np.array([2.0], np.float16).view(np.uint8)
    row[36:68] = 1
    x = np.concatenate([np.ones(32), np.arange(32)]).astype(np.float32)
    assert orc.dot_q8_0(row, x) == -8.0 + 992.0
    # negative quants are signed: -128 * 1 with d = 1
    row2 = np.zeros(Q8B, np.uint8)
    row2[0:2] = np.array([1.0], np.float16).view(np.uint8)
    row2[2] = 0x80
    assert orc.dot_q8_0(row2, np.ones(32, np.float32)) == -128.0


def test_q8_dot_and_axpy_against_f64(orc):
    rng = np.random.default_rng(21)
    for hd in (32, 256, 512):
        row = orc.quantize_q8_0(rng.standard_normal(hd).astype(np.float32))
        x = rng.standard_normal(hd).astype(np.float32)
        deq = deq_rows(row, 1, hd)[0]
        want = float(deq @ x.astype(np.float64))
        bound = 4 * hd * np.finfo(np.float32).eps * float(np.abs(deq * x).sum())
        assert abs(orc.dot_q8_0(row, x) - want) <= bound
        base = rng.standard_normal(hd).astype(np.float32)
        w = np.float32(rng.uniform(0.01, 1))
        got = orc.axpy_q8_0(row, float(w), base.copy())
        want = base.astype(np.float64) + float(w) * deq
        err = np.abs(got - want)
        assert np.all(err <= 3 * np.finfo(np.float32).eps * (np.abs(want) + float(w) * np.abs(deq)))
        # w = 0 leaves out unchanged
        assert np.array_equal(orc.axpy_q8_0(row, 0.0, base.copy()), base)


def test_attention_against_exact_f64(orc):
    rng = np.random.default_rng(22)
    # (heads, kv heads, head dim, window, ring capacity, filled positions, queries)
    for nh, nkv, hd, win, cap, total, n in [(4, 2, 64, 0, 40, 37, 3), (8, 2, 128, 16, 20, 45, 4),
                                            (2, 2, 32, 0, 9, 9, 1), (6, 3, 64, 5, 7, 30, 2)]:
        kc, vc = ring(orc, rng, total, cap, nkv, hd)
        q = (rng.standard_normal(n * nh * hd) * 0.2).astype(np.float32)
        got = orc.attention(q, kc, vc, nh, nkv, hd, cap, win, total - n, n)
        want = attention_f64(q, kc, vc, nh, nkv, hd, cap, win, total - n, n)
        assert rel(got, want) < 2e-6, (nh, nkv, hd, win, cap, total, n)


def test_attention_fixed_cases(orc):
    rng = np.random.default_rng(23)
    nh, nkv, hd, cap = 4, 2, 64, 8
    kc, vc = ring(orc, rng, 8, cap, nkv, hd)
    q = (rng.standard_normal(nh * hd)).astype(np.float32)
    # position 0 sees one key: softmax weight 1 and the value row exactly (d * 1 * q per element)
    out = orc.attention(q, kc, vc, nh, nkv, hd, cap, 0, 0, 1)[0]
    V = deq_rows(vc, cap * nkv, hd)
    for h in range(nh):
        assert np.array_equal(out[h], V[h // 2].astype(np.float32))
    # a window of 1 at any position also sees only its own key
    out = orc.attention(q, kc, vc, nh, nkv, hd, cap, 1, 5, 1)[0]
    for h in range(nh):
        assert np.array_equal(out[h], V[5 * nkv + h // 2].astype(np.float32))
    # a zero query scores every key 0: the mean of the value rows
    out = orc.attention(np.zeros(nh * hd, np.float32), kc, vc, nh, nkv, hd, cap, 0, 6, 1)[0]
    for h in range(nh):
        rows = np.arange(7) * nkv + h // 2
        assert np.allclose(out[h], V[rows].mean(0), rtol=0, atol=1e-5)


def test_attention_window_heads_and_ring_invariance(orc):
    rng = np.random.default_rng(24)
    nh, nkv, hd, win, cap, total, n = 8, 4, 64, 6, 10, 20, 2
    kc, vc = ring(orc, rng, total, cap, nkv, hd)
    q = (rng.standard_normal(n * nh * hd) * 0.5).astype(np.float32)
    p0 = total - n
    base = orc.attention(q, kc, vc, nh, nkv, hd, cap, win, p0, n)
    row = hd // QK * Q8B
    # rewriting a position older than every query's window changes nothing; one inside does
    old = p0 + 1 - win - 1  # the key just outside the first query's window
    for cache in ("k", "v"):
        k2, v2 = kc.copy(), vc.copy()
        tgt = k2 if cache == "k" else v2
        o = ((old % cap) * nkv + 1) * row
        tgt[o + 2:o + row] = rng.integers(0, 256, row - 2, dtype=np.uint8)
        assert np.array_equal(orc.attention(q, k2, v2, nh, nkv, hd, cap, win, p0, n), base)
        o = ((p0 % cap) * nkv + 1) * row
        tgt[o + 2:o + 34] = rng.integers(0, 256, 32, dtype=np.uint8)
        changed = orc.attention(q, k2, v2, nh, nkv, hd, cap, win, p0, n)
        # kv head 1 serves query heads 2 and 3 only
        assert not np.array_equal(changed[:, 2:4], base[:, 2:4])
        assert np.array_equal(np.delete(changed, [2, 3], axis=1), np.delete(base, [2, 3], axis=1))
    # the same positions in a larger ring (other slots) give the same result, bit for bit
    cap2 = 23
    k3, v3 = np.zeros(cap2 * nkv * row, np.uint8), np.zeros(cap2 * nkv * row, np.uint8)
    for p in range(p0 + 1 - win, total):
        for g in range(nkv):
            a, b = ((p % cap) * nkv + g) * row, ((p % cap2) * nkv + g) * row
            k3[b:b + row], v3[b:b + row] = kc[a:a + row], vc[a:a + row]
    assert np.array_equal(orc.attention(q, k3, v3, nh, nkv, hd, cap2, win, p0, n), base)


def test_reference_test_generator_is_marsaglia_xorshift64(orc):
    # runtime/tests/hip_ops.rs:9-22: xorshift64 with shifts 13, 7, 17 (Marsaglia 2003), the top 24
    # bits of each state scaled to [-1, 1), times scale; stated again here with Python integers
    def py_vec(state, n, scale):
        out = []
        for _ in range(n):
            state ^= (state << 13) & 0xFFFFFFFFFFFFFFFF
            state ^= state >> 7
            state ^= (state << 17) & 0xFFFFFFFFFFFFFFFF
            out.append(np.float32(np.float32(state >> 40) / np.float32(1 << 24) * np.float32(2) - np.float32(1))
                       * np.float32(scale))
        return np.array(out, np.float32), state

    for seed, scale in [(3, 1.0), (5, 0.2), (17, 2.0)]:
        r = orc.TestRng(seed)
        a = r.vec(700, scale)
        b = r.vec(300, scale)
        want, _ = py_vec(seed, 1000, scale)
        assert np.array_equal(np.concatenate([a, b]), want)
    # values lie in [-1, 1) and the draws are not degenerate
    v = orc.TestRng(99).vec(100000, 1.0)
    assert v.min() >= -1.0 and v.max() < 1.0 and abs(float(v.mean())) < 0.02


def test_reference_test_caches_hold_the_latest_position_of_each_slot(orc):
    # the ring fixture of runtime/tests/hip_ops.rs:229-241: every (position, kv head) draws a key
    # row then a value row; slot p % cap keeps the last position written to it
    nkv, hd, cap, total = 2, 64, 5, 8
    row = hd // QK * Q8B
    kc, vc = orc.test_q8_caches(orc.TestRng(7), total, cap, nkv, hd)
    r = orc.TestRng(7)
    want_k, want_v = {}, {}
    for p in range(total):
        for g in range(nkv):
            want_k[(p % cap, g)] = orc.quantize_q8_0(r.vec(hd, 1.0))
            want_v[(p % cap, g)] = orc.quantize_q8_0(r.vec(hd, 1.0))
    for (slot, g), kr in want_k.items():
        o = (slot * nkv + g) * row
        assert np.array_equal(kc[o:o + row], kr) and np.array_equal(vc[o:o + row], want_v[(slot, g)])
