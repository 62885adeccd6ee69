"""Pins the CPU oracle (oracle/moe_oracle.c) before the GPU tests compare the HIP path with it.

Each check comes from outside the oracle's own formula: the reference's literal known answers
(runtime/src/ops.rs:358-447, runtime/src/expert_kernel.rs:261-401,
tests/research/test_correctness_oracle.py, research/fixtures/scalar-operators-v1.json, copied
here as literals), numpy's independent implementations (IEEE half conversion, float32 sequential
accumulate, stable argsort), f64 brute force, and exhaustive sweeps. Planted mistakes (a dropped
term, a wrong rounding mode, a transposed operand, a reordered fold) fail at least one test in
test_oracle_mutations.py.
"""
import math
import struct

import numpy as np
import pytest

QK, Q4B, Q8B = 32, 18, 34


def h16(bits):
    return np.array([bits], np.uint16).view(np.float16)[0]


# ---------------- f16 codecs (runtime/src/ops.rs:7-59) ----------------

def test_f16_reference_known_answers(orc):
    # runtime/src/ops.rs:358-368
    for h in [0, 0x3C00, 0xBC00, 0x7BFF, 0x0001, 0x03FF, 0x0400, 0x7C00, 0x3555]:
        assert orc.f32_to_f16(orc.f16_to_f32(h)) == h
    assert orc.f16_to_f32(0x3C00) == 1.0
    assert orc.f32_to_f16(65520.0) == 0x7C00
    assert orc.f32_to_f16(1.0 + 1.0 / 2048.0) == 0x3C00
    assert orc.f32_to_f16(1.0 + 3.0 / 2048.0) == 0x3C02
    v = np.float32(5.9604645e-8)
    assert np.float32(orc.f16_to_f32(orc.f32_to_f16(float(v)))) == v


def test_f16_to_f32_exhaustive_against_numpy(orc):
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even_against_numpy(orc):
    rng = np.random.default_rng(11)
    # random bit patterns across the whole f32 range, plus every f16 midpoint neighbourhood
    xs = rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    # exact midpoints between consecutive finite f16 values (normal and subnormal), representable
    # in f32, and their f32 neighbours on either side
    h = np.arange(0, 0x7BFF, dtype=np.uint16)
    lo, hi = h.view(np.float16).astype(np.float64), (h + 1).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32).view(np.uint32)
    xs = np.concatenate([xs, mids.view(np.float32), (mids + 1).view(np.float32), (mids - 1).view(np.float32)])
    xs = np.concatenate([xs, -xs])
    xs = xs[~np.isnan(xs)]
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)
    assert orc.f32_to_f16(float("nan")) & 0x7E00 == 0x7E00


# ---------------- Q4_0 decode and dots (runtime/src/ops.rs:67-92, 249-266) ----------------

def test_q4_all_nibbles_block_known_answer(orc):
    # tests/research/test_correctness_oracle.py:13-18
    packed = bytes((15 - i) * 16 + i for i in range(16))
    for scale in [0.0, -0.0, 1.0, -2.0, 2**-24, 65504.0]:
        blk = np.frombuffer(struct.pack("<e", scale) + packed, np.uint8)
        got = orc.dequant_q4_0(blk, 32)
        want = [scale * i for i in range(-8, 8)] + [scale * i for i in range(7, -9, -1)]
        assert np.array_equal(got, np.array(want, np.float32))


def _q4_rows(rng, rows, k, scales=None):
    nb = k // QK
    out = np.empty((rows, nb, Q4B), np.uint8)
    d = rng.uniform(0.005, 0.02, (rows, nb)).astype(np.float16) if scales is None else scales
    out[:, :, :2] = np.asarray(d, np.float16).reshape(rows, nb, 1).view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = rng.integers(0, 256, (rows, nb, 16), dtype=np.uint8)
    return out.reshape(rows, nb * Q4B)


def _deq_np(rows, k):
    """numpy dequantisation of Q4_0 rows (independent of the oracle)."""
    r = rows.reshape(rows.shape[0], k // QK, Q4B)
    d = r[:, :, :2].copy().view(np.float16).astype(np.float64)
    qs = r[:, :, 2:]
    lo = (qs & 15).astype(np.int64) - 8
    hi = (qs >> 4).astype(np.int64) - 8
    vals = np.concatenate([lo, hi], axis=2)  # elements 0..15 then 16..31
    return vals, d  # integer values [rows, nb, 32] and scales [rows, nb, 1]


def test_q4_dots_against_f64_brute_force(orc):
    rng = np.random.default_rng(3)
    k = 96
    rows = _q4_rows(rng, 5, k)
    x = (np.sin(np.arange(2 * k) * 0.37)).astype(np.float32).reshape(2, k)
    vals, d = _deq_np(rows, k)
    deq = (vals * d).reshape(5, k)
    exact = deq @ x.astype(np.float64).T  # [rows, tokens]
    mm = orc.matmul_q4_0(rows, k, x, 2, 5)
    for r in range(5):
        for t in range(2):
            dot = orc.dot_q4_0(rows[r], x[t])
            assert abs(dot - exact[r, t]) < 1e-4
            assert abs(mm[t, r] - exact[r, t]) < 1e-4
    # matmul is dequantise-then-sequential-fold: equal to numpy's float32 accumulate of the products
    deq32 = orc.dequant_q4_0(rows[2], k)
    seq = np.add.accumulate(np.concatenate([[np.float32(-0.0)], deq32 * x[1]]).astype(np.float32))[-1]
    assert mm[1, 2] == seq


# ---------------- Q8_0 quantisation (runtime/src/ops.rs:95-105) ----------------

def _q8(blocks):
    b = blocks.reshape(-1, Q8B)
    return b[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1), b[:, 2:].view(np.int8)


def test_quantize_q8_0_rounds_half_away_from_zero(orc):
    # amax = 127 gives d = 1 and id = 1 exactly, so v * id = v: ties decide the rounding mode.
    x = np.zeros(32, np.float32)
    x[:8] = [127, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5]
    d, q = _q8(orc.quantize_q8_0(x))
    assert d[0] == 1.0
    assert list(q[0, :8]) == [127, 3, -3, 1, -1, 2, -2, 127]


def test_quantize_q8_0_edges(orc):
    x = np.zeros(4 * 32, np.float32)
    x[32:64] = np.linspace(-3, 3, 32)
    x[64] = np.nan                      # f32::max ignores NaN; `as i8` maps NaN to 0
    x[65:96] = 0.25
    x[96] = np.inf                      # d = inf, id = 0, inf * 0 = NaN -> 0
    x[97:128] = 1.0
    d, q = _q8(orc.quantize_q8_0(x))
    assert d[0] == 0.0 and not q[0].any()
    assert abs(d[1] - np.float16(3.0 / 127)) == 0 and q[1, 0] == -127 and q[1, 31] == 127
    assert q[2, 0] == 0 and list(q[2, 1:4]) == [127, 127, 127]
    assert np.isinf(d[3]) and not q[3].any()


def test_quantize_q8_0_invariants(orc):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(88 * 32) * rng.uniform(1e-3, 1e3, 88 * 32)).astype(np.float32)
    xb = x.reshape(88, 32)
    d16, q = _q8(orc.quantize_q8_0(x))
    amax = np.abs(xb).max(axis=1)
    d32 = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(d16, d32.astype(np.float16).astype(np.float32))  # stored scale = f16(RNE)(amax/127)
    assert np.all(np.abs(q).max(axis=1) == 127)                              # the amax element maps to +-127
    err = np.abs(xb - q.astype(np.float32) * d32[:, None])
    assert np.all(err <= d32[:, None] * 0.5000001 + 1e-30)                    # within half a step


def test_q8_round_trip_reference_bounds(orc):
    # runtime/src/ops.rs:383-390: dot_q8_0 of the quantised sin row with ones ~ sum(x) within 0.05
    x = np.sin(np.arange(64) * 0.37).astype(np.float32)
    d, q = _q8(orc.quantize_q8_0(x))
    back = sum(float(d[b]) * float(q[b].astype(np.float32).sum()) for b in range(2))
    assert abs(back - float(x.sum())) < 0.05


# ---------------- Q4 x Q8 dot (runtime/src/expert_kernel.rs:147-191) ----------------

def _blocksums_np(row, xq, k):
    vals, _ = _deq_np(row.reshape(1, -1), k)
    q = xq.reshape(-1, Q8B)[:, 2:].view(np.int8).astype(np.int64)
    return (vals[0] * q).sum(axis=1)


@pytest.mark.parametrize("k", [32, 96, 704, 2816])
def test_q8_dot_matches_exact_integer_reference(orc, k):
    # runtime/src/expert_kernel.rs:302-356, including the extreme quants
    state = [5]

    def nxt():
        s = state[0]
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        state[0] = s
        return s

    scales = [0.0, 0.01, -0.1, 0.00000006, 3.0]
    for it in range(0, 64):
        x = (np.sin((np.arange(k) + it) * 0.37) * (1 + np.arange(k) % 5)).astype(np.float32)
        xq = orc.quantize_q8_0(x)
        row = np.empty((k // QK, Q4B), np.uint8)
        for i in range(k // QK):
            row[i, :2] = np.frombuffer(struct.pack("<e", scales[(it + i) % 5]), np.uint8)
            row[i, 2:] = [nxt() & 0xFF for _ in range(16)]
        if it % 7 == 0:
            row[:, 2:] = 0
            xq.reshape(-1, Q8B)[:, 2:] = 0x81 if it % 2 == 0 else 0x7F
        row = row.reshape(-1)
        sums = orc.q4q8_block_sums(row, xq, k)
        assert np.array_equal(sums, _blocksums_np(row, xq, k))
        dw = row.reshape(-1, Q4B)[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
        dx = xq.reshape(-1, Q8B)[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
        vals, _ = _deq_np(row.reshape(1, -1), k)
        qx = xq.reshape(-1, Q8B)[:, 2:].view(np.int8).astype(np.int64)
        exact = float((sums * dw * dx).sum())
        mag = float((np.abs(vals[0] * qx).sum(axis=1) * np.abs(dw * dx)).sum())
        for v in (orc.dot_q8_scalar(row, xq, k), orc.dot_q8_avx2_order(row, xq, k)):
            assert abs(v - exact) <= 4e-6 * mag + 1e-30


def test_q8_dot_scalar_is_the_block_order_fold(orc):
    # The scalar dot is the sequential f32 fold of sumi * (dw * dx) in block order: equal to
    # numpy's float32 accumulate over the same per-block terms.
    rng = np.random.default_rng(9)
    k = 2816
    row = _q4_rows(rng, 1, k)[0]
    xq = orc.quantize_q8_0(rng.standard_normal(k).astype(np.float32))
    sums = orc.q4q8_block_sums(row, xq, k)
    dw = row.reshape(-1, Q4B)[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    dx = xq.reshape(-1, Q8B)[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    terms = sums.astype(np.float32) * (dw * dx)
    seq = np.add.accumulate(np.concatenate([[np.float32(0)], terms]).astype(np.float32))[-1]
    assert orc.dot_q8_scalar(row, xq, k) == seq


def test_q8_dot_tracks_f32_dot(orc):
    # runtime/src/expert_kernel.rs:358-382
    k = 2816
    x = (np.cos(np.arange(k) * 0.011) * 0.5).astype(np.float32)
    xq = orc.quantize_q8_0(x)
    row = np.empty((k // QK, Q4B), np.uint8)
    for i in range(k // QK):
        row[i, :2] = np.frombuffer(struct.pack("<e", 0.02), np.uint8)
        row[i, 2:] = [(i * 31 + j * 7) & 0xFF for j in range(16)]
    row = row.reshape(-1)
    ref = orc.dot_q4_0(row, x)
    deq = orc.dequant_q4_0(row, k)
    bound = sum(np.abs(deq[b * 32:(b + 1) * 32]).sum() * np.abs(x[b * 32:(b + 1) * 32]).max() / 127.0
                for b in range(k // QK))
    assert abs(orc.dot_q8_scalar(row, xq, k) - ref) <= bound


# ---------------- router, softmax, top-k, selection (ops.rs:131-187, exec.rs:493-517) ----------------

def test_matvec_is_a_sequential_f32_fold(orc):
    # tests/research/test_correctness_oracle.py:26 gives [1, 6] in binary64; the f32 sequential fold
    # loses the 1 against 1e16 (pairwise or wider sums would not).
    w = np.array([[1e16, 1, -1e16], [1, 2, 3]], np.float32)
    assert list(orc.matvec_f32(w, np.ones(3, np.float32))) == [0.0, 6.0]
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((16, 2816)) * 0.02).astype(np.float32)
    x = rng.standard_normal(2816).astype(np.float32)
    got = orc.matvec_f32(w, x)
    for r in range(16):
        prods = (w[r] * x).astype(np.float32)
        seq = np.add.accumulate(np.concatenate([[np.float32(-0.0)], prods]).astype(np.float32))[-1]
        assert got[r] == seq


def test_rms_norm_known_answers(orc):
    # runtime/src/ops.rs:407-410
    s = math.sqrt(12.5)
    got = orc.rms_norm(np.array([3, 4], np.float32), np.array([1, 2], np.float32), 0.0)
    assert abs(got[0] - 3 / s) < 1e-6 and abs(got[1] - 8 / s) < 1e-6
    # tests/research/test_correctness_oracle.py:91-93
    got = orc.rms_norm(np.array([3, 4], np.float32), np.array([2, -1], np.float32), 0.5)
    assert abs(got[0] - 6 / math.sqrt(13)) < 1e-6 and abs(got[1] + 4 / math.sqrt(13)) < 1e-6
    assert list(orc.rms_norm(np.zeros(2, np.float32), None, 1e-6)) == [0.0, 0.0]
    # research/fixtures/scalar-operators-v1.json "rms", criterion 1e-5 + 1e-4 |ref|
    x = np.array([1, -2, 3, -4], np.float64)
    w = np.array([0.25, 0.5, 1, 2], np.float64)
    ref = x / np.sqrt((x * x).mean() + 1e-6) * w
    got = orc.rms_norm(x.astype(np.float32), w.astype(np.float32), 1e-6)
    assert np.all(np.abs(got - ref) <= 1e-5 + 1e-4 * np.abs(ref))


def _gelu64(x):
    return 0.5 * x * (1 + math.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))


def test_gelu_fixture_and_limits(orc):
    # research/fixtures/scalar-operators-v1.json "gelu_tanh" inputs, criterion 1e-5 + 1e-4 |ref|
    for v in [-8, -4, -2, -1, -0.25, 0, 0.25, 1, 2, 4, 8, 16]:
        ref = _gelu64(v)
        assert abs(orc.gelu(v) - ref) <= 1e-5 + 1e-4 * abs(ref)
    assert orc.gelu(-10.0) == 0.0 or abs(orc.gelu(-10.0)) < 1e-20
    assert orc.gelu(10.0) == 10.0 and orc.gelu(0.0) == 0.0
    assert abs((orc.gelu(1.0) - orc.gelu(-1.0)) - 1.0) < 1e-6  # tests/research/test_correctness_oracle.py:159
    # gated FFN of the fixture: input [2,-1], up = I, gate = swap, down = [[3, 4]]
    gate, up = [-1.0, 2.0], [2.0, -1.0]
    h = [np.float32(orc.gelu(g)) * np.float32(u) for g, u in zip(gate, up)]
    out = 3 * float(h[0]) + 4 * float(h[1])
    assert abs(out - (6 * _gelu64(-1) - 4 * _gelu64(2))) < 1e-5


def test_softmax_fixture(orc):
    x = np.array([10000, 10001, 9999, -10000], np.float64)
    ref = np.exp(x - x.max()) / np.exp(x - x.max()).sum()
    got = orc.softmax(x.astype(np.float32))
    assert np.all(np.abs(got - ref) <= 1e-6)
    p = orc.softmax(np.array([1, 2, 3], np.float32))  # runtime/src/ops.rs:411-413
    assert abs(p.sum() - 1) < 1e-6 and p[2] > p[1]


def test_top_k_ties_and_total_order(orc):
    assert orc.top_k([0.1, 0.5, 0.5, 0.2], 3) == [1, 2, 3]  # runtime/src/ops.rs:414
    nan, neg_nan = float("nan"), -float("nan")
    # total_cmp: -NaN < -inf < ... < -0.0 < +0.0 < ... < +inf < +NaN
    x = np.array([0.0, -0.0, 1.0, nan, -np.inf, neg_nan, np.inf], np.float32)
    x[5] = np.array([0xFFC00000], np.uint32).view(np.float32)[0]
    assert orc.top_k(x, 7) == [3, 6, 2, 0, 1, 4, 5]


def test_select_experts_known_answers(orc):
    # tests/research/test_correctness_oracle.py:72-80: softmax [.2,.6,.2], top-2 = (1, 0) -> (.75, .25)
    ids, w, p = orc.select_experts(np.array([[0, math.log(3), 0]], np.float32), 2)
    assert list(ids[0]) == [1, 0]
    assert np.allclose(p[0], [0.2, 0.6, 0.2], atol=1e-7)
    assert np.allclose(w[0], [0.75, 0.25], atol=1e-7)
    # the 2^-14 clamp on the selected sum (exec.rs:124-125): 20000 equal logits give p = 5e-5
    ids, w, p = orc.select_experts(np.zeros((1, 20000), np.float32), 1)
    assert ids[0, 0] == 0
    assert abs(w[0, 0] - np.float32(p[0, 0]) / np.float32(6.103515625e-05)) <= 1e-7


# ---------------- plan (exec.rs:540-558) ----------------

def test_moe_plan_is_a_stable_sort(orc):
    rng = np.random.default_rng(4)
    for n_exp, pairs in [(4, 8), (128, 256), (128, 4096)]:
        ids = rng.zipf(1.3, pairs) % n_exp
        order, pos_of, gs = orc.moe_plan(ids, n_exp)
        want = np.argsort(ids, kind="stable")
        assert np.array_equal(order, want)
        assert np.array_equal(pos_of[order], np.arange(pairs))
        assert np.array_equal(gs, np.concatenate([[0], np.cumsum(np.bincount(ids, minlength=n_exp))]))


# ---------------- experts and the whole layer (exec.rs:572-640) ----------------

def _small_layer(rng, n_exp, d, ff):
    gu = {e: _q4_rows(rng, 2 * ff, d).reshape(-1) for e in range(n_exp)}
    dn = {e: _q4_rows(rng, d, ff).reshape(-1) for e in range(n_exp)}
    return gu, dn


def test_experts_q8_against_f64_pipeline(orc):
    rng = np.random.default_rng(8)
    n_exp, d, ff, used, n_tok = 4, 256, 64, 2, 3
    gu, dn = _small_layer(rng, n_exp, d, ff)
    x = rng.standard_normal((n_tok, d)).astype(np.float32)
    ids = np.array([[1, 3], [3, 0], [1, 2]], np.uint32)
    wts = np.array([[0.7, 0.3], [0.5, 0.5], [0.9, 0.1]], np.float32)
    ds = np.array([1.0, 0.5, 2.0, 1.25], np.float32)
    out, g, h, y = orc.experts_q8(gu, dn, ds, x, d, ff, ids, wts, n_exp, intermediates=True)
    order, pos_of, _ = orc.moe_plan(ids, n_exp)
    for k, pair in enumerate(order):
        t, e = pair // used, int(ids.reshape(-1)[pair])
        xq = orc.quantize_q8_0(x[t])
        vals, dw = _deq_np(gu[e].reshape(2 * ff, -1), d)
        q = xq.reshape(-1, Q8B)[:, 2:].view(np.int8).astype(np.float64)
        dx = xq.reshape(-1, Q8B)[:, :2].copy().view(np.float16).astype(np.float64).reshape(1, -1, 1)
        gu64 = (vals * dw * q[None] * dx).sum(axis=(1, 2))
        mag = (np.abs(vals * dw * q[None] * dx)).sum(axis=(1, 2))
        assert np.all(np.abs(g[k] - gu64) <= 4e-6 * mag + 1e-30)
        h64 = np.array([_gelu64(a) for a in g[k][:ff].astype(np.float64)]) * g[k][ff:]
        assert np.all(np.abs(h[k] - h64) <= 1e-5 * (1 + np.abs(h64)))
        hq = orc.quantize_q8_0(h[k])
        vals, dw = _deq_np(dn[e].reshape(d, -1), ff)
        q = hq.reshape(-1, Q8B)[:, 2:].view(np.int8).astype(np.float64)
        dx = hq.reshape(-1, Q8B)[:, :2].copy().view(np.float16).astype(np.float64).reshape(1, -1, 1)
        y64 = (vals * dw * q[None] * dx).sum(axis=(1, 2))
        mag = (np.abs(vals * dw * q[None] * dx)).sum(axis=(1, 2))
        assert np.all(np.abs(y[k] - y64) <= 4e-6 * mag + 1e-30)
    # slot-order combine, first term assigned, (y * scale) * weight: the expected values of the
    # reference's bitwise combine test (runtime/tests/hip_ops.rs:421-439)
    for t in range(n_tok):
        o = None
        for j in range(used):
            p = t * used + j
            v = y[pos_of[p]] * ds[ids[t, j]] * wts[t, j]
            o = v if o is None else (o + v).astype(np.float32)
        assert np.array_equal(out[t], o)


def test_experts_q8_batch_invariance(orc):
    # runtime/tests/exec.rs batch invariance and ops.rs:417-447 multi-segment == single
    rng = np.random.default_rng(12)
    n_exp, d, ff = 4, 256, 64
    gu, dn = _small_layer(rng, n_exp, d, ff)
    x = rng.standard_normal((3, d)).astype(np.float32)
    ids = np.array([[0, 2], [2, 1], [0, 1]], np.uint32)
    wts = np.array([[0.6, 0.4], [0.5, 0.5], [0.2, 0.8]], np.float32)
    all3 = orc.experts_q8(gu, dn, None, x, d, ff, ids, wts, n_exp)
    for t in range(3):
        one = orc.experts_q8(gu, dn, None, x[t:t + 1], d, ff, ids[t:t + 1], wts[t:t + 1], n_exp)
        assert np.array_equal(one[0], all3[t])


def test_moe_layer_composes_router_selection_and_experts(orc):
    rng = np.random.default_rng(13)
    n_exp, d, ff, used = 4, 256, 64, 2
    gu, dn = _small_layer(rng, n_exp, d, ff)
    w_r = (rng.standard_normal((n_exp, d)) * 0.02).astype(np.float32)
    bias = rng.standard_normal(n_exp).astype(np.float32)
    x = rng.standard_normal((2, d)).astype(np.float32)
    for pre in (False, True):
        ids, w, out = orc.moe_layer(w_r, bias, gu, dn, None, x, n_exp, d, ff, used, pre_norm=pre)
        xin = np.stack([orc.rms_norm(r, None, 1e-6) for r in x]) if pre else x
        lg = orc.router_logits(w_r, bias, xin, n_exp, d)
        ids2, w2, _ = orc.select_experts(lg, used)
        assert np.array_equal(ids, ids2) and np.array_equal(w, w2)
        assert np.array_equal(out, orc.experts_q8(gu, dn, None, xin, d, ff, ids2, w2, n_exp))


def test_cpu_baseline_matches_oracle(orc):
    rng = np.random.default_rng(14)
    n_exp, d, ff, used = 8, 512, 128, 4
    gu, dn = _small_layer(rng, n_exp, d, ff)
    w_r = (rng.standard_normal((n_exp, d)) * 0.02).astype(np.float32)
    x = rng.standard_normal((5, d)).astype(np.float32)
    ids, w, out = orc.moe_layer(w_r, None, gu, dn, None, x, n_exp, d, ff, used)
    cpb = orc.CpuBaseline(3)
    cpb.prepare(gu, dn, n_exp)
    ids2, w2, out2 = cpb.layer(w_r, None, None, x, d, ff, used)
    cpb.close()
    assert np.array_equal(ids, ids2) and np.array_equal(w, w2)
    rms = float(np.sqrt((out.astype(np.float64) ** 2).mean()))
    assert np.max(np.abs(out2 - out)) <= 1e-5 * rms
