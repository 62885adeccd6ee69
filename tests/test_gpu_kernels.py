"""Per-stage parity of the HIP kernels against the CPU oracle (GPU).

The stages follow the reference's conformance tests (runtime/tests/hip_ops.rs:56-81, 402-443) and
the build's rules: Q8_0 bytes and per-block int32 Q4xQ8 sums are bit-exact when both sides see
the same inputs; f32 results agree within 1e-3 of the reference output's RMS (and within the
reference's own per-row summation bound 4e-6 * sum|w x| * d, expert_kernel.rs:346-348).
"""
import numpy as np
import pytest

from rosevine_amd import hip
from rosevine_amd.hip import DevBuf

pytestmark = pytest.mark.gpu

QK, Q4B, Q8B = 32, 18, 34


def dev(a):
    return DevBuf.from_array(np.ascontiguousarray(a))


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def pack_np(rows, n_out, k, fmt):
    """numpy statement of the packed layout in include/rvmoe.h (index arithmetic only)."""
    nb = k // QK
    blk = rows.reshape(n_out, nb, Q4B)
    if fmt == hip.PACK_GATE_UP:
        T, S = n_out // 64, nb
        t, s, l = np.meshgrid(np.arange(T), np.arange(S), np.arange(64), indexing="ij")
        row = np.where(l < 32, 32 * t + l, n_out // 2 + 32 * t + (l - 32))
        b = s
    else:
        T, S = n_out // 32, nb // 2
        t, s, l = np.meshgrid(np.arange(T), np.arange(S), np.arange(64), indexing="ij")
        row = 32 * t + (l & 31)
        b = (l >> 5) * S + s
    sel = blk[row, b]  # [T, S, 64, 18]
    nib = (sel[..., 2:] ^ 0x88).reshape(-1)
    scl = sel[..., :2].reshape(-1)
    return np.concatenate([nib, scl])


def rand_q4(rng, n_out, k, lo=0.005, hi=0.02):
    nb = k // QK
    out = np.empty((n_out, nb, Q4B), np.uint8)
    d = rng.uniform(lo, hi, (n_out, nb)).astype(np.float16)
    out[:, :, :2] = d.reshape(n_out, nb, 1).view(np.uint8).reshape(n_out, nb, 2)
    out[:, :, 2:] = rng.integers(0, 256, (n_out, nb, 16), dtype=np.uint8)
    return out.reshape(-1)


def packed(rows, n_out, k, fmt):
    src = dev(rows)
    dst = DevBuf(rows.nbytes)
    hip.pack_q4(src, dst, 1, n_out, k, fmt)
    return dst


def test_synth_device_matches_host(gpu):
    for n_mat, n_out, k in [(2, 64, 256), (1, 1408, 2816), (3, 2816, 704)]:
        n = n_mat * n_out * (k // QK) * Q4B
        buf = DevBuf(n)
        hip.synth_q4(buf, n_mat, n_out, k, 3, 77)
        assert np.array_equal(buf.download(np.uint8, n), hip.synth_q4_host(n_mat, n_out, k, 3, 77))


@pytest.mark.parametrize("fmt,n_out,k", [(hip.PACK_GATE_UP, 1408, 2816), (hip.PACK_ROWS32, 2816, 704),
                                         (hip.PACK_GATE_UP, 128, 256), (hip.PACK_ROWS32, 64, 64)])
def test_pack_layout(gpu, fmt, n_out, k):
    rows = rand_q4(np.random.default_rng(n_out + k), n_out, k)
    dst = packed(rows, n_out, k, fmt)
    assert np.array_equal(dst.download(np.uint8, rows.size), pack_np(rows, n_out, k, fmt))


def test_quantize_q8_0_bitexact(gpu, orc):
    rng = np.random.default_rng(21)
    rows, k = 7, 2816
    x = (rng.standard_normal((rows, k)) * rng.uniform(1e-6, 1e4, (rows, 1))).astype(np.float32)
    x[0, :32] = 0.0                                    # zero block
    x[1, :32] = 0.0
    x[1, 0] = 127.0
    x[1, 1:9] = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5]  # exact ties
    x[2, 5] = np.nan                                   # NaN ignored by amax, quantised to 0
    x[3, 40] = np.inf                                  # d = inf
    x[4, 64:96] = rng.standard_normal(32) * 1e-40      # subnormal inputs, subnormal f16 scale
    x[5, 96:128] = rng.standard_normal(32) * 3e7       # f16 scale overflow to inf
    xd, q = dev(x), DevBuf(rows * (k // QK) * Q8B)
    hip.quantize_q8_0(xd, q, rows, k)
    got = q.download(np.uint8, rows * (k // QK) * Q8B).reshape(rows, -1)
    for r in range(rows):
        assert np.array_equal(got[r], orc.quantize_q8_0(x[r])), r


@pytest.mark.parametrize("fmt,n_out,k", [(hip.PACK_GATE_UP, 1408, 2816), (hip.PACK_ROWS32, 2816, 704)])
def test_block_sums_bitexact(gpu, orc, fmt, n_out, k):
    rng = np.random.default_rng(k)
    rows = rand_q4(rng, n_out, k)
    xq = orc.quantize_q8_0(rng.standard_normal(k).astype(np.float32) * 3)
    # extremes: every weight -8 against activations of +-127 (runtime/src/expert_kernel.rs:322-326)
    rows2 = rows.copy().reshape(n_out, -1, Q4B)
    rows2[:, :, 2:] = 0
    xq2 = xq.copy().reshape(-1, Q8B)
    xq2[::2, 2:] = 0x81
    xq2[1::2, 2:] = 0x7F
    for w_rows, a in ((rows, xq), (rows2.reshape(-1), xq2.reshape(-1))):
        wd = packed(w_rows, n_out, k, fmt)
        sums = DevBuf(n_out * (k // QK) * 4)
        hip.q4q8_block_sums(wd, fmt, dev(a), sums, n_out, k)
        got = sums.download(np.int32, n_out * (k // QK)).reshape(n_out, -1)
        rb = w_rows.reshape(n_out, -1)
        want = np.stack([orc.q4q8_block_sums(rb[r], a, k) for r in range(n_out)])
        assert np.array_equal(got, want)


@pytest.mark.parametrize("fmt,n_out,k", [(hip.PACK_GATE_UP, 1408, 2816), (hip.PACK_ROWS32, 2816, 704),
                                         (hip.PACK_GATE_UP, 128, 256)])
def test_q4q8_mm_matches_oracle_and_is_batch_invariant(gpu, orc, fmt, n_out, k):
    rng = np.random.default_rng(n_out * 7 + k)
    rows = rand_q4(rng, n_out, k)
    wd = packed(rows, n_out, k, fmt)
    n_in = 8
    x = rng.standard_normal((n_in, k)).astype(np.float32)
    xq = np.concatenate([orc.quantize_q8_0(x[t]) for t in range(n_in)])
    y = DevBuf(n_in * n_out * 4)
    hip.q4q8_mm(wd, fmt, dev(xq), y, n_out, k, n_in)
    got = y.download(np.float32, n_in * n_out).reshape(n_in, n_out)
    rb = rows.reshape(n_out, -1)
    qb = xq.reshape(n_in, -1)
    want = np.array([[orc.dot_q8_scalar(rb[r], qb[t], k) for r in range(n_out)] for t in range(n_in)], np.float32)
    # the same block terms folded in the same order: bit-exact (and so within any tolerance)
    assert np.array_equal(got, want)
    y1 = DevBuf(n_out * 4)
    hip.q4q8_mm(wd, fmt, dev(qb[n_in - 1]), y1, n_out, k, 1)
    assert np.array_equal(y1.download(np.float32, n_out), got[n_in - 1])


def test_geglu_q8_0_bitexact(gpu, orc):
    rng = np.random.default_rng(31)
    rows, ff = 24, 704
    gu = (rng.standard_normal((rows, 2 * ff)) * 2).astype(np.float32)
    gu[0, :64] = np.linspace(-30, 30, 64)           # tanh saturation and both signs
    gu[1, :32] = rng.standard_normal(32) * 1e-30    # tiny gate values
    hq = DevBuf(rows * (ff // QK) * Q8B)
    hip.geglu_q8_0(dev(gu), hq, rows, ff)
    got = hq.download(np.uint8, rows * (ff // QK) * Q8B).reshape(rows, -1)
    h = orc.geglu_split(gu, ff)
    for r in range(rows):
        assert np.array_equal(got[r], orc.quantize_q8_0(h[r])), r


def test_gelu_matches_the_host_libm_bitwise(gpu, orc):
    """rvh_geglu_split over 4M gate values spanning the float range: the device tanhf equals the
    host C library's (the reference's f32::tanh) on every one."""
    rng = np.random.default_rng(32)
    n = 1 << 22
    bits = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    g = bits.view(np.float32).copy()
    g[: n // 2] = (rng.standard_normal(n // 2) * 4).astype(np.float32)  # the range GELU sees
    g[~np.isfinite(g)] = 1.0
    ff = 1 << 11
    gu = np.concatenate([g.reshape(-1, ff), np.ones((n // ff, ff), np.float32)], axis=1)
    out = DevBuf(n * 4)
    hip.geglu_split(dev(gu), out, n // ff, ff)
    got = out.download(np.float32, n).reshape(-1, ff)
    want = orc.geglu_split(gu, ff)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), np.argwhere(~same)[:5]


def test_reference_ops(gpu, orc):
    rng = np.random.default_rng(41)
    # rvh_q4_mm against ops::matmul_q4_0 (runtime/tests/hip_ops.rs:56-81): rel L2 < 1e-5, batch invariance
    # shapes of the reference model's projections (contract.rs:41-62: q/k/v, output, dense FFN),
    # block-column counts 1 .. 4, k past one column group (9216), rows not a multiple of 4, and
    # 1, 2, 4 and 8 rows per wave; one token runs a one-token kernel, bitwise the batched one
    for n_out, k, tokens in [(1408, 2816, [1, 7]), (2816, 704, [1, 7]), (2048, 2816, [1, 9]),
                             (2816, 2112, [1, 3]), (1001, 8192, [1, 2]), (300, 9216, [1, 8]),
                             (4100, 256, [1, 2]), (9000, 256, [1, 9]), (16387, 256, [1, 3])]:
        for n_in in tokens:
            w = rand_q4(rng, n_out, k, 0.01, 0.03)
            x = rng.uniform(-1, 1, (n_in, k)).astype(np.float32)
            want = orc.matmul_q4_0(w, k, x, n_in, n_out)
            y = DevBuf(n_in * n_out * 4)
            wd = dev(w)
            hip.q4_mm(wd, dev(x), y, n_out, k, n_in)
            got = y.download(np.float32, n_in * n_out).reshape(n_in, n_out)
            rel = np.sqrt(((got - want).astype(np.float64) ** 2).sum() / (want.astype(np.float64) ** 2).sum())
            assert rel < 1e-5
            if n_in > 1:
                y1 = DevBuf(n_out * 4)
                hip.q4_mm(wd, dev(x[-1]), y1, n_out, k, 1)
                assert np.array_equal(y1.download(np.float32, n_out), got[-1])
            # rvh_q4_mv: the same result up to summation order (rvhip.h:46-48)
            ymv = DevBuf(n_in * n_out * 4)
            hip.q4_mv(wd, dev(x), ymv, n_out, k, n_in)
            got_mv = ymv.download(np.float32, n_in * n_out).reshape(n_in, n_out)
            rel = np.sqrt(((got_mv - want).astype(np.float64) ** 2).sum() / (want.astype(np.float64) ** 2).sum())
            assert rel < 1e-5
    # rvh_geglu_split rel < 1e-6 and rvh_moe_combine bitwise (runtime/tests/hip_ops.rs:402-439)
    e, fe, used, n = 2816, 704, 8, 3
    pairs = n * used
    gu = rng.uniform(-2, 2, (pairs, 2 * fe)).astype(np.float32)
    want_h = orc.geglu_split(gu, fe)
    h = DevBuf(pairs * fe * 4)
    hip.geglu_split(dev(gu), h, pairs, fe)
    got_h = h.download(np.float32, pairs * fe).reshape(pairs, fe)
    assert np.array_equal(got_h, want_h)  # the reference asks rel < 1e-6; the libm restatement is exact
    y = rng.uniform(-1, 1, (pairs, e)).astype(np.float32)
    pos = np.arange(pairs, dtype=np.int32)[::-1].copy()
    scale = rng.uniform(-1, 1, pairs).astype(np.float32)
    weight = rng.uniform(-1, 1, pairs).astype(np.float32)
    want = np.zeros((n, e), np.float32)
    for t in range(n):
        for j in range(used):
            p = t * used + j
            c = (y[pos[p]] * scale[p]) * weight[p]
            want[t] = c if j == 0 else want[t] + c
    out = DevBuf(n * e * 4)
    hip.moe_combine(dev(y), pairs, dev(pos), dev(scale), dev(weight), out, n, used, e)
    assert np.array_equal(out.download(np.float32, n * e).reshape(n, e), want)
    # rvh_rms_norm, rvh_f32_mm, rvh_gather_rows
    xr = rng.standard_normal((3, e)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, e).astype(np.float32)
    o = DevBuf(3 * e * 4)
    hip.rms_norm(dev(xr), o, dev(g), 3, e, 1e-6, 0.5)
    got = o.download(np.float32, 3 * e).reshape(3, e)
    for t in range(3):
        assert np.max(np.abs(got[t] - orc.rms_norm(xr[t], g, 1e-6, 0.5))) <= 2e-6 * np.abs(got[t]).max()
    wr = (rng.standard_normal((128, e)) * 0.02).astype(np.float32)
    lg = DevBuf(3 * 128 * 4)
    hip.f32_mm(dev(wr), dev(xr), lg, 128, e, 3)
    got = lg.download(np.float32, 3 * 128).reshape(3, 128)
    for t in range(3):
        assert np.max(np.abs(got[t] - orc.matvec_f32(wr, xr[t]))) <= 1e-5
    idx = np.array([2, 0, 2, 1], np.int32)
    dst = DevBuf(4 * e * 4)
    hip.gather_rows(dev(xr), 3, dev(idx), dst, 4, e)
    assert np.array_equal(dst.download(np.float32, 4 * e).reshape(4, e), xr[idx])


def test_out_of_range_calls_are_refused(gpu):
    small = DevBuf(64)
    with pytest.raises(hip.BoundsError):
        hip.q4_mm(small, small, small, 1 << 20, 2816, 1)
    with pytest.raises(hip.DeviceError) as e:
        hip.check(hip.lib().rvm_q4q8_mm(small.ptr, 9, small.ptr, small.ptr, 64, 64, 1))
    assert e.value.code == 1


def dequant_q4(w, n_out, k):
    """[n_out][k] f32 weights (n - 8) * d of Q4_0 rows (runtime/src/ops.rs:83-92; exact in f32)."""
    blk = w.reshape(n_out, k // QK, Q4B)
    d = blk[:, :, :2].copy().view(np.float16).astype(np.float32)  # [n_out, nb, 1]
    q = blk[:, :, 2:]
    n = np.concatenate([q & 0xF, q >> 4], axis=2).astype(np.float32) - 8.0  # elements j, then 16 + j
    return (n * d).reshape(n_out, k)


@pytest.mark.parametrize("n_out,k", [
    (16389, 2816),   # the output head's width (contract.rs:41-62), rows past a 64-row workgroup
    (16400, 4096),   # two steps' worth of blocks per K group more
    (16384, 2112),   # 66 blocks: a last step with two live K groups
    (16390, 8192),   # the largest k of this path
    (16387, 2080),   # 65 blocks: rows not on a dword boundary (the unaligned loads)
    (20000, 96),     # 3 blocks
])
def test_q4_mm_many_rows_matches_oracle(gpu, orc, n_out, k):
    """rvh_q4_mm from 16384 rows (int8 digits of x on the matrix cores) against ops::matmul_q4_0
    (runtime/tests/hip_ops.rs:56-81): rel L2 < 1e-5 and batch invariance; the same matrix 2 bytes
    past a dword boundary (the unaligned loads) gives the same bits."""
    rng = np.random.default_rng(n_out + k)
    w = rand_q4(rng, n_out, k, 0.01, 0.03)
    x = rng.uniform(-1, 1, (3, k)).astype(np.float32)
    want = orc.matmul_q4_0(w, k, x, 3, n_out)
    wd, xd, y = dev(w), dev(x), DevBuf(3 * n_out * 4)
    hip.q4_mm(wd, xd, y, n_out, k, 3)
    got = y.download(np.float32, 3 * n_out).reshape(3, n_out)
    rel = np.sqrt(((got - want).astype(np.float64) ** 2).sum() / (want.astype(np.float64) ** 2).sum())
    assert rel < 1e-5, rel
    y1 = DevBuf(n_out * 4)
    hip.q4_mm(wd, dev(x[2]), y1, n_out, k, 1)
    assert np.array_equal(y1.download(np.float32, n_out), got[2])
    off = DevBuf(w.nbytes + 2)
    off.upload(w, 2)
    y2 = DevBuf(n_out * 4)
    hip.check(hip.lib().rvh_q4_mm(off.at(2, w.nbytes), xd.at(2 * k * 4, k * 4), y2.at(0, n_out * 4), n_out, k, 1))
    assert np.array_equal(y2.download(np.float32, n_out), got[2])


@pytest.mark.parametrize("n_out,k", [(2048, 2816), (2816, 2112), (1000, 4096), (300, 704), (4100, 256)])
def test_q4_mm_unaligned_matrix_gives_the_same_bits(gpu, n_out, k):
    """rvh_q4_mm under 16384 rows: the matrix 2 bytes past a dword boundary (2-byte-aligned loads)
    gives the bits of the aligned copy (dword-aligned loads and byte permutes), 1 and 3 tokens."""
    rng = np.random.default_rng(n_out + 7 * k)
    w = rand_q4(rng, n_out, k, 0.01, 0.03)
    wd = dev(w)
    off = DevBuf(w.nbytes + 2)
    off.upload(w, 2)
    for n_in in (1, 3):
        x = dev(rng.uniform(-1, 1, (n_in, k)).astype(np.float32))
        ya, yb = DevBuf(n_in * n_out * 4), DevBuf(n_in * n_out * 4)
        hip.q4_mm(wd, x, ya, n_out, k, n_in)
        hip.check(hip.lib().rvh_q4_mm(off.at(2, w.nbytes), x.at(0, n_in * k * 4), yb.at(0, n_in * n_out * 4), n_out,
                                      k, n_in))
        assert np.array_equal(ya.download(np.float32, n_in * n_out), yb.download(np.float32, n_in * n_out))


def test_q4_mm_many_rows_shape_sweep(gpu, orc):
    """rvh_q4_mm from 16384 rows on seeded shapes (k of 1 to 256 blocks, odd and even block counts,
    rows not a multiple of the 128-row workgroup, 1 to 4 tokens) against ops::matmul_q4_0 within
    relative L2 1e-5, and each token's row against its one-token call bit for bit."""
    rng = np.random.default_rng(2026)
    for _ in range(6):
        n_out = int(rng.integers(16384, 20000))
        k = 32 * int(rng.integers(1, 257))
        n_in = int(rng.integers(1, 5))
        w = rand_q4(rng, n_out, k, 0.005, 0.05)
        x = (rng.standard_normal((n_in, k)) * rng.uniform(0.1, 3.0)).astype(np.float32)
        want = orc.matmul_q4_0(w, k, x, n_in, n_out)
        wd, y = dev(w), DevBuf(n_in * n_out * 4)
        hip.q4_mm(wd, dev(x), y, n_out, k, n_in)
        got = y.download(np.float32, n_in * n_out).reshape(n_in, n_out)
        rel = np.sqrt(((got - want).astype(np.float64) ** 2).sum() / (want.astype(np.float64) ** 2).sum())
        assert rel < 1e-5, (n_out, k, n_in, rel)
        y1 = DevBuf(n_out * 4)
        hip.q4_mm(wd, dev(x[n_in - 1]), y1, n_out, k, 1)
        assert np.array_equal(y1.download(np.float32, n_out), got[n_in - 1]), (n_out, k, n_in)


def test_q4_mm_many_rows_activation_edge_cases(gpu):
    """The int8 digits of x across a block's range: zero and subnormal blocks, one large element
    among tiny ones, values near 1e30, and a spread of 12 decades; each row within the reference's
    summation bound 4e-6 sum|w x| of the exact product (expert_kernel.rs:346-348). (An element
    below 2^-4 of its block's largest is held to 2^-28 of that largest.) A non-finite activation
    makes every row NaN."""
    n_out, k = 16384, 2816
    rng = np.random.default_rng(77)
    w = rand_q4(rng, n_out, k, 0.01, 0.03)
    x = rng.uniform(-1, 1, (3, k)).astype(np.float32)
    x[0, 0:32] = 0.0
    x[0, 32:64] = rng.uniform(-1, 1, 32) * np.float32(1e-40)   # subnormal
    x[0, 64:96] = rng.uniform(-1, 1, 32) * np.float32(1e-20)
    x[0, 70] = 1e3                                              # one large element among tiny ones
    x[0, 96:128] = rng.uniform(-1, 1, 32) * np.float32(1e30)
    x[0, 128:160] = -0.0
    x[1] = (rng.uniform(-1, 1, k) * 10.0 ** rng.uniform(-6, 6, k)).astype(np.float32)
    x[2, 5 * 32 + 7] = np.inf
    wf = dequant_q4(w, n_out, k).astype(np.float64)
    y = DevBuf(3 * n_out * 4)
    hip.q4_mm(dev(w), dev(x), y, n_out, k, 3)
    got = y.download(np.float32, 3 * n_out).reshape(3, n_out)
    for t in range(2):
        xt = x[t].astype(np.float64)
        exact = wf @ xt
        bound = 4e-6 * (np.abs(wf) @ np.abs(xt)) + 1e-37
        err = np.abs(got[t].astype(np.float64) - exact)
        assert (err <= bound).all(), (t, np.argmax(err - bound), float(np.max(err / bound)))
    assert np.isnan(got[2]).all()


def test_q4_mm_n_with_a_many_row_matrix(gpu):
    """rvm_q4_mm_n with a matrix of 16384+ rows among smaller ones: each output is rvh_q4_mm's."""
    rows, k = (2048, 16400, 1000), 2816
    rng = np.random.default_rng(5)
    ws = [hip.DevBuf(r * (k // 32) * 18) for r in rows]
    for i, (w, r) in enumerate(zip(ws, rows)):
        hip.synth_q4(w, 1, r, k, 9, 70 + i)
    for n_in in (1, 2):
        x = dev((rng.standard_normal((n_in, k)) * 0.5).astype(np.float32))
        ys = [hip.DevBuf(n_in * r * 4) for r in rows]
        hip.q4_mm_n(ws, x, ys, list(rows), k, n_in)
        for w, yb, r in zip(ws, ys, rows):
            y1 = hip.DevBuf(n_in * r * 4)
            hip.q4_mm(w, x, y1, r, k, n_in)
            assert np.array_equal(yb.download(np.float32, n_in * r), y1.download(np.float32, n_in * r)), (r, n_in)


@pytest.mark.parametrize("rows,k", [
    ((4096, 2048, 2048), 2816),   # q, k, v of a sliding-window layer (contract.rs:41-62)
    ((2112, 2112), 2816),         # gate and up
    ((5, 33, 64, 130), 96),       # four matrices, row counts that split workgroups, a short k
    ((1000,), 4096),              # one matrix
])
def test_q4_mm_n_equals_one_call_per_matrix(gpu, rows, k):
    """rvm_q4_mm_n: each matrix's output is rvh_q4_mm's, bit for bit, for one and for three tokens."""
    rng = np.random.default_rng(sum(rows) + k)
    ws = [hip.DevBuf(r * (k // 32) * 18) for r in rows]
    for i, (w, r) in enumerate(zip(ws, rows)):
        hip.synth_q4(w, 1, r, k, 7, 50 + i)
    for n_in in (1, 3):
        x = dev((rng.standard_normal((n_in, k)) * 0.5).astype(np.float32))
        ys = [hip.DevBuf(n_in * r * 4) for r in rows]
        hip.q4_mm_n(ws, x, ys, list(rows), k, n_in)
        for w, y, r in zip(ws, ys, rows):
            y1 = hip.DevBuf(n_in * r * 4)
            hip.q4_mm(w, x, y1, r, k, n_in)
            assert np.array_equal(y.download(np.float32, n_in * r), y1.download(np.float32, n_in * r)), (rows, r, n_in)
