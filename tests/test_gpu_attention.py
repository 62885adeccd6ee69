"""Decode attention on the GPU against the CPU oracle (runtime/tests/hip_ops.rs:228-400 cases).

Key/value quantisation is bit-exact (it is elementwise); attention agrees with the oracle's CPU
attention (hip_ops.rs:245-271) within the reference's relative L2 bound of 1e-5, and with exact
f64 attention over the same caches at depth. Ranges beyond the ring are rejected.
"""
import numpy as np
import pytest

from rosevine_amd import hip
from rosevine_amd.hip import DevBuf, DeviceError

pytestmark = pytest.mark.gpu

QK, Q8B = 32, 34


def dev(a):
    return DevBuf.from_array(np.ascontiguousarray(a))


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(np.sqrt(((a - b) ** 2).sum() / max((b ** 2).sum(), 1e-300)))


def q8_ring(orc, rng, cap, nkv, hd, scale=1.0):
    """A ring whose every slot holds a quantised random row (the latest position of that slot)."""
    k = (rng.standard_normal(cap * nkv * hd) * scale).astype(np.float32)
    v = (rng.standard_normal(cap * nkv * hd) * scale).astype(np.float32)
    return orc.quantize_q8_0(k), orc.quantize_q8_0(v)


def run_split(q, kc, vc, n_tok, nh, nkv, hd, p0, cap, win):
    dq, dk, dv = dev(q), dev(kc), dev(vc)
    out = DevBuf(n_tok * nh * hd * 4)
    part = DevBuf(hip.attention_split_scratch(n_tok, nh, hd) * 4)
    chunks = hip.attention_split(dq, dk, dv, out, part, n_tok, nh, nkv, hd, p0, cap, win)
    return chunks, out.download(np.float32, n_tok * nh * hd).reshape(n_tok, nh, hd)


def run_attention(q, kc, vc, n_tok, nh, nkv, hd, p0, cap, win):
    out = DevBuf(n_tok * nh * hd * 4)
    scores = DevBuf(n_tok * nh * cap * 4)
    hip.attention(dev(q), dev(kc), dev(vc), out, scores, n_tok, nh, nkv, hd, p0, cap, win, cap)
    return out.download(np.float32, n_tok * nh * hd).reshape(n_tok, nh, hd)


def test_kv_store_and_attention_match_cpu_across_the_ring(gpu, orc):
    # runtime/tests/hip_ops.rs:328-400 with its inputs (its generator, seed 3): a sliding window
    # of 1024 in a ring of 1028 that wraps, written 4 tokens at a time
    r = orc.TestRng(3)
    nh, nkv, hd, win = 16, 8, 256, 1024
    cap, total, n = win + 4, 1030, 4
    row = hd // QK * Q8B
    kv = r.vec(total * nkv * hd, 1.0).reshape(total, nkv, hd)
    vv = r.vec(total * nkv * hd, 1.0).reshape(total, nkv, hd)
    kc = np.zeros(cap * nkv * row, np.uint8)
    vc = np.zeros(cap * nkv * row, np.uint8)
    dk, dvv = dev(kv), dev(vv)
    dkc, dvc = dev(kc), dev(vc)
    q = r.vec(n * nh * hd, 0.2)
    p0 = 0
    while p0 < total:
        m = min(n, total - p0)
        for t in range(m):
            o = ((p0 + t) % cap) * nkv * row
            kc[o:o + nkv * row] = orc.quantize_q8_0(kv[p0 + t])
            vc[o:o + nkv * row] = orc.quantize_q8_0(vv[p0 + t])
        hip.kv_store(dk, dvv, dkc, dvc, m, nkv, hd, p0, cap, k_off=p0 * nkv * hd * 4, v_off=p0 * nkv * hd * 4)
        p0 += m
    # quantisation is elementwise and must be bitwise identical
    assert np.array_equal(dkc.download(np.uint8, kc.size), kc)
    assert np.array_equal(dvc.download(np.uint8, vc.size), vc)

    p0 = total - n
    want = orc.attention(q, kc, vc, nh, nkv, hd, cap, win, p0, n)
    out = DevBuf(n * nh * hd * 4)
    scores = DevBuf(n * nh * cap * 4)
    hip.attention(dev(q), dkc, dvc, out, scores, n, nh, nkv, hd, p0, cap, win, cap)
    assert rel(out.download(np.float32, want.size), want) < 1e-5
    # a key range beyond the ring is rejected rather than read
    with pytest.raises(DeviceError):
        hip.attention(dev(q), dkc, dvc, out, scores, n, nh, nkv, hd, p0, cap, 0, cap)


def test_split_attention_matches_cpu_and_the_one_chunk_kernel(gpu, orc):
    # runtime/tests/hip_ops.rs:273-326, case by case with its inputs (its generator, seed 5):
    # (name, heads, kv heads, head dim, window, ring capacity, filled positions, queries, chunks)
    r = orc.TestRng(5)
    cases = [
        ("local ring wrap", 16, 8, 256, 1024, 1028, 1030, 4, 16),
        ("global decode", 16, 2, 512, 0, 5000, 5000, 1, 64),
        ("global batch of 8", 16, 2, 512, 0, 5000, 5000, 8, 8),
        ("global prefill microbatch", 16, 2, 512, 0, 5000, 5000, 64, 1),
        ("short context", 16, 2, 512, 0, 100, 3, 1, 1),
        ("ragged chunks", 16, 2, 512, 0, 200, 129, 1, 3),
    ]
    for name, nh, nkv, hd, win, cap, total, n, chunks in cases:
        print(f"[attn] {name}", flush=True)
        kc, vc = orc.test_q8_caches(r, total, cap, nkv, hd)
        q = r.vec(n * nh * hd, 0.2)
        p0 = total - n
        want = orc.attention(q, kc, vc, nh, nkv, hd, cap, win, p0, n)
        c, got = run_split(q, kc, vc, n, nh, nkv, hd, p0, cap, win)
        assert c == chunks, name
        assert rel(got, want) < 1e-5, name
        one = run_attention(q, kc, vc, n, nh, nkv, hd, p0, cap, win)
        assert rel(got, one) < 1e-5, name
        assert rel(one, want) < 1e-5, name


def test_split_attention_rejects_ranges_beyond_the_ring(gpu):
    nh, nkv, hd, cap = 16, 8, 256, 64
    row = hd // QK * Q8B
    dq = dev(np.zeros(nh * hd, np.float32))
    kc, vc = dev(np.zeros(cap * nkv * row, np.uint8)), dev(np.zeros(cap * nkv * row, np.uint8))
    out = DevBuf(nh * hd * 4)
    part = DevBuf(hip.attention_split_scratch(1, nh, hd) * 4)
    with pytest.raises(DeviceError):
        hip.attention_split(dq, kc, vc, out, part, 1, nh, nkv, hd, cap, cap, 0)
    # a window that fits the ring is accepted at the same position
    hip.attention_split(dq, kc, vc, out, part, 1, nh, nkv, hd, cap, cap, cap)
    hip.sync()


@pytest.mark.parametrize("nh,nkv,hd,win,cap,total,n,n_chunks", [
    (12, 4, 64, 0, 300, 300, 3, 5),      # 3 query heads per kv head: one head per workgroup
    (6, 1, 96, 50, 64, 200, 2, 1),       # 6 per kv head (2 per workgroup), hd not a multiple of 64
    (32, 2, 128, 0, 700, 650, 1, 7),     # 16 per kv head
    (8, 8, 32, 0, 90, 90, 5, 4),         # one block per head: waves 1-3 score nothing
    (16, 2, 288, 0, 130, 130, 2, 9),     # two dimension groups, the second partly used
    (16, 4, 384, 33, 40, 1000, 3, 3),    # window, wrapped ring
    (4, 2, 160, 0, 20, 20, 1, 50),       # more chunks than keys: empty chunks merge to nothing
    (8, 2, 512, 0, 1, 1, 1, 1),          # one key: the value row itself
    (16, 2, 512, 0, 5000, 5000, 1, 200),  # 129 .. 320 chunks: the eight-wave merge
    (8, 2, 256, 0, 2600, 2600, 1, 320),  # its largest count
    (4, 2, 64, 0, 150, 150, 1, 250),     # there, with 100 empty chunks
    (4, 2, 64, 0, 400, 400, 1, 321),     # past it: the batched merge
])
def test_split_attention_shapes_and_chunkings(gpu, orc, nh, nkv, hd, win, cap, total, n, n_chunks):
    print(f"[attn] shape {nh}/{nkv}/{hd} win {win} cap {cap} total {total} n {n} chunks {n_chunks}", flush=True)
    rng = np.random.default_rng(nh * 1000 + hd)
    kc, vc = q8_ring(orc, rng, cap, nkv, hd)
    q = (rng.standard_normal(n * nh * hd) * 0.3).astype(np.float32)
    p0 = total - n
    want = orc.attention(q, kc, vc, nh, nkv, hd, cap, win, p0, n)
    dq, dk, dv = dev(q), dev(kc), dev(vc)
    out = DevBuf(n * nh * hd * 4)
    part = DevBuf(n * nh * n_chunks * (hd + 2) * 4)
    hip.attn_split(dq, dk, dv, out, part, n, nh, nkv, hd, p0, cap, win, n_chunks)
    if n_chunks > 1:
        hip.attn_combine(part, out, n * nh, hd, n_chunks)
    got = out.download(np.float32, want.size).reshape(want.shape)
    assert rel(got, want) < 1e-5
    # the same call again gives the same bits
    hip.attn_split(dq, dk, dv, out, part, n, nh, nkv, hd, p0, cap, win, n_chunks)
    if n_chunks > 1:
        hip.attn_combine(part, out, n * nh, hd, n_chunks)
    assert np.array_equal(out.download(np.float32, want.size).reshape(want.shape), got)


def test_split_attention_against_f64_in_the_peaked_regime(gpu, orc):
    # runtime/tests/hip_ops.rs:488-527 with its inputs (its generator, seed 17): global layer shape
    # at depth 16384, queries from near-uniform (scale 0.05) to sharply peaked (2.0) scores, against
    # exact f64 attention over the same caches. Its criterion is at most twice the error of its
    # one-pass kernel, published for these inputs (docs/split-k-attention.md:90-96).
    r = orc.TestRng(17)
    nh, nkv, hd, depth = 16, 2, 512, 16384
    kc, vc = orc.test_q8_caches(r, depth, depth, nkv, hd)

    def deq(c):
        blk = c.reshape(depth * nkv, hd // QK, Q8B)
        d = blk[:, :, :2].copy().view(np.float16).astype(np.float64)
        return (blk[:, :, 2:].view(np.int8).astype(np.float64) * d).reshape(depth, nkv, hd)

    K, V = deq(kc), deq(vc)
    published_one_pass = {0.05: 2.3e-6, 0.2: 2.4e-6, 0.5: 1.9e-6, 1.0: 1.1e-6, 2.0: 1.2e-6}
    for scale in (0.05, 0.2, 0.5, 1.0, 2.0):
        q = r.vec(nh * hd, scale)
        want = np.empty((nh, hd))
        for h in range(nh):
            g = h // (nh // nkv)
            s = K[:, g] @ q[h * hd:(h + 1) * hd].astype(np.float64)
            e = np.exp(s - s.max())
            want[h] = (e / e.sum()) @ V[:, g]
        _, got = run_split(q, kc, vc, 1, nh, nkv, hd, depth - 1, depth, 0)
        err = rel(got, want)
        print(f"[attn] peaked regime scale {scale}: rel {err:.2e}", flush=True)
        assert err <= 2.0 * published_one_pass[scale]


@pytest.mark.parametrize("nh,nkv,hd,win,cap,pos,n_chunks", [
    (16, 2, 512, 0, 6000, 5000, 64),     # the new key alone in stage 0 of the last chunk's 24 keys
    (16, 2, 512, 0, 6000, 5000, 128),    # a chunk of one key (the new one); chunks past it empty
    (16, 2, 512, 0, 6000, 5000, 16),     # the new key in stage 9 of its chunk
    (16, 2, 512, 0, 6000, 5000, 1),      # one chunk: no merge
    (16, 8, 256, 1024, 1028, 2000, 32),  # sliding window over a wrapped ring, 32-key chunks
    (16, 8, 256, 1024, 1028, 2000, 16),  # the new key at the end of stage 1
    (16, 8, 256, 1024, 1028, 2000, 3),   # three chunks
    (8, 8, 512, 0, 600, 500, 12),        # one head per kv head: 12 chunks, uneven per merging wave
    (4, 4, 256, 0, 40, 20, 32),          # 21 keys over 32 chunks: chunks of one key, the rest empty
    (32, 2, 512, 0, 300, 250, 7),        # 16 heads of a kv head per workgroup, two head groups
    (8, 4, 128, 0, 300, 250, 5),         # another head dimension: the three operations in sequence
    (16, 2, 512, 0, 6000, 5000, 200),    # 200 chunks of 26 keys: the eight-wave merge
    (16, 8, 256, 1024, 1028, 2000, 256),  # the sliding window in 256 chunks of 4 keys
])
def test_decode_entry_matches_store_split_and_merge(gpu, orc, nh, nkv, hd, win, cap, pos, n_chunks):
    """rvm_attn_decode: the ring bytes and the output equal rvh_kv_store + rvh_attn_split +
    rvh_attn_combine bit for bit. The token's ring slot starts as 0xff bytes (NaN scales), so a stale
    copy of it that reached the computation would show. A second call on the same rings (the new
    row already in place) gives the same bits."""
    print(f"[attn decode] {nh}/{nkv}/{hd} win {win} cap {cap} pos {pos} chunks {n_chunks}", flush=True)
    rng = np.random.default_rng(pos + n_chunks + hd)
    kc, vc = q8_ring(orc, rng, cap, nkv, hd)
    row = hd // QK * Q8B
    sl = pos % cap
    for c in (kc, vc):
        c[sl * nkv * row:(sl + 1) * nkv * row] = 0xff
    q = (rng.standard_normal(nh * hd) * 0.3).astype(np.float32)
    kv = rng.standard_normal((2, nkv * hd)).astype(np.float32)
    dq, dk, dv = dev(q), dev(kv[0]), dev(kv[1])
    part = DevBuf(nh * n_chunks * (hd + 2) * 4)
    # the three operations
    kc1, vc1, out1 = dev(kc), dev(vc), DevBuf(nh * hd * 4)
    hip.kv_store(dk, dv, kc1, vc1, 1, nkv, hd, pos, cap)
    hip.attn_split(dq, kc1, vc1, out1, part, 1, nh, nkv, hd, pos, cap, win, n_chunks)
    if n_chunks > 1:
        hip.attn_combine(part, out1, nh, hd, n_chunks)
    # the fused entry
    kc2, vc2, out2 = dev(kc), dev(vc), DevBuf(nh * hd * 4)
    hip.attn_decode(dq, dk, dv, kc2, vc2, out2, part, nh, nkv, hd, pos, cap, win, n_chunks)
    assert np.array_equal(kc2.download(np.uint8, kc.size), kc1.download(np.uint8, kc.size))
    assert np.array_equal(vc2.download(np.uint8, vc.size), vc1.download(np.uint8, vc.size))
    got, want = out2.download(np.float32, nh * hd), out1.download(np.float32, nh * hd)
    assert np.all(np.isfinite(got))
    assert np.array_equal(got, want)
    out3 = DevBuf(nh * hd * 4)
    hip.attn_decode(dq, dk, dv, kc2, vc2, out3, part, nh, nkv, hd, pos, cap, win, n_chunks)
    assert np.array_equal(out3.download(np.float32, nh * hd), want)
    # and the oracle's attention over the stored ring
    ref = orc.attention(q, kc1.download(np.uint8, kc.size), vc1.download(np.uint8, vc.size), nh, nkv, hd, cap, win,
                        pos, 1)
    assert rel(got, ref) < 1e-5
