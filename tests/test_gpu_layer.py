"""End-to-end parity of the MoE layer on the GPU against the CPU oracle.

Rules: top-k expert ids are bit-exact; f32 outputs agree within max-abs 1e-3 of the output's RMS.
The expert intermediates (gate/up rows, GeGLU, the Q8_0 down inputs, the down rows) are the
reference's bits, so the outputs differ only through the last bits of the routing weights: the
tests also hold them to 2e-5 of the RMS, which any quantisation flip would exceed.
Workloads are the seeded synthetic configurations at the reference's shapes (128 experts, top-8,
d = 2816, ff = 704): single-token decode, a ragged 32-token decode batch with Zipf(1.1)
popularity, a 512-token prefill, and a teacher-forced multi-layer stack with router bias and
an RMSNorm between layers; and 16-expert layers of other widths through each batched path.
Size-independent properties (batch invariance, graph replays) cover what the oracle is too slow
to check in full.
"""
import numpy as np
import pytest

from layer_util import D, FF, N_EXP, SEED, TOP_K, HostExperts, assert_close, dev, get_layer, oracle_layer
from rosevine_amd import hip, moe, synth
from rosevine_amd.hip import DevBuf

pytestmark = pytest.mark.gpu


def test_router_certified_ids_match_oracle(gpu, orc):
    for bias in (False, True):
        key = get_layer(0, bias=bias)
        L, router, b = key[0], key[1], key[2]
        n = moe.FOLD_MIN_TOKENS - 1  # the certified path (larger batches fold every logit)
        x = synth.tokens(SEED + 1, n)
        ws = moe.Workspace(L, n)
        ids, w, lg = moe.router_select(L, dev(x), n, ws, with_logits=True)
        want_lg = orc.router_logits(router, b, x, N_EXP, D)
        want_ids, want_w, _ = orc.select_experts(want_lg, TOP_K)
        assert np.array_equal(ids, want_ids.astype(np.int32))
        assert np.max(np.abs(w - want_w)) <= 1e-5
        print(f"[router] bias={bias} tokens={n} exactness fallbacks={ws.fallbacks()}", flush=True)
        # the reference-order path: logits bit-exact, same ids
        ws2 = moe.Workspace(L, n)
        ids2, w2, lg2 = moe.router_select(L, dev(x), n, ws2, flags=hip.EXACT_SELECT, with_logits=True)
        assert np.array_equal(lg2, want_lg)
        assert np.array_equal(ids2, want_ids.astype(np.int32))
        assert np.array_equal(w2, want_w)
        assert ws2.fallbacks() == n


def test_router_exact_candidates_match_the_full_exact_path(gpu, orc):
    """EXACT_SELECT without logits takes the candidate path (exact folds of the experts that can
    reach the top k, ranking certified for any softmax denominator); with logits every expert is
    folded. Both give the reference's ids; the candidate path's weights are tolerance class."""
    for bias in (False, True):
        key = get_layer(0, bias=bias)
        L, router, b = key[0], key[1], key[2]
        n = moe.FOLD_MIN_TOKENS - 1
        x = synth.tokens(SEED + 2, n)
        want_ids, want_w, _ = orc.select_experts(orc.router_logits(router, b, x, N_EXP, D), TOP_K)
        ws = moe.Workspace(L, n)
        ids, w = moe.router_select(L, dev(x), n, ws, flags=hip.EXACT_SELECT)
        ws2 = moe.Workspace(L, n)
        ids2, w2, _ = moe.router_select(L, dev(x), n, ws2, flags=hip.EXACT_SELECT, with_logits=True)
        assert np.array_equal(ids, want_ids.astype(np.int32))
        assert np.array_equal(ids2, ids)
        assert np.max(np.abs(w - w2)) <= 1e-6
        assert np.max(np.abs(w - want_w)) <= 1e-6
        assert ws.fallbacks() == n


def test_router_ties_go_to_the_lower_index(gpu, orc):
    rng = np.random.default_rng(5)
    router = (rng.standard_normal((N_EXP, D)) * 0.02).astype(np.float32)
    router[[7, 50, 51]] = router[3]          # identical logits: only the index can order them
    router[[90, 91]] = router[12]
    L = moe.MoeLayer(N_EXP, TOP_K, D, FF, router)
    for n in (moe.FOLD_MIN_TOKENS - 1, moe.FOLD_MIN_TOKENS):  # certified path, then the fold path
        x = synth.tokens(7, n)
        ws = moe.Workspace(L, n)
        ids, w = moe.router_select(L, dev(x), n, ws)
        want_ids, want_w, _ = orc.select_experts(orc.router_logits(router, None, x, N_EXP, D), TOP_K)
        assert np.array_equal(ids, want_ids.astype(np.int32))
        assert np.max(np.abs(w - want_w)) <= 1e-5
        assert (ws.fallbacks() > 0) == (n < moe.FOLD_MIN_TOKENS)


@pytest.mark.parametrize("n,bias,pre", [(256, False, False), (1000, True, False), (333, True, True)])
def test_router_fold_path_is_the_references_bits(gpu, orc, n, bias, pre):
    """From FOLD_MIN_TOKENS tokens every logit is folded in the reference's order: logits, ids
    and weights are the oracle's bit for bit (ragged last token tile, router bias, pre-norm)."""
    key = get_layer(0, bias=bias)
    L, router, b = key[0], key[1], key[2]
    x = synth.tokens(SEED + 11, n)
    print(f"[fold] {n} tokens bias={bias} pre_norm={pre}", flush=True)
    ws = moe.Workspace(L, n)
    flags = hip.PRE_NORM if pre else 0
    ids, w, lg = moe.router_select(L, dev(x), n, ws, flags=flags, with_logits=True)
    xin = np.stack([orc.rms_norm(r, None, 1e-6) for r in x]) if pre else x
    want_lg = orc.router_logits(router, b, xin, N_EXP, D)
    want_ids, want_w, _ = orc.select_experts(want_lg, TOP_K)
    assert np.array_equal(lg, want_lg)
    assert np.array_equal(ids, want_ids.astype(np.int32))
    assert np.array_equal(w, want_w)
    assert ws.fallbacks() == 0


def test_plan_matches_oracle(gpu, orc):
    rng = np.random.default_rng(6)
    # up to 8192 pairs a wave keeps its ids in registers between the count and the placement; above
    # that it reads them in batches (9001 and 40000: partial and several batches per wave)
    for n_pairs in [8, 256, 1000, 3000, 4096, 8192, 9001, 40000]:
        ids = (rng.zipf(1.2, n_pairs) % N_EXP).astype(np.int32)
        order, pos_of, gs = DevBuf(n_pairs * 4), DevBuf(n_pairs * 4), DevBuf((N_EXP + 1) * 4)
        hip.moe_plan(dev(ids), n_pairs, N_EXP, order, pos_of, gs)
        o, p, g = orc.moe_plan(ids.astype(np.uint32), N_EXP)
        assert np.array_equal(order.download(np.int32, n_pairs), o.astype(np.int32))
        assert np.array_equal(pos_of.download(np.int32, n_pairs), p.astype(np.int32))
        assert np.array_equal(gs.download(np.int32, N_EXP + 1), g.astype(np.int32))
        if n_pairs > 4096:  # a few ids out of range among them: a stable sort of the others
            ids[rng.integers(0, n_pairs, 7)] = -1
            hip.moe_plan(dev(ids), n_pairs, N_EXP, order, pos_of, gs)
            keep = np.flatnonzero(ids >= 0)
            o = keep[np.argsort(ids[keep], kind="stable")]
            p = np.full(n_pairs, -1, np.int64)
            p[o] = np.arange(o.size)
            g = np.concatenate([[0], np.cumsum(np.bincount(ids[keep], minlength=N_EXP))])
            assert np.array_equal(order.download(np.int32, o.size), o.astype(np.int32))
            assert np.array_equal(pos_of.download(np.int32, n_pairs), p.astype(np.int32))
            assert np.array_equal(gs.download(np.int32, N_EXP + 1), g.astype(np.int32))
    # 256 experts (one thread of the plan's workgroup per expert, the group starts' last entry
    # included)
    for n_pairs in [700, 1024, 1025]:
        ids = (rng.zipf(1.1, n_pairs) % 256).astype(np.int32)
        order, pos_of, gs = DevBuf(n_pairs * 4), DevBuf(n_pairs * 4), DevBuf(257 * 4)
        hip.moe_plan(dev(ids), n_pairs, 256, order, pos_of, gs)
        o, p, g = orc.moe_plan(ids.astype(np.uint32), 256)
        assert np.array_equal(order.download(np.int32, n_pairs), o.astype(np.int32)), n_pairs
        assert np.array_equal(pos_of.download(np.int32, n_pairs), p.astype(np.int32)), n_pairs
        assert np.array_equal(gs.download(np.int32, 257), g.astype(np.int32)), n_pairs
    # ids outside [0, n_exp) are left out of the plan
    ids = np.array([3, -1, 3, 200, 0], np.int32)
    order, pos_of, gs = DevBuf(20), DevBuf(20), DevBuf((N_EXP + 1) * 4)
    hip.moe_plan(dev(ids), 5, N_EXP, order, pos_of, gs)
    assert list(pos_of.download(np.int32, 5)) == [1, -1, 2, -1, 0]
    assert list(order.download(np.int32, 3)) == [4, 0, 2]
    assert gs.download(np.int32, N_EXP + 1)[-1] == 3


@pytest.mark.parametrize("bias,ds,pre", [(False, False, False), (True, True, True)])
def test_decode_matches_oracle(gpu, orc, bias, ds, pre):
    key = get_layer(0, bias=bias, ds=ds)
    L = key[0]
    n = 16
    x = synth.tokens(SEED + 2, n)
    ids_ref, _, out_ref, _ = oracle_layer(orc, key, x, pre_norm=pre)
    ws = moe.Workspace(L, 1)
    xd, out = dev(x), DevBuf(n * D * 4)
    flags = hip.PRE_NORM if pre else 0
    for t in range(n):
        moe.decode(L, xd, out, ws, flags=flags, x_off=t * D * 4, out_off=t * D * 4)
        ids_dev = ws.selection(L, 1)[0][0]
        assert np.array_equal(ids_dev, ids_ref[t].astype(np.int32)), t
    got = out.download(np.float32, n * D).reshape(n, D)
    for t in range(n):
        assert_close(got[t], out_ref[t], f"token {t}")


def test_forward_ragged_zipf_matches_oracle_and_decode(gpu, orc):
    rng = np.random.default_rng(8)
    router = synth.router_weights(SEED, 0)
    bias = synth.zipf_bias(SEED)
    L = moe.MoeLayer(N_EXP, TOP_K, D, FF, router, bias)
    L.synth_weights(SEED, synth.gate_up_stream(0), synth.down_stream(0))
    key = (L, router, bias, None, HostExperts(SEED, synth.gate_up_stream(0), 2 * FF, D),
           HostExperts(SEED, synth.down_stream(0), D, FF))
    n = 32
    x = synth.tokens(SEED + 3, n)
    ids_ref, _, out_ref, _ = oracle_layer(orc, key, x)
    distinct = len(set(ids_ref.reshape(-1).tolist()))
    print(f"[forward] 32 tokens, {distinct} distinct experts, max group {np.bincount(ids_ref.reshape(-1)).max()}",
          flush=True)
    ws = moe.Workspace(L, n)
    xd, out = dev(x), DevBuf(n * D * 4)
    moe.forward(L, xd, out, n, ws)
    got = out.download(np.float32, n * D).reshape(n, D)
    for t in range(n):
        assert_close(got[t], out_ref[t], f"token {t}")
    # batch invariance: each token's row equals its single-token decode bitwise
    ws1, o1 = moe.Workspace(L, 1), DevBuf(D * 4)
    for t in [0, 13, 31]:
        moe.decode(L, xd, o1, ws1, x_off=t * D * 4)
        assert np.array_equal(o1.download(np.float32, D), got[t]), t
    del rng


@pytest.mark.parametrize("n,extras", [(2, False), (5, False), (5, True), (127, False), (127, True), (128, False)])
def test_forward_batch_sizes_are_batch_invariant(gpu, n, extras):
    """Batches on both sides of the tile-size switch (4-pair tiles below 8 pairs per expert on
    average: 127 tokens and fewer; 32-pair tiles from 128 tokens): groups of one pair up to full
    tiles, with and without router bias and down scales. Every checked token's row equals its
    single-token decode bit for bit."""
    L = get_layer(0, bias=extras, ds=extras)[0]
    x = synth.tokens(SEED + 7, n)
    print(f"[batch] {n} tokens", flush=True)
    ws = moe.Workspace(L, n)
    xd, out = dev(x), DevBuf(n * D * 4)
    moe.forward(L, xd, out, n, ws)
    got = out.download(np.float32, n * D).reshape(n, D)
    ws1, o1 = moe.Workspace(L, 1), DevBuf(D * 4)
    for t in sorted({0, 1, n // 2, n - 1}):
        moe.decode(L, xd, o1, ws1, x_off=t * D * 4)
        assert np.array_equal(o1.download(np.float32, D), got[t]), t


def test_prefill_512_matches_oracle_and_decode(gpu, orc):
    """512 tokens take the fold path: ids, weights and outputs are the oracle's bit for bit; each sampled
    token has its single-token decode's ids, and its row agrees with the decode row (whose
    weights come from the certified estimates) and with the oracle."""
    key = get_layer(0)
    L = key[0]
    n = 512
    x = synth.tokens(SEED + 4, n)
    ws = moe.Workspace(L, n)
    xd, out = dev(x), DevBuf(n * D * 4)
    moe.forward(L, xd, out, n, ws)
    got = out.download(np.float32, n * D).reshape(n, D)
    ids, w = ws.selection(L, n)
    want_ids, want_w, _ = orc.select_experts(orc.router_logits(key[1], None, x, N_EXP, D), TOP_K)
    assert np.array_equal(ids, want_ids.astype(np.int32))
    assert np.array_equal(w, want_w)
    ws1, o1 = moe.Workspace(L, 1), DevBuf(D * 4)
    for t in range(0, n, 37):
        moe.decode(L, xd, o1, ws1, x_off=t * D * 4)
        assert np.array_equal(ws1.selection(L, 1)[0][0], ids[t]), t
        assert_close(o1.download(np.float32, D), got[t], f"decode row {t}")
    sub = [0, 255, 511]
    _, _, out_ref, _ = oracle_layer(orc, key, x[sub])
    for i, t in enumerate(sub):
        assert_close(got[t], out_ref[i], f"token {t}")
        assert np.array_equal(got[t], out_ref[i]), f"token {t}: not the oracle's bits"


def test_prefill_512_skewed_routing_matches_oracle(gpu, orc):
    """512 tokens with the 30-layer configuration's per-expert router bias N(0,1): groups from 0 to a
    few hundred pairs, some experts empty (config 4's ragged groups). Ids and weights are the
    oracle's for every token; output rows are the oracle's bits for the tokens at the first and last
    pairs of the 32-pair gate/up and 48-pair down tiles of the largest group, and for the tokens of
    the smallest non-empty groups."""
    key = get_layer(0, bias=True)
    L = key[0]
    n = 512
    x = synth.tokens(SEED + 40, n)
    ws = moe.Workspace(L, n)
    xd, out = dev(x), DevBuf(n * D * 4)
    moe.forward(L, xd, out, n, ws)
    got = out.download(np.float32, n * D).reshape(n, D)
    ids, w = ws.selection(L, n)
    want_ids, want_w, _ = orc.select_experts(orc.router_logits(key[1], key[2], x, N_EXP, D), TOP_K)
    assert np.array_equal(ids, want_ids.astype(np.int32))
    assert np.array_equal(w, want_w)
    counts = np.bincount(ids.reshape(-1), minlength=N_EXP)
    print(f"[prefill skewed] groups {counts.min()}..{counts.max()}, {(counts == 0).sum()} empty experts",
          flush=True)
    assert counts.max() > 100 and (counts == 0).sum() > 0
    big = int(np.argmax(counts))
    pairs = np.flatnonzero(ids.reshape(-1) == big)  # the group in plan order (stable by pair index)
    edges = {0, len(pairs) - 1}
    for tile in (32, 48):
        for start in range(tile, len(pairs), tile):
            edges |= {start - 1, start}
    toks = {int(pairs[i]) // TOP_K for i in edges}
    small = [e for e in np.argsort(counts, kind="stable") if counts[e] > 0][:3]
    toks |= {int(p) // TOP_K for e in small for p in np.flatnonzero(ids.reshape(-1) == e)[:1]}
    sub = sorted(toks)[:24]
    _, _, out_ref, _ = oracle_layer(orc, key, x[sub])
    for i, t in enumerate(sub):
        assert np.array_equal(got[t], out_ref[i]), f"token {t}: not the oracle's bits"


def test_forward_fold_path_ragged_pre_norm_matches_oracle_bitwise(gpu, orc):
    """300 tokens (a ragged last tile of 44) with pre-norm, router bias and down scales: the fold
    path's Q8_0 blocks of the normed input (formed by the router fold, token g of each tile by
    workgroup g) feed the experts, and the first and last tokens of every tile are the oracle's
    bits."""
    key = get_layer(0, bias=True, ds=True)
    L = key[0]
    n = 300
    x = synth.tokens(SEED + 12, n)
    print(f"[fold forward] {n} tokens pre_norm bias ds", flush=True)
    ws = moe.Workspace(L, n)
    xd, out = dev(x), DevBuf(n * D * 4)
    moe.forward(L, xd, out, n, ws, flags=hip.PRE_NORM)
    got = out.download(np.float32, n * D).reshape(n, D)
    sub = [0, 63, 64, 127, 191, 255, 256, 299]
    _, _, out_ref, _ = oracle_layer(orc, key, x[sub], pre_norm=True)
    for i, t in enumerate(sub):
        assert_close(got[t], out_ref[i], f"token {t}")
        assert np.array_equal(got[t], out_ref[i]), f"token {t}: not the oracle's bits"


def test_graph_replays_match_eager(gpu):
    key = get_layer(0)
    L = key[0]
    n = 4
    x = synth.tokens(SEED + 5, n)
    xd = dev(x)
    ws = moe.Workspace(L, 1)
    eager = DevBuf(n * D * 4)
    for t in range(n):
        moe.decode(L, xd, eager, ws, x_off=t * D * 4, out_off=t * D * 4)
    want = eager.download(np.float32, n * D)
    s = hip.Stream()
    s.use()
    try:
        out = DevBuf(n * D * 4)
        hip.Graph.begin()
        for t in range(n):
            moe.decode(L, xd, out, ws, x_off=t * D * 4, out_off=t * D * 4)
        g = hip.Graph.end()
        for rep in range(3):
            out.upload(np.zeros(n * D, np.float32))
            g.launch()
            assert np.array_equal(out.download(np.float32, n * D), want), rep
            moe.decode(L, xd, eager, ws)  # eager work between replays
            hip.sync()
        g.close()
    finally:
        hip.Stream.use_default()
        hip.sync()
        s.close()


def test_stack_teacher_forced(gpu, orc):
    """Three layers with router bias and RMSNorm between layers: each layer's ids are exact and
    its output within tolerance, given the previous layer's device output as input."""
    x = synth.tokens(SEED + 6, 4)
    cur = x
    for layer in range(3):
        key = get_layer(layer, bias=True)
        L = key[0]
        pre = layer > 0
        ids_ref, _, out_ref, _ = oracle_layer(orc, key, cur, pre_norm=pre)
        ws = moe.Workspace(L, 4)
        xd, out = dev(cur), DevBuf(4 * D * 4)
        moe.forward(L, xd, out, 4, ws, flags=hip.PRE_NORM if pre else 0)
        got = out.download(np.float32, 4 * D).reshape(4, D)
        ids_dev = ws.selection(L, 4)[0]
        assert np.array_equal(ids_dev, ids_ref.astype(np.int32)), layer
        for t in range(4):
            assert_close(got[t], out_ref[t], f"layer {layer} token {t}")
        cur = got



@pytest.mark.parametrize("d,ff", [(512, 128), (1024, 256)])
@pytest.mark.parametrize("n", [8, 64, 300])
def test_forward_small_shapes_match_oracle(gpu, orc, d, ff, n):
    """rvm_moe_forward at shapes other than the reference's, through each batched path: 8 tokens of
    16 experts at top-4 take the 4-pair tiles, 64 the 16x16 MFMA tiles after the certified
    selection, 300 the MFMA tiles after the exact logits (the tile loops' whole chunks at other
    block counts, the down rows' two halves at other widths). Ids are the oracle's; outputs agree
    with the oracle, bit for bit on the exact-logit path."""
    n_exp, top_k = 16, 4
    rng = np.random.default_rng([SEED, d, ff, 93])
    gate_up = hip.synth_q4_host(n_exp, 2 * ff, d, SEED, 5000 + d + ff)
    down = hip.synth_q4_host(n_exp, d, ff, SEED, 6000 + d + ff)
    router = synth.router_weights(SEED, 7, n_exp, d)
    dscale = rng.uniform(0.5, 1.5, n_exp).astype(np.float32)
    L = moe.MoeLayer(n_exp, top_k, d, ff, router, None, dscale)
    L.load_q4(gate_up, down)
    x = synth.tokens(SEED + 31 + n, n, d=d)
    ws = moe.Workspace(L, n)
    xd, out = dev(x), DevBuf(n * d * 4)
    moe.forward(L, xd, out, n, ws)
    got = out.download(np.float32, n * d).reshape(n, d)
    ids, w = ws.selection(L, n)
    want_ids, want_w, _ = orc.select_experts(orc.router_logits(router, None, x, n_exp, d), top_k)
    assert np.array_equal(ids, want_ids.astype(np.int32))
    rows = lambda raw, n_out, k: raw.reshape(n_exp, n_out * (k // 32) * 18)
    gu = {e: rows(gate_up, 2 * ff, d)[e] for e in range(n_exp)}
    dn = {e: rows(down, d, ff)[e] for e in range(n_exp)}
    want = orc.experts_q8(gu, dn, dscale, x, d, ff, want_ids, want_w, n_exp)
    for t in range(n):
        assert_close(got[t], want[t], f"d {d} ff {ff} n {n} token {t}")
    if n >= 256:
        assert np.array_equal(w, want_w)
        assert np.array_equal(got, want.astype(np.float32)), "not the oracle's bits"
