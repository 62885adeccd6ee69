"""The stack executor (rvm_session_*) on the GPU: device calls per layer, parity, graph capture.

The reference's executor, per layer with device-resident experts, issues 22 launches for its MoE
block (router norm and GEMV, expert-input norm, gather, 8 per-expert gate/up GEMVs, GeGLU, 8 down
GEMVs, combine), one blocking device-to-host copy of the router logits and four host-to-device
metadata uploads, counted by hand in runtime/tests/exec.rs:521-543. A session issues only the
kernels of one rvm_moe_* call per layer, from device memory to device memory: 3 launches for a
decode token (router statistics, gate/up with the selection, down fold), 6 for a batch below
RVM_FOLD_MIN_TOKENS, and no transfer and no synchronisation at all, which the library's own
per-thread counters (rvm_counters) confirm, and which lets one graph hold the whole stack.
"""
import numpy as np
import pytest

from layer_util import D, FF, N_EXP, SEED, TOP_K, assert_close, dev, get_layer, oracle_layer
from rosevine_amd import hip, moe, session, synth
from rosevine_amd.hip import DevBuf

pytestmark = pytest.mark.gpu

N_LAYERS = 30
REF_PER_LAYER = {"launches": 2 + 1 + 1 + TOP_K + 1 + TOP_K + 1, "d2h": 1, "h2d": 4}


def chain(keys, x, n_tok, ws):
    """The same stack as single rvm_moe_* calls with host downloads between layers."""
    cur = x
    for l, key in enumerate(keys):
        L = key[0]
        xd, out = dev(cur), DevBuf(n_tok * D * 4)
        moe.forward(L, xd, out, n_tok, ws, flags=hip.PRE_NORM if l > 0 else 0)
        cur = out.download(np.float32, n_tok * D).reshape(n_tok, D)
    return cur


def test_session_decode_stack30(gpu, orc):
    keys = [get_layer(l, bias=True) for l in range(N_LAYERS)]
    s = session.Session([k[0] for k in keys], max_tokens=4, eps=1e-6)
    x = synth.tokens(SEED + 300, 2)
    xd, out = dev(x), DevBuf(2 * D * 4)
    for t in range(2):
        hip.sync()
        hip.reset_counters()
        s.eval(xd, out, 1, x_off=t * D * 4, out_off=t * D * 4)
        c = hip.counters()
        assert c == {"launches": 3 * N_LAYERS, "h2d": 0, "d2h": 0, "d2d": 0, "syncs": 0, "graphs": 0}, c
        print(f"[session] token {t}: {c['launches'] / N_LAYERS:.0f} launches per layer, no transfer or sync "
              f"(the reference: {REF_PER_LAYER})", flush=True)
    got = out.download(np.float32, 2 * D).reshape(2, D)
    # the same computations as single decode calls, bit for bit; the last layer against the oracle
    ws = moe.Workspace(keys[0][0], 4)
    for t in range(2):
        cur = x[t:t + 1]
        for l, key in enumerate(keys):
            if l == N_LAYERS - 1:
                ids_ref, _, out_ref, _ = oracle_layer(orc, key, cur, pre_norm=True)
                assert_close(got[t], out_ref[0], f"token {t} last layer")
            xdev, o1 = dev(cur), DevBuf(D * 4)
            moe.decode(key[0], xdev, o1, ws, flags=hip.PRE_NORM if l > 0 else 0)
            cur = o1.download(np.float32, D).reshape(1, D)
        assert np.array_equal(cur[0], got[t]), t
    ids, _ = s.selection(1)
    assert np.array_equal(ids[0], ids_ref[0].astype(np.int32))


def test_session_batch_and_graph(gpu):
    keys = [get_layer(l, bias=True) for l in range(4)]
    s = session.Session([k[0] for k in keys], max_tokens=8, eps=1e-6)
    n = 5
    x = synth.tokens(SEED + 301, n)
    xd, out = dev(x), DevBuf(n * D * 4)
    hip.sync()
    hip.reset_counters()
    s.eval(xd, out, n)
    c = hip.counters()
    assert c == {"launches": 6 * 4, "h2d": 0, "d2h": 0, "d2d": 0, "syncs": 0, "graphs": 0}, c
    got = out.download(np.float32, n * D).reshape(n, D)
    # below RVM_FOLD_MIN_TOKENS a token's row does not depend on its batch: each equals its decode
    o1 = DevBuf(D * 4)
    for t in (0, n - 1):
        s.eval(xd, o1, 1, x_off=t * D * 4)
        assert np.array_equal(o1.download(np.float32, D), got[t]), t
    assert np.array_equal(got, chain(keys, x, n, moe.Workspace(keys[0][0], n)))
    # the whole stack in one graph, replayed with eager work between the replays
    st = hip.Stream()
    st.use()
    try:
        g_out = DevBuf(n * D * 4)
        hip.Graph.begin()
        s.eval(xd, g_out, n)
        g = hip.Graph.end()
        for rep in range(3):
            g_out.upload(np.zeros(n * D, np.float32))
            g.launch()
            assert np.array_equal(g_out.download(np.float32, n * D).reshape(n, D), got), rep
            s.eval(xd, o1, 1, x_off=D * 4)
            hip.sync()
        g.close()
    finally:
        hip.Stream.use_default()
        hip.sync()
        st.close()


def test_session_with_block_norms(gpu, orc):
    """Each layer with the reference block's router and expert norms, from the hidden row: the same
    bits as the per-layer rvm_moe_block_decode calls, and the first layer against the oracle."""
    keys = [get_layer(l, bias=True) for l in range(3)]
    norms, gains = [], []
    for l in range(3):
        rng = np.random.default_rng([SEED, l, 41])
        gr, ge = rng.uniform(0.5, 1.5, D).astype(np.float32), rng.uniform(0.5, 1.5, D).astype(np.float32)
        gains.append((gr, ge))
        norms.append(moe.BlockNorms(D, gr, ge, 1e-6))
    s = session.Session([k[0] for k in keys], max_tokens=2, norms=norms)
    o = synth.tokens(SEED + 302, 1) * np.float32(2.0)
    od, out = dev(o), DevBuf(D * 4)
    hip.sync()
    hip.reset_counters()
    s.eval(od, out, 1)
    assert hip.counters()["launches"] == 9 and hip.counters()["syncs"] == 0
    got = out.download(np.float32, D)
    ws, cur = moe.Workspace(keys[0][0], 1), od
    for l, key in enumerate(keys):
        nxt = DevBuf(D * 4)
        moe.block_decode(key[0], norms[l], cur, nxt, ws)
        if l == 0:
            L, router, b, dsc, gu, dn = key
            post = float(np.float32(1.0) / np.sqrt(np.float32(D)))
            rx = orc.rms_norm(o[0], gains[0][0], 1e-6, post)
            ex = orc.rms_norm(o[0], gains[0][1], 1e-6)
            ids, w, _ = orc.select_experts(orc.router_logits(router, b, rx[None], N_EXP, D), TOP_K)
            for e in ids[0]:  # regenerate the selected host experts
                gu[int(e)], dn[int(e)]
            want = orc.experts_q8(gu, dn, dsc, ex[None], D, FF, ids, w, N_EXP)[0]
            assert_close(nxt.download(np.float32, D), want, "layer 0")
        cur = nxt
    assert np.array_equal(cur.download(np.float32, D), got)


def test_session_layer_ranges_equal_the_whole_evaluation(gpu):
    """rvm_session_eval_range: the layers evaluated in ranges, with a caller's cancel check between
    ranges (runtime/src/hip_exec.rs:645-655), give the whole evaluation's bits, for a decode token and
    for a batch; an evaluation stopped after a range leaves the next one, from layer 0, unaffected;
    the span probe's events bracket each layer's router and expert work."""
    keys = [get_layer(l, bias=True) for l in range(4)]
    s = session.Session([k[0] for k in keys], max_tokens=8, eps=1e-6)
    for n in (1, 5):
        print(f"[session] layer ranges, {n} tokens", flush=True)
        x = synth.tokens(SEED + 303 + n, n)
        xd, whole, ranged = dev(x), DevBuf(n * D * 4), DevBuf(n * D * 4)
        s.eval(xd, whole, n)
        want = whole.download(np.float32, n * D)
        s.eval_range(xd, None, n, 0, 2)  # cancelled after two layers
        hip.reset_counters()
        for l0, l1 in [(0, 1), (1, 3), (3, 4)]:
            s.eval_range(xd if l0 == 0 else None, ranged if l1 == 4 else None, n, l0, l1)
        assert hip.counters()["syncs"] == 0
        assert np.array_equal(ranged.download(np.float32, n * D), want), n
        with pytest.raises(hip.BoundsError):
            s.eval_range(None, ranged, n, 2, 4)  # the evaluation ended: a new one starts at layer 0
    # span events: router, then experts, per layer
    ev = [hip.Event() for _ in range(2 * len(keys) + 1)]
    s.probe(ev)
    x = synth.tokens(SEED + 310, 1)
    xd, out = dev(x), DevBuf(D * 4)
    s.eval(xd, out, 1)
    ev[-1].synchronize()
    s.probe(None)
    probed = out.download(np.float32, D)
    for l in range(len(keys)):
        router, experts = ev[2 * l].elapsed_ms(ev[2 * l + 1]), ev[2 * l + 1].elapsed_ms(ev[2 * l + 2])
        assert router >= 0.0 and experts > 0.0, (l, router, experts)
    s.eval(xd, out, 1)  # the probe is off again; the events changed nothing
    assert np.array_equal(out.download(np.float32, D), probed)
