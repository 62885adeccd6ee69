"""Every outcome of the single-token decode selection, through rvm_moe_decode, against the oracle.

rvm_moe_decode's gate/up workgroups compute the experts of the f64-estimate ranking while
workgroup 0 certifies it or recomputes the reference's selection (runtime/src/exec.rs:507-517;
ops.rs:170-187). When the two differ, workgroup 0 computes the missing experts itself into
correction rows and the down fold reads each slot's h rows through a map. Router rows built on
the CPU (tests/routing_cases.py) force each outcome for one token:

- the exact selection swaps an expert of the ranking for another (a correction row);
- the same experts in another slot order (moved h rows);
- tied f32 keys, so that every workgroup computes experts 0..k-1 and the selected experts come
  from correction rows (the full exact path: the output is the oracle's bits);
- RVM_EXACT_SELECT on every token (also at widths of one, two and four 256-column chunks of the
  candidates' folds).

Each case asserts that a fallback was taken, that the ids are the oracle's, and that the output
agrees with the oracle (the layer tolerance, and bitwise where the full exact path ran).
Then config 2's stream of 10,000 iid tokens runs through decode with every token's ids compared
with the oracle's (about 2% of them fall back), and the 30-layer stack of config 3 (router bias
N(0,1), RMSNorm eps 1e-6 between layers, all 12.9 GB resident) runs token by token with every
layer's ids and output checked against the oracle given the device's own input (teacher-forced).
"""
import numpy as np
import pytest

import routing_cases as rc
from layer_util import D, FF, N_EXP, SEED, TOP_K, assert_close, dev, get_layer, oracle_layer, rms
from rosevine_amd import hip, moe, synth
from rosevine_amd.hip import DevBuf

pytestmark = pytest.mark.gpu


def decode_one(L, x, flags=0):
    ws = moe.Workspace(L, 1)
    xd, out = dev(x.reshape(1, D)), DevBuf(D * 4)
    moe.decode(L, xd, out, ws, flags=flags)
    ids, w = ws.selection(L, 1)
    return out.download(np.float32, D), ids[0], w[0], ws.fallbacks()


@pytest.mark.parametrize("kind", ["swap_set", "reorder", "tie"])
@pytest.mark.parametrize("extras", [False, True])
def test_decode_forced_fallback_matches_oracle(gpu, orc, kind, extras):
    """A constructed router row makes the certificate fail for one token with the given outcome;
    with extras the layer has a router bias and down scales."""
    key = get_layer(0, bias=extras, ds=extras)
    L, router, b, dsc, gu, dn = key
    for tok in range(3):
        x = synth.tokens(50 + tok, 1)[0]
        r2, b2, spec, ex, (a, bb) = rc.find_case(orc, router, b, x, kind, seed=tok)
        print(f"[fallback] {kind} extras={extras} token {tok}: ranking {spec}, exact {ex}, row {bb} ~ row {a}",
              flush=True)
        L.router.upload(r2)
        if b2 is not None:
            L.bias.upload(b2)
        try:
            got, ids, w, fb = decode_one(L, x)
        finally:
            L.router.upload(router)
            if b is not None:
                L.bias.upload(b)
        ids_ref, w_ref, out_ref, _ = oracle_layer(orc, (L, r2, b2, dsc, gu, dn), x[None, :])
        assert fb == 1, f"no fallback taken ({fb})"
        assert ids.tolist() == ex == [int(v) for v in ids_ref[0]]
        assert np.max(np.abs(w - w_ref[0])) <= 1e-6
        assert_close(got, out_ref[0], f"{kind} token {tok}")
        if kind == "tie":  # the full exact path: the reference's weights, so the reference's bits
            assert np.array_equal(w, w_ref[0])
            assert np.array_equal(got, out_ref[0])


def test_decode_exact_select_flag_matches_oracle(gpu, orc):
    """RVM_EXACT_SELECT through decode: every token takes the exact path (the candidates' logits
    folded in the reference's order)."""
    key = get_layer(0, bias=True, ds=True)
    L = key[0]
    n = 8
    x = synth.tokens(SEED + 21, n)
    ids_ref, w_ref, out_ref, _ = oracle_layer(orc, key, x)
    ws = moe.Workspace(L, 1)
    xd, out = dev(x), DevBuf(n * D * 4)
    for t in range(n):
        moe.decode(L, xd, out, ws, flags=hip.EXACT_SELECT, x_off=t * D * 4, out_off=t * D * 4)
        ids, w = ws.selection(L, 1)
        assert np.array_equal(ids[0], ids_ref[t].astype(np.int32)), t
        assert np.max(np.abs(w[0] - w_ref[t])) <= 1e-6, t
    assert ws.fallbacks() == n
    got = out.download(np.float32, n * D).reshape(n, D)
    for t in range(n):
        assert_close(got[t], out_ref[t], f"token {t}")


def test_decode_ids_config2_stream_10k(gpu, orc):
    """Config 2's 10,000 iid tokens (the benchmark's stream) through decode: every token's ids
    are the oracle's; the outputs of the tokens that fell back are checked against the oracle."""
    key = get_layer(0)
    L, router = key[0], key[1]
    n = 10000
    x = synth.tokens(SEED + 100, n)
    want_ids, want_w, _ = orc.select_experts(orc.router_logits(router, None, x, N_EXP, D), TOP_K)
    ws = moe.Workspace(L, 1)
    xd, out = dev(x), DevBuf(n * D * 4)
    got_ids = np.empty((n, TOP_K), np.int32)
    got_w = np.empty((n, TOP_K), np.float32)
    fell = np.zeros(n, bool)
    prev = 0
    for t in range(n):
        moe.decode(L, xd, out, ws, x_off=t * D * 4, out_off=t * D * 4)
        ids, w = ws.selection(L, 1)
        got_ids[t], got_w[t] = ids[0], w[0]
        c = ws.fallbacks()
        fell[t], prev = c > prev, c
        if t % 2500 == 2499:
            print(f"[sweep] {t + 1} tokens, {int(fell.sum())} fallbacks", flush=True)
    bad = np.where(np.any(got_ids != want_ids.astype(np.int32), axis=1))[0]
    assert bad.size == 0, f"{bad.size} tokens with other ids, first {bad[:8].tolist()}"
    assert np.max(np.abs(got_w - want_w)) <= 1e-5
    assert fell.sum() > 0
    sub = np.where(fell)[0][:24]
    got = out.download(np.float32, n * D).reshape(n, D)
    _, _, out_ref, _ = oracle_layer(orc, key, x[sub])
    for i, t in enumerate(sub):
        assert_close(got[t], out_ref[i], f"fallback token {t}")


def test_stack30_decode_teacher_forced(gpu, orc):
    """Config 3: 30 layers, each with its own seeded experts, router and per-expert router bias
    N(0,1), single-token decode, RMSNorm (eps 1e-6) of the previous layer's output as the layer
    input from layer 1 on. Per layer, ids are the oracle's and the output agrees with it; the
    same 30 layers captured in one graph give the same final output bit for bit."""
    n_layers, n_tok = 30, 2
    keys = [get_layer(l, bias=True) for l in range(n_layers)]
    resident = sum(k[0].weight_bytes for k in keys)
    print(f"[stack30] {resident / 1e9:.2f} GB of experts resident", flush=True)
    x = synth.tokens(SEED + 300, n_tok)
    ws = moe.Workspace(keys[0][0], 1)
    xd, out = DevBuf(D * 4), DevBuf(D * 4)
    finals = []
    for t in range(n_tok):
        cur = x[t]
        for l, key in enumerate(keys):
            L, pre = key[0], l > 0
            ids_ref, _, out_ref, _ = oracle_layer(orc, key, cur[None, :], pre_norm=pre)
            xd.upload(np.ascontiguousarray(cur, np.float32))
            moe.decode(L, xd, out, ws, flags=hip.PRE_NORM if pre else 0)
            got = out.download(np.float32, D)
            ids = ws.selection(L, 1)[0][0]
            assert np.array_equal(ids, ids_ref[0].astype(np.int32)), (t, l)
            assert_close(got, out_ref[0], f"token {t} layer {l}")
            cur = got
        finals.append(cur)
        print(f"[stack30] token {t}: 30 layers match, final rms {rms(cur):.4g}", flush=True)
    # the device-only chain (no host round trip between layers) in one captured graph
    s = hip.Stream()
    s.use()
    try:
        bufs = [DevBuf(D * 4) for _ in range(2)]
        xs, ys = dev(x), DevBuf(n_tok * D * 4)
        hip.Graph.begin()
        for t in range(n_tok):
            moe.decode(keys[0][0], xs, bufs[0], ws, x_off=t * D * 4)
            for l in range(1, n_layers):
                moe.decode(keys[l][0], bufs[(l - 1) % 2], bufs[l % 2], ws, flags=hip.PRE_NORM)
            hip.copy(ys, bufs[(n_layers - 1) % 2], D * 4, dst_off=t * D * 4)
        g = hip.Graph.end()
        g.launch()
        hip.sync()
        assert np.array_equal(ys.download(np.float32, n_tok * D).reshape(n_tok, D), np.stack(finals))
        g.close()
    finally:
        hip.Stream.use_default()
        hip.sync()
        s.close()


@pytest.mark.parametrize("d,ff", [(256, 64), (512, 128), (1024, 128)])
def test_decode_exact_select_small_widths(gpu, orc, d, ff):
    """RVM_EXACT_SELECT through decode at widths of one, two and four 256-column chunks of the
    candidates' exact folds (the ring of chunk loads runs past the row's end and reloads its last
    chunk, unused): ids and weights are the oracle's, outputs within the layer tolerance."""
    n_exp, top_k, n = 16, 4, 6
    rng = np.random.default_rng([SEED, d, 91])
    gate_up = hip.synth_q4_host(n_exp, 2 * ff, d, SEED, 3000 + d)
    down = hip.synth_q4_host(n_exp, d, ff, SEED, 4000 + d)
    router = synth.router_weights(SEED, 5, n_exp, d)
    dscale = rng.uniform(0.5, 1.5, n_exp).astype(np.float32)
    L = moe.MoeLayer(n_exp, top_k, d, ff, router, None, dscale)
    L.load_q4(gate_up, down)
    x = synth.tokens(SEED + 23 + d, n, d=d)
    ws = moe.Workspace(L, 1)
    xd, out = dev(x), DevBuf(n * d * 4)
    ids_ref, w_ref, _ = orc.select_experts(orc.router_logits(router, None, x, n_exp, d), top_k)
    for t in range(n):
        moe.decode(L, xd, out, ws, flags=hip.EXACT_SELECT, x_off=t * d * 4, out_off=t * d * 4)
        ids, w = ws.selection(L, 1)
        assert np.array_equal(ids[0], ids_ref[t].astype(np.int32)), (d, t)
        assert np.max(np.abs(w[0] - w_ref[t])) <= 1e-6, (d, t)
    assert ws.fallbacks() == n
    got = out.download(np.float32, n * d).reshape(n, d)
    rows = lambda raw, n_out, k: raw.reshape(n_exp, n_out * (k // 32) * 18)
    gu = {e: rows(gate_up, 2 * ff, d)[e] for e in range(n_exp)}
    dn = {e: rows(down, d, ff)[e] for e in range(n_exp)}
    want = orc.experts_q8(gu, dn, dscale, x, d, ff, ids_ref, w_ref, n_exp)
    for t in range(n):
        assert_close(got[t], want[t], f"d {d} token {t}")
