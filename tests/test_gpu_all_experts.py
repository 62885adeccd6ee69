"""Every expert of a layer, every row, through each fused path (the reference's all-experts sweep,
runtime/examples/expert_validate.rs:31-95, done through the layer entry points).

The router is rigged so that routing covers all 128 experts: expert e's row gets a tag weight on
coordinate e // 8 (1 + e % 8 / 50, so the group's logits are distinct), and token t carries 40 on
the tag coordinate of group t % 16, so its top 8 are that group. The other coordinates hold the
reference sweep's three input patterns (expert_validate.rs:36-46) in turn. Decode (16 tokens), a
small batch (4-pair tiles), a batch with 8 pairs per expert (16-pair MFMA tiles) and a batch on
the fold path (16 pairs per expert) then run every gate/up row and every down row of every
expert: the ids are the oracle's; the fold path's outputs are the oracle's bits, which pins each
expert's rows (a wrong row of any expert changes some token's output); the other paths agree with
the oracle within the contract's tolerance and with decode bit for bit. Layers 0 and 29 of the
seeded stack (their own weight streams).

The tagged logits are near 40, and the reference folds them in f32 from a prefix that reaches 40
at the first coordinates, so its rounding error is far larger than for N(0, 1) tokens; the
certified paths take the routing weights from the f64 estimates, which differ from the
reference's by that error. Their outputs stay within the 1e-3 contract (measured 4.4e-4 of the
RMS on both layers, against 2e-5 for the N(0, 1) tokens of the other tests).
"""
import numpy as np
import pytest

from layer_util import D, FF, N_EXP, SEED, TOP_K, HostExperts, dev, rms
from rosevine_amd import hip, moe, synth
from rosevine_amd.hip import DevBuf

pytestmark = pytest.mark.gpu

GROUPS = N_EXP // TOP_K  # 16 groups of 8 experts


def sweep_patterns(k):
    """The reference sweep's three input patterns (expert_validate.rs:36-46), in f32."""
    i = np.arange(k)
    f = i.astype(np.float32)
    return [np.sin(f * np.float32(0.37)).astype(np.float32),
            ((i * 7919 % 10007).astype(np.float32) / np.float32(5003.5) - np.float32(1.0)).astype(np.float32),
            (np.cos(f * np.float32(1.117)) + np.float32(0.3) * np.sin(f * np.float32(0.031))).astype(np.float32)]


def assert_contract(got, want, what):
    err, r = float(np.max(np.abs(got - want))), rms(want)
    assert err <= 1e-3 * r, f"{what}: max|diff| {err:.3g} > 1e-3 * rms {r:.3g}"
    return err / r


def rigged(layer):
    router = synth.router_weights(SEED, layer).copy()
    for e in range(N_EXP):
        router[e, e // TOP_K] += np.float32(1.0) + np.float32(e % TOP_K) / np.float32(50.0)
    pats = sweep_patterns(D)

    def tokens(n):
        x = np.empty((n, D), np.float32)
        for t in range(n):
            x[t] = pats[(t // GROUPS) % 3]
            x[t, :GROUPS] = 0.0
            x[t, t % GROUPS] = 40.0
        return x
    return router, tokens


@pytest.mark.parametrize("layer", [0, 29])
def test_every_expert_every_row(gpu, orc, layer):
    router, tokens = rigged(layer)
    dsc = np.random.default_rng([SEED, layer, 9]).uniform(0.5, 1.5, N_EXP).astype(np.float32)
    L = moe.MoeLayer(N_EXP, TOP_K, D, FF, router, None, dsc)
    L.synth_weights(SEED, synth.gate_up_stream(layer), synth.down_stream(layer))
    gu = HostExperts(SEED, synth.gate_up_stream(layer), 2 * FF, D)
    dn = HostExperts(SEED, synth.down_stream(layer), D, FF)
    for e in range(N_EXP):
        gu[e], dn[e]
    n_fold = 256
    x = tokens(n_fold)
    lg = orc.router_logits(router, None, x, N_EXP, D)
    ids_ref, w_ref, _ = orc.select_experts(lg, TOP_K)
    assert sorted(set(ids_ref[:GROUPS].reshape(-1).tolist())) == list(range(N_EXP))
    for t in range(n_fold):
        assert sorted(ids_ref[t].tolist()) == list(range(TOP_K * (t % GROUPS), TOP_K * (t % GROUPS + 1)))
    out_ref = orc.experts_q8(gu, dn, dsc, x, D, FF, ids_ref, w_ref, N_EXP)
    print(f"[all experts] layer {layer}: oracle done", flush=True)
    xd = dev(x)
    ws = moe.Workspace(L, n_fold)
    # decode: the 16 groups, one token each
    dec = DevBuf(GROUPS * D * 4)
    for t in range(GROUPS):
        moe.decode(L, xd, dec, ws, x_off=t * D * 4, out_off=t * D * 4)
        ids, _ = ws.selection(L, 1)
        assert np.array_equal(ids[0], ids_ref[t].astype(np.int32)), t
    dec_rows = dec.download(np.float32, GROUPS * D).reshape(GROUPS, D)
    worst = max(assert_contract(dec_rows[t], out_ref[t], f"layer {layer} decode token {t}") for t in range(GROUPS))
    # 4-pair tiles (16 tokens) and 16-pair MFMA tiles (128 tokens: 8 pairs per expert)
    for n in (GROUPS, 8 * GROUPS):
        out = DevBuf(n * D * 4)
        moe.forward(L, xd, out, n, ws)
        ids, _ = ws.selection(L, n)
        assert np.array_equal(ids, ids_ref[:n].astype(np.int32)), n
        got = out.download(np.float32, n * D).reshape(n, D)
        assert np.array_equal(got[:GROUPS], dec_rows), n
        worst = max([worst] + [assert_contract(got[t], out_ref[t], f"layer {layer} batch {n} token {t}")
                               for t in range(n)])
    # the fold path: every output the oracle's bits
    out = DevBuf(n_fold * D * 4)
    moe.forward(L, xd, out, n_fold, ws)
    ids, _ = ws.selection(L, n_fold)
    assert np.array_equal(ids, ids_ref.astype(np.int32))
    got = out.download(np.float32, n_fold * D).reshape(n_fold, D)
    bad = [t for t in range(n_fold) if not np.array_equal(got[t], out_ref[t])]
    assert not bad, f"layer {layer}: tokens {bad[:8]} differ from the oracle's bits"
    print(f"[all experts] layer {layer}: certified paths within {worst:.2e} of the RMS; fold path bitwise",
          flush=True)
