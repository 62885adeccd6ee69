"""The MoE block entry points (rvm_moe_block_decode / rvm_moe_block_forward) against the oracle
composed as the reference's executor composes the block.

The reference routes on rms_norm(o) * (1/sqrt(d)) * gate_inp_scale and runs the experts on
rms_norm(o, pre_ffw_norm_2) (runtime/src/exec.rs:465-468 and 493-503; on the device
runtime/src/hip_exec.rs:784-842). The oracle forms the two inputs with orc_rms_norm (the router's
((o * s) * post) * g order, exec.rs:498-500), then its router, selection and Q8_0 expert path.
Ids are exact; outputs are within the layer tolerance, and bit for bit where the selection is
the reference's arithmetic (the fold path of large batches). The batch sizes cover every path:
single-token decode, the 4-pair tiles of small batches, the certified selection with 16-pair MFMA
tiles, and the fold path (with a ragged last token tile).
"""
import numpy as np
import pytest

from layer_util import D, FF, N_EXP, SEED, TOP_K, assert_close, dev, get_layer
from rosevine_amd import hip, moe, synth
from rosevine_amd.hip import DevBuf

pytestmark = pytest.mark.gpu

EPS = 1e-6


def norms_for(layer):
    rng = np.random.default_rng([SEED, layer, 40])
    g_router = rng.uniform(0.5, 1.5, D).astype(np.float32)  # ffn_gate_inp.scale
    g_expert = rng.uniform(0.5, 1.5, D).astype(np.float32)  # pre_ffw_norm_2.weight
    return g_router, g_expert


def oracle_block(orc, key, o, g_router, g_expert):
    L, router, b, dsc, gu, dn = key
    post = np.float32(1.0) / np.sqrt(np.float32(D))  # 1.0 / (n_embd as f32).sqrt()
    rx = np.stack([orc.rms_norm(r, g_router, EPS, float(post)) for r in o])
    ex = np.stack([orc.rms_norm(r, g_expert, EPS) for r in o])
    lg = orc.router_logits(router, b, rx, N_EXP, D)
    ids, w, _ = orc.select_experts(lg, TOP_K)
    for e in set(int(v) for v in ids.reshape(-1)):
        gu[e], dn[e]
    out = orc.experts_q8(gu, dn, dsc, ex, D, FF, ids, w, N_EXP)
    return ids, w, out


def test_block_decode_routes_on_the_router_norm(gpu, orc):
    key = get_layer(0, bias=True, ds=True)
    L = key[0]
    g_router, g_expert = norms_for(0)
    norms = moe.BlockNorms(D, g_router, g_expert, EPS)
    n = 12
    o = synth.tokens(SEED + 30, n) * np.float32(3.0)
    ids_ref, w_ref, out_ref = oracle_block(orc, key, o, g_router, g_expert)
    ws = moe.Workspace(L, 1)
    od, out = dev(o), DevBuf(n * D * 4)
    for t in range(n):
        moe.block_decode(L, norms, od, out, ws, o_off=t * D * 4, out_off=t * D * 4)
        ids, w = ws.selection(L, 1)
        assert np.array_equal(ids[0], ids_ref[t].astype(np.int32)), t
        assert np.max(np.abs(w[0] - w_ref[t])) <= 1e-5, t
    got = out.download(np.float32, n * D).reshape(n, D)
    for t in range(n):
        assert_close(got[t], out_ref[t], f"token {t}")
    # the single-input path routes on the expert norm: another selection for most tokens
    ws1, o1 = moe.Workspace(L, 1), DevBuf(D * 4)
    differ = 0
    for t in range(n):
        moe.decode(L, od, o1, ws1, flags=hip.PRE_NORM, x_off=t * D * 4)
        differ += not np.array_equal(ws1.selection(L, 1)[0][0], ids_ref[t].astype(np.int32))
    assert differ > 0


def test_block_decode_exact_select(gpu, orc):
    key = get_layer(0, bias=True, ds=True)
    L = key[0]
    g_router, g_expert = norms_for(0)
    norms = moe.BlockNorms(D, g_router, g_expert, EPS)
    n = 4
    o = synth.tokens(SEED + 31, n)
    ids_ref, w_ref, out_ref = oracle_block(orc, key, o, g_router, g_expert)
    ws = moe.Workspace(L, 1)
    od, out = dev(o), DevBuf(n * D * 4)
    for t in range(n):
        moe.block_decode(L, norms, od, out, ws, flags=hip.EXACT_SELECT, o_off=t * D * 4, out_off=t * D * 4)
        assert np.array_equal(ws.selection(L, 1)[0][0], ids_ref[t].astype(np.int32)), t
    assert ws.fallbacks() == n
    got = out.download(np.float32, n * D).reshape(n, D)
    for t in range(n):
        assert_close(got[t], out_ref[t], f"token {t}")


@pytest.mark.parametrize("n", [5, 40, 300])
def test_block_forward_matches_oracle(gpu, orc, n):
    """5 tokens: 4-pair tiles; 40: certified selection, MFMA tiles; 300: the fold path (router input
    rows written by the prep kernel, the experts' Q8_0 blocks of the other norm), whose selection
    and outputs are the oracle's bits."""
    key = get_layer(0, bias=True, ds=True)
    L = key[0]
    g_router, g_expert = norms_for(0)
    norms = moe.BlockNorms(D, g_router, g_expert, EPS)
    o = synth.tokens(SEED + 32, n) * np.float32(2.0)
    print(f"[block] forward {n} tokens", flush=True)
    ws = moe.Workspace(L, n)
    od, out = dev(o), DevBuf(n * D * 4)
    moe.block_forward(L, norms, od, out, n, ws)
    got = out.download(np.float32, n * D).reshape(n, D)
    ids, w = ws.selection(L, n)
    sub = sorted({0, 1, n // 2, n - 1} | ({63, 64, 255, 256} if n > 256 else set()))
    ids_ref, w_ref, out_ref = oracle_block(orc, key, o[sub], g_router, g_expert)
    for i, t in enumerate(sub):
        assert np.array_equal(ids[t], ids_ref[i].astype(np.int32)), t
        assert_close(got[t], out_ref[i], f"token {t}")
        if n >= moe.FOLD_MIN_TOKENS:
            assert np.array_equal(w[t], w_ref[i]), t
            assert np.array_equal(got[t], out_ref[i]), f"token {t}: not the oracle's bits"
    # every token's row equals its single-token block decode (the selection arithmetic of the fold
    # path differs from decode's certified estimates, so from 256 tokens rows agree to tolerance)
    ws1, o1 = moe.Workspace(L, 1), DevBuf(D * 4)
    for t in sub:
        moe.block_decode(L, norms, od, o1, ws1, o_off=t * D * 4)
        assert np.array_equal(ws1.selection(L, 1)[0][0], ids[t]), t
        row = o1.download(np.float32, D)
        if n < moe.FOLD_MIN_TOKENS:
            assert np.array_equal(row, got[t]), t
        else:
            assert_close(row, got[t], f"decode row {t}")


def test_block_entries_reject_bad_norms(gpu):
    L = get_layer(0)[0]
    ws = moe.Workspace(L, 2)
    od, out = DevBuf(2 * D * 4), DevBuf(2 * D * 4)
    bad = moe.BlockNorms(D, None, None, eps=float("nan"))
    with pytest.raises(hip.DeviceError):
        moe.block_decode(L, bad, od, out, ws)
    good = moe.BlockNorms(D, None, None)
    with pytest.raises(hip.DeviceError):  # RVM_PRE_NORM is implied, not a flag of these entries
        moe.block_forward(L, good, od, out, 2, ws, flags=hip.PRE_NORM)
