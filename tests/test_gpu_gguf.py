"""The GGUF binding of a layer's MoE tensors (rvm_gguf_bind_moe) on the GPU.

Images are built in memory with the reference's tensor names and ggml shapes
(blk.L.ffn_gate_up_exps.weight [d, 2ff, n_exp], ffn_down_exps.weight [ff, d, n_exp], both Q4_0;
ffn_gate_inp.weight [d, n_exp] and ffn_down_exps.scale [n_exp], F32; runtime/src/contract.rs:66-70,
runtime/src/model.rs:33-40). The bound layer's packed expert planes must be byte for byte the repack
of the same raw rows (rvm_pack_q4 on a device copy), its router and scales the image's floats, and a
decode through it must equal the oracle (small layer) and the synthetic layer's decode bit for bit
(the reference's shape: 128 experts, d = 2816, ff = 704, 428 MB of experts).
"""
import numpy as np
import pytest

from gguf_builder import moe_layer_image
from layer_util import assert_close, dev
from rosevine_amd import gguf, hip, moe, synth
from rosevine_amd.hip import DevBuf

pytestmark = pytest.mark.gpu


def small_tensors(seed, layer, n_exp=16, d=512, ff=128):
    rng = np.random.default_rng([seed, layer, 77])
    return {"n_exp": n_exp, "d": d, "ff": ff,
            "gate_up": hip.synth_q4_host(n_exp, 2 * ff, d, seed, 1000 + 2 * layer),
            "down": hip.synth_q4_host(n_exp, d, ff, seed, 2000 + 2 * layer),
            "router": synth.router_weights(seed, layer, n_exp, d),
            "down_scale": rng.uniform(0.5, 1.5, n_exp).astype(np.float32)}


def test_bind_small_layers_match_the_raw_rows_and_the_oracle(gpu, orc):
    n_exp, top_k, d, ff = 16, 4, 512, 128
    layers = {0: small_tensors(5, 0), 3: small_tensors(5, 3)}
    img = moe_layer_image(layers, extra_f32={"blk.3.pre_ffw_norm_2.weight": np.ones(d, np.float32)})
    g = gguf.Gguf(img)
    for L, t in layers.items():
        bound = g.bind_layer(L, n_exp, top_k, d, ff)
        want = moe.MoeLayer(n_exp, top_k, d, ff, t["router"], None, t["down_scale"])
        want.load_q4(t["gate_up"], t["down"])
        hip.sync()
        for a, b, n in ((bound.gate_up, want.gate_up, want.gu_bytes), (bound.down, want.down, want.dn_bytes),
                        (bound.router, want.router, n_exp * d * 4), (bound.down_scale, want.down_scale, n_exp * 4)):
            assert np.array_equal(a.download(np.uint8, n), b.download(np.uint8, n)), L
        x = synth.tokens(40 + L, 3, d=d)
        ws = moe.Workspace(bound, 1)
        xd, out = dev(x), DevBuf(3 * d * 4)
        for i in range(3):
            moe.decode(bound, xd, out, ws, x_off=i * d * 4, out_off=i * d * 4)
        got = out.download(np.float32, 3 * d).reshape(3, d)
        rows = lambda raw, n_out, k: raw.reshape(n_exp, n_out * (k // 32) * 18)
        gu = {e: rows(t["gate_up"], 2 * ff, d)[e] for e in range(n_exp)}
        dn = {e: rows(t["down"], d, ff)[e] for e in range(n_exp)}
        ids, w, _ = orc.select_experts(orc.router_logits(t["router"], None, x, n_exp, d), top_k)
        want_out = orc.experts_q8(gu, dn, t["down_scale"], x, d, ff, ids, w, n_exp)
        for i in range(3):
            assert_close(got[i], want_out[i], f"layer {L} token {i}")
    # other tensors stay readable; shape mismatches and missing tensors are refused
    typ, shape, _, view = g.tensor("blk.3.pre_ffw_norm_2.weight")
    assert typ == gguf.F32 and shape == [d] and np.array_equal(view.view(np.float32), np.ones(d, np.float32))
    with pytest.raises(gguf.GgufError, match="tensor shape or type mismatch"):
        g.bind_layer(0, n_exp, top_k, d, 2 * ff)
    with pytest.raises(gguf.GgufError, match="missing tensor"):
        g.bind_layer(1, n_exp, top_k, d, ff)


def test_bind_the_reference_shape(gpu):
    """128 experts x (1408 x 2816 + 2816 x 704) Q4_0 from an image: the same bytes on the device as
    the synthetic generator's layer, and the same decode bits."""
    E, K, D, FF = synth.N_EXP, synth.TOP_K, synth.D, synth.FF
    seed, layer = 0, 0
    t = {"n_exp": E, "d": D, "ff": FF,
         "gate_up": hip.synth_q4_host(E, 2 * FF, D, seed, synth.gate_up_stream(layer)),
         "down": hip.synth_q4_host(E, D, FF, seed, synth.down_stream(layer)),
         "router": synth.router_weights(seed, layer), "down_scale": None}
    img = moe_layer_image({7: t})
    print(f"[gguf] image {len(img) / 1e6:.1f} MB", flush=True)
    g = gguf.Gguf(img)
    bound = g.bind_layer(7, E, K, D, FF, down_scale=False)
    want = moe.MoeLayer(E, K, D, FF, t["router"])
    want.synth_weights(seed, synth.gate_up_stream(layer), synth.down_stream(layer))
    hip.sync()
    assert np.array_equal(bound.gate_up.download(np.uint8, want.gu_bytes), want.gate_up.download(np.uint8, want.gu_bytes))
    assert np.array_equal(bound.down.download(np.uint8, want.dn_bytes), want.down.download(np.uint8, want.dn_bytes))
    x = synth.tokens(9, 4)
    xd = dev(x)
    outs = []
    for L in (bound, want):
        ws, out = moe.Workspace(L, 1), DevBuf(4 * D * 4)
        for i in range(4):
            moe.decode(L, xd, out, ws, x_off=i * D * 4, out_off=i * D * 4)
        outs.append(out.download(np.float32, 4 * D))
    assert np.array_equal(outs[0], outs[1])
