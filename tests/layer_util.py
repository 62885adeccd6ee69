"""Shared helpers of the GPU layer tests: seeded device layers at the reference's shapes, their
host-side Q4_0 experts for the oracle, and the tolerance check.

Rules: top-k expert ids are bit-exact; f32 outputs agree within max-abs 1e-3 of the output's RMS.
The expert intermediates (gate/up rows, GeGLU, the Q8_0 down inputs, the down rows) are the
reference's bits, so outputs differ only through the last bits of the routing weights; the tests
also hold them to 2e-5 of the RMS, which any quantisation flip would exceed.
"""
import numpy as np

from rosevine_amd import moe, synth
from rosevine_amd.hip import DevBuf

N_EXP, TOP_K, D, FF = synth.N_EXP, synth.TOP_K, synth.D, synth.FF
SEED = 0


def dev(a):
    return DevBuf.from_array(np.ascontiguousarray(a))


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def assert_close(got, want, what):
    err, r = float(np.max(np.abs(got - want))), rms(want)
    assert err <= 1e-3 * r, f"{what}: max|diff| {err:.3g} > 1e-3 * rms {r:.3g}"
    assert err <= 2e-5 * r, f"{what}: max|diff| {err:.3g} > 2e-5 * rms {r:.3g}"


class HostExperts(dict):
    """Reference-layout Q4_0 experts regenerated on the host on first use."""

    def __init__(self, seed, stream0, n_out, k):
        super().__init__()
        self.args = (seed, stream0, n_out, k)

    def __missing__(self, e):
        seed, stream0, n_out, k = self.args
        v = synth.host_expert(seed, stream0, int(e), n_out, k)
        self[e] = v
        return v


_layers = {}


def get_layer(layer=0, bias=False, ds=False):
    """(device layer, router, bias, down scales, host gate_up experts, host down experts) of the
    seeded layer `layer`, built once per process."""
    key = (layer, bias, ds)
    if key not in _layers:
        router = synth.router_weights(SEED, layer)
        b = synth.router_bias(SEED, layer) if bias else None
        dsc = np.random.default_rng([SEED, layer, 9]).uniform(0.5, 1.5, N_EXP).astype(np.float32) if ds else None
        L = moe.MoeLayer(N_EXP, TOP_K, D, FF, router, b, dsc)
        L.synth_weights(SEED, synth.gate_up_stream(layer), synth.down_stream(layer))
        gu = HostExperts(SEED, synth.gate_up_stream(layer), 2 * FF, D)
        dn = HostExperts(SEED, synth.down_stream(layer), D, FF)
        _layers[key] = (L, router, b, dsc, gu, dn)
    return _layers[key]


def oracle_layer(orc, key, x, pre_norm=False):
    """The oracle's ids, weights, outputs and logits for tokens x through layer `key`."""
    L, router, b, dsc, gu, dn = key
    xin = np.stack([orc.rms_norm(r, None, 1e-6) for r in x]) if pre_norm else x
    lg = orc.router_logits(router, b, xin, N_EXP, D)
    ids, w, _ = orc.select_experts(lg, TOP_K)
    for e in set(int(v) for v in ids.reshape(-1)):
        gu[e], dn[e]
    out = orc.experts_q8(gu, dn, dsc, xin, D, FF, ids, w, N_EXP)
    return ids, w, out, lg
