"""rvm_moe_decode_static, the decode entry point that allocates nothing, against rvm_moe_decode.

Both run the same kernels; the static variant's scratch is the library's static device array
instead of a caller workspace, so its outputs must equal rvm_moe_decode's bit for bit. The calls
come in a row on one GPU with different shapes (the reference's shape, then a smaller layer, then
the reference's shape again with a token whose selection falls back to the exact path), so each
call runs on what the previous one left in the array. A captured graph of static calls is
replayed with eager work between the replays.
"""
import ctypes as C
import os
import re

import numpy as np
import pytest

import routing_cases as rc
from layer_util import D, dev, get_layer
from rosevine_amd import hip, moe, synth
from rosevine_amd.hip import DevBuf, RvmLayer

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def static_scratch_bytes():
    text = open(os.path.join(ROOT, "include", "rvmoe.h")).read()
    m = re.search(r"#define RVM_STATIC_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    return int(m.group(1)) << int(m.group(2))


def test_static_scratch_covers_every_supported_decode_shape(rvlib):
    """The largest layer the entry points accept (256 experts, top-8, d = 256 * 16, ff = 64 * 16)
    needs no more decode scratch than the static array holds."""
    fake = 0x1000  # never dereferenced: the size query only validates the pointers are set
    for n_exp, top_k, d, ff in [(256, 8, 4096, 1024), (128, 8, 2816, 704), (16, 4, 512, 128)]:
        L = RvmLayer(n_exp, top_k, d, ff, fake, None, fake, fake, None)
        n = C.c_size_t()
        assert rvlib.rvm_moe_workspace_bytes(C.byref(L), 1, C.byref(n)) == 0
        assert n.value <= static_scratch_bytes(), (n_exp, top_k, d, ff, n.value)


def small_layer():
    n_exp, top_k, d, ff = 16, 4, 512, 128
    L = moe.MoeLayer(n_exp, top_k, d, ff, synth.router_weights(3, 0, n_exp, d))
    L.synth_weights(3, synth.gate_up_stream(0), synth.down_stream(0))
    return L


def both(L, x, flags=0):
    xd = dev(x.reshape(1, -1))
    ws = moe.Workspace(L, 1)
    a, b = DevBuf(L.d * 4), DevBuf(L.d * 4)
    moe.decode(L, xd, a, ws, flags=flags)
    moe.decode_static(L, xd, b, flags=flags)
    return a.download(np.float32, L.d), b.download(np.float32, L.d), ws.fallbacks()


@pytest.mark.gpu
def test_static_decode_equals_workspace_decode(gpu, orc):
    big = get_layer(0, bias=True, ds=True)
    L, router, bias = big[0], big[1], big[2]
    small = small_layer()
    print("[no-alloc] call 1: 128 experts, d 2816, pre-norm", flush=True)
    want, got, _ = both(L, synth.tokens(61, 1)[0], flags=hip.PRE_NORM)
    assert np.array_equal(got, want)
    print("[no-alloc] call 2: 16 experts, d 512", flush=True)
    want, got, _ = both(small, synth.tokens(62, 1, d=small.d)[0])
    assert np.array_equal(got, want)
    print("[no-alloc] call 3: 128 experts, tied router rows (the exact path, correction rows)", flush=True)
    x = synth.tokens(51, 1)[0]
    r2, b2, spec, ex, _ = rc.find_case(orc, router, bias, x, "tie", seed=1)
    L.router.upload(r2)
    L.bias.upload(b2)
    try:
        want, got, fb = both(L, x)
    finally:
        L.router.upload(router)
        L.bias.upload(bias)
    assert fb == 1
    assert np.array_equal(got, want)


@pytest.mark.gpu
def test_static_decode_graph_replays(gpu):
    L = get_layer(0)[0]
    n = 3
    x = synth.tokens(63, n)
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
            moe.decode_static(L, xd, out, x_off=t * D * 4, out_off=t * D * 4)
        g = hip.Graph.end()
        for rep in range(3):
            out.upload(np.zeros(n * D, np.float32))
            g.launch()
            assert np.array_equal(out.download(np.float32, n * D), want), rep
            moe.decode_static(L, xd, eager, x_off=D * 4)  # eager work on the same scratch between replays
            hip.sync()
        g.close()
    finally:
        hip.Stream.use_default()
        hip.sync()
        s.close()
