"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

On the CPU: the oracle still reproduces every fixture bit for bit. On the GPU: the HIP path
reproduces them through the C ABI (codecs and block sums bit-exact, expert ids bit-exact,
layer outputs within max-abs 1e-3 (and 2e-5) of their RMS), with no oracle call at run time.
"""
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
NAMES = ["codecs", "q4q8", "layer"]


def load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def same_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype != b.dtype or a.shape != b.shape:
        return False
    if a.dtype.kind == "f":
        return np.array_equal(a.view(np.uint8), b.view(np.uint8))
    return np.array_equal(a, b)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_the_fixture(orc, name):
    from golden import make_golden
    want = load(name)
    got = make_golden.make(name)
    assert sorted(got) == sorted(want)
    for k in want:
        assert same_bits(got[k], want[k]), f"{name}.{k} changed"


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


@pytest.mark.gpu
def test_gpu_codecs_fixture(gpu):
    from rosevine_amd import hip
    from rosevine_amd.hip import DevBuf
    f = load("codecs")
    x = f["x"]
    xq = DevBuf(f["xq"].nbytes)
    hip.quantize_q8_0(DevBuf.from_array(x), xq, x.shape[0], x.shape[1])
    assert np.array_equal(xq.download(np.uint8, f["xq"].size).reshape(f["xq"].shape), f["xq"])


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["gate_up", "rows32"])
def test_gpu_q4q8_fixture(gpu, fmt):
    from rosevine_amd import hip
    from rosevine_amd.hip import DevBuf
    f = load("q4q8")
    n_out, k = int(f["n_out"]), int(f["k"])
    form = hip.PACK_GATE_UP if fmt == "gate_up" else hip.PACK_ROWS32
    packed = DevBuf(hip.q4_packed_bytes(1, n_out, k, form))
    hip.pack_q4(DevBuf.from_array(f["w"]), packed, 1, n_out, k, form)
    xq = DevBuf.from_array(f["xq"])
    y = DevBuf(2 * n_out * 4)
    hip.q4q8_mm(packed, form, xq, y, n_out, k, 2)
    assert same_bits(y.download(np.float32, 2 * n_out).reshape(2, n_out), f["y"])
    sums = DevBuf(n_out * (k // 32) * 4)
    hip.q4q8_block_sums(packed, form, xq, sums, n_out, k)
    assert np.array_equal(sums.download(np.int32, n_out * (k // 32)).reshape(n_out, -1), f["sums"])


@pytest.mark.gpu
def test_gpu_layer_fixture(gpu):
    from rosevine_amd import hip, moe
    from rosevine_amd.hip import DevBuf
    f = load("layer")
    n_exp, top_k, d, ff, n_tok = (int(v) for v in f["shape"])
    L = moe.MoeLayer(n_exp, top_k, d, ff, f["router"], f["bias"], f["down_scale"])
    L.load_q4(f["gate_up"], f["down"])
    ws = moe.Workspace(L, n_tok)
    x = DevBuf.from_array(f["x"])
    out = DevBuf(n_tok * d * 4)
    moe.forward(L, x, out, n_tok, ws)
    ids, w = ws.selection(L, n_tok)
    assert np.array_equal(ids, f["ids"])
    got = out.download(np.float32, n_tok * d).reshape(n_tok, d)
    err, r = float(np.max(np.abs(got - f["out"]))), rms(f["out"])
    assert err <= 1e-3 * r and err <= 2e-5 * r, (err, r)
    # each token alone through the decode entry point gives the same rows bit for bit
    for t in range(n_tok):
        o1 = DevBuf(d * 4)
        moe.decode(L, x, o1, ws, x_off=t * d * 4)
        assert same_bits(o1.download(np.float32, d), got[t])
    # exact selection: the logits are the reference's bits
    ids2, w2, lg = moe.router_select(L, x, n_tok, ws, flags=hip.EXACT_SELECT, with_logits=True)
    assert np.array_equal(ids2, f["ids"])
    assert same_bits(np.asarray(lg, np.float32).reshape(n_tok, n_exp), f["logits"])
