"""The CPU construction of the decode fallback cases (tests/routing_cases.py), checked on the CPU.

For each outcome, the constructed router must give the claimed ranking under the f64 estimate
(computed here independently: exact rational sums of the f32 products, rounded once to f32), and
the claimed selection under the oracle; and the outcome must hold (the expert set changes, the
slot order changes, or two keys tie). These are the preconditions the GPU tests rely on.
"""
from fractions import Fraction

import numpy as np
import pytest

import routing_cases as rc
from rosevine_amd import synth


def exact_keys(router, bias, x):
    """f32 keys of the exact sums (Fractions), rounded once: the ideal the f64 sums approximate."""
    p = router.astype(np.float32) * x.astype(np.float32)[None, :]
    keys = []
    for e in range(router.shape[0]):
        s = sum((Fraction(float(v)) for v in p[e]), Fraction(0))
        if bias is not None:
            s += Fraction(float(np.float32(bias[e])))
        keys.append(np.float32(float(s)))
    return np.array(keys, np.float32)


@pytest.mark.parametrize("kind", ["swap_set", "reorder", "tie"])
@pytest.mark.parametrize("with_bias", [False, True])
def test_constructed_cases_hold(orc, kind, with_bias):
    router = synth.router_weights(0, 0)
    bias = synth.router_bias(0, 0) if with_bias else None
    x = synth.tokens(50, 1)[0]
    r2, b2, spec, ex, (a, b) = rc.find_case(orc, router, bias, x, kind, seed=0)
    assert np.array_equal(np.delete(r2, b, axis=0), np.delete(router, b, axis=0))
    keys, _, _ = rc.s_keys(r2, b2, x)
    assert np.array_equal(keys, exact_keys(r2, b2, x))  # the f64 sums round to the exact sums' keys
    ids, w, lg = rc.exact_selection(orc, r2, b2, x, 8)
    assert ids == ex and len(set(ex)) == 8
    top = sorted(range(len(keys)), key=lambda e: (-float(keys[e]), e))[:9]
    if kind == "tie":
        assert spec == list(range(8))
        assert any(keys[top[i]] == keys[top[i + 1]] for i in range(8))
        assert set(ex) != set(range(8))
    else:
        assert spec == top[:8] and keys[top[7]] > keys[top[8]]
        assert len(set(keys[top[:8]].tolist())) == 8
        if kind == "swap_set":
            assert set(spec) != set(ex) and b in spec and a in ex
        else:
            assert set(spec) == set(ex) and spec != ex
