"""Where one decode token's time goes: the phase stamps of the diagnostic build.

Build and run (from the repository root, on a GPU):

    python -m rosevine_amd.build --trace
    RVM_LIB=rosevine_amd/librvmoe_trace.so python -m rosevine_amd.phase_trace [--tokens 64]

The decode workload of bench.py (one layer: 128 experts, top-8, d = 2816, ff = 704; fresh
x ~ N(0, 1) per token) is captured as one graph of --tokens back-to-back decode calls and replayed;
after the last replay the stamps of its last call are read (rvm_phase_trace): every workgroup of
k_router, k_gateup_decode and k_down_fold records the 100 MHz realtime counter at its entry and at
the points named below. The last call is a token whose router certificate passes, then (in a
second graph) one whose certificate fails, so that workgroup 0 computes the exact selection.
Printed: each point's earliest, median and latest workgroup, in microseconds from the first
k_router workgroup's entry, and the graph's event time per call.
The stamps cost a few vector stores per workgroup; the diagnostic build is for this table only.
"""
from __future__ import annotations

import argparse
import sys

import numpy as np

from . import hip, moe, synth

TRACE_WG, TRACE_PT = 4096, 8

# (kernel index, point, label, workgroups: "all", "stats" (the router's statistics workgroups),
# "tiles" (gate/up workgroups 1..), "wg0")
POINTS = [
    (0, 0, "k_router entry", "all"),
    (0, 2, "k_router: router row and x loaded (statistics workgroups)", "stats"),
    (0, 1, "k_router done (statistics or Q8_0 blocks stored)", "all"),
    (1, 0, "k_gateup_decode entry", "all"),
    (1, 1, "tile: expert known (ranking done)", "tiles"),
    (1, 2, "tile: wave 0's block terms formed (its weights arrived)", "tiles"),
    (1, 3, "tile: h block ready (all waves' weights, fold, GeGLU, Q8_0)", "tiles"),
    (1, 4, "tile: down terms stored", "tiles"),
    (1, 1, "workgroup 0: ranking and certificate done", "wg0"),
    (1, 2, "workgroup 0: ids and weights published", "wg0"),
    (2, 0, "k_down_fold entry", "all"),
    (2, 3, "k_down_fold: down terms loaded", "all"),
    (2, 1, "k_down_fold: slot rows folded", "all"),
    (2, 2, "k_down_fold: output stored", "all"),
]


def read_stamps() -> np.ndarray:
    buf = np.zeros(3 * TRACE_WG * TRACE_PT, np.uint64)
    rc = hip.lib().rvm_phase_trace(buf.ctypes.data, buf.nbytes)
    if rc != 0:
        raise SystemExit(f"rvm_phase_trace returned {rc}: load the diagnostic build "
                         "(python -m rosevine_amd.build --trace; RVM_LIB=rosevine_amd/librvmoe_trace.so)")
    return buf.reshape(3, TRACE_WG, TRACE_PT).astype(np.int64)


def trace_token(L, ws, x, out, n: int, last: int):
    """Graph of n decode calls (tokens 0 .. n-2, then token `last`), replayed; the stamps of its last
    call and the graph's event time per call."""
    nb = L.d * 4
    st = hip.Stream()
    st.use()
    hip.Graph.begin()
    for t in list(range(n - 1)) + [last]:
        moe.decode(L, x, out, ws, x_off=t * nb, out_off=0)
    g = hip.Graph.end()
    for _ in range(3):
        g.launch()
    hip.sync()
    e0, e1 = hip.Event(), hip.Event()
    e0.record()
    g.launch()
    e1.record()
    e1.synchronize()
    us_tok = e0.elapsed_ms(e1) * 1e3 / n
    s = read_stamps()
    g.close()
    hip.Stream.use_default()
    st.close()
    return s, us_tok


def table(s: np.ndarray, E: int, K: int, D: int, FF: int) -> None:
    n_router = E + (D // 32 + 1) // 2  # statistics workgroups, then the Q8_0 workgroups
    sizes = [n_router, 1 + K * (2 * FF // 64), D // 32]
    t0 = s[0, :n_router, 0].min()
    print("| point | workgroups | first us | median us | last us |")
    print("| --- | --- | --- | --- | --- |")
    for k, p, label, rng in POINTS:
        v = s[k, :sizes[k], p]
        if rng == "tiles":
            v = v[1:]
        elif rng == "stats":
            v = v[:E]
        elif rng == "wg0":
            v = v[:1]
        us = (v - t0) * 0.01
        print(f"| {label} | {len(v)} | {us.min():.2f} | {np.median(us):.2f} | {us.max():.2f} |")


def stack_trace(seed: int, n: int) -> None:
    """A layer in the middle of a decode stack (router bias, RMSNorm between layers, cold weights): a
    3-layer session evaluated over layers 0 and 1 only (rvm_session_eval_range), so that the stamps
    left are layer 1's, whose router reads layer 0's output. The graph time is per token (two
    layers)."""
    from . import session

    E, K, D, FF = synth.N_EXP, synth.TOP_K, synth.D, synth.FF
    layers = []
    for l in range(3):
        L = moe.MoeLayer(E, K, D, FF, synth.router_weights(seed, l), synth.router_bias(seed, l))
        L.synth_weights(seed, synth.gate_up_stream(l), synth.down_stream(l))
        layers.append(L)
    s = session.Session(layers, max_tokens=1, eps=1e-6)
    x = hip.DevBuf.from_array(synth.tokens(seed + 300, n))
    hip.sync()
    st = hip.Stream()
    st.use()
    hip.Graph.begin()
    for t in range(n):
        s.eval_range(x, None, 1, 0, 2, x_off=t * D * 4)
    g = hip.Graph.end()
    for _ in range(3):
        g.launch()
    hip.sync()
    e0, e1 = hip.Event(), hip.Event()
    e0.record()
    g.launch()
    e1.record()
    e1.synchronize()
    us_tok = e0.elapsed_ms(e1) * 1e3 / n
    v = read_stamps()
    g.close()
    hip.Stream.use_default()
    st.close()
    print(f"\nlayer 1 of a decode stack (last of a {n}-token graph; graph {us_tok:.2f} us per token of 2 layers)")
    table(v, E, K, D, FF)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--tokens", type=int, default=64, help="decode calls per captured graph")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--stack", action="store_true", help="a fused layer in the middle of a decode stack")
    args = ap.parse_args()
    if args.stack:
        stack_trace(args.seed, args.tokens)
        return 0
    E, K, D, FF = synth.N_EXP, synth.TOP_K, synth.D, synth.FF
    L = moe.MoeLayer(E, K, D, FF, synth.router_weights(args.seed, 0))
    L.synth_weights(args.seed, synth.gate_up_stream(0), synth.down_stream(0))
    ws = moe.Workspace(L, 1)
    n = args.tokens
    x = hip.DevBuf.from_array(synth.tokens(args.seed + 100, n))
    out = hip.DevBuf(D * 4)
    hip.sync()
    # which tokens the router certificate passes (the fallback counter counts the others)
    passed, failed = [], []
    for t in range(n):
        f0 = ws.fallbacks()
        moe.decode(L, x, out, ws, x_off=t * D * 4)
        hip.sync()
        (passed if ws.fallbacks() == f0 else failed).append(t)
    passed, failed = (passed or [None])[0], (failed or [None])[0]
    for kind, t in (("certified selection", passed), ("certificate failed: exact selection in workgroup 0", failed)):
        if t is None:
            continue
        s, us_tok = trace_token(L, ws, x, out, n, t)
        print(f"\n{kind} (token {t}, last of a {n}-call graph; graph {us_tok:.2f} us per call)")
        table(s, E, K, D, FF)
    sys.stdout.flush()
    return 0


if __name__ == "__main__":
    sys.exit(main())
