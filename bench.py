#!/usr/bin/env python3
"""MoE-layer decode throughput on one MI355X: the batch-1 decode workload of 10k back-to-back
tokens through one quantized MoE layer (128 experts, top-8, d = 2816, ff = 704, Q4_0 weights,
Q8_0 activations, GeGLU, f32 slot-order combine), each token a fresh x ~ N(0, 1) with iid
router logits (W_r ~ N(0, 0.02)).

A step is one token through the layer (router, top-8, gate_up, GeGLU, down, combine). All
inputs are resident in HBM before timing; the tokens are replayed from captured HIP graphs on
one stream and timed with HIP events on that stream. One JSON line is printed.

Roofline: the algorithmic bytes of one token are the 8 selected experts' Q4_0 weights
(8 x 3,345,408 B) plus the f32 router (1,441,792 B) = 28,205,056 B; achieved = bytes / time per
token, against MI355X's 8 TB/s HBM peak.

cpu_baseline: the reference's CPU expert path (oracle/cpu_baseline.c: persistent worker pool,
avx2_q8 kernel) on this host's cores for a bounded sample of the same token stream.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer decode tokens/s + achieved HBM GB/s (% of peak), batch 1"
HBM_PEAK_GBS = 8000.0
EXPERT_BYTES = 2816 // 32 * 18 * 1408 + 704 // 32 * 18 * 2816  # 3,345,408
ROUTER_BYTES = 128 * 2816 * 4  # 1,441,792
# HBM bytes one decode call moves (read + written), from rocprofv3 FETCH_SIZE and WRITE_SIZE passes over
# this workload calibrated against a device copy of known size (profiles/decode_hbm_traffic.md).
MEASURED_TRAFFIC = 33_696_704


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_baseline(seed: int, n_tokens: int, seconds: float, threads: int):
    import numpy as np

    from oracle import oracle as orc
    from rosevine_amd import hip, synth

    gu = hip.synth_q4_host(synth.N_EXP, 2 * synth.FF, synth.D, seed, synth.gate_up_stream(0))
    dn = hip.synth_q4_host(synth.N_EXP, synth.D, synth.FF, seed, synth.down_stream(0))
    gu_rows = gu.reshape(synth.N_EXP, -1)
    dn_rows = dn.reshape(synth.N_EXP, -1)
    router = synth.router_weights(seed, 0)
    x = synth.tokens(seed, n_tokens)
    pool = orc.CpuBaseline(threads)
    pool.prepare({e: gu_rows[e] for e in range(synth.N_EXP)}, {e: dn_rows[e] for e in range(synth.N_EXP)},
                 synth.N_EXP)
    out = np.empty((1, synth.D), np.float32)
    ids = np.empty((1, synth.TOP_K), np.uint32)
    w = np.empty((1, synth.TOP_K), np.float32)
    for t in range(2):  # warmup
        pool.layer(router, None, None, x[t], synth.D, synth.FF, synth.TOP_K, out, ids, w)
    done, t0 = 0, time.perf_counter()
    while done < n_tokens and time.perf_counter() - t0 < seconds:
        pool.layer(router, None, None, x[done], synth.D, synth.FF, synth.TOP_K, out, ids, w)
        done += 1
    dt = time.perf_counter() - t0
    pool.close()
    return {"value": round(done / dt, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{done} decode tokens of the same workload in {dt:.1f} s "
                      f"({'avx2_q8' if orc.CpuBaseline.uses_avx2() else 'scalar'} kernel, {threads} threads)"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10000, help="timed tokens")
    ap.add_argument("--warmup", type=int, default=200, help="untimed tokens")
    ap.add_argument("--graph-chunk", type=int, default=500, help="tokens per captured graph")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline sample time")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only copy this many bytes device-to-device 5 times (the calibration of the HBM "
                         "byte counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the MoE path runs on one "
              "MI355X; see the sharding notes in DESIGN.md)", file=sys.stderr)
        return 2

    import numpy as np

    from rosevine_amd import hip, moe, synth

    hip.init(0)
    if args.copy_bytes:
        a, b = hip.DevBuf(args.copy_bytes), hip.DevBuf(args.copy_bytes)
        for _ in range(5):
            hip.copy(b, a, args.copy_bytes)
        hip.sync()
        log(f"[bench] copied {args.copy_bytes} bytes 5 times")
        return 0
    K, W = args.steps, args.warmup
    log(f"[bench] layer 128x(1408x2816 + 2816x704) Q4_0, tokens {W}+{K}")
    router = synth.router_weights(args.seed, 0)
    layer = moe.MoeLayer(synth.N_EXP, synth.TOP_K, synth.D, synth.FF, router)
    layer.synth_weights(args.seed, synth.gate_up_stream(0), synth.down_stream(0))
    x = synth.tokens(args.seed + 100, W + K)
    xd = hip.DevBuf.from_array(x)
    out = hip.DevBuf((W + K) * synth.D * 4)
    ws = moe.Workspace(layer, 1)
    hip.sync()

    stream = hip.Stream()
    stream.use()
    nb = synth.D * 4

    def capture(t0: int, n: int) -> hip.Graph:
        hip.Graph.begin()
        for t in range(t0, t0 + n):
            moe.decode(layer, xd, out, ws, x_off=t * nb, out_off=t * nb)
        return hip.Graph.end()

    ch = max(1, args.graph_chunk)
    warm = [capture(t, min(ch, W - t)) for t in range(0, W, ch)]
    timed = [capture(W + t, min(ch, K - t)) for t in range(0, K, ch)]
    log(f"[bench] captured {len(warm) + len(timed)} graphs")
    for g in warm:
        g.launch()
    hip.sync()
    fb0 = ws.fallbacks()

    e0, e1 = hip.Event(), hip.Event()
    hip.sync()
    e0.record()
    for g in timed:
        g.launch()
    e1.record()
    e1.synchronize()
    hip.sync()
    ms = e0.elapsed_ms(e1)
    fallbacks = ws.fallbacks() - fb0
    for g in warm + timed:
        g.close()
    hip.Stream.use_default()
    stream.close()
    y = out.download(np.float32, synth.D, offset=(W + K - 1) * nb)
    if not np.all(np.isfinite(y)):
        log("[bench] non-finite output")
        return 1

    ms_per_step = ms / K
    tok_s = K / (ms / 1e3)
    bytes_tok = synth.TOP_K * EXPERT_BYTES + ROUTER_BYTES
    achieved = bytes_tok / (ms_per_step / 1e3) / 1e9
    log(f"[bench] {ms_per_step * 1e3:.2f} us/token, {tok_s:.0f} tokens/s, {achieved:.0f} GB/s, "
        f"router fallbacks {fallbacks}/{K}")

    cpu = None
    if not args.no_cpu:
        threads = max(1, min(os.cpu_count() or 1, 16))
        log(f"[bench] CPU baseline on {threads} threads for up to {args.cpu_seconds} s")
        cpu = cpu_baseline(args.seed, 100000, args.cpu_seconds, threads)

    line = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xint8->int32, f32",
        "data": "synthetic (seeded Q4_0 experts, N(0,1) tokens, N(0,0.02) router)",
        "config": {"workload": "single MoE layer, batch-1 decode, 10k back-to-back tokens, iid routing",
                   "n_exp": synth.N_EXP, "top_k": synth.TOP_K, "d": synth.D, "ff": synth.FF,
                   "tokens": K, "graph_tokens": ch, "router_fallbacks": fallbacks},
        "roofline": {"bound": "hbm", "kernel": "rvm_moe_decode (k_router + k_gateup_decode + k_down_fold)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": MEASURED_TRAFFIC,
                     "bytes_per_launch": bytes_tok},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
