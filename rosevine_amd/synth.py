"""Seeded synthetic MoE workloads (the benchmark and test inputs; no model artifact is used).

Shapes follow the reference's MoE contract: 128 experts, top-8, d = 2816, expert ff = 704,
gate and up fused into one 1408-row Q4_0 matrix per expert (runtime/src/contract.rs:12-22,
66-70; runtime/src/model.rs:33-40).

- Q4_0 experts: the counter-based generator of rvm_synth_q4 (scale f16(U(0.005, 0.02)), uniform
  nibble bytes); layer l's gate_up experts use streams gate_up_stream(l) + e, its down experts
  down_stream(l) + e, so any expert can be regenerated on the host alone (rvm_synth_q4_host).
- Router W_r ~ N(0, 0.02), tokens x ~ N(0, 1), per-expert router bias ~ N(0, 1): numpy PCG64
  streams keyed by (seed, layer, purpose).
- Zipf(s) popularity: a per-expert logit bias -s * ln(1 + rank(e)), with a seeded rank order.
"""
from __future__ import annotations

import numpy as np

N_EXP, TOP_K, D, FF = 128, 8, 2816, 704


def gate_up_stream(layer: int) -> int:
    return (2 * layer) << 32


def down_stream(layer: int) -> int:
    return (2 * layer + 1) << 32


def router_weights(seed: int, layer: int, n_exp: int = N_EXP, d: int = D) -> np.ndarray:
    rng = np.random.default_rng([seed, layer, 1])
    return rng.standard_normal((n_exp, d), dtype=np.float32) * np.float32(0.02)


def router_bias(seed: int, layer: int, n_exp: int = N_EXP) -> np.ndarray:
    rng = np.random.default_rng([seed, layer, 2])
    return rng.standard_normal(n_exp, dtype=np.float32)


def zipf_bias(seed: int, n_exp: int = N_EXP, s: float = 1.1) -> np.ndarray:
    rng = np.random.default_rng([seed, 0, 5])
    rank = rng.permutation(n_exp)
    return (-s * np.log1p(rank)).astype(np.float32)


def tokens(seed: int, n_tok: int, d: int = D, stream: int = 3) -> np.ndarray:
    rng = np.random.default_rng([seed, stream])
    return rng.standard_normal((n_tok, d), dtype=np.float32)


def host_expert(seed: int, stream0: int, e: int, n_out: int, k: int) -> np.ndarray:
    """Expert e of a generated stack, in the reference Q4_0 row layout."""
    from . import hip
    return hip.synth_q4_host(1, n_out, k, seed, stream0 + e)
