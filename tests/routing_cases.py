"""Router rows built on the CPU to force each outcome of the decode selection's exactness check.

The decode path ranks the experts by S, the f64 sum of the reference's f32 products
W_r[e][i] * x[i] (plus the bias), keyed by the f32 value of S; it certifies that ranking, or
recomputes the selection in the reference's order (runtime/src/ops.rs:321-326 fold, exec.rs:507-517
softmax and top-k). The experts that the gate/up workgroups compute come from the S ranking
("spec" ids; experts 0 .. k-1 when two f32 keys at the top ranks tie), and workgroup 0 maps the
reference's selection onto them, computing any expert the ranking missed itself.

A near-copy of one expert's router row, placed in another expert's row, makes the two logits
differ by a few f32 ulps, where the f64 sum and the sequential f32 fold can order them
differently. `find_case` searches small perturbations of such a copy until the S ranking and
the oracle's selection show the requested outcome:

- "swap_set": the S ranking's top k holds an expert that the reference does not select (the
  reference's k-th expert must be computed in a correction row);
- "reorder": the same experts, in another slot order (the down fold reads moved h rows);
- "tie": two experts of the top k have equal f32 keys, so every gate/up workgroup computes
  experts 0 .. k-1 and the selected ones come from correction rows.
"""
from __future__ import annotations

import numpy as np


def s_keys(router: np.ndarray, bias, x: np.ndarray):
    """f32 keys of S per expert (the f32 products summed in f64, the bias added in f64), S, and
    a bound on how far another f64 summation order can move S: any order of n terms is within
    (n - 1) 2^-53 sum|p| of the exact sum, so two orders are within twice that, and the bias
    add rounds once more."""
    p = (router.astype(np.float32) * x.astype(np.float32)[None, :]).astype(np.float64)
    s = p.sum(axis=1)
    bnd = 2.0 * (p.shape[1] - 1) * 2.0 ** -53 * np.abs(p).sum(axis=1)
    if bias is not None:
        s = s + np.asarray(bias, np.float64)
        bnd = bnd * (1 + 2.0 ** -52) + np.abs(s) * 2.0 ** -52
    return s.astype(np.float32), s, bnd


def s_ranking(router, bias, x, top_k):
    """(spec ids, ties, robust): the ids every gate/up workgroup computes. The rank of an
    expert is the number of experts with a larger f32 key; a rank below top_k held by more than
    one expert is a tie. robust is False when the f64 sum of an expert that can take part in
    ranks 0 .. top_k - 1 lies so close to an f32 rounding boundary that another summation order
    could round it to another key. Those are the experts whose key is at least the (top_k + 1)-th
    largest: a key strictly below that one moves by at most one f32 step under another order and
    stays below the top_k-th key."""
    keys, s, bnd = s_keys(router, bias, x)
    near = keys >= np.sort(keys)[::-1][top_k]
    robust = np.array_equal(np.float32(s + bnd)[near], keys[near]) and np.array_equal(np.float32(s - bnd)[near],
                                                                                       keys[near])
    rank = np.array([(keys > k).sum() for k in keys])
    hits = [int((rank == r).sum()) for r in range(top_k)]
    ties = any(h != 1 for h in hits)
    if ties:
        return list(range(top_k)), True, robust
    return [int(np.where(rank == r)[0][0]) for r in range(top_k)], False, robust


def exact_selection(orc, router, bias, x, top_k):
    n_exp, d = router.shape
    lg = orc.router_logits(router, bias, x[None, :], n_exp, d)
    ids, w, _ = orc.select_experts(lg, top_k)
    return [int(v) for v in ids[0]], w[0], lg[0]


def find_case(orc, router, bias, x, kind, seed=0, top_k=8, tries=4000):
    """A copy of router with row b replaced by a perturbed copy of row a (and, with a bias,
    bias[b] by bias[a]), such that the decode selection meets `kind` for token x. Returns
    (router, bias, spec ids, exact ids, (a, b))."""
    rng = np.random.default_rng(seed)
    exact, _, _ = exact_selection(orc, router, bias, x, top_k)
    n_exp = router.shape[0]
    outside = [e for e in range(n_exp) if e not in exact]
    src_rank = {"swap_set": top_k - 1, "reorder": top_k // 2, "tie": 1}[kind]
    a = exact[src_rank]
    for t in range(tries):
        b = outside[rng.integers(len(outside))]
        r2 = router.copy()
        b2 = None if bias is None else np.array(bias, np.float32)
        if b2 is not None:
            b2[b] = b2[a]
        if kind == "tie":
            r2[b] = r2[a]
        else:
            sigma = 10.0 ** rng.uniform(-10.5, -8.0)
            r2[b] = (r2[a] + rng.standard_normal(r2.shape[1]) * sigma).astype(np.float32)
        spec, ties, robust = s_ranking(r2, b2, x, top_k)
        if not robust:
            continue
        ex, _, _ = exact_selection(orc, r2, b2, x, top_k)
        if kind == "tie":
            ok = ties and set(ex) != set(range(top_k))
        elif kind == "swap_set":
            ok = not ties and set(spec) != set(ex) and a in ex and b in spec
        else:
            ok = not ties and set(spec) == set(ex) and spec != ex and a in ex and b in ex
        if ok:
            return r2, b2, spec, ex, (a, b)
    raise RuntimeError(f"no {kind} case found in {tries} tries")
