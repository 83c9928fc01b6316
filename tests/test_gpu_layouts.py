"""Every MFMA tile layout and unit order of the expert kernel, pinned by
expert row counts chosen at their boundaries.

Routing comes from crafted logits (moe_route_logits): each token's four
experts get logits 2..5, the others -4, so the per-expert counts are exactly
the ones asked for.  Under the forced 64-row plan the counts 1-16, 17-32,
33-48, 49-64 take the 16-row skinny, narrow, 3-block skinny and wide layouts
(and counts above 64 add units of each size); under the forced 128-row plan
units of at most 64 rows run as 64-row tiles, 65-80 rows as 5-block 16-row
skinny tiles, 81-96 as narrow tiles over three row blocks, 97-112 as 7-block
skinny tiles, 113-127 as wide tiles, 128 as full tiles, and the last units'
gate/up and down tiles as half-width tiles (the 128-row plan splits the
last units' gate/up tiles up to 1024 tokens, the 64-row plan up to 128).  A
second count set, with
every expert under 64 tokens, takes the longest-first unit order of the
64-row plan.  The reference y comes from the oracle's own routing of the same
logits, dispatch, expert and combine functions.
"""
import sys

import numpy as np
import pytest

from conftest import bits

RTOL, ATOL = 1e-3, 1e-4
E, K = 32, 4

# counts at the layout boundaries (mixed sizes) and a set of small experts
MIXED = [1, 2, 15, 16, 17, 20, 31, 32, 33, 40, 47, 48, 49, 56, 63, 64,
         65, 72, 80, 95, 96, 97, 112, 127, 128, 129, 160, 192, 200, 255, 256, 0]
SMALL = [1, 3, 8, 15, 16, 17, 18, 24, 31, 32, 33, 34, 40, 47, 48, 49,
         50, 55, 60, 63, 64, 5, 9, 12, 20, 28, 36, 44, 52, 58, 61, 0]


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def routing_for_counts(counts):
    """Token -> 4 distinct experts such that expert e is chosen by exactly
    counts[e] tokens (the last nonzero count is adjusted so the sum is a
    multiple of 4).  Returns (T, choice [T][4], counts)."""
    counts = list(counts)
    s = sum(counts)
    last = max(i for i, c in enumerate(counts) if c > 0)
    counts[last] += (-s) % K
    T = sum(counts) // K
    assert max(counts) <= T
    free = [K] * T
    choice = [[] for _ in range(T)]
    for e in sorted(range(E), key=lambda i: (-counts[i], i)):
        # the tokens with the most free slots take this expert
        toks = sorted(range(T), key=lambda t: (-free[t], t))[:counts[e]]
        for t in toks:
            choice[t].append(e)
            free[t] -= 1
    assert all(f == 0 for f in free)
    return T, np.array(choice, np.int32), counts


def crafted_logits(choice, seed):
    T = choice.shape[0]
    rng = np.random.default_rng(seed)
    lg = np.full((T, E), -4.0, np.float32)
    for t in range(T):
        lg[t, choice[t]] = rng.permutation(np.array([2.0, 3.0, 4.0, 5.0], np.float32))
    return lg


def oracle_from_logits(O, w, x, logits, residual):
    idx, wt, counts = O.route(logits, w["bias"])
    offsets, pos, slot_token = O.dispatch(idx, E)
    S = int(offsets[E])
    sorted_out = np.zeros((S, x.shape[1]), np.float32)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi > lo:
            rows = np.ascontiguousarray(x[slot_token[lo:hi]])
            inter = O.expert_w1w3(rows, w["w1"][e], w["w3"][e])
            sorted_out[lo:hi] = O.expert_w2(inter, w["w2"][e])
    y = O.combine(sorted_out, pos, wt, residual)
    return idx, wt, counts, y


def test_routing_for_counts_is_exact():
    for cs in (MIXED, SMALL):
        T, choice, counts = routing_for_counts(cs)
        got = np.bincount(choice.reshape(-1), minlength=E)
        assert list(got) == counts
        assert all(len(set(r)) == K for r in choice.tolist())


@pytest.mark.gpu
@pytest.mark.parametrize("name,cs,plan", [("mixed", MIXED, 64), ("mixed", MIXED, 128),
                                          ("small", SMALL, 64), ("small", SMALL, 128)])
def test_tile_layouts(name, cs, plan, real_weights, oracle_mod):
    from final_amd import SparseMoeBlock, hip
    from final_amd import workloads as W
    w = real_weights
    T, choice, counts = routing_for_counts(cs)
    lg = crafted_logits(choice, seed=plan)
    x = W.gen_x(T, seed=70 + plan)
    r = W.gen_x(T, seed=71 + plan)
    say(f"[layouts] counts={name} T={T} forced plan={plan}")
    blk = SparseMoeBlock(max_tokens=T)
    try:
        blk.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
        blk.force_tile_rows(plan)
        dl = hip.DeviceArray.from_numpy(lg)
        dx = hip.DeviceArray.from_numpy(x)
        dr = hip.DeviceArray.from_numpy(r)
        dy = hip.DeviceArray((T, W.H))
        blk.route_logits(dl, T)
        blk.experts(dx, dy, T, residual=dr)
        hip.synchronize()
        blk.check_device()
        rt = blk.last_routing()
        y = dy.download()
    finally:
        blk.close()
    idx, wt, rcounts, ref = oracle_from_logits(oracle_mod, w, x, lg, r)
    assert list(rcounts) == counts
    assert np.array_equal(rt["idx"], idx) and np.array_equal(rt["counts"], rcounts)
    assert np.array_equal(bits(rt["w"]), bits(wt))
    np.testing.assert_allclose(y, ref, rtol=RTOL, atol=ATOL)
