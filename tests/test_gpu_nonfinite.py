"""Non-finite router inputs on the HIP path, compared with the oracle.

The reference's top-4 (moe_router_topk_kernel, layer.cu:452-476) inserts a
score only when it is strictly above the running fourth score, which starts at
the -1e30 sentinel: a NaN score (NaN logit, or NaN bias) or a score <= -1e30
(a -inf or -1e30 bias) is never selected, and a token with fewer than four
selectable experts keeps -1 / 0.0 in the empty ranks.  A token with no
selectable expert gets the empty combine sum: y = residual + 0.0f.

Both routers are covered: the expert-split decode router (T <= 256, top-4 as a
rank count) and the 64-token router (T > 256, and every moe_route_logits call).
moe_forward of 21-256 tokens under the 32/64-row plans routes from score
bounds: a row with a non-finite input or bias has infinite bounds, so every
expert stays possible for it and gets a slot (up to 32 per token), and the
expert kernel's exact routing picks from the logits (T=64, 200 and the forced
plans below; all 32 for every token in test_forward_no_expert_selected at
T=8 under the 64-row plan).
Routing (idx, w, counts) is compared bit for bit; y within rtol 1e-3 /
atol 1e-4 with NaN positions equal (rows of tokens whose inputs hold +-inf are
NaN in both).
"""
import sys

import numpy as np
import pytest

from conftest import bits

RTOL, ATOL = 1e-3, 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def block(real_weights):
    from final_amd import SparseMoeBlock
    w = real_weights
    b = SparseMoeBlock(max_tokens=2048)
    b.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
    yield b
    b.close()


def check_routing(rt, idx, w, counts):
    assert np.array_equal(rt["idx"], idx), "routing indices differ"
    assert np.array_equal(rt["counts"], counts), "expert counts differ"
    assert np.array_equal(bits(rt["w"]), bits(w)), "routing weights differ"


def crafted_logits(T, seed):
    """Logit rows cycling through: all NaN; NaN but for two experts; +inf on
    three experts and -inf elsewhere with one NaN; all equal (ties); all -inf
    (p = 0, the bias decides); finite."""
    rng = np.random.RandomState(seed)
    lg = (rng.randn(T, 32) * 2.0).astype(np.float32)
    for t in range(T):
        kind = t % 6
        if kind == 0:
            lg[t, :] = np.nan
        elif kind == 1:
            keep = rng.choice(32, 2, replace=False)
            row = np.full(32, np.nan, np.float32)
            row[keep] = lg[t, keep]
            lg[t] = row
        elif kind == 2:
            lg[t, :] = -np.inf
            lg[t, rng.choice(32, 3, replace=False)] = np.inf
            lg[t, rng.randint(32)] = np.nan
        elif kind == 3:
            lg[t, :] = 0.5
        elif kind == 4:
            lg[t, :] = -np.inf
    return lg


@pytest.mark.gpu
@pytest.mark.parametrize("T", [6, 300])
def test_route_logits_nonfinite(T, block, real_weights, oracle_mod):
    from final_amd import hip
    lg = crafted_logits(T, seed=T)
    say(f"[nonfinite logits] T={T}")
    dl = hip.DeviceArray.from_numpy(lg)
    block.route_logits(dl, T)
    rt = block.last_routing()
    idx, w, counts = oracle_mod.route(lg, real_weights["bias"])
    check_routing(rt, idx, w, counts)
    assert (idx[::6] == -1).all(), "an all-NaN row selects nothing"
    assert (idx[1::6, 2:] == -1).all() and (idx[1::6, :2] >= 0).all()


def nonfinite_bias(base):
    """Experts 0-5 NaN, 6-11 -inf, 12 exactly -1e30: none selectable; the
    other 19 keep their bias."""
    b = np.array(base, np.float32).copy()
    b[0:6] = np.nan
    b[6:12] = -np.inf
    b[12] = np.float32(-1e30)
    return b


def nonfinite_x(T, seed):
    """Token rows: every 7th holds a NaN (all logits NaN: no expert); every
    7th from 3 holds +inf and -inf (each logit NaN or +-inf); the rest
    N(0, 1)."""
    from final_amd import workloads as W
    x = W.gen_x(T, seed=seed)
    x[0::7, 5] = np.nan
    x[3::7, 100] = np.inf
    x[3::7, 901] = -np.inf
    return x


@pytest.mark.gpu
@pytest.mark.parametrize("T,plan", [(1, -1), (8, -1), (64, -1), (200, -1), (300, -1),
                                    (1000, -1), (8, 64), (300, 0), (200, 32)])
def test_forward_nonfinite(T, plan, block, real_weights, oracle_mod):
    """NaN / -inf / -1e30 biases and NaN / +-inf token rows through
    moe_forward with a residual: routing bit-exact on every token, y within
    tolerance (NaN where the oracle has NaN)."""
    from final_amd import hip
    from final_amd import workloads as W
    w = dict(real_weights)
    w["bias"] = nonfinite_bias(real_weights["bias"])
    block.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
    block.force_tile_rows(plan)
    try:
        x = nonfinite_x(T, seed=60 + T)
        r = W.gen_x(T, seed=61 + T)
        say(f"[nonfinite forward] T={T} plan={block.plan(T)}")
        dx = hip.DeviceArray.from_numpy(x)
        dr = hip.DeviceArray.from_numpy(r)
        dy = hip.DeviceArray((T, W.H))
        block.forward_gpu(dx, dy, T, residual=dr)
        hip.synchronize()
        block.check_device()
        rt = block.last_routing()
        y = dy.download()
    finally:
        block.force_tile_rows(-1)
        rw = real_weights
        block.set_weights(rw["gate"], rw["bias"], rw["w1"], rw["w3"], rw["w2"])
    ref = oracle_mod.moe_forward(x, w["gate"], w["bias"], w["w1"], w["w3"], w["w2"], residual=r)
    check_routing(rt, ref["idx"], ref["w"], ref["counts"])
    assert (ref["idx"][ref["idx"] >= 0] >= 13).all(), "experts 0-12 are never selectable"
    assert (ref["idx"][0::7] == -1).all()
    np.testing.assert_allclose(y, ref["y"], rtol=RTOL, atol=ATOL, equal_nan=True)
    # a token with no expert keeps its residual (plus 0.0f)
    np.testing.assert_array_equal(y[0::7], r[0::7] + np.float32(0.0))


@pytest.mark.gpu
@pytest.mark.parametrize("T,plan", [(8, -1), (8, 64), (300, -1), (128, 0)])
def test_forward_no_expert_selected(T, plan, block, real_weights, oracle_mod):
    """Every token row NaN: no expert is selected anywhere (no slot, no row
    task).  Every kernel plan must still finish and write y = residual + 0."""
    from final_amd import hip
    from final_amd import workloads as W
    block.force_tile_rows(plan)
    try:
        x = np.full((T, W.H), np.nan, np.float32)
        r = W.gen_x(T, seed=70 + T)
        say(f"[no expert] T={T} plan={block.plan(T)}")
        dx = hip.DeviceArray.from_numpy(x)
        dr = hip.DeviceArray.from_numpy(r)
        dy = hip.DeviceArray((T, W.H))
        block.forward_gpu(dx, dy, T, residual=dr)
        hip.synchronize()
        block.check_device()
        rt = block.last_routing()
    finally:
        block.force_tile_rows(-1)
    assert (rt["idx"] == -1).all() and (rt["counts"] == 0).all()
    assert (bits(rt["w"]) == 0).all()
    np.testing.assert_array_equal(dy.download(), r + np.float32(0.0))
