"""Parity of the HIP path (through the C-ABI) with the CPU oracle.

Bar: routing indices, per-expert counts and gate logits bit-exact; expert
weights bit-exact (same arithmetic as the reference router); y within
rtol 1e-3 / atol 1e-4 in fp32 (the tolerance the MoE block is specified to).
"""
import sys

import numpy as np
import pytest

from conftest import bits

RTOL, ATOL = 1e-3, 1e-4
MAX_TOKENS = 16384


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def block(real_weights):
    from final_amd import SparseMoeBlock
    w = real_weights
    b = SparseMoeBlock(max_tokens=MAX_TOKENS)
    b.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
    yield b
    b.close()


def oracle_forward(O, w, x, residual=None, token_mask=None):
    return O.moe_forward(x, w["gate"], w["bias"], w["w1"], w["w3"], w["w2"],
                         residual=residual, token_mask=token_mask)


def check_routing(rt, ref):
    assert np.array_equal(bits(rt["logits"]), bits(ref["logits"])), "gate logits differ"
    assert np.array_equal(rt["idx"], ref["idx"]), "routing indices differ"
    assert np.array_equal(rt["counts"], ref["counts"]), "expert counts differ"
    assert np.array_equal(bits(rt["w"]), bits(ref["w"])), "routing weights differ"


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 8, 64, 100, 128, 160, 256, 1000, 4096])
def test_forward_matches_oracle(T, block, real_weights, oracle_mod):
    from final_amd import workloads as W
    say(f"[parity] T={T} plan={block.plan(T)}")
    x = W.gen_x(T)
    y = block.forward(x)
    rt = block.last_routing()
    ref = oracle_forward(oracle_mod, real_weights, x)
    check_routing(rt, ref)
    np.testing.assert_allclose(y, ref["y"], rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
@pytest.mark.parametrize("plan", [0, 32, 64, 128])
def test_every_kernel_plan(plan, block, real_weights, oracle_mod):
    from final_amd import workloads as W
    T = 200
    say(f"[plan] T={T} forced plan={plan}")
    x = W.gen_x(T, seed=3)
    block.force_tile_rows(plan)
    try:
        y = block.forward(x)
    finally:
        block.force_tile_rows(-1)
    ref = oracle_forward(oracle_mod, real_weights, x)
    check_routing(block.last_routing(), ref)
    np.testing.assert_allclose(y, ref["y"], rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [6000, 8200])
def test_router_block_splits(T, block, real_weights, oracle_mod):
    """Large batches split each 64-token router block's experts over 4, 2 or 1
    blocks (6000 tokens: 94 token blocks, split in 2; 8200: 129, unsplit;
    4096 in test_forward_matches_oracle: split in 4).  Routing and y checked
    on every token."""
    from final_amd import workloads as W
    say(f"[router split] T={T} plan={block.plan(T)}")
    x = W.gen_x(T, seed=5)
    y = block.forward(x)
    rt = block.last_routing()
    ref = oracle_forward(oracle_mod, real_weights, x)
    check_routing(rt, ref)
    np.testing.assert_allclose(y, ref["y"], rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
def test_zipf_skew_t16384(block, real_weights, oracle_mod):
    """Skewed routing: Zipf(1.2) expert frequencies, 3 empty experts, one expert
    taking nearly every token.  Routing and y checked on all 16384 tokens."""
    from final_amd import workloads as W
    T = 16384
    w = dict(real_weights)
    w["bias"] = W.zipf_bias()
    say(f"[zipf] T={T} plan={block.plan(T)}")
    block.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
    try:
        x = W.gen_x(T)
        y = block.forward(x)
        rt = block.last_routing()
    finally:
        rw = real_weights
        block.set_weights(rw["gate"], rw["bias"], rw["w1"], rw["w3"], rw["w2"])
    ref = oracle_forward(oracle_mod, w, x)
    check_routing(rt, ref)
    assert (rt["counts"] == 0).sum() >= 3
    np.testing.assert_allclose(y, ref["y"], rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
def test_streaming_four_experts(block, real_weights, oracle_mod):
    """Every token routed to the same four experts (bias +10) under the
    weight-streaming plan: few row tasks per expert, so blocks claim down
    tasks of an expert while its gate/up tasks are still running, the case
    where a block must finish its own gate/up task before waiting for the
    down task's inputs.  T = 200 also runs several token groups per task."""
    from final_amd import workloads as W
    w = dict(real_weights)
    bias = np.array(real_weights["bias"], np.float32).copy()
    hot = [3, 7, 19, 28]
    bias[hot] += 10.0
    w["bias"] = bias
    block.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
    block.force_tile_rows(0)
    try:
        for T in (1, 8, 31, 32, 64, 200):
            say(f"[four experts] T={T} plan=0")
            x = W.gen_x(T, seed=11)
            y = block.forward(x)
            rt = block.last_routing()
            ref = oracle_forward(oracle_mod, w, x)
            check_routing(rt, ref)
            assert sorted(np.nonzero(rt["counts"])[0].tolist()) == hot
            np.testing.assert_allclose(y, ref["y"], rtol=RTOL, atol=ATOL)
    finally:
        block.force_tile_rows(-1)
        rw = real_weights
        block.set_weights(rw["gate"], rw["bias"], rw["w1"], rw["w3"], rw["w2"])


@pytest.mark.gpu
@pytest.mark.parametrize("T", [32, 40, 48, 57, 64])
def test_streaming_wide_tasks(T, block, real_weights, oracle_mod):
    """32-64 tokens under the weight-streaming plan (forced: the automatic
    plan takes 64-row MFMA tiles from 11 tokens): 64-row tasks, streamed as
    four 16-row groups that reuse one load of the token rows when every
    expert holds at most 16 tokens, else as four row groups at once over two
    token passes (one expert made hot by a bias so it holds all T tokens)."""
    from final_amd import workloads as W
    assert block.plan(T) == 64
    block.force_tile_rows(0)
    try:
        x = W.gen_x(T, seed=40 + T)
        say(f"[wide tasks] T={T} natural routing, plan=0")
        y = block.forward(x)
        rt = block.last_routing()
        ref = oracle_forward(oracle_mod, real_weights, x)
        check_routing(rt, ref)
        block.check_device()
        np.testing.assert_allclose(y, ref["y"], rtol=RTOL, atol=ATOL)
        w = dict(real_weights)
        bias = np.array(real_weights["bias"], np.float32).copy()
        bias[5] += 2.0
        w["bias"] = bias
        block.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
        say(f"[wide tasks] T={T} expert 5 hot, plan=0")
        y = block.forward(x)
        rt = block.last_routing()
        block.check_device()
    finally:
        block.force_tile_rows(-1)
        rw = real_weights
        block.set_weights(rw["gate"], rw["bias"], rw["w1"], rw["w3"], rw["w2"])
    ref = oracle_forward(oracle_mod, w, x)
    check_routing(rt, ref)
    assert rt["counts"][5] == T
    np.testing.assert_allclose(y, ref["y"], rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
def test_gate_up_half_tiles(block, real_weights, oracle_mod):
    """The 64-row plan up to 128 tokens runs its last eight units' gate/up
    work as two half-width tiles each, and their down tiles wait for both.
    Forced onto that plan: 1 token (four units, all split), 5 tokens, 128
    tokens with natural routing (eight of some 32 units split), and 128
    tokens on four hot experts (two units each: all eight split, two per
    expert)."""
    from final_amd import workloads as W
    hot = [2, 13, 21, 30]
    bias = np.array(real_weights["bias"], np.float32).copy()
    bias[hot] += 10.0
    cases = [(1, None), (5, None), (128, None), (128, bias)]
    block.force_tile_rows(64)
    try:
        for T, b in cases:
            w = dict(real_weights)
            if b is not None:
                w["bias"] = b
            block.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
            say(f"[half tiles] T={T} plan=64 hot={b is not None}")
            x = W.gen_x(T, seed=60 + T)
            y = block.forward(x)
            rt = block.last_routing()
            block.check_device()
            ref = oracle_forward(oracle_mod, w, x)
            check_routing(rt, ref)
            if b is not None:
                assert sorted(np.nonzero(rt["counts"])[0].tolist()) == hot
            np.testing.assert_allclose(y, ref["y"], rtol=RTOL, atol=ATOL)
    finally:
        block.force_tile_rows(-1)
        rw = real_weights
        block.set_weights(rw["gate"], rw["bias"], rw["w1"], rw["w3"], rw["w2"])


@pytest.mark.gpu
def test_residual_fused_and_in_place(block, real_weights, oracle_mod):
    """y = residual + MoE(x) (the decoder layer's add, layer.cu:1917), also
    with y aliasing the residual buffer."""
    from final_amd import hip
    from final_amd import workloads as W
    T = 300
    x = W.gen_x(T, seed=7)
    r = W.gen_x(T, seed=8)
    ref = oracle_forward(oracle_mod, real_weights, x, residual=r)
    dx = hip.DeviceArray.from_numpy(x)
    dr = hip.DeviceArray.from_numpy(r)
    dy = hip.DeviceArray((T, W.H))
    block.forward_gpu(dx, dy, T, residual=dr)
    hip.synchronize()
    np.testing.assert_allclose(dy.download(), ref["y"], rtol=RTOL, atol=ATOL)
    block.forward_gpu(dx, dr, T, residual=dr)  # in place
    hip.synchronize()
    block.check_device()
    np.testing.assert_allclose(dr.download(), ref["y"], rtol=RTOL, atol=ATOL)


def _norm_weight(H):
    return (1.0 + 0.1 * np.random.RandomState(17).randn(H)).astype(np.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 8, 64, 100, 256, 4096])
def test_forward_norm_matches_oracle(T, block, real_weights, oracle_mod):
    """out = h + MoE(rmsnorm(h)) (DecoderLayer steps 4-6, layer.cu:1903-1918):
    the normalised rows and the routing bit-exact, out within tolerance.  T <=
    256 normalises inside the router, larger T in its own kernel."""
    from final_amd import workloads as W
    w = real_weights
    nw = _norm_weight(W.H)
    block.set_norm_weight(nw)
    say(f"[norm] T={T} plan={block.plan(T)}")
    h = W.gen_x(T, seed=21) * np.float32(2.5)
    out = block.forward_norm(h)
    xn = block.last_normed()
    rt = block.last_routing()
    ref = oracle_mod.moe_forward_norm(h, nw, w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
    assert np.array_equal(bits(xn), bits(ref["xn"])), "normalised rows differ"
    check_routing(rt, ref)
    np.testing.assert_allclose(out, ref["y"], rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
def test_forward_norm_in_place(block, real_weights, oracle_mod):
    """out aliasing h, as the reference's layer output (layer.cu:1917)."""
    from final_amd import hip
    from final_amd import workloads as W
    w = real_weights
    nw = _norm_weight(W.H)
    block.set_norm_weight(nw)
    for T in (8, 300):
        h = W.gen_x(T, seed=23)
        ref = oracle_mod.moe_forward_norm(h, nw, w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
        dh = hip.DeviceArray.from_numpy(h)
        block.forward_norm_gpu(dh, dh, T)
        hip.synchronize()
        block.check_device()
        np.testing.assert_allclose(dh.download(), ref["y"], rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [8, 300])
def test_route_serves_one_experts_launch(T, block, real_weights, oracle_mod):
    """The weight-streaming plan's readers wait for the rows the router
    prepared, and every plan's task counters are reset by the router, so one
    moe_route serves one moe_experts; a second launch without a new route is
    rejected, and routing again restores the result."""
    from final_amd import _native, hip
    from final_amd import workloads as W
    x = W.gen_x(T, seed=31)
    ref = oracle_forward(oracle_mod, real_weights, x)
    dx = hip.DeviceArray.from_numpy(x)
    dy = hip.DeviceArray((T, W.H))
    say(f"[one route, one experts] T={T} plan={block.plan(T)}")
    block.route(dx, T)
    block.experts(dx, dy, T)
    with pytest.raises(_native.MoeError) as e:
        block.experts(dx, dy, T)
    assert e.value.status == _native.MOE_ERR_INVALID_ARG
    hip.synchronize()
    block.check_device()
    np.testing.assert_allclose(dy.download(), ref["y"], rtol=RTOL, atol=ATOL)
    dy2 = hip.DeviceArray((T, W.H))
    block.route(dx, T)
    block.experts(dx, dy2, T)
    hip.synchronize()
    block.check_device()
    np.testing.assert_allclose(dy2.download(), ref["y"], rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
def test_readback_checks_token_count(block, real_weights):
    """moe_last_normed / moe_last_routing copy the rows of the call that
    produced them and take the caller's row count: a count other than the
    stored one is rejected (nothing is copied), so a buffer sized for another
    batch can never be overrun.  Sequences: forward_norm(300) then forward(8)
    then the normalised rows; a route that succeeded followed by an experts
    call that failed (x aliasing y) then the routing."""
    from final_amd import _native, hip
    from final_amd import workloads as W
    L = _native.lib()
    block.set_norm_weight(_norm_weight(W.H))
    h = W.gen_x(300, seed=91)
    block.forward_norm(h)
    x8 = W.gen_x(8, seed=92)
    block.forward(x8)
    assert block.last_normed().shape == (300, W.H)
    small = np.empty((8, W.H), np.float32)
    assert L.moe_last_normed(block._ctx, small.ctypes.data, 8, None) == _native.MOE_ERR_INVALID_ARG
    assert block.last_routing()["idx"].shape == (8, 4)
    idx = np.empty((300, 4), np.int32)
    assert L.moe_last_routing(block._ctx, idx.ctypes.data, None, None, None, 300,
                              None) == _native.MOE_ERR_INVALID_ARG
    dx = hip.DeviceArray.from_numpy(W.gen_x(40, seed=93))
    with pytest.raises(_native.MoeError):
        block.forward_gpu(dx, dx, 40)  # route succeeds, experts rejects x == y
    hip.synchronize()
    assert block.last_routing()["idx"].shape == (40, 4)
    assert L.moe_last_routing(block._ctx, idx.ctypes.data, None, None, None, 8,
                              None) == _native.MOE_ERR_INVALID_ARG


def _forward_vs_route_experts(block, w, T, x, r, label, lazy=False):
    """y and routing of moe_forward (deferred decode routing) and of moe_route +
    moe_experts (the router finishes and plans) on the same inputs."""
    from final_amd import hip
    from final_amd import workloads as W
    block.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
    dx = hip.DeviceArray.from_numpy(x)
    dr = hip.DeviceArray.from_numpy(r)
    say(f"[{label}] T={T} lazy={lazy} moe_forward")
    block.set_lazy_chains(lazy)
    try:
        dy1 = hip.DeviceArray((T, W.H))
        block.forward_gpu(dx, dy1, T, residual=dr)
        hip.synchronize()
        block.check_device()
        rt1 = block.last_routing()
        rt1["plan_counts"] = block.last_plan_counts()
    finally:
        block.set_lazy_chains(False)
    say(f"[{label}] T={T} moe_route + moe_experts")
    dy2 = hip.DeviceArray((T, W.H))
    block.route(dx, T)
    block.experts(dx, dy2, T, residual=dr)
    hip.synchronize()
    block.check_device()
    rt2 = block.last_routing()
    return dy1.download(), rt1, dy2.download(), rt2


def _check_same(y1, rt1, y2, rt2, tiled=False):
    """The routing bit for bit; y bit for bit, except under an MFMA plan
    (tiled) whose routing from score bounds planned a slot for an expert a
    token did not take (a near-tie at the 4th place): that row changes its
    expert's row count, and so possibly its tiles' MFMA shape, which sets the
    rounding of the k-sums; y then agrees within the parity tolerance (and
    each run matches the oracle, checked by the callers)."""
    for k in ("idx", "counts"):
        assert np.array_equal(rt1[k], rt2[k])
    for k in ("w", "logits"):
        assert np.array_equal(bits(rt1[k]), bits(rt2[k]))
    extra = int(rt1["plan_counts"].sum()) - int(rt1["counts"].sum())
    assert extra >= 0
    if tiled and extra > 0:
        np.testing.assert_allclose(y1, y2, rtol=RTOL, atol=ATOL)
    else:
        assert np.array_equal(bits(y1), bits(y2))


@pytest.mark.gpu
@pytest.mark.parametrize("lazy", [False, True])
@pytest.mark.parametrize("T", [1, 3, 8])
def test_forward_routes_in_expert_kernel(T, lazy, block, real_weights, oracle_mod):
    """One decode token block under the streaming plan: moe_forward's router
    writes only bounds of each score (double sums of the gate products and a
    bound of the FMA chain's rounding), the expert kernel plans a slot for
    every expert they leave possible for a token, streams, computes the
    logits in chain jobs meanwhile and ranks and weights each token from its
    logits in the combine.  Its
    routing (idx, w, counts, logits) and y must be bit-identical to moe_route
    + moe_experts, where the router computes the logits and routes, and
    match the oracle.  A hot expert (bias +10) makes several tokens share an
    expert, so the in-block ranks and slots are exercised.  lazy: the chain
    jobs are left to the combine's waits, which run them one wave each (the
    path of blocks that start late)."""
    from final_amd import workloads as W
    w = dict(real_weights)
    bias = np.array(real_weights["bias"], np.float32).copy()
    bias[11] += 10.0
    w["bias"] = bias
    try:
        assert block.plan(T) == 0
        x = W.gen_x(T, seed=60 + T)
        r = W.gen_x(T, seed=70 + T)
        y1, rt1, y2, rt2 = _forward_vs_route_experts(block, w, T, x, r, "deferred routing", lazy)
    finally:
        rw = real_weights
        block.set_weights(rw["gate"], rw["bias"], rw["w1"], rw["w3"], rw["w2"])
    _check_same(y1, rt1, y2, rt2)
    assert rt1["counts"][11] == T
    ref = oracle_forward(oracle_mod, w, x, residual=r)
    check_routing(rt1, ref)
    np.testing.assert_allclose(y1, ref["y"], rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
def test_forward_routing_random_batches(block, real_weights, oracle_mod):
    """48 random decode batches of 1-8 tokens through moe_forward's routing
    from score bounds: with these weights about 4 % of random tokens have a
    4th/5th score gap inside the bounds and get a slot for a 5th (or 6th)
    possible expert, so 10 of these 48 batches plan more slots than their
    top-4 (by the bound restated on the CPU).  Each must give the routing
    (idx, w, counts, logits) and y of moe_route + moe_experts bit for bit
    (a row's arithmetic does not depend on its slot), and the oracle's
    routing."""
    from final_amd import workloads as W
    w = real_weights
    rng = np.random.default_rng(2024)
    for i in range(48):
        T = 1 + i % 8
        x = rng.standard_normal((T, W.H)).astype(np.float32)
        r = rng.standard_normal((T, W.H)).astype(np.float32)
        y1, rt1, y2, rt2 = _forward_vs_route_experts(block, w, T, x, r, f"random batch {i}")
        _check_same(y1, rt1, y2, rt2)
        check_routing(rt1, oracle_forward(oracle_mod, w, x, residual=r))


@pytest.mark.gpu
@pytest.mark.parametrize("lazy", [False, True])
@pytest.mark.parametrize("T", [1, 8])
def test_forward_routing_tie_plans_both(T, lazy, block, real_weights, oracle_mod):
    """A score tie at the top-4 boundary, which no bound can separate: token
    0's fifth expert gets the gate row and bias of its fourth, so their
    logits and scores are equal.  The expert kernel plans slots for both,
    and the combine keeps the lower index once the chain jobs (run by the
    waits when lazy) give the logits: the reference's tie rule (strict '>'
    insertion), bit-identical to moe_route + moe_experts and to the
    oracle."""
    from final_amd import workloads as W
    x = W.gen_x(T, seed=90 + T)
    r = W.gen_x(T, seed=95 + T)
    w = dict(real_weights)
    ref0 = oracle_forward(oracle_mod, w, x)
    l0 = np.asarray(ref0["logits"][0], np.float64)
    score = 1.0 / (1.0 + np.exp(-l0)) + np.asarray(w["bias"], np.float64)
    order = np.argsort(-score, kind="stable")
    e4, e5 = int(order[3]), int(order[4])
    gate = np.array(w["gate"], np.float32).copy()
    bias = np.array(w["bias"], np.float32).copy()
    gate[e5] = gate[e4]
    bias[e5] = bias[e4]
    w["gate"], w["bias"] = gate, bias
    try:
        assert block.plan(T) == 0
        y1, rt1, y2, rt2 = _forward_vs_route_experts(block, w, T, x, r, "tie", lazy)
    finally:
        rw = real_weights
        block.set_weights(rw["gate"], rw["bias"], rw["w1"], rw["w3"], rw["w2"])
    _check_same(y1, rt1, y2, rt2)
    lg = rt1["logits"]
    assert lg[0, e4] == lg[0, e5]
    assert min(e4, e5) in rt1["idx"][0].tolist() and max(e4, e5) not in rt1["idx"][0].tolist()
    ref = oracle_forward(oracle_mod, w, x, residual=r)
    check_routing(rt1, ref)
    np.testing.assert_allclose(y1, ref["y"], rtol=RTOL, atol=ATOL)


def _ref_scores(O, w, x):
    """The reference's scores sigmoid(logit) + bias in float32 (layer.cu:434,
    462) from the oracle's bit-exact logits."""
    lg = O.gate_logits(x, w["gate"]).astype(np.float64)
    e = np.exp(-lg).astype(np.float32)
    p = (np.float32(1.0) / (np.float32(1.0) + e)).astype(np.float32)
    return (p + np.asarray(w["bias"], np.float32)).astype(np.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [11, 16, 21, 33, 48, 64, 100, 129, 200, 256])
def test_forward_random_batches_mfma(T, block, real_weights, oracle_mod):
    """Random N(0, 1) batches under the 64-row MFMA plan.  moe_forward's
    router writes score bounds and plans a slot for every expert they leave
    possible (several token blocks, each finished by its last block); the
    expert kernel's dispatch tasks compute the logits and the exact top-4.
    Its routing (idx, w, counts, logits) must be bit-identical to moe_route
    + moe_experts, where the router computes the logits first, y too when no
    extra slot was planned (_check_same), and both must match the oracle."""
    from final_amd import workloads as W
    w = real_weights
    assert block.plan(T) == 64
    rng = np.random.default_rng(700 + T)
    x = rng.standard_normal((T, W.H)).astype(np.float32)
    r = rng.standard_normal((T, W.H)).astype(np.float32)
    y1, rt1, y2, rt2 = _forward_vs_route_experts(block, w, T, x, r, "random batch mfma")
    say(f"[random batch mfma] T={T} slots planned {int(rt1['plan_counts'].sum())} "
        f"for {int(rt1['counts'].sum())} routed")
    _check_same(y1, rt1, y2, rt2, tiled=True)
    ref = oracle_forward(oracle_mod, w, x, residual=r)
    check_routing(rt1, ref)
    np.testing.assert_allclose(y1, ref["y"], rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(y2, ref["y"], rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
@pytest.mark.parametrize("T,plan", [(64, -1), (256, -1), (16, 64), (5, 128), (40, 32)])
def test_forward_routing_ties_many_blocks(T, plan, block, real_weights, oracle_mod):
    """Exact 4th-place ties in several token blocks: expert b gets the gate
    row and bias of expert a, the pair chosen on the oracle's scores so that
    a and b share the 4th place for as many tokens as possible.  Each tied
    token keeps the lower index (the strict '>' insertion of
    layer.cu:465-476), under the 64-row plan of the decode router's several
    token blocks and under forced MFMA plans at small T (the 128-row plan
    keeps the full router).  No score bound separates an exact tie, so
    moe_forward's routing from bounds plans a slot for both experts of each
    tied token, and the dispatch tasks' exact routing keeps one."""
    from final_amd import workloads as W
    rng = np.random.default_rng(800 + T)
    x = rng.standard_normal((T, W.H)).astype(np.float32)
    r = rng.standard_normal((T, W.H)).astype(np.float32)
    w = dict(real_weights)
    sc = _ref_scores(oracle_mod, w, x)
    best = None
    for a in range(32):
        for b in range(32):
            if a == b:
                continue
            others = np.ones(32, bool)
            others[[a, b]] = False
            above = (sc[:, others] > sc[:, a:a + 1]).sum(1)
            n = int((above == 3).sum())
            if best is None or n > best[0]:
                best = (n, a, b)
    n, a, b = best
    gate = np.array(w["gate"], np.float32).copy()
    bias = np.array(w["bias"], np.float32).copy()
    gate[b] = gate[a]
    bias[b] = bias[a]
    w["gate"], w["bias"] = gate, bias
    sc2 = _ref_scores(oracle_mod, w, x)
    tied = [t for t in range(T) if (sc2[t] > sc2[t, a]).sum() == 3]
    say(f"[ties] T={T} plan={plan} pair=({a},{b}) tied tokens={tied}")
    assert len(tied) >= 1 and (T < 64 or len({t // 8 for t in tied}) >= 2)
    block.force_tile_rows(plan)
    try:
        y1, rt1, y2, rt2 = _forward_vs_route_experts(block, w, T, x, r, "ties")
    finally:
        block.force_tile_rows(-1)
        rw = real_weights
        block.set_weights(rw["gate"], rw["bias"], rw["w1"], rw["w3"], rw["w2"])
    # no bound separates an exact tie: under the 32- and 64-row plans, which
    # route from score bounds, each tied token has both experts planned
    if (plan if plan > 0 else block.plan(T)) in (32, 64):
        assert int(rt1["plan_counts"].sum()) >= int(rt1["counts"].sum()) + len(tied)
    _check_same(y1, rt1, y2, rt2, tiled=True)
    for t in tied:
        assert min(a, b) in rt1["idx"][t].tolist() and max(a, b) not in rt1["idx"][t].tolist()
    ref = oracle_forward(oracle_mod, w, x, residual=r)
    check_routing(rt1, ref)
    np.testing.assert_allclose(y1, ref["y"], rtol=RTOL, atol=ATOL)
