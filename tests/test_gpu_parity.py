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
@pytest.mark.parametrize("T", [1, 8, 64, 100, 256, 1000, 4096])
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
