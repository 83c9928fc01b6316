"""Committed golden fixtures (tests/golden/, made by make_fixtures.py) against
the generator and the CPU oracle.  These hold the inputs and the oracle's
routing/outputs to fixed bits across builds and hosts; the GPU path is held to
the same fixtures in test_gpu_golden.py."""
import hashlib
import json
import os

import numpy as np
import pytest

from conftest import bits

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def inputs():
    with open(os.path.join(HERE, "inputs.json")) as f:
        return json.load(f)


def test_generator_reproduces_inputs(inputs, real_weights):
    from final_amd import workloads as W
    w = real_weights
    assert sha(w["gate"]) == inputs["gate"]["sha256"]
    assert sha(w["bias"]) == inputs["bias"]["sha256"]
    for name in ("w1", "w3", "w2"):
        for e in (0, 31):
            assert sha(w[name][e]) == inputs[f"{name}[{e}]"]["sha256"], (name, e)
    assert sha(W.gen_x(4096)) == inputs["x[4096]"]["sha256"]
    assert sha(W.zipf_bias()) == inputs["zipf_bias"]["sha256"]


def test_generator_independent_of_threads():
    from final_amd import workloads as W
    a = W.normal(3, 77, 1.0, 3_000_001, first=5)
    W.set_threads(1)
    try:
        b = W.normal(3, 77, 1.0, 3_000_001, first=5)
    finally:
        W.set_threads(0)
    assert np.array_equal(bits(a), bits(b))
    c = W.normal(3, 77, 1.0, 10)  # element i is the same whatever the window
    assert np.array_equal(bits(c[5:]), bits(a[:5]))
    assert abs(float(a.mean())) < 3e-3 and abs(float(a.std()) - 1.0) < 3e-3


def test_oracle_t64_matches_fixture(real_weights, oracle_mod):
    from final_amd import workloads as W
    g = load("moe_seed0.npz")
    w = real_weights
    x = W.gen_x(64)
    r = oracle_mod.moe_forward(x, w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
    assert np.array_equal(r["idx"], g["idx"][:64].astype(np.int32))
    assert np.array_equal(bits(r["w"]), g["w_bits"][:64])
    assert np.array_equal(bits(r["logits"]), g["logits_bits_t64"])
    assert np.array_equal(r["counts"], g["counts_t64"])
    rows = g["y_rows"]
    first = rows[rows < 64]
    assert np.array_equal(bits(r["y"][first]), bits(g["y"][: len(first)]))


def test_oracle_t4096_routing_and_rows_match_fixture(real_weights, oracle_mod):
    from final_amd import workloads as W
    g = load("moe_seed0.npz")
    w = real_weights
    x = W.gen_x(4096)
    mask = np.zeros(4096, np.uint8)
    mask[g["y_rows"]] = 1
    r = oracle_mod.moe_forward(x, w["gate"], w["bias"], w["w1"], w["w3"], w["w2"], token_mask=mask)
    assert np.array_equal(r["idx"], g["idx"].astype(np.int32))
    assert np.array_equal(bits(r["w"]), g["w_bits"])
    for T in (1, 8, 64, 256, 4096):
        assert np.array_equal(np.bincount(r["idx"][:T].ravel(), minlength=32), g[f"counts_t{T}"])
    assert np.array_equal(bits(r["y"][g["y_rows"]]), bits(g["y"]))


def test_oracle_zipf_matches_fixture(real_weights, oracle_mod):
    from final_amd import workloads as W
    g = load("moe_zipf16384.npz")
    w = dict(real_weights)
    w["bias"] = W.zipf_bias()
    x = W.gen_x(16384)
    mask = np.zeros(16384, np.uint8)
    mask[g["y_rows"][:4]] = 1
    r = oracle_mod.moe_forward(x, w["gate"], w["bias"], w["w1"], w["w3"], w["w2"], token_mask=mask)
    assert np.array_equal(r["idx"], g["idx"].astype(np.int32))
    assert np.array_equal(bits(r["w"]), g["w_bits"])
    assert np.array_equal(r["counts"], g["counts"])
    assert (g["counts"] == 0).sum() >= 3
    assert np.array_equal(bits(r["y"][g["y_rows"][:4]]), bits(g["y"][:4]))


def test_fma_vs_muladd_gate_does_not_change_routing(real_weights, oracle_mod):
    """The reference's CPU test path may accumulate the gate with mul+add
    instead of FMA; on these workloads that changes no routing decision."""
    from final_amd import workloads as W
    x = W.gen_x(4096)
    w = real_weights
    a = oracle_mod.route(oracle_mod.gate_logits(x, w["gate"]), w["bias"])[0]
    b = oracle_mod.route(oracle_mod.gate_logits(x, w["gate"], muladd=True), w["bias"])[0]
    assert np.array_equal(a, b)
