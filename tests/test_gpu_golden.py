"""The HIP path against the committed golden fixtures (no oracle at run time):
routing bit-exact for every token, y within 1e-3 rel / 1e-4 abs on the stored
rows and by per-row checksums for all 4096 tokens."""
import os

import numpy as np
import pytest

from conftest import bits

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
RTOL, ATOL = 1e-3, 1e-4


@pytest.fixture(scope="module")
def block(real_weights):
    from final_amd import SparseMoeBlock
    w = real_weights
    b = SparseMoeBlock(max_tokens=16384)
    b.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
    yield b
    b.close()


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 8, 64, 256, 4096])
def test_gpu_matches_seed0_fixture(T, block):
    from final_amd import workloads as W
    g = np.load(os.path.join(HERE, "moe_seed0.npz"), allow_pickle=False)
    print(f"[golden] T={T}", flush=True)
    y = block.forward(W.gen_x(T))
    rt = block.last_routing()
    assert np.array_equal(rt["idx"], g["idx"][:T].astype(np.int32))
    assert np.array_equal(bits(rt["w"]), g["w_bits"][:T])
    assert np.array_equal(rt["counts"], g[f"counts_t{T}"])
    rows = g["y_rows"]
    sel = rows < T
    np.testing.assert_allclose(y[rows[sel]], g["y"][sel], rtol=RTOL, atol=ATOL)
    cs = g["y_checksum"][:T]
    y64 = y.astype(np.float64)
    # |sum(y) - sum(ref)| <= sum(|y - ref|) <= H * (atol + rtol*max|ref|)
    assert np.all(np.abs(y64.sum(axis=1) - cs[:, 0]) <= y.shape[1] * (ATOL + RTOL * np.abs(y64).max(axis=1)))
    assert np.allclose((y64 * y64).sum(axis=1), cs[:, 1], rtol=4 * RTOL)


@pytest.mark.gpu
def test_gpu_matches_zipf_fixture(block, real_weights):
    from final_amd import workloads as W
    g = np.load(os.path.join(HERE, "moe_zipf16384.npz"), allow_pickle=False)
    w = real_weights
    print("[golden] zipf T=16384", flush=True)
    block.set_weights(w["gate"], W.zipf_bias(), w["w1"], w["w3"], w["w2"])
    try:
        y = block.forward(W.gen_x(16384))
        rt = block.last_routing()
    finally:
        block.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
    assert np.array_equal(rt["idx"], g["idx"].astype(np.int32))
    assert np.array_equal(bits(rt["w"]), g["w_bits"])
    assert np.array_equal(rt["counts"], g["counts"])
    np.testing.assert_allclose(y[g["y_rows"]], g["y"], rtol=RTOL, atol=ATOL)
