"""Dense SwiGLU FFN of the first layers (MLP::forward_gpu, layer.cu:1231-1269)
through the C-ABI (moe_dense_*), against the oracle's restatement.

Bar: y within rtol 1e-3 / atol 1e-4 in fp32.  The HIP path cuts the
intermediate dimension into 4 chunks and adds their partial down-projections,
so its k-sums are ordered differently from the reference's single chains;
only the tolerance is expected, not bit equality.
"""
import sys

import numpy as np
import pytest

RTOL, ATOL = 1e-3, 1e-4
H, I = 2048, 7168


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dense_weights():
    rng = np.random.default_rng(2024)
    w1 = rng.standard_normal((I, H), dtype=np.float32) * np.float32(0.02)
    w3 = rng.standard_normal((I, H), dtype=np.float32) * np.float32(0.02)
    w2 = rng.standard_normal((H, I), dtype=np.float32) * np.float32(0.02)
    return w1, w3, w2


@pytest.fixture(scope="module")
def mlp(dense_weights):
    from final_amd import DenseMLP
    m = DenseMLP(H, I, max_tokens=2048)
    m.set_weights(*dense_weights)
    yield m
    m.close()


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 8, 31, 32, 48, 64, 100, 150, 192, 256, 1000, 2048])
def test_dense_matches_oracle(T, mlp, dense_weights, oracle_mod):
    from final_amd import workloads as W
    say(f"[dense] T={T} plan={mlp.plan(T)}")
    if T <= 192:
        # weight streaming, 4 chunks of 1792; above 64 tokens in several
        # 64-token groups per task
        assert mlp.plan(T) == 0
    x = W.gen_x(T, seed=31)
    y = mlp.forward(x)
    ref = oracle_mod.dense_mlp(x, *dense_weights)
    np.testing.assert_allclose(y, ref, rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
def test_dense_residual_in_place(mlp, dense_weights, oracle_mod):
    from final_amd import hip
    from final_amd import workloads as W
    T = 40
    x = W.gen_x(T, seed=32)
    r = W.gen_x(T, seed=33)
    ref = oracle_mod.dense_mlp(x, *dense_weights, residual=r)
    dx = hip.DeviceArray.from_numpy(x)
    dr = hip.DeviceArray.from_numpy(r)
    mlp.forward_gpu(dx, dr, T, residual=dr)
    hip.synchronize()
    mlp.check_device()
    np.testing.assert_allclose(dr.download(), ref, rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
def test_dense_context_rejects_moe_calls(mlp):
    from final_amd import _native
    L = _native.lib()
    assert L.moe_forward(mlp._ctx, None, None, None, 1, None) == _native.MOE_ERR_INVALID_ARG
    assert L.moe_route(mlp._ctx, None, 1, None) == _native.MOE_ERR_INVALID_ARG
    assert L.moe_dense_forward(mlp._ctx, None, None, None, 0, None) == 0  # T = 0: no-op
