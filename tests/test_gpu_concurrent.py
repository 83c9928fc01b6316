"""Two MoE contexts whose persistent expert kernels run at the same time on two
streams, so neither has the whole chip: each kernel's grid is sized to fill
every CU, and blocks that find no free CU start only when the other kernel's
blocks exit.  Every task is claimed from the queue by a running block, so a
block that is not resident owns nothing another block waits for
(tests/test_protocol_model.py explores that protocol on the CPU); here both
kernels must finish with no device-side wait timeout and match the oracle.
"""
import sys

import numpy as np
import pytest

RTOL, ATOL = 1e-3, 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.gpu
@pytest.mark.parametrize("ta,tb", [(64, 8), (64, 1024), (128, 96)])
def test_two_contexts_two_streams(ta, tb, real_weights, oracle_mod):
    from final_amd import SparseMoeBlock, hip
    from final_amd import workloads as W
    w = real_weights
    say(f"[concurrent] T={ta} and T={tb} on two streams")
    blocks, streams, xs, ds = [], [], [], []
    for T in (ta, tb):
        b = SparseMoeBlock(max_tokens=max(T, 64))
        b.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
        blocks.append(b)
        streams.append(hip.Stream())
        x = W.gen_x(T + 16)[16:]  # two different token sets
        xs.append(x)
        ds.append((hip.DeviceArray.from_numpy(x), hip.DeviceArray((T, W.H))))
    say(f"[concurrent] plans {[b.plan(T) for b, T in zip(blocks, (ta, tb))]}")
    for _ in range(6):  # interleaved launches; the streams overlap on the device
        for b, s, (dx, dy), T in zip(blocks, streams, ds, (ta, tb)):
            b.forward_gpu(dx, dy, T, stream=s)
    for s in streams:
        s.synchronize()
    for b, s, (dx, dy), x in zip(blocks, streams, ds, xs):
        b.check_device(s)  # raises on a device-side wait timeout
        ref = oracle_mod.moe_forward(x, w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
        rt = b.last_routing()
        assert np.array_equal(rt["idx"], ref["idx"]) and np.array_equal(rt["counts"], ref["counts"])
        np.testing.assert_allclose(dy.download(), ref["y"], rtol=RTOL, atol=ATOL)
    for b in blocks:
        b.close()
