"""moe_forward_noalloc (the entry point that allocates nothing) against
moe_forward through the C-ABI.

moe_forward_noalloc runs the router and expert kernels of moe_route +
moe_experts on a per-GPU device array instead of the context's scratch, so
its y must equal theirs bit for bit.  moe_forward routes batches of up to
256 tokens from score bounds (inside the experts launch for a decode batch
of up to 8 tokens under the weight-streaming plan, with the same arithmetic
per row; under an MFMA plan with a slot for every expert the bounds leave
possible): its routing must equal theirs bit for bit, and its y too unless it
planned a slot for an expert a token did not take, which can change that
expert's tile shape and so the rounding of its k-sums (then within the
parity tolerance).  Two calls in a row, the second with fewer tokens (the
array keeps the first call's contents), and the size limit.
"""
import sys

import numpy as np
import pytest

from conftest import bits

RTOL, ATOL = 1e-3, 1e-4


def same_as_forward(z, y, rt_fwd, plan_counts, T, tiled):
    """z (noalloc) against moe_forward's y: bit for bit unless moe_forward's
    MFMA plan (tiled) held more slots than its routing (see the module
    docstring)."""
    if tiled and int(plan_counts.sum()) > int(rt_fwd["counts"].sum()):
        np.testing.assert_allclose(z, y, rtol=RTOL, atol=ATOL)
    else:
        assert np.array_equal(bits(z), bits(y)), f"T={T}: noalloc y differs from moe_forward"


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.gpu
def test_noalloc_matches_forward(real_weights):
    from final_amd import SparseMoeBlock, _native, hip
    from final_amd import workloads as W
    L = _native.lib()
    w = real_weights
    blk = SparseMoeBlock(max_tokens=256)
    try:
        blk.set_weights(w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
        for T in (128, 8, 1):
            say(f"[noalloc] T={T} plan={blk.plan(T)}")
            x = W.gen_x(T, seed=300 + T)
            r = W.gen_x(T, seed=400 + T)
            dx = hip.DeviceArray.from_numpy(x)
            dr = hip.DeviceArray.from_numpy(r)
            dy = hip.DeviceArray((T, W.H))
            dv = hip.DeviceArray((T, W.H))
            dz = hip.DeviceArray((T, W.H))
            blk.forward_gpu(dx, dy, T, residual=dr)
            hip.synchronize()
            rt_fwd = blk.last_routing()
            pc_fwd = blk.last_plan_counts()
            blk.route(dx, T)
            blk.experts(dx, dv, T, residual=dr)
            _native.check(L.moe_forward_noalloc(blk._ctx, dx.ptr, dz.ptr, dr.ptr, T, None),
                          "moe_forward_noalloc")
            hip.synchronize()
            blk.check_device()
            y, v, z = dy.download(), dv.download(), dz.download()
            assert np.isfinite(z).all()
            assert np.array_equal(bits(z), bits(v)), f"T={T}: noalloc y differs from route + experts"
            same_as_forward(z, y, rt_fwd, pc_fwd, T, blk.plan(T) > 0)
            rt = blk.last_routing()  # moe_route's, the same as moe_forward's
            assert np.array_equal(rt["idx"], rt_fwd["idx"])
            assert np.array_equal(bits(rt["w"]), bits(rt_fwd["w"]))
            assert np.array_equal(bits(rt["logits"]), bits(rt_fwd["logits"]))
        # a forced MFMA plan on the same array, after the streaming calls
        blk.force_tile_rows(64)
        try:
            T = 100
            say(f"[noalloc] T={T} plan={blk.plan(T)}")
            x = W.gen_x(T, seed=500)
            dx = hip.DeviceArray.from_numpy(x)
            dy = hip.DeviceArray((T, W.H))
            dv = hip.DeviceArray((T, W.H))
            dz = hip.DeviceArray((T, W.H))
            blk.forward_gpu(dx, dy, T)
            hip.synchronize()
            rt_fwd = blk.last_routing()
            pc_fwd = blk.last_plan_counts()
            blk.route(dx, T)
            blk.experts(dx, dv, T)
            _native.check(L.moe_forward_noalloc(blk._ctx, dx.ptr, dz.ptr, None, T, None),
                          "moe_forward_noalloc")
            hip.synchronize()
            blk.check_device()
            assert np.array_equal(bits(dz.download()), bits(dv.download()))
            same_as_forward(dz.download(), dy.download(), rt_fwd, pc_fwd, T, True)
        finally:
            blk.force_tile_rows(-1)
        big = hip.DeviceArray((129, W.H))
        out = hip.DeviceArray((129, W.H))
        assert L.moe_forward_noalloc(blk._ctx, big.ptr, out.ptr, None, 129,
                                     None) == _native.MOE_ERR_TOO_MANY_TOKENS
        assert L.moe_forward_noalloc(blk._ctx, big.ptr, big.ptr, None, 4,
                                     None) == _native.MOE_ERR_INVALID_ARG
    finally:
        blk.close()
