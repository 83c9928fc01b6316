"""bench.py's command-line contract pieces that need no GPU: the one-GPU
refusal and the CPU baseline object."""
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "ONE GPU" in r.stderr
    assert r.stdout == ""


def test_cpu_baseline_object():
    sys.path.insert(0, ROOT)
    import bench
    from final_amd import workloads as W
    w = W.gen_weights(0)
    x = W.gen_x(4)
    cb = bench.cpu_baseline(w, x, 2, single_tokens=2)
    assert cb["kind"] == "port" and cb["unit"] == "tokens/s" and cb["cores"] == 2
    assert cb["value"] > 0 and "4 tokens" in cb["sample"]
    st = cb["single_thread"]
    assert st["value"] > 0 and st["unit"] == "tokens/s" and "first 2 tokens" in st["sample"]
    host = cb["host"]
    assert host["nproc"] == os.cpu_count() and isinstance(host["model"], str)


def test_roofline_bound_follows_intensity():
    """The primary bound is MFMA at or above the fp32 ridge (157.3 TFLOP/s over
    8 TB/s = 19.66 FLOP/B) and HBM below it, whatever kernel plan ran; within
    2x of the ridge the other bound is reported as well."""
    sys.path.insert(0, ROOT)
    import bench
    from final_amd import workloads as W
    ridge = bench.PEAK_MFMA_F32_TFLOPS * 1e3 / bench.PEAK_HBM_GBS
    assert abs(ridge - 19.6625) < 1e-3
    # T=4096: far above the ridge -> MFMA, no secondary
    r = bench.roofline(128, 100 * 1e9, 1e9, 1.0, "none")
    assert r["bound"] == "mfma" and "secondary" not in r
    assert r["kernel"] == "expert_mfma_kernel<128>"
    assert abs(r["achieved"] - 100.0) < 1e-9 and r["per_launch"] == {"flop": 100 * 1e9}
    # an MFMA plan below the ridge (T=256-like intensity 16) -> HBM primary
    r = bench.roofline(64, 16e9, 1e9, 1.0, "none")
    assert r["bound"] == "hbm" and r["kernel"] == "expert_mfma_kernel<64>"
    assert abs(r["achieved"] - 1000.0) < 1e-9 and r["per_launch"] == {"bytes": 1e9}
    assert r["secondary"]["bound"] == "mfma" and abs(r["secondary"]["achieved"] - 16.0) < 1e-9
    # streaming plan at decode intensity -> HBM, no secondary
    r = bench.roofline(0, 1e9, 1e9, 1.0, "none")
    assert r["bound"] == "hbm" and r["kernel"] == "expert_ring_kernel" and "secondary" not in r
    # the expert kernel's accounting with all 32 experts active: 16.0 FLOP/B
    # at T=256 (below the ridge), 244 at T=4096 (above)
    counts = np.ones(W.E, np.int64)
    for T, ai in ((256, 16.0), (4096, 244.4)):
        flops = T * (W.flops_per_token() - 2 * W.H * W.E)
        nbytes = W.algorithmic_bytes(counts, T) - (W.E * W.H * 4 + W.E * 4)
        assert abs(flops / nbytes - ai) < 0.1
