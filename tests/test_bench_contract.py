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
