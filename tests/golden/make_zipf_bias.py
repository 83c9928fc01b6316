"""Calibrates the expert_bias of the skewed workload (zipf_t16384) and writes
final_amd/data/zipf_bias.json.

Target: tokens-per-expert fractions from final_amd.workloads.zipf_targets
(Zipf(1.2) over 29 experts in a fixed scrambled rank order, head water-filled
at one selection per token, experts 5, 17 and 30 never chosen).  The routing
of the workload's own 16384 tokens is evaluated with the CPU oracle's router
(a restatement of the reference's, layer.cu:439-499) and the bias is moved by
stochastic approximation until the counts track the targets.

Run:  python tests/golden/make_zipf_bias.py
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from final_amd import workloads as W  # noqa: E402
from oracle import oracle as O  # noqa: E402


def main():
    O.build()
    T = W.WORKLOADS["zipf_t16384"].T
    L = __import__("final_amd")._native.lib()
    gate = W.normal(0, L.moe_synth_stream_gate(), W.WEIGHT_STD, W.E * W.H).reshape(W.E, W.H)
    x = W.gen_x(T)
    logits = O.gate_logits(x, gate)
    tgt = W.zipf_targets()
    zero = tgt == 0
    b = np.where(zero, -10.0, 0.0).astype(np.float32)
    lr = 0.5
    for it in range(400):
        _, _, counts = O.route(logits, b)
        frac = counts / T
        err = tgt - frac
        b = np.where(zero, -10.0, b + lr * err).astype(np.float32)
        if it % 50 == 0:
            print(it, float(np.abs(err).max()))
        lr = max(0.05, lr * 0.99)
    _, _, counts = O.route(logits, b)
    out = {"bias": [float(v) for v in b], "counts_t16384": counts.tolist(),
           "targets": [float(v) for v in tgt], "zero_experts": [int(i) for i in np.where(zero)[0]],
           "note": "expert_bias for zipf_t16384; made by tests/golden/make_zipf_bias.py"}
    os.makedirs(os.path.dirname(W.ZIPF_BIAS_PATH), exist_ok=True)
    with open(W.ZIPF_BIAS_PATH, "w") as f:
        json.dump(out, f, indent=1)
    print("counts", counts.tolist())
    print("targets", np.round(tgt * T).astype(int).tolist())


if __name__ == "__main__":
    main()
