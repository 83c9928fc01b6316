"""Writes the golden fixtures of the MoE block under tests/golden/.

The reference ships no vectors for this path, so these are produced by the
CPU oracle (pinned by tests/test_oracle_pinning.py) on the seeded synthetic
workloads and committed, so that later builds of the oracle, the generator and
the HIP path are held to the same bits:

  inputs.json          sha256 + first values of every generated tensor
  moe_seed0.npz        x seed 0, first 4096 tokens (T = 1, 8, 64, 256, 4096 are
                       prefixes of it): routing of all 4096 tokens, y of the
                       first 16 tokens and of every 128th, per-row checksums
  moe_zipf16384.npz    skewed workload: routing of all 16384 tokens, y of every
                       512th token

Run:  python tests/golden/make_fixtures.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from final_amd import workloads as W  # noqa: E402
from oracle import oracle as O  # noqa: E402

PREFIXES = (1, 8, 64, 256, 4096)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def input_digest(w, x4096, x16384):
    d = {}
    for name in ("gate", "bias"):
        d[name] = {"sha256": sha(w[name]), "head": w[name].ravel()[:4].tolist()}
    for name in ("w1", "w3", "w2"):
        for e in (0, 31):
            d[f"{name}[{e}]"] = {"sha256": sha(w[name][e]), "head": w[name][e].ravel()[:4].tolist()}
    d["x[4096]"] = {"sha256": sha(x4096), "head": x4096.ravel()[:4].tolist()}
    d["x[16384]"] = {"sha256": sha(x16384), "head": x16384.ravel()[:4].tolist()}
    d["zipf_bias"] = {"sha256": sha(W.zipf_bias()), "head": W.zipf_bias()[:4].tolist()}
    return d


def rows_checksum(y: np.ndarray) -> np.ndarray:
    y64 = y.astype(np.float64)
    return np.stack([y64.sum(axis=1), (y64 * y64).sum(axis=1)], axis=1)


def main():
    O.build()
    w = W.gen_weights(0)
    x = W.gen_x(4096)
    xz = W.gen_x(16384)

    with open(os.path.join(HERE, "inputs.json"), "w") as f:
        json.dump(input_digest(w, x, xz), f, indent=1)

    r = O.moe_forward(x, w["gate"], w["bias"], w["w1"], w["w3"], w["w2"])
    sample = np.r_[np.arange(16), np.arange(128, 4096, 128)]
    counts = {f"counts_t{T}": np.bincount(r["idx"][:T].ravel(), minlength=W.E).astype(np.int32)
              for T in PREFIXES}
    np.savez_compressed(
        os.path.join(HERE, "moe_seed0.npz"),
        idx=r["idx"].astype(np.uint8), w_bits=r["w"].view(np.uint32),
        logits_bits_t64=r["logits"][:64].view(np.uint32), y_rows=sample.astype(np.int32),
        y=r["y"][sample], y_checksum=rows_checksum(r["y"]), **counts)

    wz = dict(w)
    wz["bias"] = W.zipf_bias()
    mask = np.zeros(16384, np.uint8)
    zs = np.arange(0, 16384, 512)
    mask[zs] = 1
    rz = O.moe_forward(xz, wz["gate"], wz["bias"], wz["w1"], wz["w3"], wz["w2"], token_mask=mask)
    np.savez_compressed(
        os.path.join(HERE, "moe_zipf16384.npz"),
        idx=rz["idx"].astype(np.uint8), w_bits=rz["w"].view(np.uint32), counts=rz["counts"],
        y_rows=zs.astype(np.int32), y=rz["y"][zs])
    print("counts t4096", counts["counts_t4096"].tolist())
    print("counts zipf", rz["counts"].tolist())


if __name__ == "__main__":
    main()
