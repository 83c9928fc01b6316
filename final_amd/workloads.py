"""Seeded synthetic MoE-block workloads (the reference ships no data files).

Shapes follow the reference model (include/config.h:5,14-17): hidden 2048,
32 experts, top-4, SwiGLU experts with intermediate 1792.  Weights ~ N(0, 0.02),
activations ~ N(0, 1), drawn by the counter-based generator of
include/moe_synth.h, so every host produces the same bits.

Workloads:
  cpu_t64        T=64, the small case the reference's tests/moe path runs
  prefill_t4096  T=4096 (batch 16 x seq 256), near-uniform expert load
  zipf_t16384    T=16384, gate bias tuned so expert selection frequency follows
                 Zipf(1.2) with the head capped and experts 5, 17, 30 unused
  decode_t{1,8,64,256}  weight-streaming shapes

expert_bias is not specified by the reference for synthetic runs; it is drawn
N(0, 0.02) with the other weights (near-uniform load) except in zipf_t16384.
"""
from __future__ import annotations

import ctypes
import json
import os
from dataclasses import dataclass

import numpy as np

from . import _native

H, I, E, K = 2048, 1792, 32, 4
WEIGHT_STD = 0.02
DATA_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data")
ZIPF_BIAS_PATH = os.path.join(DATA_DIR, "zipf_bias.json")


@dataclass(frozen=True)
class Workload:
    name: str
    T: int
    seed: int = 0
    bias: str = "normal"  # "normal" | "zipf"
    kind: str = "moe"     # "moe" | "dense" (the dense FFN of layers 0-1, I = DENSE_I)


WORKLOADS = {
    "cpu_t64": Workload("cpu_t64", 64),
    "prefill_t4096": Workload("prefill_t4096", 4096),
    "zipf_t16384": Workload("zipf_t16384", 16384, bias="zipf"),
    "decode_t1": Workload("decode_t1", 1),
    "decode_t8": Workload("decode_t8", 8),
    "decode_t64": Workload("decode_t64", 64),
    "decode_t256": Workload("decode_t256", 256),
    "dense_t1": Workload("dense_t1", 1, kind="dense"),
    "dense_t64": Workload("dense_t64", 64, kind="dense"),
    "dense_t4096": Workload("dense_t4096", 4096, kind="dense"),
}

DENSE_I = 7168  # INTERMEDIATE_SIZE, reference include/config.h:6


def normal(seed: int, stream: int, std: float, n: int, first: int = 0) -> np.ndarray:
    out = np.empty((n,), np.float32)
    _native.lib().moe_synth_normal(seed, stream, std, first, out.ctypes.data, n)
    return out


def set_threads(n: int) -> None:
    _native.lib().moe_synth_set_threads(int(n))


def gen_weights(seed: int = 0, h: int = H, inter: int = I, e: int = E,
                bias: str = "normal") -> dict:
    """gate [E][H], bias [E], w1/w3 [E][I][H], w2 [E][H][I] (fp32)."""
    L = _native.lib()
    gate = normal(seed, L.moe_synth_stream_gate(), WEIGHT_STD, e * h).reshape(e, h)
    if bias == "zipf":
        b = zipf_bias(e)
    else:
        b = normal(seed, L.moe_synth_stream_bias(), WEIGHT_STD, e)
    w1 = np.empty((e, inter, h), np.float32)
    w3 = np.empty((e, inter, h), np.float32)
    w2 = np.empty((e, h, inter), np.float32)
    for x in range(e):
        L.moe_synth_normal(seed, L.moe_synth_stream_w1(x), WEIGHT_STD, 0, w1[x].ctypes.data, inter * h)
        L.moe_synth_normal(seed, L.moe_synth_stream_w3(x), WEIGHT_STD, 0, w3[x].ctypes.data, inter * h)
        L.moe_synth_normal(seed, L.moe_synth_stream_w2(x), WEIGHT_STD, 0, w2[x].ctypes.data, h * inter)
    return {"gate": gate, "bias": b, "w1": w1, "w3": w3, "w2": w2}


def gen_dense_weights(seed: int = 0, h: int = H, inter: int = DENSE_I) -> dict:
    """Dense FFN weights N(0, 0.02): w1, w3 [I][H], w2 [H][I], drawn from
    streams past the 32 experts' (expert ids 32..34 of the same generator)."""
    L = _native.lib()
    w1 = normal(seed, L.moe_synth_stream_w1(E), WEIGHT_STD, inter * h).reshape(inter, h)
    w3 = normal(seed, L.moe_synth_stream_w3(E + 1), WEIGHT_STD, inter * h).reshape(inter, h)
    w2 = normal(seed, L.moe_synth_stream_w2(E + 2), WEIGHT_STD, h * inter).reshape(h, inter)
    return {"w1": w1, "w3": w3, "w2": w2}


def gen_x(T: int, seed: int = 0, h: int = H, e: int = E) -> np.ndarray:
    """x [T][H] ~ N(0,1); the first rows of a longer x are the same tokens."""
    L = _native.lib()
    return normal(seed, L.moe_synth_stream_x(e), 1.0, T * h).reshape(T, h)


def zipf_bias(e: int = E) -> np.ndarray:
    if not os.path.exists(ZIPF_BIAS_PATH):
        raise RuntimeError(f"missing {ZIPF_BIAS_PATH} (tests/golden/make_zipf_bias.py writes it)")
    with open(ZIPF_BIAS_PATH) as f:
        d = json.load(f)
    b = np.array(d["bias"], dtype=np.float32)
    assert b.shape == (e,)
    return b


def zipf_targets(e: int = E, s: float = 1.2, zero=(5, 17, 30), T: int = 1) -> np.ndarray:
    """Target tokens-per-expert fractions (sum = K): Zipf(s) over the active
    experts in a fixed scrambled rank order, water-filled so no expert exceeds
    one selection per token."""
    active = [x for x in range(e) if x not in zero]
    rng = np.random.default_rng(12345)
    order = rng.permutation(active)  # order[r] = expert of rank r+1
    z = np.array([(r + 1.0) ** -s for r in range(len(order))])
    q = K * z / z.sum()
    for _ in range(64):  # water-fill the cap at 1.0
        over = q > 1.0
        if not over.any():
            break
        excess = (q[over] - 1.0).sum()
        q[over] = 1.0
        free = ~over & (q < 1.0)
        q[free] += excess * q[free] / q[free].sum()
    tgt = np.zeros((e,), np.float64)
    tgt[order] = q
    return tgt


def flops_per_token(h: int = H, inter: int = I, e: int = E, k: int = K) -> int:
    """Gate 2*H*E plus k experts of 2*2*H*I (W1, W3) + 2*I*H (W2)."""
    return 2 * h * e + k * (2 * 2 * h * inter + 2 * inter * h)


def algorithmic_bytes(counts: np.ndarray, T: int, h: int = H, inter: int = I, e: int = E,
                      residual: bool = False) -> int:
    """Weights of every active expert + gate + bias + x + y (+ residual)."""
    active = int((np.asarray(counts) > 0).sum())
    per_expert = 3 * h * inter * 4
    return active * per_expert + e * h * 4 + e * 4 + T * h * 4 * (3 if residual else 2)
