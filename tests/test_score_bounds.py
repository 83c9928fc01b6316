"""The score bounds of the deferred decode routing (score_bounds in
final_amd/csrc/moe_kernels.hip), restated in numpy and checked against the
oracle's bit-exact FMA chains (orc_gate_logits, layer.cu:109-127) and
sigmoid (orc_sigmoid, layer.cu:434): the chain's logit must lie within the
radius around the product sum, and score = sigmoid + bias within the
bounds.  Rows with heavy cancellation (alternating large products) put the
chain's rounding error at its largest relative to the sum."""
import numpy as np

U = 2.0 ** -24


def _radius(m, H, n):
    gh = H * U / (1 - H * U)
    gn = n * U / (1 - n * U)
    return (gh + gn) / (1 - gn) * 1.0001 * m + 1e-37


def _bounds(s, m, H, n, bias):
    r = _radius(m, H, n)
    pl = 1.0 / (1.0 + np.exp(-(s - r))) * (1 - 2.0 ** -20)
    ph = 1.0 / (1.0 + np.exp(-(s + r))) * (1 + 2.0 ** -20)
    # float rounding toward -inf / +inf of pl / ph, then the float add
    lo = np.float32(pl)
    lo = np.where(lo.astype(np.float64) > pl, np.nextafter(lo, np.float32(-np.inf)), lo)
    hi = np.float32(ph)
    hi = np.where(hi.astype(np.float64) < ph, np.nextafter(hi, np.float32(np.inf)), hi)
    return (lo + bias).astype(np.float32), (hi + bias).astype(np.float32)


def _rows(rng, T, H, kind):
    if kind == "normal":
        return rng.standard_normal((T, H)).astype(np.float32)
    if kind == "cancel":  # large alternating products that cancel
        v = rng.uniform(50, 60, (T, H)).astype(np.float32)
        v[:, 1::2] *= -1
        return v
    return (rng.standard_normal((T, H)) * 10.0 ** rng.uniform(-6, 3, (T, H))).astype(np.float32)


def test_chain_logits_within_radius(oracle_mod):
    O = oracle_mod
    rng = np.random.default_rng(5)
    H, E = 2048, 32
    worst = 0.0
    for kind in ("normal", "cancel", "scaled"):
        x = _rows(rng, 16, H, kind)
        g = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        if kind == "cancel":
            g = np.abs(g) + np.float32(0.01)
        lg = O.gate_logits(x, g).astype(np.float64)  # bit-exact chains
        prod = x.astype(np.float64)[:, None, :] * g.astype(np.float64)[None, :, :]
        s = prod.sum(-1)
        m = np.abs(prod).sum(-1)
        # the decode router's rounding depths: H / (4 tpp) FMAs per chain, 2
        # adds and log2(tpp) shuffle levels for tpp = 8 .. 64 threads per pair
        for n in (H // 32 + 5, H // 64 + 6, H // 128 + 7, H // 256 + 8):
            r = _radius(m, H, n)
            err = np.abs(lg - s)
            assert np.all(err <= r), (kind, n, float((err / r).max()))
            worst = max(worst, float((err / r).max()))
    # the radius is a bound, not an estimate: the real error sits well inside
    assert worst < 0.5


def test_scores_within_bounds(oracle_mod):
    O = oracle_mod
    rng = np.random.default_rng(6)
    H, E = 2048, 32
    x = _rows(rng, 8, H, "normal")
    g = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.3).astype(np.float32)
    lg = O.gate_logits(x, g)
    prod = x.astype(np.float64)[:, None, :] * g.astype(np.float64)[None, :, :]
    lo, hi = _bounds(prod.sum(-1), np.abs(prod).sum(-1), H, H // 32 + 5, bias)
    for t in range(8):
        for e in range(E):
            sc = np.float32(O.sigmoid(float(lg[t, e])) + bias[e])
            assert lo[t, e] <= sc <= hi[t, e], (t, e)
    # and the top-4 sets these bounds settle are the exact ones
    for t in range(8):
        above = np.array([np.sum((hi[t] >= lo[t, e]) & (np.arange(E) != e)) for e in range(E)])
        chosen = np.nonzero(above < 4)[0]
        if len(chosen) == 4:
            sc = np.array([np.float32(O.sigmoid(float(v))) for v in lg[t]], np.float32) + bias
            order = sorted(range(E), key=lambda e: (-sc[e], e))
            assert sorted(order[:4]) == chosen.tolist()
