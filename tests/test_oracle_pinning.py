"""Pins the CPU oracle (oracle/moe_oracle.c) before anything is compared to it.

The reference holds no test vectors for this path (its tests/moe is closed
objects, its CPU forward is an empty stub, layer.cu:1499-1503), so every
oracle function is pinned here by something independent of its own code:
exact rational arithmetic for the FMA chains, brute-force sorting for the
router, a float64 model for the experts, and closed-form special cases of the
whole block.  A plausible slip (reordered k, mul+add instead of fma, a tie
broken the wrong way, w normalised by the wrong sum, W1/W3 swapped, a dropped
residual) fails at least one test.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from conftest import bits

TOPK = 4


# ---------------------------------------------------------------------------
# exact float32 arithmetic
# ---------------------------------------------------------------------------

def f32_round(q: Fraction) -> np.float32:
    """Round an exact rational to the nearest float32 (ties to even)."""
    if q == 0:
        return np.float32(0.0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)  # subnormals share the minimum exponent
    ulp = Fraction(2) ** (e - 23)
    m = a / ulp
    n = math.floor(m)
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return np.float32(sign * float(n * ulp))


def fma_exact(a, b, c) -> np.float32:
    return f32_round(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def chain(xs, ws) -> np.float32:
    acc = np.float32(0.0)
    for x, w in zip(xs, ws):
        acc = fma_exact(x, w, acc)
    return acc


def ulp32(v: float) -> float:
    return float(np.spacing(np.float32(abs(v))))


def test_f32_round_self_check():
    rng = np.random.default_rng(0)
    for _ in range(200):
        v = float(rng.standard_normal()) * 10.0 ** int(rng.integers(-30, 30))
        assert f32_round(Fraction(v)) == np.float32(v)  # double -> float32 is one rounding
    assert f32_round(Fraction(1) + Fraction(2) ** -24) == np.float32(1.0)  # tie to even
    assert f32_round(Fraction(1) + Fraction(3) * Fraction(2) ** -24) == np.float32(1.0 + 2 ** -22)


# ---------------------------------------------------------------------------
# a1: FMA-chain GEMM (layer.cu:109-127, 913-952, 1084-1106)
# ---------------------------------------------------------------------------

def test_gemm_chain_is_sequential_fma(oracle_mod):
    rng = np.random.default_rng(1)
    A = rng.standard_normal((5, 37)).astype(np.float32)
    B = (rng.standard_normal((6, 37)) * 0.3).astype(np.float32)
    C = oracle_mod.gemm_nt_chain(A, B)
    for m in range(5):
        for n in range(6):
            assert bits(C[m, n]) == bits(chain(A[m], B[n])), (m, n)


def test_gemm_chain_differs_from_other_orders(oracle_mod):
    """The sequential chain is not the reversed chain nor mul+add: the check
    above would catch either (guards the test's own power)."""
    rng = np.random.default_rng(2)
    A = rng.standard_normal((1, 300)).astype(np.float32)
    B = rng.standard_normal((8, 300)).astype(np.float32)
    C = oracle_mod.gemm_nt_chain(A, B)
    rev = [chain(A[0][::-1], B[n][::-1]) for n in range(8)]
    assert any(bits(C[0, n]) != bits(rev[n]) for n in range(8))
    muladd = oracle_mod.gate_logits(A, B, muladd=True)
    assert any(bits(C[0, n]) != bits(muladd[0, n]) for n in range(8))


def test_gemm_scalar_and_vector_paths_identical(oracle_mod):
    rng = np.random.default_rng(3)
    A = rng.standard_normal((70, 300)).astype(np.float32)
    B = (rng.standard_normal((75, 300)) * 0.02).astype(np.float32)
    C1 = oracle_mod.gemm_nt_chain(A, B)
    oracle_mod.force_scalar(True)
    try:
        C2 = oracle_mod.gemm_nt_chain(A, B)
    finally:
        oracle_mod.force_scalar(False)
    assert np.array_equal(bits(C1), bits(C2))


def test_gemm_close_to_float64(oracle_mod):
    rng = np.random.default_rng(4)
    A = rng.standard_normal((40, 2048)).astype(np.float32)
    B = (rng.standard_normal((33, 2048)) * 0.02).astype(np.float32)
    C = oracle_mod.gemm_nt_chain(A, B).astype(np.float64)
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    bound = 2048 * 2 ** -24 * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64).T)
    assert np.all(np.abs(C - ref) <= bound)


def test_gate_closed_forms(oracle_mod):
    rng = np.random.default_rng(5)
    E, H = 32, 64
    gate = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = np.zeros((H + 1, H), np.float32)
    for k in range(H):
        x[k, k] = 1.0  # basis vector picks column k exactly
    lg = oracle_mod.gate_logits(x, gate)
    for k in range(H):
        assert np.array_equal(bits(lg[k]), bits(gate[:, k]))
    assert np.all(lg[H] == 0.0)  # x = 0


# ---------------------------------------------------------------------------
# a2: sigmoid with a double exp (layer.cu:434), silu (layer.cu:728)
# ---------------------------------------------------------------------------

def test_sigmoid_values(oracle_mod):
    assert oracle_mod.sigmoid(0.0) == 0.5
    assert oracle_mod.sigmoid(200.0) == 1.0
    assert oracle_mod.sigmoid(-200.0) == 0.0
    xs = np.linspace(-30, 30, 4001).astype(np.float32)
    ys = np.array([oracle_mod.sigmoid(float(v)) for v in xs])
    assert np.all(np.diff(ys) >= 0)  # monotone
    for v, y in zip(xs[::50], ys[::50]):
        # three float roundings (exp result, add, divide): within 1.5 ulp
        exact = 1.0 / (1.0 + math.exp(-float(v)))
        assert abs(y - exact) <= 1.5 * ulp32(exact) + 1e-45, v
    # symmetry sigma(-x) = 1 - sigma(x) up to the two roundings
    for v in xs[::97]:
        assert abs(oracle_mod.sigmoid(float(v)) + oracle_mod.sigmoid(-float(v)) - 1.0) <= 2 ** -23


def test_silu_values(oracle_mod):
    assert oracle_mod.silu(0.0) == 0.0
    for v in np.linspace(-20, 20, 201):
        v = float(np.float32(v))
        exact = v / (1.0 + math.exp(-v))
        assert abs(oracle_mod.silu(v) - exact) <= 4 * ulp32(exact) + 1e-30


# ---------------------------------------------------------------------------
# a3: router (layer.cu:439-499)
# ---------------------------------------------------------------------------

def brute_route(logits, bias):
    """Top-4 by full sort: score descending, lower expert first on ties."""
    T, E = logits.shape
    idx = np.full((T, TOPK), -1, np.int64)
    probs = np.zeros((T, TOPK), np.float64)
    for t in range(T):
        p = [1.0 / (1.0 + math.exp(-float(l))) for l in logits[t]]
        score = [np.float32(np.float32(pp) + np.float32(b)) for pp, b in zip(p, bias)]
        order = sorted(range(E), key=lambda e: (-float(score[e]), e))
        idx[t] = order[:TOPK]
        probs[t] = [p[e] for e in order[:TOPK]]
    return idx, probs


def test_router_matches_brute_force(oracle_mod):
    rng = np.random.default_rng(6)
    T, E = 500, 32
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.02).astype(np.float32)
    idx, w, counts = oracle_mod.route(logits, bias)
    bidx, bp = brute_route(logits, bias)
    assert np.array_equal(idx, bidx)
    wref = bp / bp.sum(axis=1, keepdims=True)
    assert np.all(np.abs(w - wref) <= 3 * 2 ** -24)
    assert np.array_equal(counts, np.bincount(idx.ravel(), minlength=E))
    assert np.all(np.abs(w.astype(np.float64).sum(axis=1) - 1.0) < 1e-6)
    for t in range(T):
        assert len(set(idx[t])) == TOPK


def test_router_ties_pick_lower_expert(oracle_mod):
    E = 32
    logits = np.zeros((3, E), np.float32)
    bias = np.zeros(E, np.float32)
    # token 0: every score equal -> experts 0..3 in index order
    # token 1: experts 31, 7, 9, 2 tied on top through the bias
    logits[1] = -5.0
    for e in (31, 7, 9, 2):
        logits[1, e] = 3.0
    # token 2: ties between a logit lead and a bias lead resolve by index
    logits[2, 10] = 1.0
    logits[2, 20] = 1.0
    idx, w, _ = oracle_mod.route(logits, bias)
    assert idx[0].tolist() == [0, 1, 2, 3]
    assert np.all(w[0] == np.float32(0.25))
    assert idx[1].tolist() == [2, 7, 9, 31]
    assert idx[2].tolist()[:2] == [10, 20] and idx[2].tolist()[2:] == [0, 1]


def test_router_bias_shifts_selection_not_weights(oracle_mod):
    E = 32
    rng = np.random.default_rng(7)
    logits = rng.standard_normal((50, E)).astype(np.float32)
    bias = np.zeros(E, np.float32)
    bias[[3, 11, 17, 29]] = 10.0  # always selected, in score order
    idx, w, counts = oracle_mod.route(logits, bias)
    assert all(set(r) == {3, 11, 17, 29} for r in idx.tolist())
    p = 1.0 / (1.0 + np.exp(-logits[:, [3, 11, 17, 29]].astype(np.float64)))
    wref = np.sort(p / p.sum(axis=1, keepdims=True), axis=1)
    assert np.allclose(np.sort(w, axis=1), wref, atol=3e-7)
    assert counts[[3, 11, 17, 29]].tolist() == [50] * 4 and counts.sum() == 200


def test_router_nan_scores_never_selected(oracle_mod):
    E = 32
    logits = np.zeros((1, E), np.float32)
    logits[0, :] = np.nan
    logits[0, [4, 9]] = 1.0
    idx, w, counts = oracle_mod.route(logits, np.zeros(E, np.float32))
    assert idx[0].tolist() == [4, 9, -1, -1]
    assert counts.sum() == 2 and w[0, 2] == 0 and w[0, 3] == 0


# ---------------------------------------------------------------------------
# a4 + a5: dispatch (layer.cu:730-768, 501-542)
# ---------------------------------------------------------------------------

def test_dispatch_is_stable_counting_sort(oracle_mod):
    rng = np.random.default_rng(8)
    T, E = 300, 32
    idx = np.array([rng.choice(E, TOPK, replace=False) for _ in range(T)], np.int32)
    offsets, pos, slot_token = oracle_mod.dispatch(idx, E)
    counts = np.bincount(idx.ravel(), minlength=E)
    assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts)
    assert offsets[-1] == T * TOPK
    flat_e = idx.ravel()
    flat_t = np.repeat(np.arange(T), TOPK)
    order = np.lexsort((flat_t, flat_e))  # by expert, then token
    assert np.array_equal(slot_token, flat_t[order])
    # pos is the inverse permutation
    assert np.array_equal(slot_token[pos.ravel()], flat_t)
    assert sorted(pos.ravel().tolist()) == list(range(T * TOPK))


# ---------------------------------------------------------------------------
# a6 + a7: experts; a8 + a9: combine
# ---------------------------------------------------------------------------

def silu64(v):
    return v / (1.0 + np.exp(-v))


def test_expert_ffn_close_to_float64(oracle_mod):
    rng = np.random.default_rng(9)
    M, H, I = 13, 256, 96
    x = rng.standard_normal((M, H)).astype(np.float32)
    w1 = (rng.standard_normal((I, H)) * 0.05).astype(np.float32)
    w3 = (rng.standard_normal((I, H)) * 0.05).astype(np.float32)
    w2 = (rng.standard_normal((H, I)) * 0.05).astype(np.float32)
    inter = oracle_mod.expert_w1w3(x, w1, w3)
    out = oracle_mod.expert_w2(inter, w2)
    x64 = x.astype(np.float64)
    i_ref = silu64(x64 @ w1.T.astype(np.float64)) * (x64 @ w3.T.astype(np.float64))
    o_ref = i_ref @ w2.T.astype(np.float64)
    assert np.allclose(inter, i_ref, rtol=1e-5, atol=1e-6)
    assert np.allclose(out, o_ref, rtol=1e-4, atol=1e-5)
    # W1 is the gated (silu) side: swapping W1 and W3 must change the result
    assert not np.allclose(oracle_mod.expert_w1w3(x, w3, w1), inter, rtol=1e-3, atol=1e-4)


def test_combine_closed_form(oracle_mod):
    rng = np.random.default_rng(10)
    T, H = 20, 64
    sorted_out = rng.standard_normal((T * TOPK, H)).astype(np.float32)
    perm = rng.permutation(T * TOPK).astype(np.int32).reshape(T, TOPK)
    w = rng.random((T, TOPK)).astype(np.float32)
    res = rng.standard_normal((T, H)).astype(np.float32)
    y = oracle_mod.combine(sorted_out, perm, w)
    yr = oracle_mod.combine(sorted_out, perm, w, residual=res)
    for t in (0, 7, 19):
        for h in (0, 31, 63):
            acc = np.float32(0.0)
            for k in range(TOPK):  # fma chain over k ascending from 0
                acc = fma_exact(sorted_out[perm[t, k], h], w[t, k], acc)
            assert bits(y[t, h]) == bits(acc)
            assert bits(yr[t, h]) == bits(np.float32(res[t, h] + acc))


# ---------------------------------------------------------------------------
# whole block: special cases with closed forms
# ---------------------------------------------------------------------------

def small_block(rng, E=32, H=128, I=64, same_experts=False):
    gate = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.02).astype(np.float32)
    if same_experts:
        w1 = np.repeat((rng.standard_normal((1, I, H)) * 0.05).astype(np.float32), E, 0)
        w3 = np.repeat((rng.standard_normal((1, I, H)) * 0.05).astype(np.float32), E, 0)
        w2 = np.repeat((rng.standard_normal((1, H, I)) * 0.05).astype(np.float32), E, 0)
    else:
        w1 = (rng.standard_normal((E, I, H)) * 0.05).astype(np.float32)
        w3 = (rng.standard_normal((E, I, H)) * 0.05).astype(np.float32)
        w2 = (rng.standard_normal((E, H, I)) * 0.05).astype(np.float32)
    return gate, bias, w1, w3, w2


def mlp64(x, w1, w3, w2):
    x64 = x.astype(np.float64)
    return (silu64(x64 @ w1.T.astype(np.float64)) * (x64 @ w3.T.astype(np.float64))) @ w2.T.astype(np.float64)


def test_block_identical_experts_is_one_mlp(oracle_mod):
    """With 32 equal experts the weights sum to 1, so y = MLP(x) whatever the
    routing picks."""
    rng = np.random.default_rng(11)
    gate, bias, w1, w3, w2 = small_block(rng, same_experts=True)
    x = rng.standard_normal((40, gate.shape[1])).astype(np.float32)
    r = oracle_mod.moe_forward(x, gate, bias, w1, w3, w2)
    assert np.allclose(r["y"], mlp64(x, w1[0], w3[0], w2[0]), rtol=1e-4, atol=1e-5)


def test_block_forced_experts_is_weighted_mix(oracle_mod):
    """Bias +10 on four experts forces them: y = sum_e w_e MLP_e(x) + residual
    with w_e = p_e / sum p."""
    rng = np.random.default_rng(12)
    gate, bias, w1, w3, w2 = small_block(rng)
    forced = [1, 6, 22, 30]
    bias = np.zeros_like(bias)
    bias[forced] = 10.0
    x = rng.standard_normal((25, gate.shape[1])).astype(np.float32)
    res = rng.standard_normal(x.shape).astype(np.float32)
    r = oracle_mod.moe_forward(x, gate, bias, w1, w3, w2, residual=res)
    logits = x.astype(np.float64) @ gate.T.astype(np.float64)
    p = 1.0 / (1.0 + np.exp(-logits[:, forced]))
    wts = p / p.sum(axis=1, keepdims=True)
    ref = res.astype(np.float64) + sum(wts[:, [i]] * mlp64(x, w1[e], w3[e], w2[e])
                                       for i, e in enumerate(forced))
    assert np.allclose(r["y"], ref, rtol=1e-4, atol=1e-5)
    assert r["counts"][forced].tolist() == [25] * 4


def test_block_pieces_compose(oracle_mod):
    """orc_moe_forward equals route -> dispatch -> experts -> combine called
    one by one, bit for bit, also with a token mask."""
    rng = np.random.default_rng(13)
    gate, bias, w1, w3, w2 = small_block(rng)
    T = 60
    x = rng.standard_normal((T, gate.shape[1])).astype(np.float32)
    full = oracle_mod.moe_forward(x, gate, bias, w1, w3, w2)
    logits = oracle_mod.gate_logits(x, gate)
    idx, w, counts = oracle_mod.route(logits, bias)
    offsets, pos, slot_token = oracle_mod.dispatch(idx, 32)
    sout = np.zeros((T * TOPK, gate.shape[1]), np.float32)
    for e in range(32):
        s0, s1 = offsets[e], offsets[e + 1]
        if s1 > s0:
            rows = x[slot_token[s0:s1]]
            sout[s0:s1] = oracle_mod.expert_w2(oracle_mod.expert_w1w3(rows, w1[e], w3[e]), w2[e])
    y = oracle_mod.combine(sout, pos, w)
    assert np.array_equal(bits(full["logits"]), bits(logits))
    assert np.array_equal(full["idx"], idx) and np.array_equal(full["counts"], counts)
    assert np.array_equal(bits(full["y"]), bits(y))
    mask = (np.arange(T) % 3 == 0).astype(np.uint8)
    part = oracle_mod.moe_forward(x, gate, bias, w1, w3, w2, token_mask=mask)
    sel = mask.astype(bool)
    assert np.array_equal(bits(part["y"][sel]), bits(y[sel]))
    assert np.all(np.isnan(part["y"][~sel]))


# ---------------------------------------------------------------------------
# Post-attention RMSNorm (rms_norm_kernel, layer.cu:144-193)
# ---------------------------------------------------------------------------

def _rms_from_total(total, H=2048):
    """rms = 1.0f / sqrtf(total / H + 1e-5f) in float32 (IEEE ops)."""
    f = np.float32
    return f(1.0) / np.sqrt(f(total) / f(H) + f(1e-5))


def test_rmsnorm_one_hot_rows(oracle_mod):
    """A single nonzero element contributes its square exactly whatever the
    reduction order: every index (one per thread, warp and stride position)
    must enter the sum once -- a dropped or doubled term fails."""
    H = 2048
    rng = np.random.RandomState(5)
    wgt = (1.0 + 0.1 * rng.randn(H)).astype(np.float32)
    cols = [0, 1, 16, 31, 32, 255, 256, 511, 1000, 1791, 2047]
    h = np.zeros((len(cols), H), np.float32)
    vals = np.float32(1.5) ** np.arange(len(cols), dtype=np.float32)
    for r, (c, v) in enumerate(zip(cols, vals)):
        h[r, c] = v
    out = oracle_mod.rmsnorm(h, wgt)
    for r, (c, v) in enumerate(zip(cols, vals)):
        rms = _rms_from_total(np.float32(v) * np.float32(v))
        want = (np.float32(v) * rms) * wgt[c]
        assert out[r, c] == want, (c, out[r, c], want)
        assert np.count_nonzero(out[r]) == 1


def _sequential_total(row):
    """float32 sum of squares in index order (the order a plain loop takes)."""
    t = np.float32(0.0)
    for v in row:
        t = np.float32(t + np.float32(v) * np.float32(v))
    return t


# Rows whose sum of squares depends on the reduction order: one large square
# (4096) and several squares of 2^-12, each half an ulp of 4096.  Added to the
# large one first, every small square is lost; the reference's order adds the
# small ones to each other first, so they survive.  Each case gives the total
# the reference's order produces (exact in float32).
_B = 2.0 ** -6   # square 2^-12


def _reverse_total(row):
    """float32 sum of squares in descending index order."""
    return _sequential_total(row[::-1])


# name -> (elements, total in the reference's order, a plausible wrong order)
_ORDER_CASES = {
    # warp tree (__shfl_down at 16, 8, 4, 2, 1): the large square at lane 0,
    # small ones at lanes 1..15 and 17..31 (lane 16 empty).  Lane 0 meets
    # lane 8 (2 small), lane 4 (4), lane 2 (8) and lane 1 (16): 4096 + 30 *
    # 2^-12 exactly; a plain loop over the lanes loses them all.
    "warp tree": ({0: 64.0, **{l: _B for l in list(range(1, 16)) + list(range(17, 32))}},
                  4096.0 + 30 * 2.0 ** -12, _sequential_total),
    # block tree over the 8 warp sums (offsets 4, 2, 1): large at warp 0,
    # one small square in each of warps 1..7 (thread 32w).  w0 + w4 loses its
    # small square; (w2 + w6) and (w1 + w5) + (w3 + w7) keep theirs:
    # 4096 + 6 * 2^-12; a plain loop over the warps loses them all.
    "block tree": ({0: 64.0, **{32 * w: _B for w in range(1, 8)}},
                   4096.0 + 6 * 2.0 ** -12, _sequential_total),
    # one thread's fma chain runs over i = t, t+256, ..., t+1792 ascending:
    # the large square first (i = 7), then seven small ones, each lost:
    # 4096.  Descending order keeps them (7 * 2^-12 first, then 4096 + 3.5
    # ulps, ties to even: 4096 + 8 * 2^-12).
    "thread chain": ({7: 64.0, **{7 + 256 * j: _B for j in range(1, 8)}},
                     4096.0, _reverse_total),
}


@pytest.mark.parametrize("case", sorted(_ORDER_CASES))
def test_rmsnorm_reduction_order(oracle_mod, case):
    """The reference's reduction order (layer.cu:157-186), each stage pinned
    by a row whose total differs from a plausible other order's by several
    ulps, enough to change rms."""
    H = 2048
    elems, total_ref, other_order = _ORDER_CASES[case]
    h = np.zeros((1, H), np.float32)
    for i, v in elems.items():
        h[0, i] = np.float32(v)
    assert np.float32(total_ref) == total_ref          # exact in float32
    total_other = other_order(h[0])
    assert total_other != np.float32(total_ref)
    rms_ref = _rms_from_total(np.float32(total_ref))
    assert rms_ref != _rms_from_total(total_other)      # distinguishable at this input
    wgt = np.ones(H, np.float32)
    out = oracle_mod.rmsnorm(h, wgt)
    i_big = max(elems, key=lambda i: elems[i])
    assert out[0, i_big] == np.float32(64.0) * rms_ref


def test_rmsnorm_matches_float64(oracle_mod):
    """Random rows: within a few float32 ulps of the float64 formula."""
    rng = np.random.RandomState(9)
    T, H = 16, 2048
    h = rng.randn(T, H).astype(np.float32) * np.float32(3.0)
    wgt = (1.0 + 0.05 * rng.randn(H)).astype(np.float32)
    out = oracle_mod.rmsnorm(h, wgt)
    h64 = h.astype(np.float64)
    ref = h64 / np.sqrt((h64 ** 2).mean(axis=1, keepdims=True) + 1e-5) * wgt
    np.testing.assert_allclose(out, ref, rtol=4e-7, atol=0)


def test_moe_forward_norm_is_norm_then_block(oracle_mod):
    """The fused-step oracle is exactly rmsnorm followed by the block with the
    pre-norm rows as the residual."""
    from final_amd import workloads as W
    rng = np.random.RandomState(3)
    T, H, I, E = 4, 64, 32, 8
    h = rng.randn(T, H).astype(np.float32)
    nw = (1.0 + 0.1 * rng.randn(H)).astype(np.float32)
    gate = (0.1 * rng.randn(E, H)).astype(np.float32)
    bias = (0.01 * rng.randn(E)).astype(np.float32)
    w1 = (0.1 * rng.randn(E, I, H)).astype(np.float32)
    w3 = (0.1 * rng.randn(E, I, H)).astype(np.float32)
    w2 = (0.1 * rng.randn(E, H, I)).astype(np.float32)
    r = oracle_mod.moe_forward_norm(h, nw, gate, bias, w1, w3, w2)
    xn = oracle_mod.rmsnorm(h, nw)
    r2 = oracle_mod.moe_forward(xn, gate, bias, w1, w3, w2, residual=h)
    assert np.array_equal(r["xn"], xn)
    assert np.array_equal(r["y"], r2["y"])
    assert np.array_equal(r["idx"], r2["idx"])


# ---------------------------------------------------------------------------
# Dense SwiGLU FFN (MLP::forward_gpu, layer.cu:1231-1269)
# ---------------------------------------------------------------------------

def test_silu_dexp_within_three_roundings(oracle_mod):
    """d_silu (layer.cu:436): exp in double, then three float roundings (the
    cast, 1.0f + e, the quotient), each at most 2^-24 relative: within
    3 * 2^-24 (plus double-rounding slack) of float64 silu; exact at 0."""
    xs = np.concatenate([np.linspace(-30, 30, 2001), [0.0, -1e-30, 1e-30, 88.0, -88.0]])
    for x in xs.astype(np.float32):
        got = np.float32(oracle_mod.silu_dexp(float(x)))
        ref = float(x) / (1.0 + math.exp(-float(x)))
        assert abs(float(got) - ref) <= 3.01 * 2.0 ** -24 * abs(ref) + 1e-45, (x, got, ref)
    assert oracle_mod.silu_dexp(0.0) == 0.0


def test_dense_mlp_matches_float64(oracle_mod):
    """Small shapes: within float32 accumulation error of the float64 SwiGLU
    MLP, with silu on the W1 branch (a W1/W3 swap would fail) and the
    residual added last."""
    rng = np.random.RandomState(11)
    T, H, I = 5, 64, 256
    x = rng.randn(T, H).astype(np.float32)
    w1 = (0.2 * rng.randn(I, H)).astype(np.float32)
    w3 = (0.2 * rng.randn(I, H)).astype(np.float32)
    w2 = (0.2 * rng.randn(H, I)).astype(np.float32)
    r = rng.randn(T, H).astype(np.float32)
    y = oracle_mod.dense_mlp(x, w1, w3, w2, residual=r)
    x64, w164, w364, w264 = (a.astype(np.float64) for a in (x, w1, w3, w2))
    g = x64 @ w164.T
    u = x64 @ w364.T
    ref = (g / (1.0 + np.exp(-g)) * u) @ w264.T + r
    np.testing.assert_allclose(y, ref, rtol=2e-5, atol=2e-5)
    swapped = oracle_mod.dense_mlp(x, w3, w1, w2, residual=r)
    assert np.abs(swapped - ref).max() > 1e-2
    # rows are independent: a token mask computes the selected rows only
    m = np.array([1, 0, 1, 0, 0], np.uint8)
    ym = oracle_mod.dense_mlp(x, w1, w3, w2, residual=r, token_mask=m)
    assert np.array_equal(ym[m.astype(bool)], y[m.astype(bool)])
    assert np.isnan(ym[~m.astype(bool)]).all()


def test_dense_mlp_is_chained_gemms(oracle_mod):
    """The three products are the pinned fma chains (gemm_nt_chain), the
    SwiGLU is d_silu(gate) * up elementwise."""
    rng = np.random.RandomState(12)
    T, H, I = 3, 32, 64
    x = rng.randn(T, H).astype(np.float32)
    w1 = (0.3 * rng.randn(I, H)).astype(np.float32)
    w3 = (0.3 * rng.randn(I, H)).astype(np.float32)
    w2 = (0.3 * rng.randn(H, I)).astype(np.float32)
    gate = oracle_mod.gemm_nt_chain(x, w1)
    up = oracle_mod.gemm_nt_chain(x, w3)
    inter = np.array([[np.float32(oracle_mod.silu_dexp(float(g))) * u for g, u in zip(gr, ur)]
                      for gr, ur in zip(gate, up)], np.float32)
    want = oracle_mod.gemm_nt_chain(inter, w2)
    assert np.array_equal(bits(oracle_mod.dense_mlp(x, w1, w3, w2)), bits(want))


# ---------------------------------------------------------------------------
# Exact rounding sequences of the activations, from decimal arithmetic
# ---------------------------------------------------------------------------

def _dec_exp_to_double(v: float) -> float:
    """exp(v) correctly rounded to double, from 60-digit decimal arithmetic
    (independent of the host's libm)."""
    import decimal
    with decimal.localcontext() as c:
        c.prec = 60
        return float(decimal.Decimal(v).exp())  # Decimal -> float rounds to nearest


def _dec_exp_to_float(v: float) -> np.float32:
    """exp(v) correctly rounded to float (one rounding from the exact value)."""
    import decimal
    with decimal.localcontext() as c:
        c.prec = 60
        e = decimal.Decimal(v).exp()
        # past the largest float plus half its ulp the nearest float is inf
        if e >= decimal.Decimal(float(np.finfo(np.float32).max)) + decimal.Decimal(2.0 ** 103):
            return np.float32(np.inf)
        # nearest float: round the exact value via the two float neighbours of
        # its double approximation (60 digits decide every tie)
        f = np.float32(float(e))
        lo, hi = sorted((f, np.nextafter(f, np.float32(np.inf) if decimal.Decimal(float(f)) < e
                                          else np.float32(-np.inf))))
        dlo, dhi = e - decimal.Decimal(float(lo)), decimal.Decimal(float(hi)) - e
        if dlo < dhi:
            return lo
        if dhi < dlo:
            return hi
        return lo if (lo.view(np.uint32) & 1) == 0 else hi


def _sweep():
    xs = np.concatenate([np.linspace(-30, 30, 6001), np.linspace(-2, 2, 4001),
                         [0.0, 1e-30, -1e-30, 1e-7, -1e-7, 88.0, -88.0, 103.0, -103.0]])
    return np.unique(xs.astype(np.float32))


def test_sigmoid_is_the_double_exp_sequence(oracle_mod):
    """d_sigmoid (layer.cu:435): e = (float)exp(-(double)x) (exp correctly
    rounded to double, then to float), then 1.0f + e and 1.0f / that, each
    rounded to float.  Bit-equal over a dense sweep.  The sweep separates this
    three-rounding sequence from a sigmoid evaluated in double and rounded
    once (which differs at thousands of points).  A correctly rounded expf in
    place of the double exp gives the same e except where the double result
    sits within half a double ulp of a float rounding boundary, which no point
    of the sweep hits: that choice is bounded (at most one float ulp in e on
    such a point) rather than pinned."""
    one = np.float32(1.0)
    d_one = 0
    for x in _sweep():
        e = np.float32(_dec_exp_to_double(-float(x)))
        ref = one / (one + e)
        got = np.float32(oracle_mod.sigmoid(float(x)))
        assert got.view(np.uint32) == ref.view(np.uint32), (x, got, ref)
        alt1 = np.float32(1.0 / (1.0 + _dec_exp_to_double(-float(x))))  # one rounding
        d_one += alt1.view(np.uint32) != ref.view(np.uint32)
    assert d_one > 100, d_one


def test_silu_dexp_is_the_double_exp_sequence(oracle_mod):
    """d_silu (layer.cu:436): x / (1.0f + (float)exp(-(double)x)), bit-equal."""
    one = np.float32(1.0)
    for x in _sweep():
        e = np.float32(_dec_exp_to_double(-float(x)))
        ref = x / (one + e)
        got = np.float32(oracle_mod.silu_dexp(float(x)))
        assert got.view(np.uint32) == ref.view(np.uint32), (x, got, ref)


def test_silu_is_the_expf_sequence(oracle_mod):
    """d_silu_opt (layer.cu:728): x / (1.0f + expf(-x)) with expf rounded
    once to float.  The host's expf is a library routine: it must agree with
    the correctly rounded exp on all but a few last-bit ties of the sweep, and
    wherever it does the rest of the sequence is bit-equal.  The sweep
    separates it from x * sigmoid(x) and from silu evaluated in double and
    rounded once (each differs at many points)."""
    one = np.float32(1.0)
    n = miss = d_mul = d_one = 0
    for x in _sweep():
        e = _dec_exp_to_float(-float(x))
        ref = x / (one + e)
        got = np.float32(oracle_mod.silu(float(x)))
        n += 1
        if got.view(np.uint32) != ref.view(np.uint32):
            miss += 1
            assert abs(float(got) - float(ref)) <= 2 * float(np.spacing(np.abs(ref))), (x, got, ref)
        d_mul += (x * (one / (one + e))).view(np.uint32) != ref.view(np.uint32)
        alt1 = np.float32(float(x) / (1.0 + _dec_exp_to_double(-float(x))))
        d_one += alt1.view(np.uint32) != ref.view(np.uint32)
    assert miss <= n // 1000, (miss, n)
    assert d_mul > 100 and d_one > 100, (d_mul, d_one)
