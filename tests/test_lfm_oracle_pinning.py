"""Pins the decoder-model oracle (oracle/lfm_oracle.c and the composition in
oracle/oracle.py) independently of its own formulas: closed forms, float64
restatements of the textbook operations, causality and sequence-boundary
invariants, and constructed routing ties.  The reference holds no vectors for
these paths (its attention keeps at most 16 positions, layer.cu:312, and its
own CPU paths are empty stubs), so these checks are what pins them; each is
chosen so that a plausible slip (a pairing of the wrong rotary columns, a
flipped rotation sign, a wrong kv-head mapping, a conv tap in the wrong
order, a missing residual) fails it.
"""
import numpy as np
import pytest

from conftest import bits

HD = 64


def rng(s):
    return np.random.default_rng(s)


def ulp(x):
    return np.spacing(np.abs(np.asarray(x, np.float32))).astype(np.float64)


# -- embedding -------------------------------------------------------------------

def test_embed_gathers_rows(oracle_mod):
    table = rng(0).standard_normal((50, 16), dtype=np.float32)
    ids = np.array([3, 0, 49, 3, -1, 50], np.int32)
    h = oracle_mod.embed(ids, table)
    assert np.array_equal(bits(h[:4]), bits(table[[3, 0, 49, 3]]))
    assert not h[4:].any()


# -- rotary tables -----------------------------------------------------------------

def test_rope_tables_closed_forms(oracle_mod):
    P = 4096
    c, s = oracle_mod.rope_tables(P)
    assert np.array_equal(c[0], np.ones(HD, np.float32)) and not s[0].any()
    assert np.array_equal(bits(c[:, :32]), bits(c[:, 32:]))
    assert np.array_equal(bits(s[:, :32]), bits(s[:, 32:]))
    # theta_j within 2 ulp of 1e6^(-2j/64); the tables within 1 ulp of the
    # float64 cos/sin of the float angle (float(i) * theta_j rounded)
    j = np.arange(32)
    th = np.array([np.float32(1e6) ** np.float32(-2.0 * k / 64) for k in j], np.float32)
    th64 = 1e6 ** (-2.0 * j / 64)
    assert np.all(np.abs(th.astype(np.float64) - th64) <= 2 * ulp(th))
    ang = (np.arange(P, dtype=np.float32)[:, None] * th[None, :]).astype(np.float32)
    for tab, fn in ((c, np.cos), (s, np.sin)):
        ref = fn(ang.astype(np.float64))
        assert np.all(np.abs(tab[:, :32].astype(np.float64) - ref) <= ulp(ref) * 1.0 + 1e-45)
    # column 0 rotates by exactly one radian per position
    np.testing.assert_allclose(c[:, 0], np.cos(np.arange(P, dtype=np.float64)), rtol=0, atol=1e-6)


# -- q/k norm + rotation ------------------------------------------------------------

def _rot64(y, c, s):
    """Complex rotation of the (d, d+32) pairs in float64."""
    z = (y[..., :32].astype(np.float64) + 1j * y[..., 32:].astype(np.float64)) * \
        (c[..., :32].astype(np.float64) + 1j * s[..., :32].astype(np.float64))
    return np.concatenate([z.real, z.imag], axis=-1)


def test_qk_norm_rope_pins(oracle_mod):
    batch, seq, heads, kvh = 2, 40, 4, 1
    T, ld = batch * seq, (heads + 2 * kvh) * HD
    qkv = (2.0 * rng(1).standard_normal((T, ld))).astype(np.float32)
    qw = rng(2).standard_normal(HD, dtype=np.float32)
    kw = rng(3).standard_normal(HD, dtype=np.float32)
    c, s = oracle_mod.rope_tables(seq)
    out = oracle_mod.qk_norm_rope(qkv, seq, qw, kw, c, s, heads, kvh, heads * HD)
    # v columns untouched
    assert np.array_equal(bits(out[:, (heads + kvh) * HD:]), bits(qkv[:, (heads + kvh) * HD:]))
    for hd in range(heads + kvh):
        cols = slice(hd * HD, (hd + 1) * HD)
        y = oracle_mod.rmsnorm(np.ascontiguousarray(qkv[:, cols]), qw if hd < heads else kw)
        pos = np.arange(T) % seq
        # position 0 is the identity: exactly the RMSNorm
        first = pos == 0
        assert np.array_equal(bits(out[first, cols]), bits(y[first]))
        # every position: the float64 complex rotation by +pos * theta_j
        ref = _rot64(y, c[pos], s[pos])
        np.testing.assert_allclose(out[:, cols], ref, rtol=0, atol=4e-6 * np.abs(y).max())
        # the rotation keeps each pair's length
        n_in = np.hypot(y[:, :32].astype(np.float64), y[:, 32:])
        n_out = np.hypot(out[:, cols][:, :32].astype(np.float64), out[:, cols][:, 32:])
        np.testing.assert_allclose(n_out, n_in, rtol=1e-6, atol=1e-6)


# -- attention ----------------------------------------------------------------------

def _attn64(qkv, batch, seq, heads, kvh):
    q_c, kv_c = heads * HD, kvh * HD
    x = qkv.astype(np.float64).reshape(batch, seq, -1)
    out = np.zeros((batch, seq, heads * HD))
    for b in range(batch):
        for h in range(heads):
            g = h // (heads // kvh)
            q = x[b, :, h * HD:(h + 1) * HD]
            k = x[b, :, q_c + g * HD:q_c + (g + 1) * HD]
            v = x[b, :, q_c + kv_c + g * HD:q_c + kv_c + (g + 1) * HD]
            sc = q @ k.T / 8.0
            sc[np.triu_indices(seq, 1)] = -np.inf
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            out[b, :, h * HD:(h + 1) * HD] = p @ v
    return out.reshape(batch * seq, -1)


@pytest.mark.parametrize("batch,seq,heads,kvh", [(2, 37, 8, 2), (1, 70, 4, 1), (3, 1, 4, 1)])
def test_attention_matches_float64_softmax(batch, seq, heads, kvh, oracle_mod):
    ld = (heads + 2 * kvh) * HD
    qkv = rng(seq).standard_normal((batch * seq, ld), dtype=np.float32)
    got = oracle_mod.attention(qkv, batch, seq, heads, kvh, heads * HD, (heads + kvh) * HD)
    np.testing.assert_allclose(got, _attn64(qkv, batch, seq, heads, kvh), rtol=1e-5, atol=2e-6)


def test_attention_closed_forms(oracle_mod):
    batch, seq, heads, kvh = 2, 33, 8, 2
    ld = (heads + 2 * kvh) * HD
    qc, vc = heads * HD, (heads + kvh) * HD
    qkv = rng(5).standard_normal((batch * seq, ld), dtype=np.float32)
    got = oracle_mod.attention(qkv, batch, seq, heads, kvh, qc, vc)
    x = qkv.reshape(batch, seq, -1)
    # the first query of a sequence sees only its own key: out = v exactly
    for h in range(heads):
        g = h // (heads // kvh)
        assert np.array_equal(bits(got.reshape(batch, seq, -1)[:, 0, h * HD:(h + 1) * HD]),
                              bits(x[:, 0, vc + g * HD:vc + (g + 1) * HD]))
    # q = 0: uniform weights, out = mean of v over the prefix
    z = qkv.copy()
    z[:, :qc] = 0
    got0 = oracle_mod.attention(z, batch, seq, heads, kvh, qc, vc).reshape(batch, seq, -1)
    v = x[:, :, vc:].astype(np.float64)
    pref = np.cumsum(v, axis=1) / np.arange(1, seq + 1)[None, :, None]
    for h in range(heads):
        g = h // (heads // kvh)
        np.testing.assert_allclose(got0[:, :, h * HD:(h + 1) * HD], pref[:, :, g * HD:(g + 1) * HD],
                                   rtol=1e-5, atol=1e-6)
    # causality: changing the last position's k and v changes no earlier output
    y = qkv.copy().reshape(batch, seq, -1)
    y[:, -1, qc:] = 100.0
    got1 = oracle_mod.attention(y.reshape(batch * seq, -1), batch, seq, heads, kvh, qc, vc)
    m = np.ones((batch, seq), bool)
    m[:, -1] = False
    assert np.array_equal(bits(got1.reshape(batch, seq, -1)[m]), bits(got.reshape(batch, seq, -1)[m]))


# -- short conv ----------------------------------------------------------------------

def test_shortconv_pins(oracle_mod):
    batch, seq, H, L = 3, 9, 16, 3
    T = batch * seq
    bcg = rng(6).standard_normal((T, 3 * H), dtype=np.float32)
    w = rng(7).standard_normal((H, L), dtype=np.float32)
    y = oracle_mod.shortconv(bcg, w, batch, seq, L)
    b3 = bcg.astype(np.float64).reshape(batch, seq, 3, H)
    bx = b3[:, :, 0] * b3[:, :, 2]
    ref = np.zeros((batch, seq, H))
    for s in range(seq):
        for k in range(L):
            p = s - (L - 1) + k
            if p >= 0:
                ref[:, s] += bx[:, p] * w[:, k]
    ref *= b3[:, :, 1]
    np.testing.assert_allclose(y.reshape(batch, seq, H), ref, rtol=1e-5, atol=1e-6)
    # impulse: B*g = 1 at one position of sequence 1 only, C = 1 -> the taps
    imp = np.zeros_like(bcg).reshape(batch, seq, 3, H)
    imp[:, :, 1] = 1.0
    imp[1, 4, 0] = 1.0
    imp[1, 4, 2] = 1.0
    yi = oracle_mod.shortconv(imp.reshape(T, -1), w, batch, seq, L).reshape(batch, seq, H)
    expect = np.zeros((batch, seq, H), np.float32)
    for d in range(L):  # output s = 4 + d uses tap k = L - 1 - d
        expect[1, 4 + d] = w[:, L - 1 - d]
    assert np.array_equal(bits(yi), bits(expect))


# -- routing guide --------------------------------------------------------------------

def _small_moe(seed, T=24, H=64, I=64, E=8):
    r = rng(seed)
    return dict(x=r.standard_normal((T, H), dtype=np.float32),
                gate=(0.2 * r.standard_normal((E, H))).astype(np.float32),
                bias=np.zeros(E, np.float32),
                w1=(0.1 * r.standard_normal((E, I, H))).astype(np.float32),
                w3=(0.1 * r.standard_normal((E, I, H))).astype(np.float32),
                w2=(0.1 * r.standard_normal((E, H, I))).astype(np.float32))


def test_guided_routing(oracle_mod):
    O = oracle_mod
    m = _small_moe(8)
    res = np.zeros_like(m["x"])
    own = O.moe_forward(m["x"], m["gate"], m["bias"], m["w1"], m["w3"], m["w2"], residual=res)
    # the own routing as guide: nothing adopted, the same y bit for bit
    y, idx, na, nh = O.moe_forward_guided(m["x"], m["gate"], m["bias"], m["w1"], m["w3"], m["w2"],
                                          res, own["idx"], 1e-4)
    assert (na, nh) == (0, 0) and np.array_equal(idx, own["idx"])
    assert np.array_equal(bits(y), bits(own["y"]))
    # a clearly worse expert in place of the 4th: not a near-tie, own kept
    g = own["idx"].copy()
    lg = own["logits"]
    sc = 1 / (1 + np.exp(-lg.astype(np.float64)))
    worst = np.argmin(sc, axis=1)
    g[:, 3] = worst
    y2, idx2, na, nh = O.moe_forward_guided(m["x"], m["gate"], m["bias"], m["w1"], m["w3"],
                                            m["w2"], res, g, 1e-4)
    assert na == 0 and nh == len(g) and np.array_equal(idx2, own["idx"])
    # a constructed tie: token 0's 4th and 5th experts get equal scores through
    # the bias; the oracle takes the lower index, the guide the other one
    p = np.array([O.sigmoid(v) for v in lg[0]], np.float32)
    order = np.argsort(-p.astype(np.float64), kind="stable")
    a, b = int(order[3]), int(order[4])
    bias = np.zeros(8, np.float32)
    bias[b] = np.float32(p[a] - p[b])
    while np.float32(p[b] + bias[b]) < p[a]:
        bias[b] = np.nextafter(bias[b], np.float32(1))
    assert np.float32(p[b] + bias[b]) == p[a]
    own3 = O.moe_forward(m["x"][:1], m["gate"], bias, m["w1"], m["w3"], m["w2"], residual=res[:1])
    lo, hi = min(a, b), max(a, b)
    assert lo in own3["idx"][0] and hi not in own3["idx"][0]
    g3 = own3["idx"].copy()
    g3[0, list(g3[0]).index(lo)] = hi
    y3, idx3, na, nh = O.moe_forward_guided(m["x"][:1], m["gate"], bias, m["w1"], m["w3"], m["w2"],
                                            res[:1], g3, 1e-6)
    assert (na, nh) == (1, 0) and np.array_equal(idx3, g3)
    assert not np.array_equal(bits(y3), bits(own3["y"]))
    # duplicates are never a top-4
    g4 = own3["idx"].copy()
    g4[0, 1] = g4[0, 0]
    *_, na, nh = O.moe_forward_guided(m["x"][:1], m["gate"], bias, m["w1"], m["w3"], m["w2"],
                                      res[:1], g4, 1.0)
    assert (na, nh) == (0, 1)


# -- decoder layer and head, against float64 ----------------------------------------

def _rms64(x, w):
    x = x.astype(np.float64)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + 1e-5) * w


def _layer64(h, w, batch, seq, c, s, idx):
    """DecoderLayer in float64 from the textbook operations, with the MoE
    routing given (idx [T][4]; weights renormalised from the sigmoid)."""
    h = h.astype(np.float64)
    xn = _rms64(h, w["op_norm"])
    if "q" in w:
        heads, kvh = w["q"].shape[0] // HD, w["k"].shape[0] // HD
        q, k, v = xn @ w["q"].T, xn @ w["k"].T, xn @ w["v"].T
        pos = np.arange(len(h)) % seq

        def nr(x, nw, n):
            x = x.reshape(len(h), n, HD)
            x = _rms64(x, nw)
            return _rot64(x, c[pos][:, None, :], s[pos][:, None, :]).reshape(len(h), n * HD)
        q, k = nr(q, w["q_norm"], heads), nr(k, w["k_norm"], kvh)
        att = _attn64(np.concatenate([q, k, v], axis=1), batch, seq, heads, kvh)
        op = att @ w["o"].T
    else:
        bcg = xn @ w["in_proj"].T
        H = h.shape[1]
        b3 = bcg.reshape(batch, seq, 3, H)
        bx = b3[:, :, 0] * b3[:, :, 2]
        conv = np.zeros((batch, seq, H))
        for t in range(seq):
            for kk in range(3):
                p = t - 2 + kk
                if p >= 0:
                    conv[:, t] += bx[:, p] * w["conv"].reshape(H, 3)[:, kk]
        op = (b3[:, :, 1] * conv).reshape(len(h), H) @ w["out_proj"].T
    h = h + op
    x2 = _rms64(h, w["ffn_norm"])
    p = 1 / (1 + np.exp(-(x2 @ w["gate"].T)))
    y = h.copy()
    for t in range(len(h)):
        pw = p[t, idx[t]]
        pw = pw / pw.sum()
        for e, wt in zip(idx[t], pw):
            a = x2[t] @ w["w1"][e].T
            g = a / (1 + np.exp(-a)) * (x2[t] @ w["w3"][e].T)
            y[t] += wt * (g @ w["w2"][e].T)
    return y


@pytest.mark.parametrize("attn", [True, False])
def test_decoder_layer_matches_float64(attn, oracle_mod):
    O = oracle_mod
    batch, seq, H, I, E = 2, 20, 256, 128, 8
    r = rng(10 + attn)
    w = {"op_norm": (1 + 0.1 * r.standard_normal(H)).astype(np.float32),
         "ffn_norm": (1 + 0.1 * r.standard_normal(H)).astype(np.float32),
         "gate": (0.05 * r.standard_normal((E, H))).astype(np.float32),
         "bias": (0.02 * r.standard_normal(E)).astype(np.float32),
         "w1": (0.05 * r.standard_normal((E, I, H))).astype(np.float32),
         "w3": (0.05 * r.standard_normal((E, I, H))).astype(np.float32),
         "w2": (0.05 * r.standard_normal((E, H, I))).astype(np.float32)}
    if attn:
        w.update(q=(0.05 * r.standard_normal((H, H))).astype(np.float32),
                 k=(0.05 * r.standard_normal((HD, H))).astype(np.float32),
                 v=(0.05 * r.standard_normal((HD, H))).astype(np.float32),
                 o=(0.05 * r.standard_normal((H, H))).astype(np.float32),
                 q_norm=(1 + 0.1 * r.standard_normal(HD)).astype(np.float32),
                 k_norm=(1 + 0.1 * r.standard_normal(HD)).astype(np.float32))
    else:
        w.update(conv=(0.3 * r.standard_normal((H, 3))).astype(np.float32),
                 in_proj=(0.05 * r.standard_normal((3 * H, H))).astype(np.float32),
                 out_proj=(0.05 * r.standard_normal((H, H))).astype(np.float32))
    h = r.standard_normal((batch * seq, H), dtype=np.float32)
    c, s = O.rope_tables(seq)
    got, info = O.decoder_layer(h, w, batch, seq, c, s)
    ref = _layer64(h, w, batch, seq, c, s, info["idx"])
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
    # the residual carries h: zero operator and expert outputs give h back exactly
    z = dict(w)
    z["w2"] = np.zeros_like(w["w2"])
    z["o" if attn else "out_proj"] = np.zeros_like(w["o" if attn else "out_proj"])
    same, _ = O.decoder_layer(h, z, batch, seq, c, s)
    assert np.array_equal(bits(same), bits(h))


def test_model_head_takes_last_tokens(oracle_mod):
    batch, seq, H, V = 3, 5, 64, 256
    h = rng(12).standard_normal((batch * seq, H), dtype=np.float32)
    nw = (1 + 0.1 * rng(13).standard_normal(H)).astype(np.float32)
    head = rng(14).standard_normal((V, H), dtype=np.float32)
    got = oracle_mod.model_head(h, nw, head, batch, seq)
    last = h.reshape(batch, seq, H)[:, -1]
    np.testing.assert_allclose(got, _rms64(last, nw) @ head.T.astype(np.float64), rtol=1e-5, atol=1e-5)
