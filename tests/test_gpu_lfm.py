"""Parity of the decoder-model kernels around the MoE block (include/lfm_capi.h)
with the CPU oracle (oracle/lfm_oracle.c, moe_oracle.c).

Bars: the embedding, the strided RMSNorm, the q/k norm + rotation and the
short-conv mix restate the reference's arithmetic exactly and are compared
bit for bit; the projection GEMM (MFMA tiles, another accumulation order than
the reference's FMA chains) and the attention (online softmax in fp32 instead
of the reference's double-precision exp and sum) within rtol 1e-3 / atol 1e-4,
the fp32 tolerance of the model.  Decoder layers are checked teacher-forced
(the oracle gets the GPU's input) with the MoE routing bit-exact except where
the oracle's own scores are tied within 1e-5 (orc_moe_forward_guided).
"""
import sys

import numpy as np
import pytest

from conftest import bits
from test_gpu_lfm_model import near_tie_gaps

RTOL, ATOL = 1e-3, 1e-4
TIE_EPS = 1e-5


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rng(seed):
    return np.random.default_rng(seed)


def dev(a):
    from final_amd import hip
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,res", [(1, 128, 32, False), (20, 256, 512, False),
                                       (64, 65536 // 16, 2048, False),
                                       (100, 3072, 2048, True), (300, 256, 64, False),
                                       (1050, 128, 2048, False), (1100, 384, 256, True),
                                       (2048, 6144, 2048, False), (4096, 2048, 2048, True)])
def test_gemm_nt(M, N, K, res, oracle_mod):
    from final_amd import hip, lfm
    say(f"[gemm] M={M} N={N} K={K} residual={res}")
    r = rng(M + N)
    A = r.standard_normal((M, K), dtype=np.float32)
    B = (0.02 * r.standard_normal((N, K))).astype(np.float32)
    R = r.standard_normal((M, N), dtype=np.float32) if res else None
    dA, dB = dev(A), dev(B)
    dC = dev(R) if res else hip.DeviceArray((M, N))
    lfm.gemm_nt(dA, dB, dC, M, N, K, R=dC if res else None)  # residual in place
    got = dC.download()
    ref = oracle_mod.gemm_nt_chain(A, B)
    if res:
        ref = oracle_mod.add(R, ref)
    np.testing.assert_allclose(got, ref, rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
def test_embedding_bit_exact_and_bad_ids(oracle_mod):
    from final_amd import hip, lfm
    V, H, T = 1000, 2048, 300
    table = rng(1).standard_normal((V, H), dtype=np.float32)
    ids = rng(2).integers(0, V, T).astype(np.int32)
    dt, di, dh = dev(table), dev(ids), hip.DeviceArray((T, H))
    flag = dev(np.zeros(1, np.int32))
    lfm.embed(di, dt, dh, T, H, V, bad_flag=flag)
    assert np.array_equal(bits(dh.download()), bits(oracle_mod.embed(ids, table)))
    assert flag.download()[0] == 0
    ids[[0, 17]] = [-1, V]
    di.upload(ids)
    lfm.embed(di, dt, dh, T, H, V, bad_flag=flag)
    got = dh.download()
    assert flag.download()[0] == 1
    assert not got[0].any() and not got[17].any()
    assert np.array_equal(bits(got), bits(oracle_mod.embed(ids, table)))


@pytest.mark.gpu
@pytest.mark.parametrize("dim,rows,stride", [(2048, 64, 512 * 2048), (64, 4096, 64), (2048, 7, 2048)])
def test_rmsnorm_rows_bit_exact(dim, rows, stride, oracle_mod):
    from final_amd import hip, lfm
    say(f"[rmsnorm] dim={dim} rows={rows} stride={stride}")
    x = (3.0 * rng(dim).standard_normal((rows - 1) * stride + dim)).astype(np.float32)
    w = rng(5).standard_normal(dim, dtype=np.float32)
    dx, dw, dy = dev(x), dev(w), hip.DeviceArray((rows, dim))
    lfm.rmsnorm(dx, dw, dy, rows, dim, x_stride=stride)
    sel = np.stack([x[r * stride:r * stride + dim] for r in range(rows)])
    assert np.array_equal(bits(dy.download()), bits(oracle_mod.rmsnorm(sel, w)))


@pytest.mark.gpu
@pytest.mark.parametrize("batch,seq", [(2, 512), (3, 37), (1, 1)])
def test_qk_norm_rope_bit_exact(batch, seq, oracle_mod):
    """GPU vs oracle bit for bit.  Both read `q1*c1 - q2*s1` (layer.cu:225-226)
    the same way (q1*c1 fused into an FMA with the rounded product q2*s1), so
    this shows that the two implementations agree, not that they match the
    reference's nvcc build, whose contraction choice nothing pins."""
    from final_amd import lfm
    say(f"[qk_norm_rope] batch={batch} seq={seq}")
    T = batch * seq
    qkv = rng(seq).standard_normal((T, lfm.QKV_COLS), dtype=np.float32)
    qw = rng(7).standard_normal(64, dtype=np.float32)
    kw = rng(8).standard_normal(64, dtype=np.float32)
    cos, sin = lfm.rope_tables(max(seq, 1))
    d = dev(qkv)
    lfm.qk_norm_rope(d, lfm.QKV_COLS, dev(qw), dev(kw), dev(cos), dev(sin), batch, seq)
    ref = oracle_mod.qk_norm_rope(qkv, seq, qw, kw, cos, sin)
    assert np.array_equal(bits(d.download()), bits(ref))


@pytest.mark.gpu
@pytest.mark.parametrize("batch,seq", [(2, 512), (4, 16), (3, 37), (2, 1), (1, 130)])
def test_attention(batch, seq, oracle_mod):
    from final_amd import hip, lfm
    say(f"[attention] batch={batch} seq={seq}")
    T = batch * seq
    qkv = rng(seq + 3).standard_normal((T, lfm.QKV_COLS), dtype=np.float32)
    d, out = dev(qkv), hip.DeviceArray((T, lfm.Q_COLS))
    lfm.attention(d, lfm.QKV_COLS, out, batch, seq)
    got = out.download()
    ref = oracle_mod.attention(qkv, batch, seq)
    np.testing.assert_allclose(got, ref, rtol=RTOL, atol=ATOL)
    # causality: the first query of every sequence attends to itself only
    v0 = qkv.reshape(batch, seq, -1)[:, 0, lfm.Q_COLS + lfm.KV_COLS:]
    for h in range(lfm.HEADS):
        g = h // 4
        np.testing.assert_allclose(got.reshape(batch, seq, -1)[:, 0, h * 64:(h + 1) * 64],
                                   v0[:, g * 64:(g + 1) * 64], rtol=1e-6, atol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("batch,seq", [(2, 512), (3, 2), (5, 1)])
def test_shortconv_bit_exact(batch, seq, oracle_mod):
    from final_amd import hip, lfm
    say(f"[shortconv] batch={batch} seq={seq}")
    H, T = lfm.HIDDEN, batch * seq
    bcg = rng(seq).standard_normal((T, 3 * H), dtype=np.float32)
    w = (0.3 * rng(9).standard_normal((H, 3))).astype(np.float32)
    y = hip.DeviceArray((T, H))
    lfm.shortconv(dev(bcg), dev(w), y, batch, seq, H)
    assert np.array_equal(bits(y.download()), bits(oracle_mod.shortconv(bcg, w, batch, seq)))


@pytest.mark.gpu
def test_device_generator_matches_host():
    from final_amd import hip, lfm
    from final_amd import workloads as W
    n, first = 1 << 20, 12345
    d = hip.DeviceArray((n,))
    lfm.synth_normal_device(d, n, 7, 99, 0.02, first)
    got = d.download()
    ref = W.normal(7, 99, 0.02, n, first)
    mism = int(np.count_nonzero(bits(got) != bits(ref)))
    say(f"[synth] device vs host mismatches: {mism} of {n}")
    assert mism <= 2  # double log/cos of two libms: a last-bit tie in float rounding at most
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=0)


# -- decoder layers, teacher-forced ---------------------------------------------

def _layer_check(model, O, layer, h_in, h_out_gpu, batch, seq, cos, sin):
    """Runs the oracle's layer on the GPU's input and compares."""
    from final_amd import lfm
    w = lfm.synth_layer_weights(model.seed, layer, model.is_attention(layer), model.is_moe(layer),
                                model.std)
    guide = model.last_routing(layer, batch * seq) if model.is_moe(layer) else None
    ref, info = O.decoder_layer(h_in, w, batch, seq, cos, sin, guide=guide, eps=TIE_EPS)
    if guide is not None:
        gaps = near_tie_gaps(info, w["bias"])
        say(f"[layer {layer}] near-ties followed: {info['adopted']} (gaps {gaps.tolist()}), "
            f"not near-ties: {info['hard']}")
        assert info["hard"] == 0, "GPU routing differs from the oracle's beyond a near-tie"
        assert len(gaps) == info["adopted"] and (gaps >= -TIE_EPS).all()
        assert info["adopted"] <= 2
    np.testing.assert_allclose(h_out_gpu, ref, rtol=RTOL, atol=ATOL)


@pytest.mark.gpu
def test_decoder_layers_teacher_forced(oracle_mod):
    """One conv and one attention layer (MoE FFN), then a dense-FFN conv layer,
    batch 2 x seq 512, each checked against the oracle on the GPU's input."""
    from final_amd import hip, lfm
    batch, seq = 2, 512
    T = batch * seq
    say("[layers] building a 3-layer synthetic model")
    model = lfm.LFM2Model(num_layers=3, layer_types=[1, 0, 1], num_dense_layers=0,
                          max_batch=batch, max_seq=seq, seed=11)
    dense = lfm.LFM2Model(num_layers=1, layer_types=[1], num_dense_layers=1,
                          max_batch=batch, max_seq=seq, seed=12)
    cos, sin = lfm.rope_tables(seq)
    ids = rng(3).integers(0, lfm.VOCAB, (batch, seq)).astype(np.int32)
    d_ids, h = dev(ids), hip.DeviceArray((T, lfm.HIDDEN))
    model.embed(d_ids, batch, seq, h)
    h_in = h.download()
    table = lfm.synth_tensor(model.seed, "embed_tokens.weight", (lfm.VOCAB, lfm.HIDDEN))
    assert np.array_equal(bits(h_in), bits(oracle_mod.embed(ids, table)))
    for layer in range(model.num_layers):
        say(f"[layers] layer {layer} attention={model.is_attention(layer)}")
        model.layer_forward(layer, h, batch, seq)
        h_out = h.download()
        _layer_check(model, oracle_mod, layer, h_in, h_out, batch, seq, cos, sin)
        h_in = h_out
    assert model.status() == 0
    say("[layers] dense-FFN layer")
    h.upload(h_in)
    dense.layer_forward(0, h, batch, seq)
    _layer_check(dense, oracle_mod, 0, h_in, h.download(), batch, seq, cos, sin)


@pytest.mark.gpu
def test_model_small_end_to_end(oracle_mod):
    """4 layers (conv, attention, conv, attention), batch 3 x seq 96: the
    one-call forward equals the layer-by-layer one bit for bit, and its
    last-token logits match the oracle run freely on the same ids (following
    the GPU's routing only on near-ties)."""
    from final_amd import hip, lfm
    batch, seq, L = 3, 96, 4
    T = batch * seq
    model = lfm.LFM2Model(num_layers=L, layer_types=[1, 0, 1, 0], num_dense_layers=0,
                          max_batch=4, max_seq=128, seed=21)
    ids = rng(4).integers(0, lfm.VOCAB, (batch, seq)).astype(np.int32)
    d_ids = dev(ids)
    logits = hip.DeviceArray((batch, lfm.VOCAB))
    model.forward(d_ids, batch, seq, logits)
    got = logits.download()
    h = hip.DeviceArray((T, lfm.HIDDEN))
    model.embed(d_ids, batch, seq, h)
    guides = {}
    for layer in range(L):
        model.layer_forward(layer, h, batch, seq)
        guides[layer] = model.last_routing(layer, T)
    model.head(h, batch, seq, logits)
    assert np.array_equal(bits(logits.download()), bits(got)), "one-call forward differs"
    cos, sin = lfm.rope_tables(seq)
    table = lfm.synth_tensor(model.seed, "embed_tokens.weight", (lfm.VOCAB, lfm.HIDDEN))
    x = oracle_mod.embed(ids, table)
    adopted = 0
    for layer in range(L):
        w = lfm.synth_layer_weights(model.seed, layer, model.is_attention(layer), True)
        x, info = oracle_mod.decoder_layer(x, w, batch, seq, cos, sin, guide=guides[layer],
                                           eps=1e-4)
        assert info["hard"] == 0
        adopted += info["adopted"]
    norm_w = lfm.synth_tensor(model.seed, "embedding_norm.weight", (lfm.HIDDEN,))
    ref = oracle_mod.model_head(x, norm_w, table, batch, seq)
    say(f"[model] near-ties followed: {adopted}; max |dlogit| {np.abs(got - ref).max():.3e}")
    np.testing.assert_allclose(got, ref, rtol=RTOL, atol=ATOL)
