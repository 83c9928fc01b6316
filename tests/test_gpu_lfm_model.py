"""The whole decoder forward at the benchmark's shape on one GPU: 24 layers (the
reference's layer types: 6 attention, 18 short conv), every FFN the MoE block,
hidden 2048, vocab 65536, synthetic N(0, 0.02) weights, batch 64 x seq 512 of
uniform random token ids.

The oracle runs two of the 64 sequences (the first and the last) through all
24 layers on its own, following the GPU's routing only where its own top-4 is
tied within 1e-4 (orc_moe_forward_guided); their last-token logits must match
the GPU's within rtol 1e-3 / atol 1e-4.  Sequences are independent in every
layer (attention and the conv stay inside a sequence, the MoE block works per
token), so two of them are a fair sample.
"""
import sys

import numpy as np
import pytest

from conftest import bits

RTOL, ATOL = 1e-3, 1e-4
TIE_EPS = 1e-4
BATCH, SEQ, LAYERS = 64, 512, 24
SAMPLE = (0, BATCH - 1)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.gpu
def test_lfm2_forward_batch64_seq512(oracle_mod):
    from final_amd import hip, lfm
    T = BATCH * SEQ
    say(f"[model] building {LAYERS} synthetic layers (batch {BATCH} x seq {SEQ})")
    model = lfm.LFM2Model(num_layers=LAYERS, num_dense_layers=0, max_batch=BATCH, max_seq=SEQ,
                          seed=0)
    ids = np.random.default_rng(0).integers(0, lfm.VOCAB, (BATCH, SEQ)).astype(np.int32)
    d_ids = hip.DeviceArray.from_numpy(ids)
    logits = hip.DeviceArray((BATCH, lfm.VOCAB))
    model.forward(d_ids, BATCH, SEQ, logits)
    got = logits.download()
    assert np.all(np.isfinite(got))
    say("[model] layer-by-layer pass (routing of the sampled sequences)")
    h = hip.DeviceArray((T, lfm.HIDDEN))
    model.embed(d_ids, BATCH, SEQ, h)
    rows = np.concatenate([np.arange(b * SEQ, (b + 1) * SEQ) for b in SAMPLE])
    guides = []
    for layer in range(LAYERS):
        model.layer_forward(layer, h, BATCH, SEQ)
        guides.append(np.ascontiguousarray(model.last_routing(layer, T)[rows]))
    model.head(h, BATCH, SEQ, logits)
    assert np.array_equal(bits(logits.download()), bits(got)), "one-call forward differs"
    assert model.status() == 0
    model.close()

    O = oracle_mod
    nb = len(SAMPLE)
    cos, sin = lfm.rope_tables(SEQ)
    table = lfm.synth_tensor(0, "embed_tokens.weight", (lfm.VOCAB, lfm.HIDDEN))
    x = O.embed(ids[list(SAMPLE)], table)
    adopted = 0
    for layer in range(LAYERS):
        w = lfm.synth_layer_weights(0, layer, lfm.LAYER_TYPES[layer] == 0, True)
        x, info = O.decoder_layer(x, w, nb, SEQ, cos, sin, guide=guides[layer], eps=TIE_EPS)
        del w
        say(f"[oracle] layer {layer}: near-ties followed {info['adopted']}, other {info['hard']}")
        assert info["hard"] == 0, f"layer {layer}: GPU routing is not a near-tie of the oracle's"
        adopted += info["adopted"]
    norm_w = lfm.synth_tensor(0, "embedding_norm.weight", (lfm.HIDDEN,))
    ref = O.model_head(x, norm_w, table, nb, SEQ)
    mine = got[list(SAMPLE)]
    err = np.abs(mine - ref)
    say(f"[model] near-ties followed over {LAYERS} layers: {adopted} of {nb * SEQ * LAYERS} "
        f"token-layers; max |dlogit| {err.max():.3e}, max rel {(err / np.abs(ref).clip(1e-3)).max():.3e}")
    assert adopted <= nb * SEQ * LAYERS // 100
    np.testing.assert_allclose(mine, ref, rtol=RTOL, atol=ATOL)
