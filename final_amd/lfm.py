"""Python host mirror of the decoder model around the MoE block over the
C-ABI of include/lfm_capi.h: the kernels of one decoder layer (projection
GEMM, embedding, RMSNorm, q/k norm + rotary, causal GQA attention, short-conv
mix) and a handle on the one-GPU LFM2Model (include/model.h; reference
src/model.cu).  Arguments mirror the C signatures: device buffers are
hip.DeviceArray (or int pointers), streams hip.Stream (or None).  Errors raise
final_amd._native.MoeError with the C status.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native
from . import hip
from .moe import _ptr, _stream

HIDDEN, VOCAB, HEADS, KV_HEADS, HEAD_DIM = 2048, 65536, 32, 8, 64
Q_COLS, KV_COLS = HEADS * HEAD_DIM, KV_HEADS * HEAD_DIM
QKV_COLS = Q_COLS + 2 * KV_COLS
MOE_I, DENSE_I, EXPERTS, CONV_L = 1792, 7168, 32, 3
ROPE_THETA = 1000000.0
# reference include/config.h:31 (0 = attention, 1 = short conv)
LAYER_TYPES = (1, 1, 0, 1, 1, 1, 0, 1, 1, 1, 0, 1, 1, 1, 0, 1, 1, 1, 0, 1, 1, 0, 1, 1)


def _ck(rc, what):
    _native.check(rc, what)


# -- kernels -----------------------------------------------------------------

def gemm_nt(A, B, C, M, N, K, R=None, stream=None):
    _ck(_native.lib().lfm_gemm_nt(_ptr(A), _ptr(B), _ptr(C), _ptr(R), M, N, K, _stream(stream)),
        "lfm_gemm_nt")


def embed(ids, table, h, num_tokens, hidden, vocab, bad_flag=None, stream=None):
    _ck(_native.lib().lfm_embed(_ptr(ids), _ptr(table), _ptr(h), num_tokens, hidden, vocab,
                                _ptr(bad_flag), _stream(stream)), "lfm_embed")


def rmsnorm(x, weight, y, rows, dim, x_stride=None, y_stride=None, stream=None):
    _ck(_native.lib().lfm_rmsnorm(_ptr(x), dim if x_stride is None else x_stride, _ptr(weight),
                                  _ptr(y), dim if y_stride is None else y_stride, rows, dim,
                                  _stream(stream)), "lfm_rmsnorm")


def qk_norm_rope(qkv, ld, q_weight, k_weight, cos, sin, batch, seq, heads=HEADS,
                 kv_heads=KV_HEADS, k_col=Q_COLS, stream=None):
    _ck(_native.lib().lfm_qk_norm_rope(_ptr(qkv), ld, _ptr(q_weight), _ptr(k_weight), _ptr(cos),
                                       _ptr(sin), batch, seq, heads, kv_heads, k_col,
                                       _stream(stream)), "lfm_qk_norm_rope")


def attention(qkv, ld, out, batch, seq, heads=HEADS, kv_heads=KV_HEADS, k_col=Q_COLS,
              v_col=Q_COLS + KV_COLS, stream=None):
    _ck(_native.lib().lfm_attention(_ptr(qkv), ld, _ptr(out), batch, seq, heads, kv_heads, k_col,
                                    v_col, _stream(stream)), "lfm_attention")


def shortconv(bcg, conv_w, y, batch, seq, hidden, kernel=CONV_L, stream=None):
    _ck(_native.lib().lfm_shortconv(_ptr(bcg), _ptr(conv_w), _ptr(y), batch, seq, hidden, kernel,
                                    _stream(stream)), "lfm_shortconv")


def rope_tables(max_pos, head_dim=HEAD_DIM, theta=ROPE_THETA):
    """Host cos/sin tables [max_pos][head_dim] (RotaryEmbedding::init_gpu)."""
    c = np.empty((max_pos, head_dim), np.float32)
    s = np.empty((max_pos, head_dim), np.float32)
    _ck(_native.lib().lfm_rope_tables(c.ctypes.data, s.ctypes.data, max_pos, head_dim, theta),
        "lfm_rope_tables")
    return c, s


# -- synthetic weights -------------------------------------------------------

def synth_stream_of(name: str) -> int:
    return int(_native.lib().lfm_synth_stream_of(name.encode()))


def synth_is_norm(name: str) -> bool:
    return bool(_native.lib().lfm_synth_is_norm(name.encode()))


def synth_normal_device(dst, n, seed, stream_id, std, first=0, stream=None):
    _ck(_native.lib().lfm_synth_normal(_ptr(dst), n, seed, stream_id, std, first, _stream(stream)),
        "lfm_synth_normal")


def synth_tensor(seed: int, name: str, shape, std: float = 0.02) -> np.ndarray:
    """The tensor `name` of a synthetic model, drawn on the device and copied
    back (ones for RMSNorm weights)."""
    out = np.empty(tuple(shape), np.float32)
    _ck(_native.lib().lfm_synth_tensor(seed, name.encode(), std, out.ctypes.data, out.size),
        "lfm_synth_tensor")
    return out


def layer_tensors(layer: int, is_attention: bool, moe: bool):
    """(name, shape) of every tensor of a decoder layer under the reference's
    names (layer.cu:1277-1298, 1508-1526, 1680-1693, 1784-1811)."""
    p = f"layers.{layer}."
    H = HIDDEN
    out = [(p + "operator_norm.weight", (H,)), (p + "ffn_norm.weight", (H,))]
    if is_attention:
        out += [(p + "self_attn.q_proj.weight", (Q_COLS, H)),
                (p + "self_attn.k_proj.weight", (KV_COLS, H)),
                (p + "self_attn.v_proj.weight", (KV_COLS, H)),
                (p + "self_attn.out_proj.weight", (H, Q_COLS)),
                (p + "self_attn.q_layernorm.weight", (HEAD_DIM,)),
                (p + "self_attn.k_layernorm.weight", (HEAD_DIM,))]
    else:
        out += [(p + "conv.conv.weight", (H, 1, CONV_L)),
                (p + "conv.in_proj.weight", (3 * H, H)),
                (p + "conv.out_proj.weight", (H, H))]
    if moe:
        out += [(p + "feed_forward.gate.weight", (EXPERTS, H)),
                (p + "feed_forward.expert_bias", (EXPERTS,))]
        for e in range(EXPERTS):
            out += [(p + f"feed_forward.experts.{e}.w1.weight", (MOE_I, H)),
                    (p + f"feed_forward.experts.{e}.w3.weight", (MOE_I, H)),
                    (p + f"feed_forward.experts.{e}.w2.weight", (H, MOE_I))]
    else:
        out += [(p + "feed_forward.w1.weight", (DENSE_I, H)),
                (p + "feed_forward.w3.weight", (DENSE_I, H)),
                (p + "feed_forward.w2.weight", (H, DENSE_I))]
    return out


def synth_layer_weights(seed: int, layer: int, is_attention: bool, moe: bool,
                        std: float = 0.02) -> dict:
    """A synthetic layer's tensors as host arrays under short names: op_norm,
    ffn_norm; q, k, v, o, q_norm, k_norm | conv, in_proj, out_proj; gate,
    bias, w1/w3 [E][I][H], w2 [E][H][I] | dense_w1, dense_w3, dense_w2."""
    p = f"layers.{layer}."
    g = lambda name, shape: synth_tensor(seed, p + name, shape, std)  # noqa: E731
    H = HIDDEN
    w = {"op_norm": g("operator_norm.weight", (H,)), "ffn_norm": g("ffn_norm.weight", (H,))}
    if is_attention:
        w.update(q=g("self_attn.q_proj.weight", (Q_COLS, H)),
                 k=g("self_attn.k_proj.weight", (KV_COLS, H)),
                 v=g("self_attn.v_proj.weight", (KV_COLS, H)),
                 o=g("self_attn.out_proj.weight", (H, Q_COLS)),
                 q_norm=g("self_attn.q_layernorm.weight", (HEAD_DIM,)),
                 k_norm=g("self_attn.k_layernorm.weight", (HEAD_DIM,)))
    else:
        w.update(conv=g("conv.conv.weight", (H, CONV_L)),
                 in_proj=g("conv.in_proj.weight", (3 * H, H)),
                 out_proj=g("conv.out_proj.weight", (H, H)))
    if moe:
        w["gate"] = g("feed_forward.gate.weight", (EXPERTS, H))
        w["bias"] = g("feed_forward.expert_bias", (EXPERTS,))
        w1 = np.empty((EXPERTS, MOE_I, H), np.float32)
        w3 = np.empty((EXPERTS, MOE_I, H), np.float32)
        w2 = np.empty((EXPERTS, H, MOE_I), np.float32)
        for e in range(EXPERTS):
            w1[e] = g(f"feed_forward.experts.{e}.w1.weight", (MOE_I, H))
            w3[e] = g(f"feed_forward.experts.{e}.w3.weight", (MOE_I, H))
            w2[e] = g(f"feed_forward.experts.{e}.w2.weight", (H, MOE_I))
        w.update(w1=w1, w3=w3, w2=w2)
    else:
        w.update(dense_w1=g("feed_forward.w1.weight", (DENSE_I, H)),
                 dense_w3=g("feed_forward.w3.weight", (DENSE_I, H)),
                 dense_w2=g("feed_forward.w2.weight", (H, DENSE_I)))
    return w


# -- the model ---------------------------------------------------------------

class LFM2Model:
    """Handle on the one-GPU model (lfm_model_*).  Synthetic weights drawn on
    the device by name; layer_types[i] 0 = attention, 1 = short conv."""

    def __init__(self, num_layers: int = 24, layer_types=None, num_dense_layers: int = 0,
                 max_batch: int = 64, max_seq: int = 512, seed: int = 0, std: float = 0.02):
        L = _native.lib()
        types = list(layer_types) if layer_types is not None else \
            [LAYER_TYPES[i % len(LAYER_TYPES)] for i in range(num_layers)]
        self._types = (ctypes.c_int * max(1, num_layers))(*types[:num_layers])
        self.layer_types = types[:num_layers]
        self.num_dense_layers = num_dense_layers
        cfg = _native.LfmModelConfig(num_layers, ctypes.cast(self._types, ctypes.c_void_p),
                                     num_dense_layers, max_batch, max_seq, seed, std)
        self._m = ctypes.c_void_p()
        _ck(L.lfm_model_create_synthetic(ctypes.byref(cfg), ctypes.byref(self._m)),
            "lfm_model_create_synthetic")
        self.num_layers, self.max_batch, self.max_seq = num_layers, max_batch, max_seq
        self.seed, self.std = seed, std

    def is_attention(self, layer: int) -> bool:
        return self.layer_types[layer] == 0

    def is_moe(self, layer: int) -> bool:
        return layer >= self.num_dense_layers

    def forward(self, ids, batch, seq, logits, stream=None):
        _ck(_native.lib().lfm_model_forward(self._m, _ptr(ids), batch, seq, _ptr(logits),
                                            _stream(stream)), "lfm_model_forward")

    def embed(self, ids, batch, seq, h, stream=None):
        _ck(_native.lib().lfm_model_embed(self._m, _ptr(ids), batch, seq, _ptr(h),
                                          _stream(stream)), "lfm_model_embed")

    def layer_forward(self, layer, h, batch, seq, stream=None):
        _ck(_native.lib().lfm_model_layer_forward(self._m, layer, _ptr(h), batch, seq,
                                                  _stream(stream)), "lfm_model_layer_forward")

    def head(self, h, batch, seq, logits, stream=None):
        _ck(_native.lib().lfm_model_head(self._m, _ptr(h), batch, seq, _ptr(logits),
                                         _stream(stream)), "lfm_model_head")

    def last_routing(self, layer: int, num_tokens: int) -> np.ndarray:
        """idx [T][4] of the MoE layer's last forward (valid until the next
        MoE layer runs)."""
        ctx = ctypes.c_void_p()
        _ck(_native.lib().lfm_model_moe(self._m, layer, ctypes.byref(ctx)), "lfm_model_moe")
        if not ctx.value:
            raise ValueError(f"layer {layer} has no MoE block")
        idx = np.empty((num_tokens, 4), np.int32)
        _ck(_native.lib().moe_last_routing(ctx, idx.ctypes.data, None, None, None, num_tokens,
                                           None), "moe_last_routing")
        return idx

    def status(self, stream=None) -> int:
        return int(_native.lib().lfm_model_status(self._m, _stream(stream)))

    def close(self) -> None:
        if self._m:
            _native.lib().lfm_model_destroy(self._m)
            self._m = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
