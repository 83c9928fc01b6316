"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check in
__graft_entry__.py and by the cpu_baseline leg of bench.py, always as the
checker.  The product package (final_amd) never imports this module.

The oracle restates the reference's MoE arithmetic (risepower20/final,
src/layer.cu:9-141, 434-542, 695-1126, 1428-1498, 1860-1880) and the decoder
around it (layer.cu:144-429, 1508-1922; model.cu:18-116, 469-559); each C
function cites the lines it follows, and decoder_layer / model_head below
compose them in DecoderLayer::forward_gpu's and worker_stage's order.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
TOPK = 4

_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (gcc, -ffp-contract=off)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        L.orc_force_scalar.argtypes = [ctypes.c_int]
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_get_threads.restype = ctypes.c_int
        L.orc_gemm_nt_chain.argtypes = [_f32p, _i64, _f32p, _i64, _i64, _f32p]
        L.orc_gate_logits.argtypes = [_f32p, _f32p, _i64, ctypes.c_int, ctypes.c_int, _f32p]
        L.orc_gate_logits_muladd.argtypes = [_f32p, _f32p, _i64, ctypes.c_int, ctypes.c_int, _f32p]
        L.orc_sigmoid.argtypes = [ctypes.c_float]
        L.orc_sigmoid.restype = ctypes.c_float
        L.orc_silu.argtypes = [ctypes.c_float]
        L.orc_silu.restype = ctypes.c_float
        L.orc_route.argtypes = [_f32p, _f32p, _i64, ctypes.c_int, _i32p, _f32p, _i32p]
        L.orc_dispatch.argtypes = [_i32p, _i64, ctypes.c_int, _i32p, _i32p, _i32p]
        L.orc_expert_w1w3.argtypes = [_f32p, _i64, _f32p, _f32p, ctypes.c_int, ctypes.c_int, _f32p]
        L.orc_expert_w2.argtypes = [_f32p, _i64, _f32p, ctypes.c_int, ctypes.c_int, _f32p]
        L.orc_combine.argtypes = [_f32p, _i32p, _f32p, _f32p, _i64, ctypes.c_int, _f32p]
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, _i64, ctypes.c_int, _f32p]
        L.orc_silu_dexp.argtypes = [ctypes.c_float]
        L.orc_silu_dexp.restype = ctypes.c_float
        L.orc_dense_mlp.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _i64, ctypes.c_int,
                                    ctypes.c_int, _f32p]
        L.orc_moe_forward.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                      _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      _u8p, _f32p, _f32p, _i32p, _f32p, _i32p]
        L.orc_moe_forward.restype = ctypes.c_int
        L.orc_moe_forward_guided.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                             _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             _i32p, ctypes.c_float, _f32p, _i32p,
                                             ctypes.POINTER(_i64), ctypes.POINTER(_i64)]
        L.orc_moe_forward_guided.restype = ctypes.c_int
        L.orc_embed.argtypes = [_i32p, _i64, _f32p, ctypes.c_int, ctypes.c_int, _f32p]
        L.orc_rope_tables.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        L.orc_qk_norm_rope.argtypes = [_f32p, ctypes.c_int, _i64, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, _f32p, _f32p, _f32p, _f32p]
        L.orc_attention.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]
        L.orc_shortconv.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, _f32p]
        L.orc_add.argtypes = [_f32p, _f32p, _i64, _f32p]
        _lib = L
    return _lib


def _f(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f32p)


def _i(a):
    if a is None:
        return None
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_i32p)


def force_scalar(on: bool) -> None:
    lib().orc_force_scalar(1 if on else 0)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def get_threads() -> int:
    return int(lib().orc_get_threads())


def gemm_nt_chain(A: np.ndarray, B: np.ndarray) -> np.ndarray:
    M, K = A.shape
    N, K2 = B.shape
    assert K == K2
    C = np.empty((M, N), np.float32)
    lib().orc_gemm_nt_chain(_f(A), M, _f(B), N, K, _f(C))
    return C


def gate_logits(x, gate, muladd: bool = False):
    T, H = x.shape
    E = gate.shape[0]
    out = np.empty((T, E), np.float32)
    fn = lib().orc_gate_logits_muladd if muladd else lib().orc_gate_logits
    fn(_f(x), _f(gate), T, H, E, _f(out))
    return out


def sigmoid(v: float) -> float:
    return float(np.float32(lib().orc_sigmoid(float(v))))


def silu(v: float) -> float:
    return float(np.float32(lib().orc_silu(float(v))))


def route(logits, bias):
    T, E = logits.shape
    idx = np.empty((T, TOPK), np.int32)
    w = np.empty((T, TOPK), np.float32)
    counts = np.empty((E,), np.int32)
    lib().orc_route(_f(logits), _f(bias), T, E, _i(idx), _f(w), _i(counts))
    return idx, w, counts


def dispatch(idx, E):
    T = idx.shape[0]
    offsets = np.empty((E + 1,), np.int32)
    pos = np.empty((T, TOPK), np.int32)
    slot_token = np.full((T * TOPK,), -1, np.int32)
    lib().orc_dispatch(_i(idx), T, E, _i(offsets), _i(pos), _i(slot_token))
    return offsets, pos, slot_token


def expert_w1w3(xrows, w1, w3):
    M, H = xrows.shape
    I = w1.shape[0]
    inter = np.empty((M, I), np.float32)
    lib().orc_expert_w1w3(_f(xrows), M, _f(w1), _f(w3), H, I, _f(inter))
    return inter


def expert_w2(inter, w2):
    M, I = inter.shape
    H = w2.shape[0]
    out = np.empty((M, H), np.float32)
    lib().orc_expert_w2(_f(inter), M, _f(w2), H, I, _f(out))
    return out


def combine(sorted_out, pos, w, residual=None):
    T = pos.shape[0]
    H = sorted_out.shape[1]
    y = np.empty((T, H), np.float32)
    lib().orc_combine(_f(sorted_out), _i(pos), _f(w), _f(residual), T, H, _f(y))
    return y


def silu_dexp(v: float) -> float:
    return float(lib().orc_silu_dexp(v))


def dense_mlp(x, w1, w3, w2, residual=None, token_mask=None):
    """Dense SwiGLU FFN (MLP::forward_gpu, layer.cu:1231-1269).  x [T][H],
    w1/w3 [I][H], w2 [H][I].  Rows of unselected tokens are NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, H = x.shape
    I = w1.shape[0]
    y = np.full((T, H), np.nan, np.float32)
    sel = np.arange(T) if token_mask is None else np.nonzero(np.asarray(token_mask))[0]
    if len(sel) == 0:
        return y
    xs = np.ascontiguousarray(x[sel])
    rs = None if residual is None else np.ascontiguousarray(np.asarray(residual, np.float32)[sel])
    ys = np.empty((len(sel), H), np.float32)
    rc = lib().orc_dense_mlp(_f(xs), _f(np.ascontiguousarray(w1, dtype=np.float32)),
                             _f(np.ascontiguousarray(w3, dtype=np.float32)),
                             _f(np.ascontiguousarray(w2, dtype=np.float32)), _f(rs),
                             len(sel), H, I, _f(ys))
    if rc != 0:
        raise RuntimeError("orc_dense_mlp failed")
    y[sel] = ys
    return y


def rmsnorm(h, weight):
    """Post-attention RMSNorm of every row of h [T][H] (layer.cu:144-193)."""
    h = np.ascontiguousarray(h, dtype=np.float32)
    T, H = h.shape
    out = np.empty((T, H), np.float32)
    lib().orc_rmsnorm(_f(h), _f(np.ascontiguousarray(weight, dtype=np.float32)), T, H, _f(out))
    return out


def moe_forward_norm(h, norm_weight, gate, bias, w1, w3, w2, token_mask=None):
    """Steps 4-6 of DecoderLayer::forward_gpu (layer.cu:1903-1918):
    out = h + MoE(rmsnorm(h)).  Returns the moe_forward dict plus xn, the
    normalised rows."""
    xn = rmsnorm(h, norm_weight)
    r = moe_forward(xn, gate, bias, w1, w3, w2, residual=h, token_mask=token_mask)
    r["xn"] = xn
    return r


def moe_forward(x, gate, bias, w1, w3, w2, residual=None, token_mask=None):
    """Full block.  w1/w3: [E][I][H], w2: [E][H][I].  Returns dict with y
    (rows of unselected tokens are NaN), logits, idx, w, counts."""
    T, H = x.shape
    E, I, _ = w1.shape
    y = np.full((T, H), np.nan, np.float32)
    logits = np.empty((T, E), np.float32)
    idx = np.empty((T, TOPK), np.int32)
    w = np.empty((T, TOPK), np.float32)
    counts = np.empty((E,), np.int32)
    mask = None
    if token_mask is not None:
        mask = np.ascontiguousarray(token_mask, dtype=np.uint8)
    rc = lib().orc_moe_forward(
        _f(x), _f(gate), _f(bias), _f(w1), _f(w3), _f(w2), _f(residual),
        T, H, I, E, mask.ctypes.data_as(_u8p) if mask is not None else None,
        _f(y), _f(logits), _i(idx), _f(w), _i(counts))
    if rc != 0:
        raise RuntimeError("orc_moe_forward failed")
    return {"y": y, "logits": logits, "idx": idx, "w": w, "counts": counts}


# ---------------------------------------------------------------------------
# Decoder model around the block (lfm_oracle.c)
# ---------------------------------------------------------------------------

HEADS, KV_HEADS, HEAD_DIM, CONV_L = 32, 8, 64, 3  # config.h:8-9,28-29
Q_COLS, KV_COLS = HEADS * HEAD_DIM, KV_HEADS * HEAD_DIM
ROPE_THETA = 1000000.0


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def embed(ids, table):
    """embedding_lookup_kernel (model.cu:18-32)."""
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    V, H = table.shape
    h = np.empty((ids.size, H), np.float32)
    lib().orc_embed(_i(ids), ids.size, _f(_c32(table)), H, V, _f(h))
    return h


def rope_tables(max_pos, head_dim=HEAD_DIM, theta=ROPE_THETA):
    """RotaryEmbedding::init_gpu's cos/sin tables [max_pos][head_dim]."""
    c = np.empty((max_pos, head_dim), np.float32)
    s_ = np.empty((max_pos, head_dim), np.float32)
    lib().orc_rope_tables(_f(c), _f(s_), max_pos, head_dim, theta)
    return c, s_


def qk_norm_rope(qkv, seq, q_weight, k_weight, cos, sin, heads=HEADS, kv_heads=KV_HEADS,
                 k_col=Q_COLS):
    """Returns a copy of qkv [T][ld] with its q/k heads normalised and rotated."""
    out = np.array(qkv, dtype=np.float32, order="C", copy=True)
    T, ld = out.shape
    lib().orc_qk_norm_rope(_f(out), ld, T, seq, heads, kv_heads, k_col, _f(_c32(q_weight)),
                           _f(_c32(k_weight)), _f(_c32(cos)), _f(_c32(sin)))
    return out


def attention(qkv, batch, seq, heads=HEADS, kv_heads=KV_HEADS, k_col=Q_COLS,
              v_col=Q_COLS + KV_COLS):
    """Causal GQA attention (fused_attn_gqa_kernel, any seq) -> [T][heads*64]."""
    qkv = _c32(qkv)
    out = np.empty((batch * seq, heads * HEAD_DIM), np.float32)
    lib().orc_attention(_f(qkv), qkv.shape[1], batch, seq, heads, kv_heads, k_col, v_col, _f(out))
    return out


def shortconv(bcg, conv_w, batch, seq, L=CONV_L):
    """ShortConv's mix (layer.cu:360-429): bcg [T][3H] -> [T][H]."""
    bcg = _c32(bcg)
    H = bcg.shape[1] // 3
    y = np.empty((batch * seq, H), np.float32)
    lib().orc_shortconv(_f(bcg), _f(_c32(conv_w).reshape(H, L)), batch, seq, H, L, _f(y))
    return y


def add(a, b):
    """add_kernel (layer.cu:1860-1880)."""
    a, b = _c32(a), _c32(b)
    out = np.empty_like(a)
    lib().orc_add(_f(a), _f(b), a.size, _f(out))
    return out


def moe_forward_guided(x, gate, bias, w1, w3, w2, residual, guide, eps):
    """moe_forward over all tokens, following guide [T][4] where it is a
    near-tie of the oracle's scores (orc_moe_forward_guided).  Returns
    (y, idx used, adopted count, count of guides that are not near-ties)."""
    T, H = x.shape
    E, I, _ = w1.shape
    y = np.empty((T, H), np.float32)
    idx = np.empty((T, TOPK), np.int32)
    na, nh = _i64(0), _i64(0)
    rc = lib().orc_moe_forward_guided(
        _f(_c32(x)), _f(gate), _f(bias), _f(w1), _f(w3), _f(w2), _f(_c32(residual)), T, H, I, E,
        _i(np.ascontiguousarray(guide, dtype=np.int32)), float(eps), _f(y), _i(idx),
        ctypes.byref(na), ctypes.byref(nh))
    if rc != 0:
        raise RuntimeError("orc_moe_forward_guided failed")
    return y, idx, int(na.value), int(nh.value)


def decoder_layer(h, w, batch, seq, cos, sin, guide=None, eps=0.0):
    """DecoderLayer::forward_gpu (layer.cu:1882-1919) on h [T][H] (T = batch*seq):
    operator norm; attention (q|k|v projections, q/k norm + rotation, causal
    GQA attention, out_proj) or short conv (in_proj, mix, out_proj); residual;
    FFN norm; MoE block (or dense FFN); residual.  w: dict of the layer's
    tensors under the reference's short names (op_norm, ffn_norm, q, k, v, o,
    q_norm, k_norm | conv, in_proj, out_proj; gate, bias, w1, w3, w2 for a MoE
    FFN with w1/w3 [E][I][H] and w2 [E][H][I], or dense_w1/w3/w2).  guide:
    routing of another implementation to follow on near-ties (MoE only).
    Returns (h', info) with the routing used and the near-tie counts; with a
    guide also the oracle's own routing (own_idx) and its gate logits."""
    h = _c32(h)
    xn = rmsnorm(h, w["op_norm"])
    if "q" in w:
        heads, kvh = w["q"].shape[0] // HEAD_DIM, w["k"].shape[0] // HEAD_DIM
        qc, kc = heads * HEAD_DIM, kvh * HEAD_DIM
        wqkv = np.ascontiguousarray(np.concatenate([w["q"], w["k"], w["v"]], axis=0))
        qkv = gemm_nt_chain(xn, wqkv)
        qkv = qk_norm_rope(qkv, seq, w["q_norm"], w["k_norm"], cos, sin, heads, kvh, qc)
        att = attention(qkv, batch, seq, heads, kvh, qc, qc + kc)
        op = gemm_nt_chain(att, _c32(w["o"]))
    else:
        bcg = gemm_nt_chain(xn, _c32(w["in_proj"]))
        mix = shortconv(bcg, w["conv"], batch, seq)
        op = gemm_nt_chain(mix, _c32(w["out_proj"]))
    h = add(h, op)
    info = {}
    if "gate" in w:
        x2 = rmsnorm(h, w["ffn_norm"])
        if guide is None:
            r = moe_forward(x2, w["gate"], w["bias"], w["w1"], w["w3"], w["w2"], residual=h)
            h, info["idx"], info["adopted"], info["hard"] = r["y"], r["idx"], 0, 0
        else:
            info["logits"] = gate_logits(x2, w["gate"])
            info["own_idx"] = route(info["logits"], w["bias"])[0]
            h, info["idx"], info["adopted"], info["hard"] = moe_forward_guided(
                x2, w["gate"], w["bias"], w["w1"], w["w3"], w["w2"], h, guide, eps)
    else:
        x2 = rmsnorm(h, w["ffn_norm"])
        h = dense_mlp(x2, w["dense_w1"], w["dense_w3"], w["dense_w2"], residual=h)
    return h, info


def model_head(h, norm_weight, head, batch, seq):
    """Final RMSNorm of each sequence's last token and the LM head
    (model.cu:481-536, lm_head_gemm_kernel's FMA chains) -> [batch][vocab]."""
    H = h.shape[1]
    last = np.ascontiguousarray(_c32(h).reshape(batch, seq, H)[:, seq - 1, :])
    return gemm_nt_chain(rmsnorm(last, norm_weight), _c32(head))
