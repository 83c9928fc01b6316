"""Python host mirror of the reference's SparseMoeBlock (include/layer.h:72-123,
src/layer.cu:1274-1503) over the C-ABI of include/moe_capi.h.

Same operations and argument meaning as the C++ class: weights in by value,
init (device allocation + upload), forward on device pointers with a stream,
plus the routing read-back the parity tests compare bit-exactly.  Errors raise
final_amd._native.MoeError carrying the C status.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native
from . import hip

TOPK = 4


def _ptr(x):
    """int pointer from a DeviceArray, an int or None."""
    if x is None:
        return None
    if isinstance(x, hip.DeviceArray):
        return x.ptr
    return int(x)


def _stream(s):
    if s is None:
        return None
    if isinstance(s, hip.Stream):
        return s.ptr
    return int(s)


class SparseMoeBlock:
    def __init__(self, hidden: int = 2048, inter: int = 1792, num_experts: int = 32,
                 top_k: int = 4, max_tokens: int = 4096):
        L = _native.lib()
        self.dims = _native.MoeDims(hidden, inter, num_experts, top_k, max_tokens)
        self._ctx = ctypes.c_void_p()
        _native.check(L.moe_create(ctypes.byref(self.dims), ctypes.byref(self._ctx)), "moe_create")
        self.hidden, self.inter, self.num_experts = hidden, inter, num_experts
        self.max_tokens = max_tokens
        self._routed_T = -1   # T of the last successful route (C side: routed_T)
        self._normed_T = -1   # T of the last successful forward_norm (C side: normed_T)

    # -- weights ------------------------------------------------------------
    def set_weights(self, gate, bias, w1, w3, w2, stream=None) -> None:
        """Host numpy weights: gate [E][H], bias [E] or None, w1/w3 [E][I][H]
        (or a list of E [I][H] arrays), w2 [E][H][I]."""
        E = self.num_experts
        keep = []

        def host_ptrs(ws):
            arrs = [np.ascontiguousarray(ws[e], dtype=np.float32) for e in range(E)]
            keep.extend(arrs)
            return (ctypes.c_void_p * E)(*[a.ctypes.data for a in arrs])

        gate = np.ascontiguousarray(gate, dtype=np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        p1, p3, p2 = host_ptrs(w1), host_ptrs(w3), host_ptrs(w2)
        _native.check(_native.lib().moe_set_weights(
            self._ctx, gate.ctypes.data, None if b is None else b.ctypes.data,
            p1, p3, p2, 0, _stream(stream)), "moe_set_weights")

    def set_weights_device(self, gate, bias, w1_ptrs, w3_ptrs, w2_ptrs, stream=None) -> None:
        """Device pointers (DeviceArray or int) per expert."""
        E = self.num_experts
        arr = lambda ps: (ctypes.c_void_p * E)(*[_ptr(p) for p in ps])
        _native.check(_native.lib().moe_set_weights(
            self._ctx, _ptr(gate), _ptr(bias), arr(w1_ptrs), arr(w3_ptrs), arr(w2_ptrs), 1,
            _stream(stream)), "moe_set_weights")

    def set_norm_weight(self, weight, stream=None) -> None:
        """The decoder layer's post-attention RMSNorm weight [H] (host numpy)."""
        w = np.ascontiguousarray(weight, dtype=np.float32)
        if w.shape != (self.hidden,):
            raise ValueError(f"norm weight must have shape ({self.hidden},)")
        _native.check(_native.lib().moe_set_norm_weight(self._ctx, w.ctypes.data, 0, _stream(stream)),
                      "moe_set_norm_weight")

    # -- forward ------------------------------------------------------------
    def forward_norm_gpu(self, h, out, num_tokens: int, stream=None) -> None:
        """out = h + MoE(rmsnorm(h)) on device buffers; out may be h."""
        # The read-backs pass these counts to the C side, which rejects a count
        # other than the one it holds, so a stale value can only fail a call.
        _native.check(_native.lib().moe_forward_norm(self._ctx, _ptr(h), _ptr(out), int(num_tokens),
                                                     _stream(stream)), "moe_forward_norm")
        self._routed_T = self._normed_T = int(num_tokens)

    def forward_norm(self, h: np.ndarray) -> np.ndarray:
        """Host convenience for forward_norm_gpu."""
        h = np.ascontiguousarray(h, dtype=np.float32)
        T = h.shape[0]
        dh = hip.DeviceArray.from_numpy(h)
        do = hip.DeviceArray((T, self.hidden))
        self.forward_norm_gpu(dh, do, T)
        hip.synchronize()
        self.check_device()
        return do.download()

    def last_normed(self, stream=None) -> np.ndarray:
        """Normalised rows of the last forward_norm ([T][H])."""
        T = max(self._normed_T, 0)
        out = np.empty((T, self.hidden), np.float32)
        _native.check(_native.lib().moe_last_normed(self._ctx, out.ctypes.data, T, _stream(stream)),
                      "moe_last_normed")
        return out

    def forward_gpu(self, x, y, num_tokens: int, residual=None, stream=None) -> None:
        """Route then run the experts (one moe_forward call, so a single
        decode token block may route inside the expert kernel)."""
        rc = _native.lib().moe_forward(self._ctx, _ptr(x), _ptr(y), _ptr(residual),
                                       int(num_tokens), _stream(stream))
        # the route may have succeeded before the experts call failed; a
        # stale count can only make a read-back fail (the C side checks it)
        self._routed_T = int(num_tokens)
        _native.check(rc, "moe_forward")

    def route(self, x, num_tokens: int, stream=None) -> None:
        _native.check(_native.lib().moe_route(self._ctx, _ptr(x), int(num_tokens), _stream(stream)),
                      "moe_route")
        self._routed_T = int(num_tokens)

    def route_forward(self, x, num_tokens: int, stream=None) -> None:
        """forward_gpu's routing launch (timing): follow with experts() on the
        same stream, x and num_tokens; together they are forward_gpu."""
        _native.check(_native.lib().moe_route_forward(self._ctx, _ptr(x), int(num_tokens),
                                                      _stream(stream)), "moe_route_forward")
        self._routed_T = int(num_tokens)

    def route_logits(self, logits, num_tokens: int, stream=None) -> None:
        _native.check(_native.lib().moe_route_logits(self._ctx, _ptr(logits), int(num_tokens),
                                                     _stream(stream)), "moe_route_logits")
        self._routed_T = int(num_tokens)

    def experts(self, x, y, num_tokens: int, residual=None, stream=None) -> None:
        _native.check(_native.lib().moe_experts(self._ctx, _ptr(x), _ptr(y), _ptr(residual),
                                                int(num_tokens), _stream(stream)), "moe_experts")

    def forward(self, x: np.ndarray, residual: np.ndarray | None = None) -> np.ndarray:
        """Host convenience: upload x (and residual), run, download y."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        dx = hip.DeviceArray.from_numpy(x)
        dy = hip.DeviceArray((T, self.hidden))
        dr = hip.DeviceArray.from_numpy(residual) if residual is not None else None
        self.forward_gpu(dx, dy, T, residual=dr)
        hip.synchronize()
        self.check_device()
        return dy.download()

    # -- inspection ---------------------------------------------------------
    def last_routing(self, stream=None) -> dict:
        T = max(self._routed_T, 0)
        idx = np.empty((T, TOPK), np.int32)
        w = np.empty((T, TOPK), np.float32)
        counts = np.empty((self.num_experts,), np.int32)
        logits = np.empty((T, self.num_experts), np.float32)
        _native.check(_native.lib().moe_last_routing(
            self._ctx, idx.ctypes.data, w.ctypes.data, counts.ctypes.data, logits.ctypes.data,
            T, _stream(stream)), "moe_last_routing")
        return {"idx": idx, "w": w, "counts": counts, "logits": logits}

    def last_plan_counts(self, stream=None):
        """Slots per expert of the last plan (the routing's counts, plus the
        speculative slots of a deferred decode routing)."""
        c = np.empty((self.num_experts,), np.int32)
        _native.check(_native.lib().moe_last_plan_counts(self._ctx, c.ctypes.data, _stream(stream)),
                      "moe_last_plan_counts")
        return c

    def check_device(self, stream=None) -> None:
        _native.check(_native.lib().moe_device_status(self._ctx, _stream(stream)), "device status")

    def plan(self, num_tokens: int) -> int:
        return int(_native.lib().moe_plan_tile_rows(self._ctx, int(num_tokens)))

    def force_tile_rows(self, rows: int) -> None:
        _native.check(_native.lib().moe_force_tile_rows(self._ctx, int(rows)), "moe_force_tile_rows")

    def set_wait_divisor(self, d: int) -> None:
        _native.check(_native.lib().moe_set_wait_divisor(self._ctx, int(d)), "moe_set_wait_divisor")

    def set_lazy_chains(self, on: bool) -> None:
        """Test hook: decode routing leaves its logit chains to the waits that
        need them (the path of an expert kernel whose blocks start late)."""
        _native.check(_native.lib().moe_set_lazy_chains(self._ctx, int(bool(on))), "moe_set_lazy_chains")

    def close(self) -> None:
        if self._ctx:
            _native.lib().moe_destroy(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DenseMLP:
    """Dense SwiGLU FFN of the first layers (reference MLP::forward_gpu,
    layer.cu:1231-1269): y = W2 (silu(W1 x) * (W3 x)) [+ residual], on the
    MoE kernels with the intermediate dimension cut into 4 chunk experts."""

    def __init__(self, hidden: int = 2048, inter: int = 7168, max_tokens: int = 4096):
        self._ctx = ctypes.c_void_p()
        _native.check(_native.lib().moe_dense_create(int(hidden), int(inter), int(max_tokens),
                                                     ctypes.byref(self._ctx)), "moe_dense_create")
        self.hidden, self.inter, self.max_tokens = hidden, inter, max_tokens

    def set_weights(self, w1, w3, w2, stream=None) -> None:
        """Host numpy: w1, w3 [I][H], w2 [H][I]."""
        w1, w3, w2 = (np.ascontiguousarray(a, dtype=np.float32) for a in (w1, w3, w2))
        _native.check(_native.lib().moe_dense_set_weights(
            self._ctx, w1.ctypes.data, w3.ctypes.data, w2.ctypes.data, 0, _stream(stream)),
            "moe_dense_set_weights")

    def forward_gpu(self, x, y, num_tokens: int, residual=None, stream=None) -> None:
        _native.check(_native.lib().moe_dense_forward(self._ctx, _ptr(x), _ptr(y), _ptr(residual),
                                                      int(num_tokens), _stream(stream)),
                      "moe_dense_forward")

    def forward(self, x: np.ndarray, residual: np.ndarray | None = None) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        dx = hip.DeviceArray.from_numpy(x)
        dy = hip.DeviceArray((T, self.hidden))
        dr = hip.DeviceArray.from_numpy(residual) if residual is not None else None
        self.forward_gpu(dx, dy, T, residual=dr)
        hip.synchronize()
        self.check_device()
        return dy.download()

    def plan(self, num_tokens: int) -> int:
        return int(_native.lib().moe_plan_tile_rows(self._ctx, int(num_tokens)))

    def check_device(self, stream=None) -> None:
        _native.check(_native.lib().moe_device_status(self._ctx, _stream(stream)), "device status")

    def close(self) -> None:
        if self._ctx:
            _native.lib().moe_destroy(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
