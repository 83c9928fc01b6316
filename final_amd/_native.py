"""ctypes binding of libfinal_amd_moe.so (the C-ABI of include/moe_capi.h and
include/moe_synth.h).  The library is built in-tree by final_amd/csrc/Makefile;
loading fails loudly when it is missing - there is no fallback path."""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfinal_amd_moe.so")

MOE_OK = 0
MOE_ERR_INVALID_ARG = 1
MOE_ERR_UNSUPPORTED = 2
MOE_ERR_HIP = 3
MOE_ERR_OUT_OF_MEMORY = 4
MOE_ERR_NOT_READY = 5
MOE_ERR_TOO_MANY_TOKENS = 6
MOE_ERR_DEVICE_TIMEOUT = 7
MOE_ERR_INTERNAL = 8

# every symbol include/moe_capi.h and include/moe_synth.h declare
CAPI_SYMBOLS = (
    "moe_create", "moe_destroy", "moe_set_weights", "moe_forward", "moe_route",
    "moe_experts", "moe_route_logits", "moe_last_routing", "moe_device_status",
    "moe_plan_tile_rows", "moe_force_tile_rows", "moe_set_wait_divisor",
    "moe_strerror", "moe_version", "moe_set_norm_weight", "moe_forward_norm",
    "moe_last_normed", "moe_dense_create", "moe_dense_set_weights", "moe_dense_forward",
    "moe_forward_noalloc", "moe_create_shared", "moe_dense_create_shared",
    "moe_set_lazy_chains", "moe_route_forward", "moe_last_plan_counts",
)
LFM_SYMBOLS = (
    "lfm_gemm_nt", "lfm_embed", "lfm_rmsnorm", "lfm_qk_norm_rope", "lfm_attention",
    "lfm_shortconv", "lfm_rope_tables", "lfm_synth_normal", "lfm_fill", "lfm_synth_stream_of",
    "lfm_synth_is_norm", "lfm_synth_tensor", "lfm_model_create_synthetic",
    "lfm_model_create_from_file", "lfm_model_destroy", "lfm_model_forward", "lfm_model_embed",
    "lfm_model_layer_forward", "lfm_model_head", "lfm_model_moe", "lfm_model_info",
    "lfm_model_status",
)
SYNTH_SYMBOLS = (
    "moe_synth_normal", "moe_synth_stream_gate", "moe_synth_stream_bias",
    "moe_synth_stream_w1", "moe_synth_stream_w3", "moe_synth_stream_w2",
    "moe_synth_stream_x", "moe_synth_set_threads",
)


class MoeDims(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("inter", ctypes.c_int),
                ("num_experts", ctypes.c_int), ("top_k", ctypes.c_int),
                ("max_tokens", ctypes.c_int)]


class LfmModelConfig(ctypes.Structure):
    _fields_ = [("num_layers", ctypes.c_int), ("layer_types", ctypes.c_void_p),
                ("num_dense_layers", ctypes.c_int), ("max_batch", ctypes.c_int),
                ("max_seq", ctypes.c_int), ("seed", ctypes.c_uint64),
                ("weight_std", ctypes.c_float)]


class MoeError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {strerror(status)} (status {status})")


_lib = None
_vp = ctypes.c_void_p
_i = ctypes.c_int


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"final_amd native library not built: {LIB_PATH} is missing "
            "(run `make -C final_amd/csrc` or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    L.moe_create.argtypes = [ctypes.POINTER(MoeDims), ctypes.POINTER(_vp)]
    L.moe_destroy.argtypes = [_vp]
    L.moe_set_weights.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp]
    L.moe_forward.argtypes = [_vp, _vp, _vp, _vp, _i, _vp]
    L.moe_forward_noalloc.argtypes = [_vp, _vp, _vp, _vp, _i, _vp]
    L.moe_route.argtypes = [_vp, _vp, _i, _vp]
    L.moe_route_forward.argtypes = [_vp, _vp, _i, _vp]
    L.moe_last_plan_counts.argtypes = [_vp, _vp, _vp]
    L.moe_experts.argtypes = [_vp, _vp, _vp, _vp, _i, _vp]
    L.moe_route_logits.argtypes = [_vp, _vp, _i, _vp]
    L.moe_last_routing.argtypes = [_vp, _vp, _vp, _vp, _vp, _i, _vp]
    L.moe_device_status.argtypes = [_vp, _vp]
    L.moe_set_norm_weight.argtypes = [_vp, _vp, _i, _vp]
    L.moe_forward_norm.argtypes = [_vp, _vp, _vp, _i, _vp]
    L.moe_last_normed.argtypes = [_vp, _vp, _i, _vp]
    L.moe_dense_create.argtypes = [_i, _i, _i, ctypes.POINTER(_vp)]
    L.moe_dense_set_weights.argtypes = [_vp, _vp, _vp, _vp, _i, _vp]
    L.moe_dense_forward.argtypes = [_vp, _vp, _vp, _vp, _i, _vp]
    L.moe_plan_tile_rows.argtypes = [_vp, _i]
    L.moe_force_tile_rows.argtypes = [_vp, _i]
    L.moe_set_wait_divisor.argtypes = [_vp, _i]
    L.moe_set_lazy_chains.argtypes = [_vp, _i]
    L.moe_strerror.argtypes = [_i]
    L.moe_strerror.restype = ctypes.c_char_p
    L.moe_version.restype = ctypes.c_char_p
    L.moe_synth_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float,
                                   ctypes.c_uint64, _vp, ctypes.c_size_t]
    for n in ("gate", "bias"):
        getattr(L, f"moe_synth_stream_{n}").restype = ctypes.c_uint64
    for n in ("w1", "w3", "w2", "x"):
        f = getattr(L, f"moe_synth_stream_{n}")
        f.argtypes = [_i]
        f.restype = ctypes.c_uint64
    L.moe_synth_set_threads.argtypes = [_i]
    L.moe_create_shared.argtypes = [ctypes.POINTER(MoeDims), _vp, ctypes.POINTER(_vp)]
    L.moe_dense_create_shared.argtypes = [_i, _i, _i, _vp, ctypes.POINTER(_vp)]
    _ll, _sz, _u64, _f = ctypes.c_longlong, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_float
    L.lfm_gemm_nt.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]
    L.lfm_embed.argtypes = [_vp, _vp, _vp, _i, _i, _i, _vp, _vp]
    L.lfm_rmsnorm.argtypes = [_vp, _ll, _vp, _vp, _ll, _i, _i, _vp]
    L.lfm_qk_norm_rope.argtypes = [_vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]
    L.lfm_attention.argtypes = [_vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp]
    L.lfm_shortconv.argtypes = [_vp, _vp, _vp, _i, _i, _i, _i, _vp]
    L.lfm_rope_tables.argtypes = [_vp, _vp, _i, _i, _f]
    L.lfm_synth_normal.argtypes = [_vp, _sz, _u64, _u64, _f, _u64, _vp]
    L.lfm_fill.argtypes = [_vp, _sz, _f, _vp]
    L.lfm_synth_stream_of.argtypes = [ctypes.c_char_p]
    L.lfm_synth_stream_of.restype = _u64
    L.lfm_synth_is_norm.argtypes = [ctypes.c_char_p]
    L.lfm_synth_tensor.argtypes = [_u64, ctypes.c_char_p, _f, _vp, _sz]
    L.lfm_model_create_synthetic.argtypes = [ctypes.POINTER(LfmModelConfig), ctypes.POINTER(_vp)]
    L.lfm_model_create_from_file.argtypes = [ctypes.c_char_p, _i, _i, ctypes.POINTER(_vp)]
    L.lfm_model_destroy.argtypes = [_vp]
    L.lfm_model_forward.argtypes = [_vp, _vp, _i, _i, _vp, _vp]
    L.lfm_model_embed.argtypes = [_vp, _vp, _i, _i, _vp, _vp]
    L.lfm_model_layer_forward.argtypes = [_vp, _i, _vp, _i, _i, _vp]
    L.lfm_model_head.argtypes = [_vp, _vp, _i, _i, _vp, _vp]
    L.lfm_model_moe.argtypes = [_vp, _i, ctypes.POINTER(_vp)]
    L.lfm_model_info.argtypes = [_vp, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i),
                                 ctypes.POINTER(_i)]
    L.lfm_model_status.argtypes = [_vp, _vp]
    _lib = L
    return L


def strerror(status: int) -> str:
    return lib().moe_strerror(int(status)).decode()


def check(status: int, what: str) -> None:
    if status != MOE_OK:
        raise MoeError(status, what)


def version() -> str:
    return lib().moe_version().decode()
