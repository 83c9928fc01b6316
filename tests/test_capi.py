"""The C-ABI library (CPU side only: no HIP call is made here).

Loads libfinal_amd_moe.so, checks that every function include/moe_capi.h and
include/moe_synth.h declare is exported, that the C++ layer interface of
include/layer.h / tensor.h / model_loader.h is exported, and that argument
validation answers with the documented status codes before touching a GPU."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_c_functions(header, prefix="moe_"):
    text = open(os.path.join(INCLUDE, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from final_amd import _native
    return _native.lib()


def test_c_symbols_exported(L):
    from final_amd import _native
    names = declared_c_functions("moe_capi.h") + declared_c_functions("moe_synth.h")
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/ but not exported"
    assert set(declared_c_functions("moe_capi.h")) == set(_native.CAPI_SYMBOLS)
    assert set(declared_c_functions("moe_synth.h")) == set(_native.SYNTH_SYMBOLS)
    lfm = declared_c_functions("lfm_capi.h", "lfm_")
    assert len(lfm) >= 20
    for n in lfm:
        assert hasattr(L, n), f"{n} declared in include/lfm_capi.h but not exported"
    assert set(lfm) == set(_native.LFM_SYMBOLS)


def test_cpp_interface_exported():
    from final_amd import _native
    out = subprocess.run(["nm", "-DC", "--defined-only", _native.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    for sig in (
        "SparseMoeBlock::SparseMoeBlock(int)",
        "SparseMoeBlock::init_gpu()",
        "SparseMoeBlock::forward_gpu(float*, float*, int, int, int, ihipStream_t*)",
        "SparseMoeBlock::forward(Tensor const&, Tensor&, Tensor&)",
        "SparseMoeBlock::route_tokens(Tensor const&, std::vector<int, std::allocator<int> >&, std::vector<float, std::allocator<float> >&)",
        "MLP::MLP(std::__cxx11::basic_string<char, std::char_traits<char>, std::allocator<char> > const&",
        "Tensor::load_from_file(",
        "Tensor::save_to_file(",
        "ModelLoader::ModelLoader(",
        "ModelLoader::load_tensor(",
        "g_model_loader",
        "RMSNorm::forward_gpu(float*, float*, int, int, ihipStream_t*)",
        "RotaryEmbedding::init_gpu()",
        "Attention::Attention(int)",
        "Attention::forward_gpu(float*, float*, float*, float*, int, int, int, ihipStream_t*)",
        "ShortConv::ShortConv(int)",
        "ShortConv::forward_gpu(float*, float*, int, int, int, ihipStream_t*)",
        "DecoderLayer::DecoderLayer(int, bool)",
        "DecoderLayer::init_gpu(int)",
        "DecoderLayer::forward_gpu(float*, float*, float*, float*, int, int, int, ihipStream_t*)",
        "LFM2Model::LFM2Model(std::__cxx11::basic_string<char, std::char_traits<char>, std::allocator<char> > const&)",
        "LFM2Model::forward(int, int, int const*, unsigned long, float*)",
        "LFM2Model::sync()",
    ):
        assert sig in out, sig


def test_statuses_and_strings(L):
    from final_amd import _native
    msgs = {s: L.moe_strerror(s).decode() for s in range(0, 9)}
    assert msgs[0] == "ok" and len(set(msgs.values())) == 9
    assert L.moe_strerror(99).decode() == "unknown status"
    assert "gfx950" in L.moe_version().decode()


def test_argument_validation_before_any_gpu_call(L):
    from final_amd import _native
    ctx = ctypes.c_void_p()
    assert L.moe_create(None, ctypes.byref(ctx)) == _native.MOE_ERR_INVALID_ARG
    bad = [
        (2048, 1792, 16, 4, 64, _native.MOE_ERR_UNSUPPORTED),   # 16 experts
        (2048, 1792, 32, 2, 64, _native.MOE_ERR_UNSUPPORTED),   # top-2
        (2000, 1792, 32, 4, 64, _native.MOE_ERR_UNSUPPORTED),   # hidden % 256
        (2048, 1800, 32, 4, 64, _native.MOE_ERR_UNSUPPORTED),   # inter % 256
        (2048, 1792, 32, 4, 0, _native.MOE_ERR_INVALID_ARG),    # no tokens
        (0, 1792, 32, 4, 64, _native.MOE_ERR_INVALID_ARG),
        (2048, 1792, 32, 4, 1 << 21, _native.MOE_ERR_INVALID_ARG),
    ]
    for h, i, e, k, t, want in bad:
        d = _native.MoeDims(h, i, e, k, t)
        assert L.moe_create(ctypes.byref(d), ctypes.byref(ctx)) == want, (h, i, e, k, t)
        assert not ctx.value
    assert L.moe_destroy(None) == _native.MOE_OK
    assert L.moe_forward(None, None, None, None, 4, None) == _native.MOE_ERR_INVALID_ARG
    assert L.moe_route(None, None, 4, None) == _native.MOE_ERR_INVALID_ARG
    assert L.moe_experts(None, None, None, None, 4, None) == _native.MOE_ERR_INVALID_ARG
    assert L.moe_route_logits(None, None, 4, None) == _native.MOE_ERR_INVALID_ARG
    assert L.moe_last_routing(None, None, None, None, None, 0, None) == _native.MOE_ERR_INVALID_ARG
    assert L.moe_device_status(None, None) == _native.MOE_ERR_INVALID_ARG
    assert L.moe_set_weights(None, None, None, None, None, None, 0, None) == _native.MOE_ERR_INVALID_ARG
    assert L.moe_plan_tile_rows(None, 64) == -1
    assert L.moe_force_tile_rows(None, 0) == _native.MOE_ERR_INVALID_ARG
    assert L.moe_set_wait_divisor(None, 2) == _native.MOE_ERR_INVALID_ARG
    assert L.moe_set_lazy_chains(None, 1) == _native.MOE_ERR_INVALID_ARG


def test_error_raises_with_status():
    from final_amd import _native
    with pytest.raises(_native.MoeError) as ei:
        _native.check(_native.MOE_ERR_TOO_MANY_TOKENS, "moe_forward")
    assert ei.value.status == _native.MOE_ERR_TOO_MANY_TOKENS
    assert "max_tokens" in str(ei.value)


def test_lfm_argument_validation_before_any_gpu_call(L):
    from final_amd import _native
    INV, UNS = _native.MOE_ERR_INVALID_ARG, _native.MOE_ERR_UNSUPPORTED
    a = 4096  # a 16-byte-aligned non-null address the checks never dereference
    assert L.lfm_gemm_nt(None, a, a + 64, None, 4, 128, 32, None) == INV
    assert L.lfm_gemm_nt(a, a, a + 64, None, -1, 128, 32, None) == INV
    assert L.lfm_gemm_nt(a, a + 64, a, None, 4, 128, 32, None) == INV      # C aliases A
    assert L.lfm_gemm_nt(a, a + 64, a + 128, None, 4, 100, 32, None) == UNS  # N % 128
    assert L.lfm_gemm_nt(a, a + 64, a + 128, None, 4, 128, 48, None) == UNS  # K % 32
    assert L.lfm_gemm_nt(a + 4, a + 64, a + 128, None, 4, 128, 32, None) == INV  # misaligned
    assert L.lfm_gemm_nt(None, None, None, None, 0, 128, 32, None) == _native.MOE_OK
    assert L.lfm_embed(None, a, a, 4, 2048, 100, None, None) == INV
    assert L.lfm_embed(a, a, a, 4, 2050, 100, None, None) == UNS
    assert L.lfm_rmsnorm(a, 10, a, a, 64, 2, 64, None) == INV             # stride < dim
    assert L.lfm_qk_norm_rope(a, 3072, a, a, a, a, 1, 4, 32, 8, 1024, None) == INV  # k_col overlaps q
    assert L.lfm_attention(a, 3072, a + 4096 * 16, 1, 4, 32, 4, 2048, 2560, None) == UNS  # 8 groups
    assert L.lfm_attention(a, 3072, a, 1, 4, 32, 8, 2048, 2560, None) == INV  # out aliases qkv
    assert L.lfm_shortconv(a, a, a + 64, 1, 4, 2050, 3, None) == UNS
    assert L.lfm_shortconv(a, a, a, 1, 4, 2048, 3, None) == INV
    assert L.lfm_model_forward(None, a, 1, 1, a, None) == INV
    assert L.lfm_model_destroy(None) == _native.MOE_OK
    assert L.lfm_model_create_synthetic(None, None) == INV
    assert L.lfm_rope_tables(None, None, 4, 64, 1e6) == INV
    assert L.lfm_synth_is_norm(b"layers.0.ffn_norm.weight") == 1
    assert L.lfm_synth_is_norm(b"layers.0.conv.in_proj.weight") == 0
    assert L.lfm_synth_stream_of(b"a") == 0xAF63DC4C8601EC8C  # FNV-1a 64 of "a"
