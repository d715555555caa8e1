"""The C ABI library loads without a GPU, exports every declared entry point, and its
host-only functions (status strings, workspace layout, argument checks) behave."""

import ctypes
import os
import re

import pytest

from sgl_asap_amd import _lib
from sgl_asap_amd.moe.experts import workspace_layout

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "afd.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(afd_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(_lib.EXPORTED)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in declared_functions():
        assert hasattr(L, name), name
    assert L.afd_abi_version() == _lib.ABI_VERSION == 6


def test_status_strings():
    L = _lib.lib()
    for st in (0, -1, -2, -3, -4, -5):
        assert L.afd_status_string(st)
    with pytest.raises(ValueError):
        _lib.check(_lib.AFD_ERR_ARG, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.AFD_ERR_UNSUPPORTED, "x")


def test_workspace_layout_dsv4_rank():
    cfg = _lib.AfdMoeCfg(4096, 2048, 8, 0, 64, _lib.AFD_W_MXFP4)
    L = workspace_layout(cfg, 16384)
    assert L["block_m"] == 128
    assert L["np_max"] == (16384 * 8 + 64 * 127 + 127) // 128 * 128
    tiles = L["np_max"] // 128
    assert L["max_tiles"] == tiles
    # MXFP4: xq / xs are the per-token e4m3 rows and their UE8M0 scales; hq holds one A tile
    # image (16896 B) per row tile and 128-wide K stage of h (+ 512 B of readable slack after
    # the last image, rounded to 256 B)
    assert L["xq"] == 0 and L["xs"] == 16384 * 4096
    assert L["counts"] - L["xs"] == 16384 * 4096 // 32
    assert L["hs"] - L["hq"] == -(-(tiles * (2048 // 128) * 16896 + 512) // 256) * 256
    offs = [L[k] for k in ("xq", "xs", "counts", "offsets", "padded_offsets", "sorted_pairs", "pair_pos",
                           "tile_expert", "num_tiles", "hist", "hq", "hs", "y")]
    assert offs == sorted(offs) and all(o % 256 == 0 for o in offs)
    assert L["total"] >= L["y"] + L["np_max"] * 4096 * 2


def test_workspace_layout_fp8_block():
    """W8A8 (FP8 block weights, fp8 activations): expert segments pad to 256 rows; hq holds one
    16 KiB FP8 image per 256-row tile and 64-wide K stage of h, hs their fp32 1x128 scales."""
    cfg = _lib.AfdMoeCfg(4096, 1536, 8, 0, 64, _lib.AFD_W_FP8_BLOCK)
    L = workspace_layout(cfg, 16384)
    assert L["block_m"] == 256
    assert L["np_max"] == (16384 * 8 + 64 * 255 + 255) // 256 * 256
    tiles = L["np_max"] // 256
    assert L["max_tiles"] == tiles
    assert L["xq"] == 0 and L["xs"] == 16384 * 4096
    assert L["counts"] - L["xs"] == 16384 * (4096 // 128) * 4
    assert L["hs"] - L["hq"] == tiles * (1536 // 64) * 256 * 64
    assert L["y"] - L["hs"] == tiles * (1536 // 128) * 256 * 4
    assert L["tile_expert"] + tiles * 4 <= L["num_tiles"]
    assert L["total"] >= L["y"] + L["np_max"] * 4096 * 2


def test_workspace_layout_bf16_activations():
    """W4A16 (MXFP4 weights, bf16 activations): xq holds a batch's bf16 rows, xs is empty, hq
    one 32 KiB bf16 A image per row tile and 128-wide K stage of h, hs empty."""
    cfg = _lib.AfdMoeCfg(4096, 2048, 8, 0, 64, _lib.AFD_W_MXFP4, _lib.AFD_ACT_SWIGLU, 0.0, 0.0,
                         _lib.AFD_WALK_STATIC, _lib.AFD_A_BF16)
    L = workspace_layout(cfg, 16384)
    tiles = L["max_tiles"]
    assert L["xq"] == 0 and L["xs"] == 16384 * 4096 * 2
    assert L["counts"] == L["xs"]  # no scales
    assert L["hs"] - L["hq"] == tiles * (2048 // 128) * 128 * 128 * 2
    assert L["y"] == L["hs"]
    fp8 = workspace_layout(_lib.AfdMoeCfg(4096, 2048, 8, 0, 64, _lib.AFD_W_MXFP4), 16384)
    assert (fp8["np_max"], fp8["max_tiles"]) == (L["np_max"], L["max_tiles"])


def test_activation_format_checks():
    out = _lib.AfdWsLayout()
    L = _lib.lib()
    unknown = _lib.AfdMoeCfg(4096, 2048, 8, 0, 64, _lib.AFD_W_MXFP4, 0, 0.0, 0.0, 0, 2)
    assert L.afd_workspace_layout(ctypes.byref(unknown), 16, ctypes.byref(out)) == _lib.AFD_ERR_UNSUPPORTED
    # W8A16: FP8 blocks with bf16 activations, the same bf16 h bytes as W4A16, no h scales
    w8 = workspace_layout(_lib.AfdMoeCfg(4096, 1536, 8, 0, 64, _lib.AFD_W_FP8_BLOCK, 0, 0.0, 0.0, 0,
                                         _lib.AFD_A_BF16), 16384)
    assert w8["xs"] - w8["xq"] == 16384 * 4096 * 2 and w8["counts"] == w8["xs"]
    assert w8["hs"] - w8["hq"] == w8["max_tiles"] * (1536 // 64) * 128 * 64 * 2 and w8["y"] == w8["hs"]
    # bf16 activations are not quantized: afd_quant_act refuses before touching any pointer
    a16 = _lib.AfdMoeCfg(256, 128, 2, 0, 8, _lib.AFD_W_MXFP4, 0, 0.0, 0.0, 0, _lib.AFD_A_BF16)
    assert L.afd_quant_act(ctypes.byref(a16), None, 0, None, None, None) == _lib.AFD_ERR_UNSUPPORTED


def test_silu_mul_argument_checks():
    """afd_silu_mul refuses bad shapes on the host, before any launch."""
    L = _lib.lib()
    assert L.afd_silu_mul(None, 0, 1536, None, None) == _lib.AFD_OK  # nothing to do
    assert L.afd_silu_mul(None, -1, 1536, None, None) == _lib.AFD_ERR_ARG
    assert L.afd_silu_mul(None, 4, 0, None, None) == _lib.AFD_ERR_ARG
    assert L.afd_silu_mul(None, 4, 1536, None, None) == _lib.AFD_ERR_ARG
    assert L.afd_silu_mul(16, 4, 1540, 16, None) == _lib.AFD_ERR_SHAPE  # inter not a multiple of 8
    assert L.afd_silu_mul(8, 4, 1536, 16, None) == _lib.AFD_ERR_SHAPE  # misaligned rows
    assert L.afd_silu_mul(16, 1 << 30, 64, 16, None) == _lib.AFD_ERR_SHAPE  # 2^33 vectors
    assert L.afd_silu_mul(16, 1 << 28, 64, 16, None) == _lib.AFD_ERR_SHAPE  # 2^31 vectors


def test_python_activation_formats():
    from sgl_asap_amd.moe.experts import ExpertWeights, moe_cfg

    mx = ExpertWeights("mxfp4", 4, 256, 128, None, None, None, None)
    fp8 = ExpertWeights("fp8_block", 4, 256, 128, None, None, None, None)
    assert moe_cfg(mx, 2, 0).act_fmt == _lib.AFD_A_FP8
    assert moe_cfg(mx, 2, 0, act_format="mxfp8").act_fmt == _lib.AFD_A_FP8
    assert moe_cfg(mx, 2, 0, act_format="bf16").act_fmt == _lib.AFD_A_BF16
    assert moe_cfg(fp8, 2, 0, act_format="fp8_1x128").act_fmt == _lib.AFD_A_FP8
    assert moe_cfg(fp8, 2, 0, act_format="bf16").act_fmt == _lib.AFD_A_BF16
    with pytest.raises(ValueError):
        moe_cfg(mx, 2, 0, act_format="fp8_1x128")
    with pytest.raises(ValueError):
        moe_cfg(fp8, 2, 0, act_format="mxfp8")


def test_bad_configs_rejected_on_host():
    out = _lib.AfdWsLayout()
    bad = [
        _lib.AfdMoeCfg(4000, 2048, 8, 0, 64, 1),  # hidden not a multiple of 256
        _lib.AfdMoeCfg(4096, 2000, 8, 0, 64, 1),  # inter not a multiple of 128
        _lib.AfdMoeCfg(16640, 2048, 8, 0, 64, 1),  # hidden above 16384
        _lib.AfdMoeCfg(4096, 16512, 8, 0, 64, 1),  # inter above 16384
        _lib.AfdMoeCfg(4096, 2048, 0, 0, 64, 1),  # topk 0
        _lib.AfdMoeCfg(4096, 2048, 8, 0, 512, 1),  # too many local experts
        _lib.AfdMoeCfg(4096, 2048, 8, 0, 64, 7),  # unknown format
        _lib.AfdMoeCfg(4096, 2048, 8, 0, 64, 1, 5),  # unknown activation
        _lib.AfdMoeCfg(4096, 2048, 8, 0, 64, 1, _lib.AFD_ACT_SITU, 0.0, 1.0),  # SiTU without beta
        _lib.AfdMoeCfg(4096, 2048, 8, 0, 64, 1, _lib.AFD_ACT_SITU, 1.0, float("inf")),
        _lib.AfdMoeCfg(4096, 2048, 8, 0, 64, 1, _lib.AFD_ACT_SWIGLU_LIMIT, 0.0, 0.0),  # no limit
        _lib.AfdMoeCfg(4096, 2048, 8, 0, 64, 1, _lib.AFD_ACT_SWIGLU_LIMIT, 0.0, float("inf")),
    ]
    for cfg in bad:
        assert _lib.lib().afd_workspace_layout(ctypes.byref(cfg), 16, ctypes.byref(out)) != 0
    widest = _lib.AfdMoeCfg(16384, 16384, 8, 0, 8, 1)
    assert _lib.lib().afd_workspace_layout(ctypes.byref(widest), 16, ctypes.byref(out)) == 0
    good = _lib.AfdMoeCfg(256, 128, 2, 0, 8, 1)
    assert _lib.lib().afd_workspace_layout(ctypes.byref(good), 1 << 17, ctypes.byref(out)) != 0
    assert _lib.lib().afd_workspace_layout(ctypes.byref(good), (1 << 17) - 1, ctypes.byref(out)) == 0


def test_situ_and_limit_configs_accepted():
    out = _lib.AfdWsLayout()
    for ok in (_lib.AfdMoeCfg(4096, 2048, 8, 0, 64, 1, _lib.AFD_ACT_SITU, 2.0, 3.0),
               _lib.AfdMoeCfg(4096, 2048, 8, 0, 64, 1, _lib.AFD_ACT_SWIGLU_LIMIT, 0.0, 10.0)):
        assert _lib.lib().afd_workspace_layout(ctypes.byref(ok), 16, ctypes.byref(out)) == 0


def test_python_activation_arguments():
    """AfdExperts' activation arguments follow FusedMoE's (activation, gemm1_alpha,
    gemm1_clamp_limit) and fail as the reference does."""
    from sgl_asap_amd.moe.experts import ExpertWeights, moe_cfg

    wts = ExpertWeights("mxfp4", 4, 256, 128, None, None, None, None)
    assert moe_cfg(wts, 2, 0).activation == _lib.AFD_ACT_SWIGLU
    c = moe_cfg(wts, 2, 0, "situ", 2.0, 3.0)
    assert (c.activation, c.act_alpha, c.act_limit) == (_lib.AFD_ACT_SITU, 2.0, 3.0)
    with pytest.raises(ValueError):
        moe_cfg(wts, 2, 0, "situ", 2.0, None)
    with pytest.raises(NotImplementedError):
        moe_cfg(wts, 2, 0, "gelu")
    # SwiGLU with a limit: gemm1_clamp_limit on "silu", or DeepSeek-V4's swiglu_limit
    c = moe_cfg(wts, 2, 0, "silu", None, 10.0)
    assert (c.activation, c.act_limit) == (_lib.AFD_ACT_SWIGLU_LIMIT, 10.0)
    for bad in (0.0, -1.0, float("inf")):
        with pytest.raises(ValueError):
            moe_cfg(wts, 2, 0, "silu", None, bad)
