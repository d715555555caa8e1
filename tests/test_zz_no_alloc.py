"""GPU: the allocation-free expert call (afd_moe_ffn_noalloc, through the C ABI) equals the
expert call with a workspace argument (afd_moe_ffn) bit for bit, on two calls in a row with
the second one smaller (the library's scratch array keeps the first call's contents), for both
weight formats; a job whose workspace would exceed the array is refused."""

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import bits16, dev, say
from sgl_asap_amd import _lib
from sgl_asap_amd import workloads as W
from sgl_asap_amd.moe.experts import AfdExperts, pack_fp8_block_experts, pack_mxfp4_experts, workspace_layout
from sgl_asap_amd.moe.topk import StandardTopKOutput

pytestmark = pytest.mark.gpu

H, I, E, K = 1024, 512, 32, 4
LOCAL = range(8, 24)
PACK = {"mxfp4": pack_mxfp4_experts, "fp8_block": pack_fp8_block_experts}


def noalloc(layer, x, ids, w, out):
    return _lib.lib().afd_moe_ffn_noalloc(
        ctypes.byref(layer.cfg), ctypes.byref(layer._wstruct), x.data_ptr(), ids.data_ptr(), w.data_ptr(),
        x.shape[0], out.data_ptr(), torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
def test_noalloc_equals_workspace_call(fmt):
    gen = W.generator("cpu", 21)
    w13, w2 = W.expert_weights(len(LOCAL), H, I, gen, "cpu")
    layer = AfdExperts(E, K, 0, LOCAL, PACK[fmt](w13, w2, device=dev()), n_max=2048)
    for n, seed in ((1500, 1), (37, 2)):  # the second call smaller than the first
        say(f"afd_moe_ffn_noalloc fmt={fmt} n={n}")
        x = W.tokens(n, H, gen, "cpu").to(dev())
        ids, w = W.route_uniform(n, E, K, gen, "cpu")
        ids, w = ids.to(torch.int32).to(dev()), w.to(torch.float32).to(dev())
        got = torch.full((n, H), 5.0, dtype=torch.bfloat16, device=dev())
        _lib.check(noalloc(layer, x, ids, w, got), "afd_moe_ffn_noalloc")
        want = layer(x, StandardTopKOutput(w, ids))
        torch.cuda.synchronize()
        assert np.array_equal(bits16(got), bits16(want)), (fmt, n)


def test_noalloc_refuses_jobs_beyond_the_scratch_array():
    say("afd_moe_ffn_noalloc: job above the scratch size is refused")
    shape = W.SHAPES["dsv4_rank"]
    cfg = _lib.AfdMoeCfg(shape.hidden, shape.inter, shape.top_k, 0, shape.num_local, _lib.AFD_W_MXFP4)
    assert workspace_layout(cfg, 568)["total"] <= _lib.AFD_NOALLOC_SCRATCH_BYTES
    assert workspace_layout(cfg, 569)["total"] > _lib.AFD_NOALLOC_SCRATCH_BYTES
    weights = _lib.AfdExpertWeights(1, 1, 1, 1)  # never read: the size check comes first
    x = torch.empty(569, shape.hidden, dtype=torch.bfloat16, device=dev())
    ids = torch.zeros(569, shape.top_k, dtype=torch.int32, device=dev())
    w = torch.zeros(569, shape.top_k, dtype=torch.float32, device=dev())
    st = _lib.lib().afd_moe_ffn_noalloc(ctypes.byref(cfg), ctypes.byref(weights), x.data_ptr(), ids.data_ptr(),
                                        w.data_ptr(), 569, x.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert st == _lib.AFD_ERR_WORKSPACE
