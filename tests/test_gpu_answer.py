"""GPU: the expert call that answers its job (afd_moe_ffn_answer). Its output equals the plain
call's bit for bit (bf16 rows and quantized rows, both weight formats), and the done word in
pinned host memory holds the reply value once the stream has passed the call; a stream parked
on that word (the A side's wait) then reads the complete output. n = 0 stores the value with a
stream store. Calls back to back on one stream and workspace each store their own value."""

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import bits16, dev, say
from sgl_asap_amd import _lib
from sgl_asap_amd import workloads as W
from sgl_asap_amd.moe.experts import AfdExperts, pack_fp8_block_experts, pack_mxfp4_experts
from sgl_asap_amd.moe.topk import StandardTopKOutput
from sgl_asap_amd.transport import hip

pytestmark = pytest.mark.gpu

H, I, E, K = 256, 128, 16, 4
LOCAL = range(4, 12)
PACK = {"mxfp4": pack_mxfp4_experts, "fp8_block": pack_fp8_block_experts}


def layer(fmt, n_max, seed=0):
    gen = W.generator("cpu", seed)
    w13, w2 = W.expert_weights(len(LOCAL), H, I, gen, "cpu")
    return AfdExperts(E, K, 0, LOCAL, PACK[fmt](w13, w2, device=dev()), n_max=n_max)


def job(n, seed):
    gen = W.generator("cpu", seed)
    x = W.tokens(n, H, gen, "cpu").to(dev())
    ids, w = W.route_uniform(n, E, K, gen, "cpu")
    return x, ids.to(torch.int32).to(dev()), w.to(torch.float32).to(dev())


def plain(experts, x, ids, w):
    out = experts(x, StandardTopKOutput(w, ids))
    torch.cuda.synchronize()
    return bits16(out)


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
@pytest.mark.parametrize("quantized", [False, True])
def test_answer_equals_plain_call_and_stores_the_reply(fmt, quantized):
    say(f"afd_moe_ffn_answer fmt={fmt} quantized={quantized}")
    experts = layer(fmt, 512)
    page = hip.HostPage(4096)
    stream = torch.cuda.current_stream().cuda_stream
    try:
        for i, (n, seed) in enumerate(((1, 1), (300, 2), (512, 3), (77, 4))):
            x, ids, w = job(n, seed)
            out = torch.full((n, H), 3.0, dtype=torch.bfloat16, device=dev())
            value = (1 << 40) + 17 * (i + 1)
            if quantized:
                xq, xs = experts.quant_act(x)
                experts.call_ptrs(n, xq.data_ptr(), xs.data_ptr(), ids.data_ptr(), w.data_ptr(), out.data_ptr(),
                                  stream, page.addr(64), value)
            else:
                experts.call_ptrs(n, x.data_ptr(), 0, ids.data_ptr(), w.data_ptr(), out.data_ptr(), stream,
                                  page.addr(64), value)
            torch.cuda.synchronize()
            assert page.load(64) == value
            assert np.array_equal(bits16(out), plain(experts, x, ids, w)), (n, seed)
    finally:
        page.release()


def test_waiting_stream_sees_the_whole_output():
    """A second stream parks on the done word (GEQ) and copies the output right after: the copy
    equals the output, for calls large enough that the wait is parked while they run."""
    say("afd_moe_ffn_answer: a parked stream reads the complete output")
    experts = layer("mxfp4", 4096)
    page = hip.HostPage(4096)
    compute, reader = torch.cuda.Stream(), torch.cuda.Stream()
    try:
        for i, (n, seed) in enumerate(((4096, 11), (1500, 12), (4096, 13))):
            x, ids, w = job(n, seed)
            out = torch.zeros(n, H, dtype=torch.bfloat16, device=dev())
            copy = torch.empty_like(out)
            value = 100 + i
            compute.wait_stream(torch.cuda.current_stream())
            reader.wait_stream(torch.cuda.current_stream())
            # the call is enqueued before the wait it satisfies (streams may share a hardware
            # queue); the wait still starts while the call runs
            experts.call_ptrs(n, x.data_ptr(), 0, ids.data_ptr(), w.data_ptr(), out.data_ptr(),
                              compute.cuda_stream, page.addr(0), value)
            hip.wait64(reader.cuda_stream, page.addr(0), value)
            with torch.cuda.stream(reader):
                copy.copy_(out)
            torch.cuda.synchronize()
            assert page.load(0) == value
            assert np.array_equal(bits16(copy), bits16(out)), (n, seed)
            assert np.array_equal(bits16(out), plain(experts, x, ids, w))
    finally:
        page.release()


def test_empty_job_stores_with_a_stream_store():
    say("afd_moe_ffn_answer: n = 0")
    experts = layer("mxfp4", 64)
    page = hip.HostPage(4096)
    try:
        ws = experts.workspace()
        stream = torch.cuda.current_stream().cuda_stream
        _lib.call("afd_moe_ffn_answer", ctypes.byref(experts.cfg), ctypes.byref(experts._wstruct),
                  ws.data_ptr(), None, None, ws.data_ptr(), ws.data_ptr(), 0, ws.data_ptr(), ws.numel(),
                  ws.data_ptr(), page.addr(8), 5, stream)
        torch.cuda.synchronize()
        assert page.load(8) == 5
        for bad in ((None, None), (ws.data_ptr(), ws.data_ptr())):  # exactly one activation form
            with pytest.raises(ValueError):
                _lib.call("afd_moe_ffn_answer", ctypes.byref(experts.cfg), ctypes.byref(experts._wstruct),
                          bad[0], bad[1], None, ws.data_ptr(), ws.data_ptr(), 0, ws.data_ptr(), ws.numel(),
                          ws.data_ptr(), page.addr(8), 5, stream)
        with pytest.raises(ValueError):  # a misaligned done word
            _lib.call("afd_moe_ffn_answer", ctypes.byref(experts.cfg), ctypes.byref(experts._wstruct),
                      ws.data_ptr(), None, None, ws.data_ptr(), ws.data_ptr(), 0, ws.data_ptr(), ws.numel(),
                      ws.data_ptr(), page.addr(8) + 4, 5, stream)
    finally:
        page.release()
