"""GPU: the expert call on a job read from a device descriptor (afd_moe_ffn_job), the form
the graph runner captures. Every call equals the by-value call on the same job bit for bit,
for jobs smaller than the capacity, quantized rows, an empty job, a descriptor rewritten
between calls and captured graphs replayed on new jobs; a descriptor size above the capacity
is clamped to it."""

import numpy as np
import pytest
import torch

from gpu_util import bits16, dev, say
from sgl_asap_amd import workloads as W
from sgl_asap_amd.moe.experts import (
    AfdExperts,
    new_job_desc,
    pack_fp8_block_experts,
    pack_mxfp4_experts,
    set_job,
)
from sgl_asap_amd.moe.topk import StandardTopKOutput

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


def direct(experts, x, ids, w):
    out = experts(x, StandardTopKOutput(w, ids))
    torch.cuda.synchronize()
    return bits16(out)


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
@pytest.mark.parametrize("quantized", [False, True])
def test_job_calls_equal_by_value_calls(fmt, quantized):
    say(f"afd_moe_ffn_job fmt={fmt} quantized={quantized}")
    experts = layer(fmt, 256)
    desc = new_job_desc(dev())
    for n, seed in ((1, 1), (100, 2), (256, 3), (0, 4), (37, 5)):
        x, ids, w = job(n, seed)
        out = torch.full((n, H), 7.0, dtype=torch.bfloat16, device=dev())
        if quantized:
            xq, xs = experts.quant_act(x)
            set_job(desc, xq=xq, xs=xs, ids=ids, w=w, out=out)
        else:
            set_job(desc, x=x, ids=ids, w=w, out=out)
        experts.call_job(desc, 256, quantized)
        torch.cuda.synchronize()
        if n:
            assert np.array_equal(bits16(out), direct(experts, x, ids, w)), n


def test_descriptor_n_above_capacity_is_clamped():
    say("afd_moe_ffn_job: n > n_cap computes the first n_cap tokens")
    experts = layer("mxfp4", 128)
    desc = new_job_desc(dev())
    x, ids, w = job(100, 9)
    out = torch.full((100, H), 3.0, dtype=torch.bfloat16, device=dev())
    set_job(desc, x=x, ids=ids, w=w, out=out)
    experts.call_job(desc, 64, False)
    torch.cuda.synchronize()
    got = bits16(out)
    assert np.array_equal(got[:64], direct(experts, x[:64].contiguous(), ids[:64].contiguous(), w[:64].contiguous()))
    assert np.all(got[64:] == bits16(torch.full((1,), 3.0, dtype=torch.bfloat16))[0])


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
def test_captured_graph_serves_new_jobs(fmt):
    """One capture at capacity 128, replayed on jobs of 5..128 tokens written into the
    descriptor, with eager calls and synchronizations between the replays."""
    say(f"graph of afd_moe_ffn_job, fmt={fmt}")
    experts = layer(fmt, 128)
    desc = new_job_desc(dev())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        experts.call_job(desc, 128)  # descriptor n = 0: a first call that does nothing
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        experts.call_job(desc, 128)
    torch.cuda.synchronize()
    for rep in range(3):
        for n in (5, 128, 64, 77):
            x, ids, w = job(n, 100 + 10 * rep + n)
            out = torch.empty(n, H, dtype=torch.bfloat16, device=dev())
            set_job(desc, x=x, ids=ids, w=w, out=out)
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(bits16(out), direct(experts, x, ids, w)), (rep, n)


def test_set_job_argument_checks():
    say("set_job argument checks")
    desc = new_job_desc(dev())
    x, ids, w = job(8, 1)
    out = torch.empty(8, H, dtype=torch.bfloat16, device=dev())
    with pytest.raises(ValueError):
        set_job(desc, ids=ids, w=w, out=out)  # no rows
    with pytest.raises(ValueError):
        set_job(desc, x=x[:4], ids=ids, w=w, out=out)  # row count
    with pytest.raises(TypeError):
        set_job(desc, x=x, ids=ids.long(), w=w, out=out)
    with pytest.raises(ValueError):
        layer("mxfp4", 16).call_job(desc, 32)  # capacity above n_max
