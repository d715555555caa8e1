"""GPU: the one-GPU AFD loop (dispatch -> arena copies + doorbell -> F job gated on the
doorbell -> reply + done flag -> combine) returns exactly what the expert call returns."""

import numpy as np
import pytest
import torch

from gpu_util import bits16, dev, say
from oracle import experts as OX
from sgl_asap_amd import workloads as W
from sgl_asap_amd.loop import OneGpuAfd
from sgl_asap_amd.moe.experts import AfdExperts, pack_mxfp4_experts
from sgl_asap_amd.moe.layer import AsapMoE
from sgl_asap_amd.moe.topk import StandardTopKOutput

pytestmark = pytest.mark.gpu

H, I, E, K = 256, 128, 16, 4
LOCAL = range(0, 8)  # this F rank owns half the experts


def make_experts(n_max, layers=(0,), seed=0):
    gen = W.generator("cpu", seed)
    out = {}
    for layer in layers:
        w13, w2 = W.expert_weights(len(LOCAL), H, I, gen, "cpu")
        out[layer] = AfdExperts(E, K, layer, LOCAL, pack_mxfp4_experts(w13, w2, device=dev()), n_max=n_max)
    return out


def job(n, seed):
    gen = W.generator("cpu", seed)
    x = W.tokens(n, H, gen, "cpu").to(dev())
    ids, w = W.route_uniform(n, E, K, gen, "cpu")
    return x, StandardTopKOutput(w.to(dev()), ids.to(dev()))


def direct(experts, layer, x, topk):
    out = experts[layer](x, topk)
    torch.cuda.synchronize()
    return bits16(out)


def test_loop_matches_expert_call():
    say("loop: single layer, single slot")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64) as afd:
        layer = AsapMoE(E, H, I, 0, top_k=K)
        for seed in range(3):
            x, topk = job(37 + seed, seed)
            out = layer(x, topk)
            torch.cuda.synchronize()
            assert np.array_equal(bits16(out), direct(experts, 0, x, topk))
        assert afd.server.stats["jobs"] == 3 and afd.server.stats["lost_messages"] == 0


def test_loop_shared_expert_add():
    say("loop: shared expert added in the combine")
    experts = make_experts(64)
    gen = W.generator("cpu", 5)
    wsh = torch.randn(H, H, generator=gen).to(torch.bfloat16).to(dev()) * 0.05

    def shared(x):
        return (x.float() @ wsh.float().T).to(torch.bfloat16)

    with OneGpuAfd(experts, n_max=64):
        layer = AsapMoE(E, H, I, 0, top_k=K, shared_experts=shared)
        x, topk = job(50, 11)
        out = layer(x, topk)
        torch.cuda.synchronize()
        routed = direct(experts, 0, x, topk)
        ref = OX.combine([routed], bits16(shared(x)))
        assert np.array_equal(bits16(out), ref)


def test_two_micro_batches_in_flight():
    say("loop: two slots in flight")
    experts = make_experts(64, layers=(0, 1))
    with OneGpuAfd(experts, n_max=64, slots=2):
        layers = [AsapMoE(E, H, I, lid, top_k=K) for lid in (0, 1)]
        for lid, layer in enumerate(layers):
            (xa, ta), (xb, tb) = job(20, 2 * lid), job(33, 2 * lid + 1)
            da = layer.dispatcher.dispatch(xa, ta, micro_batch=0)
            db = layer.dispatcher.dispatch(xb, tb, micro_batch=1)
            oa = layer.dispatcher.combine(da)
            ob = layer.dispatcher.combine(db)
            torch.cuda.synchronize()
            assert np.array_equal(bits16(oa), direct(experts, lid, xa, ta))
            assert np.array_equal(bits16(ob), direct(experts, lid, xb, tb))


def test_sequence_wrap():
    say("loop: seq_base 2^32 - 3, eight messages across the wrap")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64, slots=1, seq_base=(1 << 32) - 3) as afd:
        layer = AsapMoE(E, H, I, 0, top_k=K)
        for seed in range(8):
            x, topk = job(16 + seed, 100 + seed)
            out = layer(x, topk)
            torch.cuda.synchronize()
            assert np.array_equal(bits16(out), direct(experts, 0, x, topk))
        assert afd.channel._seq[0] == 5  # 2^32 - 3 + 8 wrapped
        assert afd.server.stats["jobs"] == 8


def test_exchange_above_n_max():
    say("loop: n > n_max is exchanged in pieces")
    experts = make_experts(128)
    with OneGpuAfd(experts, n_max=48):
        layer = AsapMoE(E, H, I, 0, top_k=K)
        x, topk = job(128, 7)
        out = layer(x, topk)
        torch.cuda.synchronize()
        assert np.array_equal(bits16(out), direct(experts, 0, x, topk))


def test_graph_buckets():
    say("loop: hip graph buckets up to 64 tokens")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64, graph_max_tokens=64) as afd:
        assert afd.scheduler.graph_runner.buckets == [1, 2, 4, 8, 16, 32, 64]
        layer = AsapMoE(E, H, I, 0, top_k=K)
        for n in (1, 3, 16, 17, 64):
            x, topk = job(n, 200 + n)
            out = layer(x, topk)
            torch.cuda.synchronize()
            assert np.array_equal(bits16(out), direct(experts, 0, x, topk)), n


def test_empty_batch():
    say("loop: empty batch")
    experts = make_experts(64)
    with OneGpuAfd(experts, n_max=64) as afd:
        layer = AsapMoE(E, H, I, 0, top_k=K)
        x, topk = job(0, 1)
        out = layer(x, topk)
        assert out.shape == (0, H) and afd.server.stats["jobs"] == 0
