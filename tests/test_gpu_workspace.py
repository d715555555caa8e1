"""GPU: the expert calls' workspaces. Layers whose calls need the same workspace size share one
buffer per stream (calls on a stream run in order); another stream or another size gets its
own buffer. Calls of different layers enqueued back to back on one stream, and on two streams
at once, give the results of isolated calls bit for bit. A graph runner keeps a workspace of
its own (its graphs capture the pointer), so its replays do not depend on the shared ones."""

import numpy as np
import pytest
import torch

from gpu_util import bits16, dev, say
from sgl_asap_amd import workloads as W
from sgl_asap_amd.moe import experts as EX
from sgl_asap_amd.moe.experts import AfdExperts, pack_mxfp4_experts
from sgl_asap_amd.moe.topk import StandardTopKOutput
from sgl_asap_amd.runner.graph_runner import FfnGraphRunner

pytestmark = pytest.mark.gpu

H, I, E, K = 512, 256, 16, 4


def layer(seed, n_max=256):
    gen = W.generator("cpu", seed)
    w13, w2 = W.expert_weights(8, H, I, gen, "cpu")
    return AfdExperts(E, K, 0, range(4, 12), pack_mxfp4_experts(w13, w2, device=dev()), n_max=n_max)


def job(n, seed):
    gen = W.generator("cpu", seed)
    x = W.tokens(n, H, gen, "cpu").to(dev())
    ids, w = W.route_uniform(n, E, K, gen, "cpu")
    return x, StandardTopKOutput(w.to(torch.float32).to(dev()), ids.to(torch.int32).to(dev()))


def test_layers_share_a_workspace_per_stream_and_size():
    say("workspaces: sharing per (stream, size), interleaved layers bit-exact")
    a, b, c = layer(1), layer(2), layer(3, n_max=512)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    assert a.workspace(s1).data_ptr() == b.workspace(s1).data_ptr()
    assert a.workspace(s1).data_ptr() != a.workspace(s2).data_ptr()
    assert c.workspace(s1).data_ptr() != a.workspace(s1).data_ptr()  # another size
    jobs = [job(n, 10 + n) for n in (200, 37, 256)]
    alone = []
    for lay in (a, b):
        for x, t in jobs:
            alone.append(bits16(lay(x, t)))
            torch.cuda.synchronize()
    # the same six calls back to back on one stream, then spread over two streams at once
    for streams in ((s1,), (s1, s2)):
        outs = []
        k = 0
        for lay in (a, b):
            for x, t in jobs:
                s = streams[k % len(streams)]
                s.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(s):
                    outs.append(lay(x, t))
                k += 1
        torch.cuda.synchronize()
        for got, want in zip(outs, alone):
            assert np.array_equal(bits16(got), want)


def test_graph_runner_keeps_its_own_workspace():
    say("workspaces: a graph runner's own buffer")
    a = layer(4)
    runner = FfnGraphRunner({0: a}, 256, a.local)
    pool = {ws.data_ptr() for ws in EX._WORKSPACES.values()}
    assert runner.ws.data_ptr() not in pool and runner.ws.numel() >= a.layout["total"]
    for n, seed in ((5, 21), (256, 22)):
        x, t = job(n, seed)
        want = bits16(a(x, t))
        out = runner.run(0, x, t.topk_ids, t.topk_weights, 0)
        torch.cuda.synchronize()
        assert np.array_equal(bits16(out), want)
