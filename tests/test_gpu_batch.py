"""GPU: batched expert calls (afd_moe_ffn_batch) and the F scheduler's batching.

One call over several jobs of a layer must give every job exactly the output of the expert
call on that job alone (bf16 bit patterns equal): the single-job call is pinned against the
oracle by test_gpu_moe / test_gpu_fullsize / test_gpu_stream, so equality pins the batch.
Covered: MXFP4 at the DeepSeek-V4 F-rank shape with Zipf(1.2) jobs of very different sizes
(one token, empty jobs, a job of whole row tiles), eight jobs (the most a batch holds), FP8
128x128-block experts, SiTU, the done counters of the answering form (including a batch of
empty jobs), the argument checks, and the scheduler packing the jobs of one poll through the
one-GPU transport."""

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import bits16, dev, say
from sgl_asap_amd import _lib
from sgl_asap_amd import workloads as W
from sgl_asap_amd.loop import OneGpuAfd
from sgl_asap_amd.moe.experts import AfdExperts, pack_fp8_block_experts, pack_mxfp4_experts, release_workspaces
from sgl_asap_amd.moe.topk import StandardTopKOutput
from sgl_asap_amd.transport.hip import HostPage

pytestmark = pytest.mark.gpu

DSV4 = W.SHAPES["dsv4_zipf"]


def make_jobs(shape, sizes, seed, device):
    jobs = []
    for j, n in enumerate(sizes):
        x, ids, w = W.job(shape, n=n, seed=seed + j, device="cpu")
        jobs.append((x.to(device), StandardTopKOutput(w.float().to(device), ids.int().to(device))))
    return jobs


def assert_batch_equals_single(layer, jobs):
    single = [bits16(layer(x, t)) for x, t in jobs]
    batched = [bits16(o) for o in layer.forward_batch(jobs)]
    torch.cuda.synchronize()
    for b, (s, o) in enumerate(zip(single, batched)):
        assert s.shape == o.shape, b
        assert np.array_equal(s, o), f"job {b} ({s.shape[0]} tokens)"


@pytest.fixture(scope="module")
def dsv4_layer():
    say("batch: packing 64 MXFP4 experts (hidden 4096, inter 2048)")
    gen = W.generator(dev(), 21)
    w13, w2 = W.expert_weights(DSV4.num_local, DSV4.hidden, DSV4.inter, gen, dev())
    layer = AfdExperts(DSV4.num_experts, DSV4.top_k, 0, DSV4.local, pack_mxfp4_experts(w13, w2), n_max=16384)
    del w13, w2
    torch.cuda.synchronize()
    yield layer
    del layer
    release_workspaces()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("sizes", [
    (1, 300, 0, 4097, 2048, 777, 5000),  # ragged, with an empty job and a one-token job
    (8192, 8192),                         # the one-GPU loop's two micro-batches in one call
    (16384,),                             # a batch of one
])
def test_mxfp4_batch_equals_single_calls(dsv4_layer, sizes):
    say(f"batch: MXFP4 dsv4 Zipf jobs {sizes}")
    jobs = make_jobs(DSV4, sizes, 700 + len(sizes), dev())
    assert_batch_equals_single(dsv4_layer, jobs)


def test_mxfp4_batch_of_eight_uniform_jobs(dsv4_layer):
    shape = W.SHAPES["dsv4_rank"]
    sizes = (64, 1, 513, 128, 2000, 129, 700, 1024)
    say(f"batch: eight uniform-routing jobs {sizes}")
    assert_batch_equals_single(dsv4_layer, make_jobs(shape, sizes, 800, dev()))


def test_batch_answers_every_job(dsv4_layer):
    """The answering form (what the scheduler enqueues): every job's output lands where its
    pointer says and every done counter holds its value afterwards; null counters skipped."""
    sizes = (3000, 10, 0, 1200)
    say(f"batch: answering form, jobs {sizes}")
    jobs = make_jobs(DSV4, sizes, 900, dev())
    single = [bits16(dsv4_layer(x, t)) for x, t in jobs]
    outs = [torch.full((x.shape[0], DSV4.hidden), -1.0, dtype=torch.bfloat16, device=dev()) for x, _ in jobs]
    page = HostPage(4096)
    try:
        rows = []
        for b, ((x, t), out) in enumerate(zip(jobs, outs)):
            done = page.addr(64 * b) if b != 1 else 0
            rows.append((x.shape[0], x.data_ptr(), 0, t.topk_ids.data_ptr(), t.topk_weights.data_ptr(),
                         out.data_ptr(), done, 1000 + b))
        stream = torch.cuda.current_stream().cuda_stream
        dsv4_layer.call_batch_ptrs(rows, stream, capacity=8192)
        torch.cuda.synchronize()
        assert [page.load(64 * b) for b in range(4)] == [1000, 0, 1002, 1003]
        for b, (s, o) in enumerate(zip(single, outs)):
            assert np.array_equal(s, bits16(o)), b
        # a batch whose jobs are all empty still answers (stream stores)
        empty = [(0, 0, 0, 0, 0, page.addr(512 + 64 * b), 7 + b) for b in range(2)]
        descs = (_lib.AfdBatchJob * 2)()
        for d, r in zip(descs, empty):
            d.n, d.done, d.value = 0, r[5], r[6]
        ws = dsv4_layer.workspace()
        _lib.call("afd_moe_ffn_batch", ctypes.byref(dsv4_layer.cfg), ctypes.byref(dsv4_layer._wstruct), descs, 2,
                  ws.data_ptr(), ws.numel(), stream)
        torch.cuda.synchronize()
        assert [page.load(512), page.load(576)] == [7, 8]
    finally:
        page.release()


def test_batch_argument_checks(dsv4_layer):
    say("batch: argument checks")
    tiny = make_jobs(DSV4, (2,) * 9, 950, dev())
    with pytest.raises(ValueError):
        dsv4_layer.forward_batch(tiny)  # nine jobs
    with pytest.raises(ValueError):
        dsv4_layer.forward_batch(make_jobs(DSV4, (9000, 8000), 960, dev()))  # 17000 > n_max
    descs = (_lib.AfdBatchJob * 1)()
    x, t = tiny[0]
    d = descs[0]
    d.x, d.ids, d.w, d.n, d.out = x.data_ptr(), t.topk_ids.data_ptr(), t.topk_weights.data_ptr(), 2, 0
    ws = dsv4_layer.workspace()
    stream = torch.cuda.current_stream().cuda_stream
    with pytest.raises(ValueError):  # no output pointer
        _lib.call("afd_moe_ffn_batch", ctypes.byref(dsv4_layer.cfg), ctypes.byref(dsv4_layer._wstruct), descs, 1,
                  ws.data_ptr(), ws.numel(), stream)
    d.out = x.data_ptr()
    d.reserved = 1
    with pytest.raises(ValueError):  # reserved field set
        _lib.call("afd_moe_ffn_batch", ctypes.byref(dsv4_layer.cfg), ctypes.byref(dsv4_layer._wstruct), descs, 1,
                  ws.data_ptr(), ws.numel(), stream)
    d.reserved = 0
    with pytest.raises(ValueError):  # workspace too small
        _lib.call("afd_moe_ffn_batch", ctypes.byref(dsv4_layer.cfg), ctypes.byref(dsv4_layer._wstruct), descs, 1,
                  ws.data_ptr(), 1024, stream)


@pytest.mark.parametrize("fmt,act", [("fp8_block", "silu"), ("mxfp4", "situ")])
def test_small_layers_batch_equals_single_calls(fmt, act):
    hidden, inter, num_experts, num_local, k = (1024, 512, 64, 16, 6) if fmt == "fp8_block" else (512, 256, 8, 8, 2)
    say(f"batch: {fmt} {act} H={hidden} I={inter} E={num_experts} local={num_local} k={k}")
    gen = W.generator("cpu", 31)
    w13, w2 = W.expert_weights(num_local, hidden, inter, gen, "cpu")
    pack = pack_fp8_block_experts if fmt == "fp8_block" else pack_mxfp4_experts
    kw = {} if act == "silu" else dict(activation="situ", gemm1_alpha=2.0, gemm1_clamp_limit=3.0)
    layer = AfdExperts(num_experts, k, 0, range(0, num_local), pack(w13, w2, device=dev()), n_max=4096, **kw)
    jobs = []
    for j, n in enumerate((333, 1, 1500, 64, 0, 900)):
        g = W.generator("cpu", 40 + j)
        x = W.tokens(n, hidden, g, "cpu")
        ids, w = W.route_zipf(n, num_experts, k, 1.1, g, "cpu")
        jobs.append((x.to(dev()), StandardTopKOutput(w.to(dev()), ids.to(dev()))))
    assert_batch_equals_single(layer, jobs)


def test_scheduler_batches_the_jobs_of_one_poll(dsv4_layer):
    """Four jobs from 2 replicas x 2 slots pending together: with batch_tokens the scheduler
    packs them (largest first) into batched calls, and every A rank's answer equals the plain
    call's bit for bit; two passes back to back before any synchronization."""
    sizes = (6000, 1700, 4097, 9000)
    say(f"batch: scheduler packing {sizes} at batch_tokens=12000")
    jobs = make_jobs(DSV4, sizes, 980, dev())
    eager = [bits16(dsv4_layer(x, t)) for x, t in jobs]
    order = [(r, mb) for r in range(2) for mb in range(2)]
    with OneGpuAfd({0: dsv4_layer}, n_max=16384, slots=2, replicas=2, batch_tokens=12000) as afd:
        main = torch.cuda.current_stream()
        sends = [torch.cuda.Stream() for _ in range(2)]
        copies = []
        for _ in range(2):
            for s in sends:
                s.wait_stream(main)
            tickets = []
            for (r, mb), (x, t) in zip(order, jobs):
                tickets.append((r, afd.channels[r].send(0, mb, x.data_ptr(), t.topk_ids.data_ptr(),
                                                        t.topk_weights.data_ptr(), x.shape[0], sends[r])))
            afd.scheduler.serve_pending()
            for r, t in tickets:
                afd.channels[r].wait(t, main)
                copies.append(afd.channels[r].result_view(0, t.slot, t.n_tokens).clone())
        torch.cuda.synchronize()
        assert afd.server.stats["jobs"] == 8
        # 9000 + 1700 and 6000 + 4097 fit 12000: two batched calls per pass
        assert afd.scheduler.batch_calls == 4
    for i, c in enumerate(copies):
        assert np.array_equal(bits16(c), eager[i % 4]), (i, sizes[i % 4])


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
def test_quantized_rows_batch_equals_single_calls(fmt):
    """Rows quantized by the A side (fp8 on the wire): the batch stages them into its
    workspace and every job's output equals afd_moe_ffn_q on that job alone."""
    hidden, inter, num_experts, num_local, k = (1024, 512, 64, 16, 6)
    say(f"batch: quantized rows, {fmt} H={hidden} I={inter} E={num_experts} local={num_local} k={k}")
    gen = W.generator("cpu", 51)
    w13, w2 = W.expert_weights(num_local, hidden, inter, gen, "cpu")
    pack = pack_fp8_block_experts if fmt == "fp8_block" else pack_mxfp4_experts
    layer = AfdExperts(num_experts, k, 0, range(0, num_local), pack(w13, w2, device=dev()), n_max=4096)
    jobs, single = [], []
    for j, n in enumerate((700, 1, 0, 1300, 64)):
        g = W.generator("cpu", 60 + j)
        x = W.tokens(n, hidden, g, "cpu").to(dev())
        ids, w = W.route_zipf(n, num_experts, k, 1.2, g, "cpu")
        topk = StandardTopKOutput(w.to(dev()), ids.to(dev()))
        xq, xs = layer.quant_act(x)
        jobs.append((xq, xs, topk, torch.empty(n, hidden, dtype=torch.bfloat16, device=dev())))
        single.append(bits16(layer.forward_q(xq, xs, topk)))
    rows = [(xq.shape[0], xq.data_ptr(), xs.data_ptr(), t.topk_ids.data_ptr(), t.topk_weights.data_ptr(),
             out.data_ptr(), 0, 0) for xq, xs, t, out in jobs if xq.shape[0] > 0]
    layer.call_batch_ptrs(rows, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    outs = [out for xq, _, _, out in jobs if xq.shape[0] > 0]
    want = [s for s, (xq, _, _, _) in zip(single, jobs) if xq.shape[0] > 0]
    for b, (s, o) in enumerate(zip(want, outs)):
        assert np.array_equal(s, bits16(o)), b


def test_scheduler_batches_fp8_wire_jobs(dsv4_layer):
    """MXFP8 on the wire: the A side quantizes before the copy and the scheduler's batched
    calls stage the arena's e4m3 rows; every answer equals the plain bf16 call's."""
    sizes = (3000, 700, 5000, 2100)
    say(f"batch: scheduler with MXFP8 on the wire, jobs {sizes}")
    jobs = make_jobs(DSV4, sizes, 990, dev())
    eager = [bits16(dsv4_layer(x, t)) for x, t in jobs]
    order = [(r, mb) for r in range(2) for mb in range(2)]
    with OneGpuAfd({0: dsv4_layer}, n_max=16384, slots=2, replicas=2, act="mxfp8", batch_tokens=16384) as afd:
        main = torch.cuda.current_stream()
        sends = [torch.cuda.Stream() for _ in range(2)]
        for s in sends:
            s.wait_stream(main)
        quantized = [dsv4_layer.quant_act(x) for x, _ in jobs]  # the A side's quantizer
        for s in sends:
            s.wait_stream(main)
        tickets = []
        for (r, mb), (x, t), (xq, xs) in zip(order, jobs, quantized):
            tickets.append((r, afd.channels[r].send(0, mb, xq.data_ptr(), t.topk_ids.data_ptr(),
                                                    t.topk_weights.data_ptr(), x.shape[0], sends[r],
                                                    xs_ptr=xs.data_ptr())))
        afd.scheduler.serve_pending()
        got = []
        for r, t in tickets:
            afd.channels[r].wait(t, main)
            got.append(afd.channels[r].result_view(0, t.slot, t.n_tokens).clone())
        torch.cuda.synchronize()
        assert afd.scheduler.batch_calls == 1  # 10800 tokens in one call
    for i, c in enumerate(got):
        assert np.array_equal(bits16(c), eager[i]), (i, sizes[i])
