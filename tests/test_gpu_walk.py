"""GPU: the two tile walks of the persistent GEMMs give identical results. "dynamic" hands
the tiles out from per-XCD counters, "static" gives each workgroup a fixed share; both run
over the same dense tile order, so every output bit must agree, for both weight formats with
fp8 or bf16 activations, for jobs from one token (8 row tiles, fewer than the 32 needed
to split the rows over the XCDs) to thousands, for skewed routing, and while another stream
holds a parked wait (a CU held by a wait kernel: the dynamic walk must still cover every
tile).

Before every call the whole workspace and the output are filled with 0xFF bytes, a NaN in
every format the kernels write there (bf16 y and h, e4m3 h, UE8M0 and fp32 scales), and the
dynamic walk runs first: a tile that a walk skipped would leave NaN rows behind, which reach
the output through the finalize, so each output is also checked to hold no NaN. (That every
tile is taken exactly once is shown on the CPU for the walk code itself,
tests/test_walk_model.py.)

The MXFP4 gate_up of the static walk with at least 3 K stages runs its copy ring on across
tiles (the next tile decoded from LDS two stages before the end, the previous tile's epilogue
inside the next tile's first stage); the dynamic walk runs tile by tile. Their equality pins
that form, down to its smallest K (hidden 512: 4 stages) and its 256-column tiles (2I not a
multiple of 512)."""

import time

import numpy as np
import pytest
import torch

from gpu_util import bits16, dev, say
from sgl_asap_amd import workloads as W
from sgl_asap_amd.moe.experts import AfdExperts, pack_fp8_block_experts, pack_mxfp4_experts
from sgl_asap_amd.moe.topk import StandardTopKOutput
from sgl_asap_amd.transport import hip

pytestmark = pytest.mark.gpu

PACK = {"mxfp4": pack_mxfp4_experts, "fp8_block": pack_fp8_block_experts}


def layer(fmt, hidden, inter, num_local, n_max, seed=0):
    """fmt: a weight format, with "_a16" for bf16 activations."""
    gen = W.generator("cpu", seed)
    w13, w2 = W.expert_weights(num_local, hidden, inter, gen, "cpu")
    act = "bf16" if fmt.endswith("_a16") else None
    pack = PACK[fmt.replace("_a16", "")]
    return AfdExperts(num_local, 8, 0, range(0, num_local), pack(w13, w2, device=dev()), n_max=n_max,
                      act_format=act)


def job(n, hidden, num_experts, seed, zipf=None):
    gen = W.generator("cpu", seed)
    x = W.tokens(n, hidden, gen, "cpu").to(dev())
    if zipf:
        ids, w = W.route_zipf(n, num_experts, 8, zipf, gen, "cpu")
    else:
        ids, w = W.route_uniform(n, num_experts, 8, gen, "cpu")
    return x, StandardTopKOutput(w.to(torch.float32).to(dev()), ids.to(torch.int32).to(dev()))


def bf16_values(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def poisoned_call(experts, x, topk):
    """The expert call with its workspace and its output filled with 0xFF bytes beforehand;
    fails if any output element is NaN."""
    experts.workspace().fill_(0xFF)
    out = torch.empty(x.shape[0], experts.hidden_size, dtype=torch.bfloat16, device=dev())
    out.view(torch.int16).fill_(-1)
    experts(x, topk, out=out)
    torch.cuda.synchronize()
    got = bits16(out)
    assert not np.isnan(bf16_values(got)).any(), f"the {experts.tile_walk} walk left NaN rows (a skipped tile)"
    return got


def both(experts, x, topk):
    """(static, dynamic) outputs, each from a poisoned workspace; the dynamic walk runs first."""
    outs = {}
    for walk in ("dynamic", "static"):
        experts.tile_walk = walk
        outs[walk] = poisoned_call(experts, x, topk)
    return outs["static"], outs["dynamic"]


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block", "mxfp4_a16", "fp8_block_a16"])
def test_walks_agree(fmt):
    experts = layer(fmt, 1024, 512, 32, 4096)
    for n, seed, zipf in ((1, 1, None), (7, 2, None), (300, 3, None), (4096, 4, None), (3000, 5, 1.2)):
        say(f"walks fmt={fmt} n={n} zipf={zipf}")
        x, topk = job(n, 1024, 32, seed, zipf)
        s, d = both(experts, x, topk)
        assert np.array_equal(s, d), (fmt, n, seed)


@pytest.mark.parametrize("hidden,inter", [(512, 384), (256, 128), (768, 256), (1536, 640)])
def test_walks_agree_across_shapes(hidden, inter):
    experts = layer("mxfp4", hidden, inter, 16, 2048, seed=hidden)
    for n, seed, zipf in ((5, 11, None), (700, 12, None), (2048, 13, 1.2)):
        say(f"walks mxfp4 H={hidden} I={inter} n={n} zipf={zipf}")
        x, topk = job(n, hidden, 16, seed, zipf)
        s, d = both(experts, x, topk)
        assert np.array_equal(s, d), (hidden, inter, n, seed)


def test_dynamic_walk_with_a_parked_wait():
    say("walks: a parked stream wait holds a CU during dynamic and static calls")
    experts = layer("mxfp4", 1024, 512, 32, 4096)
    x, topk = job(4096, 1024, 32, 9)
    ref = both(experts, x, topk)[0]
    page = hip.HostPage(4096)
    other = torch.cuda.Stream()
    try:
        for walk in ("dynamic", "static"):
            experts.tile_walk = walk
            page.store(0, 0)
            other.wait_stream(torch.cuda.current_stream())
            hip.wait64(other.cuda_stream, page.addr(0), 1)  # parked until the host stores 1
            out = experts(x, topk)
            done = torch.cuda.Event()
            done.record()
            # the call normally finishes while the wait is parked; the host releases the wait
            # after at most 10 s in any case (were the two streams on one hardware queue, the
            # call would queue behind the wait), so nothing can hang
            deadline = time.monotonic() + 10.0
            while not done.query() and time.monotonic() < deadline:
                time.sleep(0.001)
            page.store(0, 1)
            torch.cuda.synchronize()
            assert np.array_equal(bits16(out), ref), walk
    finally:
        page.store(0, 1)
        torch.cuda.synchronize()
        page.release()
