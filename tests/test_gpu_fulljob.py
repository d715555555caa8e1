"""GPU: whole full-size jobs against the fp32 CPU oracle, every token.

The full-size layers of DeepSeek-V4-Flash's F rank (16384 tokens, 64 local of 256 experts,
top-8, MXFP4 weights, MXFP8 activations) and of the ERNIE-style FP8-block layer (16384
tokens, 64 experts all local, top-8 under Zipf(1.1) routing, FP8 1x128 activations), each
job through the expert call and through the oracle, all 16384 tokens compared (rel-L2 <=
1e-2, tokens with no local expert exactly zero): with SwiGLU, with the model family's own
activation (SwiGLU limited to 1.5; SiTU) and with bf16 activations. The weights are drawn so
that the format holds them exactly (``test_gpu_large.exact_weights``), so the oracle takes
them as drawn and no CPU weight quantization is needed.
"""

import time

import pytest
import torch

from gpu_util import dev, say
from oracle import experts as OX
from sgl_asap_amd import workloads as W
from sgl_asap_amd.moe.experts import AfdExperts
from sgl_asap_amd.moe.topk import StandardTopKOutput
from test_gpu_fullsize import MODEL_ACTIVATION
from test_gpu_large import exact_weights, oracle_act, packed
from test_gpu_moe import assert_close

pytestmark = pytest.mark.gpu

CASES = [  # shape, activation format (None: the weight format's fp8 form), activation
    ("dsv4_rank", None, "swiglu"),
    ("dsv4_rank", None, "model"),
    ("dsv4_rank", "bf16", "swiglu"),
    ("ernie_fp8", None, "swiglu"),
    ("ernie_fp8", None, "model"),
    ("ernie_fp8", "bf16", "swiglu"),
]


@pytest.fixture(scope="module")
def layers():
    """name -> (shape, packed weights, host weights, job); one shape held at a time."""
    held = {}

    def get(name):
        if name not in held:
            held.clear()
            shape = W.SHAPES[name]
            w13, w2 = exact_weights(shape.fmt, shape.num_local, shape.hidden, shape.inter, seed=81, device=dev())
            weights = packed(shape.fmt, w13, w2)
            host = (w13.cpu().numpy(), w2.cpu().numpy())
            del w13, w2
            x, ids, w = W.job(shape, seed=82, device="cpu")
            held[name] = (shape, weights, host, (x, ids.to(torch.int32), w.to(torch.float32)))
        return held[name]

    yield get
    held.clear()


@pytest.mark.parametrize("name,act_format,act", CASES)
def test_whole_job_against_the_oracle(layers, name, act_format, act):
    shape, weights, (w13, w2), (x, ids, w) = layers(name)
    kw, oact = MODEL_ACTIVATION[name] if act == "model" else ({}, {})
    say(f"{name}: {shape.tokens} tokens, {shape.fmt}, act_format={act_format} {kw}, every token against the oracle")
    experts = AfdExperts(shape.num_experts, shape.top_k, 0, shape.local, weights, n_max=shape.tokens,
                         act_format=act_format, **kw)
    out = experts(x.to(dev()), StandardTopKOutput(w.to(dev()), ids.to(dev())))
    torch.cuda.synchronize()
    del experts
    t0 = time.time()
    ref = OX.moe_ffn(x, ids.numpy(), w.numpy(), w13, w2, shape.local.start,
                     act=oracle_act(shape.fmt, act_format), **oact)
    say(f"  oracle {time.time() - t0:.1f} s")
    assert_close(out, ref, ids.numpy(), shape.local)
