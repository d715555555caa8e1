"""GPU parity of the whole expert call (afd_moe_ffn) against the fp32 CPU oracle.

Bars: routing and the activation quantization bit-exact; the output within rel-L2 <= 1e-2
of the oracle (the oracle applies the same quantizers at the same points, so the remaining
difference is fp32 summation order and the occasional quantization-boundary flip); tokens
with no local expert exactly zero.
"""

import numpy as np
import pytest
import torch

import layouts as L
from gpu_util import bits16, dev, rel_l2, say, u8
from oracle import experts as OX
from oracle import formats as F
from oracle import routing as R
from sgl_asap_amd import workloads as W
from sgl_asap_amd.moe.experts import AfdExperts, pack_fp8_block_experts, pack_mxfp4_experts
from sgl_asap_amd.moe.topk import StandardTopKOutput

pytestmark = pytest.mark.gpu

REL_L2_TOL = 1e-2


def deq_weights(w13, w2, fmt):
    """Dequantized logical weights as the oracle sees them."""
    if fmt == "mxfp4":
        c13, s13 = F.mx_quantize(w13.numpy(), "e2m1")
        c2, s2 = F.mx_quantize(w2.numpy(), "e2m1")
        return F.mx_dequantize(c13, s13, "e2m1"), F.mx_dequantize(c2, s2, "e2m1")
    c13, s13 = F.fp8_block_quantize_2d(w13.numpy())
    c2, s2 = F.fp8_block_quantize_2d(w2.numpy())
    return F.fp8_block_dequantize_2d(c13, s13), F.fp8_block_dequantize_2d(c2, s2)


def run_case(hidden, inter, num_experts, e_lo, num_local, k, n, fmt, seed, zipf=None, situ=None,
             swiglu_limit=None, walk="static", act_format=None):
    """situ: None for SwiGLU, else SiTU's (gemm1_alpha, gemm1_clamp_limit); swiglu_limit:
    SwiGLU with that limit (DeepSeek-V4's FusedMoE argument); walk: the GEMMs' tile walk;
    act_format: "bf16" for bf16 activations, None for the weight format's fp8 form."""
    say(f"moe fmt={fmt} H={hidden} I={inter} E={num_experts} local=[{e_lo},{e_lo + num_local}) k={k} n={n} seed={seed} situ={situ} swiglu_limit={swiglu_limit} walk={walk} act_format={act_format}")
    gen = W.generator("cpu", seed)
    x = W.tokens(n, hidden, gen, "cpu")
    if zipf is None:
        ids, w = W.route_uniform(n, num_experts, k, gen, "cpu")
    else:
        ids, w = W.route_zipf(n, num_experts, k, zipf, gen, "cpu")
    w13, w2 = W.expert_weights(num_local, hidden, inter, gen, "cpu")
    pack = pack_mxfp4_experts if fmt == "mxfp4" else pack_fp8_block_experts
    weights = pack(w13, w2, device=dev())
    local = range(e_lo, e_lo + num_local)
    act_kw = {} if situ is None else dict(activation="situ", gemm1_alpha=situ[0], gemm1_clamp_limit=situ[1])
    if swiglu_limit is not None:
        act_kw = dict(swiglu_limit=swiglu_limit)
    experts = AfdExperts(num_experts, k, 0, local, weights, n_max=max(n, 1), act_format=act_format, **act_kw)
    experts.tile_walk = walk
    out = experts(x.to(dev()), StandardTopKOutput(w.to(dev()), ids.to(dev())))
    torch.cuda.synchronize()
    w13d, w2d = deq_weights(w13, w2, fmt)
    act = "bf16" if act_format == "bf16" else "mxfp8" if fmt == "mxfp4" else "fp8_1x128"
    oact = {} if situ is None else dict(activation="situ", act_alpha=situ[0], act_limit=situ[1])
    if swiglu_limit is not None:
        oact = dict(activation="swiglu_limit", act_limit=swiglu_limit)
    ref, parts = OX.moe_ffn(x, ids.numpy(), w.numpy(), w13d, w2d, e_lo, act=act, return_parts=True, **oact)
    return experts, out, ref, parts, (x, ids, w)


def assert_close(out, ref, ids, local):
    got = F.bf16_to_f32(bits16(out))
    want = F.bf16_to_f32(ref)
    err = rel_l2(got, want)
    say(f"rel_l2={err:.3e}")
    assert err <= REL_L2_TOL, err
    none_local = ~((ids >= local.start) & (ids < local.stop)).any(axis=1)
    assert not got[none_local].any(), "tokens with no local expert must be exactly 0"
    return err


def test_tiny_layer_mxfp4():
    """The tiny CPU-runnable layer: H256 I128, 8 experts, top-2, 64 tokens."""
    s = W.SHAPES["tiny"]
    experts, out, ref, parts, (x, ids, w) = run_case(s.hidden, s.inter, s.num_experts, 0, s.num_local, s.top_k, s.tokens, "mxfp4", seed=0)
    assert_close(out, ref, ids.numpy(), s.local)
    # intermediates: the routing and the quantized token rows are bit-exact
    n, k = ids.shape
    pos = experts.ws_view("pair_pos", torch.int32, n * k, n).cpu().numpy()
    assert np.array_equal(pos, parts["route"]["pair_pos"])
    codes = u8(experts.ws_view("xq", torch.uint8, n * s.hidden, n)).reshape(n, s.hidden)
    scales = u8(experts.ws_view("xs", torch.uint8, n * s.hidden // 32, n)).reshape(n, -1, 4)
    q_ref, s_ref = F.mx_quantize(F.bf16_to_f32(bits16(x)), "e4m3")
    assert np.array_equal(codes, q_ref)
    # scales in stage order: within each 128-wide K stage, block j at byte (2 (j & 1) | j >> 1)
    assert np.array_equal(scales[..., L.SCALE_ORDER].reshape(n, -1), s_ref)


@pytest.mark.parametrize(
    "hidden,inter,num_experts,e_lo,num_local,k,n,seed",
    [
        (512, 256, 32, 8, 16, 4, 300, 1),
        (256, 128, 16, 0, 16, 8, 1, 2),
        (1024, 512, 64, 16, 16, 6, 513, 3),
        (2048, 1024, 32, 0, 8, 8, 256, 4),
        (4096, 512, 256, 0, 4, 8, 64, 10),
    ],
)
def test_mxfp4_layers(hidden, inter, num_experts, e_lo, num_local, k, n, seed):
    experts, out, ref, parts, (x, ids, w) = run_case(hidden, inter, num_experts, e_lo, num_local, k, n, "mxfp4", seed)
    assert_close(out, ref, ids.numpy(), range(e_lo, e_lo + num_local))


@pytest.mark.parametrize(
    "hidden,inter,num_experts,num_local,k,n,seed,zipf",
    [
        (512, 256, 8, 8, 2, 200, 5, None),
        (1024, 384, 16, 16, 8, 700, 6, 1.1),
    ],
)
def test_fp8_block_layers(hidden, inter, num_experts, num_local, k, n, seed, zipf):
    experts, out, ref, parts, (x, ids, w) = run_case(hidden, inter, num_experts, 0, num_local, k, n, "fp8_block", seed, zipf)
    assert_close(out, ref, ids.numpy(), range(0, num_local))


def test_no_local_pairs_is_zero():
    say("moe no local pairs")
    gen = W.generator("cpu", 9)
    x = W.tokens(40, 256, gen, "cpu")
    ids = torch.full((40, 2), 12, dtype=torch.int32)
    w = torch.ones(40, 2)
    w13, w2 = W.expert_weights(8, 256, 128, gen, "cpu")
    experts = AfdExperts(16, 2, 0, range(0, 8), pack_mxfp4_experts(w13, w2, device=dev()), n_max=64)
    out = experts(x.to(dev()), StandardTopKOutput(w.to(dev()), ids.to(dev())))
    torch.cuda.synchronize()
    assert not bits16(out).any()


def test_repeat_call_is_deterministic():
    say("moe determinism")
    experts, out, ref, parts, (x, ids, w) = run_case(512, 256, 32, 0, 32, 4, 333, "mxfp4", seed=11)
    again = experts(x.to(dev()), StandardTopKOutput(w.to(dev()), ids.to(dev())))
    torch.cuda.synchronize()
    assert np.array_equal(bits16(out), bits16(again))


@pytest.mark.parametrize(
    "fmt,alpha,limit,seed",
    [
        ("mxfp4", 2.0, 3.0, 21),
        ("mxfp4", 0.5, 0.25, 22),  # both tanh branches mostly saturated
        ("fp8_block", 2.0, 3.0, 23),
    ],
)
def test_situ_layers(fmt, alpha, limit, seed):
    """SiTU (ERNIE 5.5's activation) through both weight formats against the oracle."""
    experts, out, ref, parts, (x, ids, w) = run_case(
        1024, 512, 32, 0, 16, 8, 384, fmt, seed, situ=(alpha, limit)
    )
    assert_close(out, ref, ids.numpy(), range(0, 16))


@pytest.mark.parametrize(
    "fmt,limit,seed",
    [
        ("mxfp4", 0.5, 31),  # binds on a large share of the gate and up values
        ("mxfp4", 1.5, 32),  # binds on the tails
        ("fp8_block", 0.5, 33),
    ],
)
def test_swiglu_limit_layers(fmt, limit, seed):
    """SwiGLU with DeepSeek-V4's swiglu_limit through both weight formats against the oracle;
    the limit must change the output (the clamps bind)."""
    experts, out, ref, parts, (x, ids, w) = run_case(1024, 512, 32, 0, 16, 8, 384, fmt, seed, swiglu_limit=limit)
    assert_close(out, ref, ids.numpy(), range(0, 16))
    plain = AfdExperts(32, 8, 0, range(0, 16), experts.weights, n_max=384)
    base = plain(x.to(dev()), StandardTopKOutput(w.to(dev()), ids.to(dev())))
    torch.cuda.synchronize()
    assert not np.array_equal(bits16(base), bits16(out))
