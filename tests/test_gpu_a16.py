"""GPU parity of the expert call with bf16 activations (W4A16: MXFP4 weights; W8A16: FP8
128x128-block weights; the activations kept bf16, h rounded to bf16) against the fp32 CPU
oracle run with ``act="bf16"`` on the dequantized weights.

Bars: routing bit-exact (the same router as the fp8 path); the output within rel-L2 <= 1e-2 of
the oracle (the weight expansion is exact, so the remaining difference is fp32 summation order
and the bf16 rounding of h and y at different sums); tokens with no local expert exactly 0;
the h images decoded from the workspace within the same bar of the oracle's h. At the
DeepSeek-V4 F-rank size (16384 tokens, MXFP4) and the ERNIE-style FP8-block size (16384
tokens, Zipf(1.1)): tokens of a few experts against the oracle, and the size-independent
properties of the fp8 path's full-size test (subset and permutation rows, doubling the
weights, the descriptor call, the static and dynamic walks bit-identical). Batched,
answering and descriptor calls are bit-identical to the plain call.
"""

import ctypes
import random

import numpy as np
import pytest
import torch

from gpu_util import bits16, dev, rel_l2, say
from oracle import experts as OX
from oracle import formats as F
from sgl_asap_amd import workloads as W
from sgl_asap_amd.moe.experts import (AfdExperts, new_job_desc, pack_fp8_block_experts, pack_mxfp4_experts,
                                      release_workspaces, set_job)
from sgl_asap_amd.moe.topk import StandardTopKOutput

pytestmark = pytest.mark.gpu

REL_L2_TOL = 1e-2


PACK = {"mxfp4": pack_mxfp4_experts, "fp8_block": pack_fp8_block_experts}


def mx_deq(w13, w2):
    c13, s13 = F.mx_quantize(w13.numpy(), "e2m1")
    c2, s2 = F.mx_quantize(w2.numpy(), "e2m1")
    return F.mx_dequantize(c13, s13, "e2m1"), F.mx_dequantize(c2, s2, "e2m1")


def fp8_deq(w13, w2):
    c13, s13 = F.fp8_block_quantize_2d(w13.numpy())
    c2, s2 = F.fp8_block_quantize_2d(w2.numpy())
    return F.fp8_block_dequantize_2d(c13, s13), F.fp8_block_dequantize_2d(c2, s2)


DEQ = {"mxfp4": mx_deq, "fp8_block": fp8_deq}


def run_case(hidden, inter, num_experts, e_lo, num_local, k, n, seed, zipf=None, situ=None,
             swiglu_limit=None, tile_walk="static", fmt="mxfp4"):
    say(f"a16 fmt={fmt} H={hidden} I={inter} E={num_experts} local=[{e_lo},{e_lo + num_local}) k={k} n={n} "
        f"seed={seed} zipf={zipf} situ={situ} swiglu_limit={swiglu_limit} walk={tile_walk}")
    gen = W.generator("cpu", seed)
    x = W.tokens(n, hidden, gen, "cpu")
    if zipf is None:
        ids, w = W.route_uniform(n, num_experts, k, gen, "cpu")
    else:
        ids, w = W.route_zipf(n, num_experts, k, zipf, gen, "cpu")
    w13, w2 = W.expert_weights(num_local, hidden, inter, gen, "cpu")
    weights = PACK[fmt](w13, w2, device=dev())
    act_kw, oact = {}, {}
    if situ is not None:
        act_kw = dict(activation="situ", gemm1_alpha=situ[0], gemm1_clamp_limit=situ[1])
        oact = dict(activation="situ", act_alpha=situ[0], act_limit=situ[1])
    if swiglu_limit is not None:
        act_kw = dict(swiglu_limit=swiglu_limit)
        oact = dict(activation="swiglu_limit", act_limit=swiglu_limit)
    experts = AfdExperts(num_experts, k, 0, range(e_lo, e_lo + num_local), weights, n_max=max(n, 1),
                         act_format="bf16", tile_walk=tile_walk, **act_kw)
    assert experts.act_format == "bf16"
    out = experts(x.to(dev()), StandardTopKOutput(w.to(dev()), ids.to(dev())))
    torch.cuda.synchronize()
    w13d, w2d = DEQ[fmt](w13, w2)
    ref, parts = OX.moe_ffn(x, ids.numpy(), w.numpy(), w13d, w2d, e_lo, act="bf16", return_parts=True, **oact)
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


def h_from_images(experts, n, rows):
    """The gate_up GEMM's h rows in padded expert order, decoded from the workspace's bf16 A
    images. MXFP4: one 32 KiB image per (row tile, 128-wide K stage), row r at r * 256 B,
    logical 16-byte chunk c at physical chunk c ^ (r % 16). FP8 block: one 16 KiB image per
    (row tile, 64-wide K stage), row r at r * 128 B, chunk c at c ^ ((r ^ (r >> 3)) % 8)."""
    inter = experts.intermediate_size
    stage_k = 128 if experts.weights.fmt == "mxfp4" else 64
    stages, chunks = inter // stage_k, stage_k // 8
    tiles = (rows + 127) // 128
    raw = experts.ws_view("hq", torch.uint8, tiles * stages * 128 * stage_k * 2, n).cpu().numpy()
    img = raw.reshape(tiles, stages, 128, chunks, 16)  # [tile][stage][row][physical chunk][byte]
    r = np.arange(128)
    swz = (r & 15) if stage_k == 128 else ((r ^ (r >> 3)) & 7)
    physical = np.arange(chunks)[None, :] ^ swz[:, None]  # physical chunk of logical chunk c
    ordered = img[:, :, r[:, None], physical, :]  # [tile][stage][row][logical chunk][byte]
    h = ordered.transpose(0, 2, 1, 3, 4).reshape(tiles * 128, stages * stage_k * 2).view(np.uint16)
    return F.bf16_to_f32(h[:rows])


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
def test_tiny_layer_a16(fmt):
    """The tiny CPU-runnable layer (H256 I128, 8 experts, top-2, 64 tokens) with bf16
    activations: output and h against the oracle, routing bit-exact."""
    s = W.SHAPES["tiny"]
    experts, out, ref, parts, (x, ids, w) = run_case(s.hidden, s.inter, s.num_experts, 0, s.num_local, s.top_k,
                                                     s.tokens, seed=0, fmt=fmt)
    assert_close(out, ref, ids.numpy(), s.local)
    n, k = ids.shape
    pos = experts.ws_view("pair_pos", torch.int32, n * k, n).cpu().numpy()
    assert np.array_equal(pos, parts["route"]["pair_pos"])
    sp = parts["route"]["sorted_pairs"]
    real = sp >= 0
    h = h_from_images(experts, n, len(sp))
    err = rel_l2(h[real], parts["h"][real])
    say(f"h rel_l2={err:.3e}")
    assert err <= REL_L2_TOL


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
def test_a16_differs_from_fp8_activations(fmt):
    """The bf16 path is not the fp8 path under another name: the same layer with fp8
    activations gives different bits, and lies farther from the bf16 oracle."""
    s = W.SHAPES["tiny"]
    experts, out, ref, parts, (x, ids, w) = run_case(s.hidden, s.inter, s.num_experts, 0, s.num_local, s.top_k,
                                                     s.tokens, seed=1, fmt=fmt)
    fp8 = AfdExperts(s.num_experts, s.top_k, 0, s.local, experts.weights, n_max=s.tokens)
    out8 = fp8(x.to(dev()), StandardTopKOutput(w.to(dev()), ids.to(dev())))
    torch.cuda.synchronize()
    assert not np.array_equal(bits16(out), bits16(out8))
    want = F.bf16_to_f32(ref)
    assert rel_l2(F.bf16_to_f32(bits16(out)), want) < rel_l2(F.bf16_to_f32(bits16(out8)), want)


@pytest.mark.parametrize(
    "hidden,inter,num_experts,e_lo,num_local,k,n,seed",
    [
        (512, 256, 32, 8, 16, 4, 300, 1),      # down N = 512: 512-column tiles; gate_up N = 512
        (256, 128, 16, 0, 16, 8, 1, 2),        # one token; 256-column tiles in both GEMMs
        (1024, 512, 64, 16, 16, 6, 513, 3),
        (2048, 1024, 32, 0, 8, 8, 256, 4),
        (4096, 512, 256, 0, 4, 8, 64, 10),
        (768, 384, 16, 0, 16, 2, 129, 5),      # down N = 768 (256-column tiles), K stages 6 / 3
    ],
)
def test_a16_layers(hidden, inter, num_experts, e_lo, num_local, k, n, seed):
    experts, out, ref, parts, (x, ids, w) = run_case(hidden, inter, num_experts, e_lo, num_local, k, n, seed)
    assert_close(out, ref, ids.numpy(), range(e_lo, e_lo + num_local))


@pytest.mark.parametrize(
    "hidden,inter,num_experts,e_lo,num_local,k,n,seed,zipf",
    [
        (512, 256, 32, 8, 16, 4, 300, 51, None),     # 512-column tiles in both GEMMs
        (256, 128, 16, 0, 16, 8, 1, 52, None),       # one token; 256-column tiles
        (1024, 384, 16, 0, 16, 8, 700, 53, 1.1),     # K blocks 8 / 3, down N = 1024
        (768, 640, 8, 0, 8, 2, 129, 54, None),       # down N = 768: 256-column tiles; 10 K stages
        (4096, 1536, 64, 0, 4, 8, 96, 55, None),     # the ERNIE-style shape on 4 experts
    ],
)
def test_w8a16_layers(hidden, inter, num_experts, e_lo, num_local, k, n, seed, zipf):
    """FP8 128x128-block weights with bf16 activations (W8A16): the block scales change every
    two 64-wide K stages, applied to the fp32 sums."""
    experts, out, ref, parts, (x, ids, w) = run_case(hidden, inter, num_experts, e_lo, num_local, k, n, seed,
                                                     zipf=zipf, fmt="fp8_block")
    assert_close(out, ref, ids.numpy(), range(e_lo, e_lo + num_local))


def draw(case: int) -> dict:
    rng = random.Random(5100 + case)
    num_experts = rng.choice([8, 16, 32, 64])
    num_local = rng.randint(1, min(num_experts, 24))
    spec = dict(
        hidden=256 * rng.randint(1, 6),
        inter=128 * rng.randint(1, 6),
        num_experts=num_experts,
        num_local=num_local,
        e_lo=rng.randint(0, num_experts - num_local),
        k=rng.randint(1, min(8, num_experts)),
        n=rng.choice([1, 2, 31, 64, 127, 128, 129, 255, 300, 777]),
        zipf=rng.choice([None, 1.2]),
        tile_walk=rng.choice(["static", "dynamic"]),
        fmt=rng.choice(["mxfp4", "fp8_block"]),
    )
    act = rng.choice(["silu", "situ", "limit"])
    if act == "situ":
        spec["situ"] = (rng.choice([0.5, 2.0]), rng.choice([0.25, 3.0]))
    if act == "limit":
        spec["swiglu_limit"] = rng.choice([0.3, 1.0])
    return spec


@pytest.mark.parametrize("case", range(24))
def test_a16_random_layer(case):
    """Seeded random shapes: both weight formats, hidden 256-1536, inter 128-768 (both tile
    widths, 1-12 K stages), token counts around the 128-row tile edge, partial local ranges,
    top-1 to top-8, uniform and Zipf routing, the three activations, both tile walks."""
    s = draw(case)
    extra = {k: s[k] for k in ("situ", "swiglu_limit") if k in s}
    experts, out, ref, parts, (x, ids, w) = run_case(
        s["hidden"], s["inter"], s["num_experts"], s["e_lo"], s["num_local"], s["k"], s["n"], 9100 + case,
        zipf=s["zipf"], tile_walk=s["tile_walk"], fmt=s["fmt"], **extra)
    assert_close(out, ref, ids.numpy(), range(s["e_lo"], s["e_lo"] + s["num_local"]))


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8_block"])
def test_a16_walks_batch_answer_descriptor_identical(fmt):
    """Static and dynamic walks, a batched call (with an empty first job), the answering call
    and the descriptor call all give the plain call's bits."""
    experts, out, ref, parts, (x, ids, w) = run_case(1024, 512, 32, 0, 16, 8, 700, seed=41, zipf=1.2, fmt=fmt)
    xd, idsd, wd = x.to(dev()), ids.to(torch.int32).to(dev()), w.to(dev())
    base = bits16(out)
    experts.tile_walk = "dynamic"
    dyn = experts(xd, StandardTopKOutput(wd, idsd))
    experts.tile_walk = "static"
    cuts = [0, 0, 250, 251, 700]  # an empty first job, then 250, 1 and 449 tokens
    jobs = [(xd[a:b], StandardTopKOutput(wd[a:b], idsd[a:b])) for a, b in zip(cuts[:-1], cuts[1:])]
    outs = experts.forward_batch(jobs)
    done = torch.zeros(1, dtype=torch.int64, device=dev())
    ans = torch.empty_like(out)
    experts.call_ptrs(700, xd.data_ptr(), 0, idsd.data_ptr(), wd.data_ptr(), ans.data_ptr(),
                      torch.cuda.current_stream().cuda_stream, done_ptr=done.data_ptr(), done_value=7)
    desc = new_job_desc(dev())
    got = torch.empty_like(out)
    set_job(desc, x=xd, ids=idsd, w=wd, out=got)
    experts.call_job(desc, 700)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(dyn), base)
    assert np.array_equal(np.concatenate([bits16(o) for o in outs]), base)
    assert np.array_equal(bits16(ans), base) and int(done.item()) == 7
    assert np.array_equal(bits16(got), base)


def test_a16_has_no_quantized_form():
    s = W.SHAPES["tiny"]
    gen = W.generator("cpu", 3)
    w13, w2 = W.expert_weights(s.num_local, s.hidden, s.inter, gen, "cpu")
    experts = AfdExperts(s.num_experts, s.top_k, 0, s.local, pack_mxfp4_experts(w13, w2, device=dev()),
                         n_max=s.tokens, act_format="bf16")
    x = W.tokens(4, s.hidden, gen, "cpu").to(dev())
    with pytest.raises(NotImplementedError):
        experts.quant_act(x)
    q = torch.zeros(4, s.hidden, dtype=torch.uint8, device=dev())
    sc = torch.zeros(4, s.hidden // 32, dtype=torch.uint8, device=dev())
    ids = torch.zeros(4, s.top_k, dtype=torch.int32, device=dev())
    w = torch.ones(4, s.top_k, device=dev())
    ws = experts.workspace()
    out = torch.empty(4, s.hidden, dtype=torch.bfloat16, device=dev())
    from sgl_asap_amd import _lib
    st = _lib.lib().afd_moe_ffn_q(ctypes.byref(experts.cfg), ctypes.byref(experts._wstruct), q.data_ptr(),
                                  sc.data_ptr(), ids.data_ptr(), w.data_ptr(), 4, ws.data_ptr(), ws.numel(),
                                  out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert st == _lib.AFD_ERR_UNSUPPORTED


@pytest.fixture(scope="module", params=["dsv4_rank", "ernie_fp8"])
def dsv4_a16(request):
    shape = W.SHAPES[request.param]
    say(f"full-size bf16-activation layer {shape.name}: packing weights")
    gen = W.generator("cpu", 1)
    w13, w2 = W.expert_weights(shape.num_local, shape.hidden, shape.inter, gen, "cpu")
    experts = AfdExperts(shape.num_experts, shape.top_k, 0, shape.local, PACK[shape.fmt](w13, w2, device=dev()),
                         n_max=shape.tokens, act_format="bf16")
    x, ids, w = W.job(shape, seed=0, device="cpu")
    job = (x.to(dev()), ids.to(torch.int32).to(dev()), w.to(torch.float32).to(dev()))
    out = experts(job[0], StandardTopKOutput(job[2], job[1]))
    torch.cuda.synchronize()
    yield shape, experts, (w13, w2), (x, ids, w), job, out
    del experts
    release_workspaces()
    torch.cuda.empty_cache()


def call(experts, x, ids, w):
    out = experts(x.contiguous(), StandardTopKOutput(w.contiguous(), ids.contiguous()))
    torch.cuda.synchronize()
    return out


def test_dsv4_a16_properties(dsv4_a16):
    shape, experts, _, _, (x, ids, w), out = dsv4_a16
    say(f"{shape.name} W4A16: subset / permutation rows, doubled weights, descriptor, dynamic walk")
    full = bits16(out)
    g = torch.Generator().manual_seed(5)
    sub = torch.randperm(shape.tokens, generator=g)[:3000].sort().values.to(dev())
    assert np.array_equal(bits16(call(experts, x[sub], ids[sub], w[sub])), full[sub.cpu().numpy()])
    perm = torch.randperm(shape.tokens, generator=g).to(dev())
    assert np.array_equal(bits16(call(experts, x[perm], ids[perm], w[perm])), full[perm.cpu().numpy()])
    assert np.array_equal(bits16(call(experts, x, ids, 2 * w)), bits16(out * 2))
    desc = new_job_desc(dev())
    got = torch.empty_like(out)
    set_job(desc, x=x, ids=ids, w=w, out=got)
    experts.call_job(desc, shape.tokens)
    experts.tile_walk = "dynamic"
    dyn = call(experts, x, ids, w)
    experts.tile_walk = "static"
    assert np.array_equal(bits16(got), full)
    assert np.array_equal(bits16(dyn), full)


def test_dsv4_a16_subset_against_oracle(dsv4_a16):
    """MXFP4: tokens whose local experts all lie in [0, 4) (plus tokens with no local expert)
    against the oracle run with those 4 experts only. FP8 blocks (every expert local, 8 per
    token): the tokens whose 8 experts are all among the 16 most used, those experts renumbered
    for the oracle (a token's result does not depend on the numbering)."""
    shape, experts, (w13, w2), (xc, idsc, wc), _, out = dsv4_a16
    a16_subset_against_oracle(shape, (w13, w2), (xc, idsc, wc), out)


# each model family's activation (DeepSeek-V4's swiglu_limit, P/srt/models/deepseek_v4.py:63, set
# low enough to clamp many of these synthetic values; ERNIE 5.5's SiTU, P/srt/models/ernie55.py:43-55)
MODEL_ACTIVATION = {
    "dsv4_rank": (dict(swiglu_limit=1.5), dict(activation="swiglu_limit", act_limit=1.5)),
    "ernie_fp8": (dict(activation="situ", gemm1_alpha=1.702, gemm1_clamp_limit=7.0),
                  dict(activation="situ", act_alpha=1.702, act_limit=7.0)),
}


def test_a16_full_size_with_model_activation(dsv4_a16):
    """The full-size job with bf16 activations and the model family's own activation, through
    the same packed weights, against the oracle subset."""
    shape, experts, (w13, w2), (xc, idsc, wc), job, base = dsv4_a16
    kw, oact = MODEL_ACTIVATION[shape.name]
    say(f"{shape.name} bf16 activations, full size, {kw}")
    act_experts = AfdExperts(shape.num_experts, shape.top_k, 0, shape.local, experts.weights,
                             n_max=shape.tokens, act_format="bf16", **kw)
    out = call(act_experts, *job)
    assert not torch.equal(out, base)  # the activation took effect
    a16_subset_against_oracle(shape, (w13, w2), (xc, idsc, wc), out, oact)


def a16_subset_against_oracle(shape, weights, job, out, oact=None):
    w13, w2 = weights
    xc, idsc, wc = job
    oact = oact or {}
    if shape.fmt != "mxfp4":
        return fp8_subset_against_oracle(shape, (w13, w2), (xc, idsc, wc), out, oact=oact)
    say(f"{shape.name} W4A16: tokens of 4 experts against the oracle")
    lo, keep = shape.local.start, 4
    ids = idsc.numpy()
    rel = ids - lo
    local = (rel >= 0) & (rel < len(shape.local))
    only_kept = ~(local & (rel >= keep)).any(axis=1)
    has_kept = (local & (rel < keep)).any(axis=1)
    sub = np.concatenate([np.nonzero(only_kept & has_kept)[0][:448], np.nonzero(only_kept & ~has_kept)[0][:64]])
    assert len(sub) >= 256
    w13d, w2d = mx_deq(w13[:keep], w2[:keep])
    ref = OX.moe_ffn(xc[sub], ids[sub].astype(np.int32), wc.numpy()[sub].astype(np.float32), w13d, w2d, lo,
                     act="bf16", **oact)
    got = bits16(out)[sub]
    err = rel_l2(F.bf16_to_f32(got), F.bf16_to_f32(ref))
    say(f"  {len(sub)} tokens, rel_l2 = {err:.2e}")
    assert err <= REL_L2_TOL
    assert not got[~has_kept[sub]].any()


def fp8_subset_against_oracle(shape, weights, job, out, keep=16, oact=None):
    w13, w2 = weights
    xc, idsc, wc = job
    rel = idsc.numpy() - shape.local.start
    counts = np.bincount(rel.ravel(), minlength=len(shape.local))
    chosen = np.argsort(-counts, kind="stable")[:keep]
    table = np.full(len(shape.local), -1, dtype=np.int64)
    table[chosen] = np.arange(keep)
    sub = np.nonzero((table[rel] >= 0).all(axis=1))[0][:256]
    say(f"{shape.name} W8A16: {len(sub)} tokens of the {keep} most used experts against the oracle")
    assert len(sub) >= 128
    w13d, w2d = fp8_deq(w13[chosen], w2[chosen])
    ids = table[rel[sub]].astype(np.int32)
    ref = OX.moe_ffn(xc[sub], ids, wc.numpy()[sub].astype(np.float32), w13d, w2d, 0, act="bf16", **(oact or {}))
    err = rel_l2(F.bf16_to_f32(bits16(out)[sub]), F.bf16_to_f32(ref))
    say(f"  {len(sub)} tokens, rel_l2 = {err:.2e}")
    assert err <= REL_L2_TOL
