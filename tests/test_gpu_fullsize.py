"""GPU: the full-size layers (one F rank of DeepSeek-V4-Flash shape, 16384 tokens, MXFP4; the
ERNIE-style FP8 block layer, Zipf(1.1) routing) checked through properties that do not need
the oracle to run the whole job:

* rows: every token's output depends on its own row, ids and weights only, so a subset of
  the job, or the job with its tokens permuted, gives the same rows bit for bit (this pins
  the routing, padding and tile walk at full size);
* weights: doubling w doubles every output exactly (products, fp32 sums and the bf16
  rounding all scale by 2);
* the job read from a device descriptor equals the by-value call;
and tokens of a few experts against the oracle on the dequantized weights (rel-L2 1e-2):
for the MXFP4 layer the tokens of 4 of its experts, for the FP8 block layer (every expert
local, 8 per token) the tokens whose 8 experts are all among its 16 most used; both again
with each model family's own activation (DeepSeek-V4: SwiGLU with a limit; ERNIE: SiTU)."""

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from gpu_util import bits16, dev, rel_l2, say
from oracle import experts as OX
from oracle import formats as F
from sgl_asap_amd import workloads as W
from sgl_asap_amd.moe.experts import AfdExperts, new_job_desc, pack_fp8_block_experts, pack_mxfp4_experts, set_job, release_workspaces
from sgl_asap_amd.moe.topk import StandardTopKOutput

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=["dsv4_rank", "ernie_fp8"])
def layer(request):
    shape = W.SHAPES[request.param]
    say(f"full-size layer {shape.name}: packing weights")
    gen = W.generator("cpu", 1)
    w13, w2 = W.expert_weights(shape.num_local, shape.hidden, shape.inter, gen, "cpu")
    pack = pack_mxfp4_experts if shape.fmt == "mxfp4" else pack_fp8_block_experts
    experts = AfdExperts(shape.num_experts, shape.top_k, 0, shape.local, pack(w13, w2, device=dev()),
                         n_max=shape.tokens)
    x, ids, w = W.job(shape, seed=0, device="cpu")
    job = (x.to(dev()), ids.to(torch.int32).to(dev()), w.to(torch.float32).to(dev()))
    out = experts(job[0], StandardTopKOutput(job[2], job[1]))
    torch.cuda.synchronize()
    yield shape, experts, (w13, w2), (x, ids, w), job, out
    del experts
    release_workspaces()  # the shared per-stream workspaces of this size
    torch.cuda.empty_cache()


def call(experts, x, ids, w):
    out = experts(x.contiguous(), StandardTopKOutput(w.contiguous(), ids.contiguous()))
    torch.cuda.synchronize()
    return out


def test_subset_and_permutation_rows(layer):
    shape, experts, _, _, (x, ids, w), out = layer
    say(f"{shape.name}: subset and permutation rows")
    full = bits16(out)
    g = torch.Generator().manual_seed(5)
    sub = torch.randperm(shape.tokens, generator=g)[:3000].sort().values.to(dev())
    assert np.array_equal(bits16(call(experts, x[sub], ids[sub], w[sub])), full[sub.cpu().numpy()])
    perm = torch.randperm(shape.tokens, generator=g).to(dev())
    assert np.array_equal(bits16(call(experts, x[perm], ids[perm], w[perm])), full[perm.cpu().numpy()])


def test_doubling_weights_doubles_output(layer):
    shape, experts, _, _, (x, ids, w), out = layer
    say(f"{shape.name}: output linear in the top-k weights")
    twice = call(experts, x, ids, 2 * w)
    assert np.array_equal(bits16(twice), bits16(out * 2))


def test_descriptor_call_equals_by_value(layer):
    shape, experts, _, _, (x, ids, w), out = layer
    say(f"{shape.name}: job descriptor at full size")
    desc = new_job_desc(dev())
    got = torch.empty_like(out)
    set_job(desc, x=x, ids=ids, w=w, out=got)
    experts.call_job(desc, shape.tokens)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(got), bits16(out))


def test_subset_against_oracle(layer):
    """Tokens whose local experts all lie in [e_lo, e_lo + 4) (plus tokens with no local
    expert), against the oracle run with those 4 experts only: the oracle's weight
    quantization of all 64 experts would take minutes on the CPU."""
    shape, experts, (w13, w2), (xc, idsc, wc), _, out = layer
    subset_against_oracle(shape, (w13, w2), (xc, idsc, wc), out)


# the activation each model family runs its experts with: DeepSeek-V4's FusedMoE passes its
# swiglu_limit (P/srt/models/deepseek_v4.py:63), ERNIE 5.5's SiTU (P/srt/models/ernie55.py:43-55);
# the limit is lower than a model's so that it clamps a good share of these synthetic gate and
# up values (N(0, ~1.3)), not only their far tails
MODEL_ACTIVATION = {
    "dsv4_rank": (dict(swiglu_limit=1.5), dict(activation="swiglu_limit", act_limit=1.5)),
    "ernie_fp8": (dict(activation="situ", gemm1_alpha=1.702, gemm1_clamp_limit=7.0),
                  dict(activation="situ", act_alpha=1.702, act_limit=7.0)),
}


def test_subset_against_oracle_with_model_activation(layer):
    """The same full-size job through the same packed weights with the model family's own
    activation (the gate_up kernels' constant-taking form), against the oracle subset."""
    shape, experts, (w13, w2), (xc, idsc, wc), job, _ = layer
    kw, oact = MODEL_ACTIVATION[shape.name]
    say(f"{shape.name}: full-size job with {kw}")
    act_experts = AfdExperts(shape.num_experts, shape.top_k, 0, shape.local, experts.weights,
                             n_max=shape.tokens, **kw)
    out = call(act_experts, *job)
    assert not torch.equal(out, layer[5])  # the activation took effect
    subset_against_oracle(shape, (w13, w2), (xc, idsc, wc), out, oact)


def subset_against_oracle(shape, weights, job, out, oact=None):
    w13, w2 = weights
    xc, idsc, wc = job
    oact = oact or {}
    if shape.fmt != "mxfp4":
        return fp8_subset_against_oracle(shape, (w13, w2), (xc, idsc, wc), out, oact=oact)
    say(f"{shape.name}: tokens of 4 experts against the oracle")
    lo, keep = shape.local.start, 4
    ids = idsc.numpy()
    rel = ids - lo
    local = (rel >= 0) & (rel < len(shape.local))
    only_kept = ~(local & (rel >= keep)).any(axis=1)
    has_kept = (local & (rel < keep)).any(axis=1)
    sub = np.concatenate([np.nonzero(only_kept & has_kept)[0][:448], np.nonzero(only_kept & ~has_kept)[0][:64]])
    assert len(sub) >= 256
    c13, s13 = F.mx_quantize(w13[:keep].numpy(), "e2m1")
    c2, s2 = F.mx_quantize(w2[:keep].numpy(), "e2m1")
    ref = OX.moe_ffn(xc[sub], ids[sub].astype(np.int32), wc.numpy()[sub].astype(np.float32),
                     F.mx_dequantize(c13, s13, "e2m1"), F.mx_dequantize(c2, s2, "e2m1"), lo, act="mxfp8", **oact)
    got = bits16(out)[sub]
    err = rel_l2(F.bf16_to_f32(got), F.bf16_to_f32(ref))
    say(f"  {len(sub)} tokens, rel_l2 = {err:.2e}")
    assert err <= 1e-2
    assert not got[~has_kept[sub]].any()  # tokens with no local expert are exactly 0


def fp8_subset_against_oracle(shape, weights, job, out, keep=16, oact=None):
    """The FP8 block layer has every expert local and 8 per token, so no token stays within
    4 experts: take the tokens whose 8 experts are all among the ``keep`` most used, renumber
    those experts 0..keep-1 (a token's result does not depend on the numbering: its pairs,
    their k order and the finalize sum are unchanged) and run the oracle with them only,
    quantizing the experts on a thread pool."""
    w13, w2 = weights
    xc, idsc, wc = job
    lo = shape.local.start
    rel = idsc.numpy() - lo
    counts = np.bincount(rel.ravel(), minlength=len(shape.local))
    chosen = np.argsort(-counts, kind="stable")[:keep]
    table = np.full(len(shape.local), -1, dtype=np.int64)
    table[chosen] = np.arange(keep)
    sub = np.nonzero((table[rel] >= 0).all(axis=1))[0][:256]
    say(f"{shape.name}: {len(sub)} tokens of the {keep} most used experts against the oracle")
    assert len(sub) >= 128

    def deq(e):
        c13, s13 = F.fp8_block_quantize_2d(w13[e:e + 1].numpy())
        c2, s2 = F.fp8_block_quantize_2d(w2[e:e + 1].numpy())
        return F.fp8_block_dequantize_2d(c13, s13)[0], F.fp8_block_dequantize_2d(c2, s2)[0]

    with ThreadPoolExecutor(8) as pool:
        parts = list(pool.map(deq, chosen.tolist()))
    w13d = np.stack([p[0] for p in parts])
    w2d = np.stack([p[1] for p in parts])
    ids = table[rel[sub]].astype(np.int32)
    ref = OX.moe_ffn(xc[sub], ids, wc.numpy()[sub].astype(np.float32), w13d, w2d, 0, act="fp8_1x128", **(oact or {}))
    err = rel_l2(F.bf16_to_f32(bits16(out)[sub]), F.bf16_to_f32(ref))
    say(f"  {len(sub)} tokens, rel_l2 = {err:.2e}")
    assert err <= 1e-2


def test_largest_job_rows_match_a_subset():
    """131071 tokens (the most a doorbell announces; token rows addressed with 32-bit byte
    offsets up to 2^29): the rows of a 2000-token subset equal the full job's bit for bit."""
    shape = W.SHAPES["dsv4_rank"]
    n = 131071
    say(f"largest job: {n} tokens, {shape.name} shape")
    gen = W.generator("cpu", 2)
    w13, w2 = W.expert_weights(shape.num_local, shape.hidden, shape.inter, gen, "cpu")
    experts = AfdExperts(shape.num_experts, shape.top_k, 0, shape.local, pack_mxfp4_experts(w13, w2, device=dev()),
                         n_max=n)
    del w13, w2
    x, ids, w = W.job(shape, n=n, seed=3, device=dev())
    ids, w = ids.to(torch.int32), w.to(torch.float32)
    full = bits16(call(experts, x, ids, w))
    sub = torch.cat([torch.arange(0, 1000), torch.arange(n - 1000, n)]).to(dev())
    assert np.array_equal(bits16(call(experts, x[sub], ids[sub], w[sub])), full[sub.cpu().numpy()])
    del experts
    release_workspaces()  # the shared per-stream workspaces of this size
    torch.cuda.empty_cache()
