"""GPU: the one-GPU AFD loop at its benchmark workload: two micro-batches of 8192 tokens
(DeepSeek-V4-Flash F-rank shape: hidden 4096, moe_intermediate 2048, 64 of 256 experts local,
top-8, Zipf(1.2) routing, MXFP4 weights), MXFP8 activations inside the expert call, bf16 or
MXFP8 activations on the wire, and a bf16 shared expert with intermediate 1536 on the
attention side.

Per micro-batch and wire format:
* the routed partial sum that landed in A's result segment equals the direct expert call on
  the same job, bit for bit;
* the layer output equals the oracle's combine of that partial sum and the shared expert's
  output, bit for bit;
* the shared expert's output is within rel-L2 1e-2 of the oracle's dense SwiGLU on a token
  subset;
* the routed partial sum is within rel-L2 1e-2 of the oracle's expert call on the tokens whose
  local experts all lie among the job's 4 most used local experts (the most used included);
  tokens without a local expert are exactly 0."""

import numpy as np
import pytest
import torch

from gpu_util import bits16, dev, rel_l2, say
from oracle import experts as OX
from oracle import formats as F
from sgl_asap_amd import workloads as W
from sgl_asap_amd.loop import OneGpuAfd
from sgl_asap_amd.moe.experts import AfdExperts, pack_mxfp4_experts, release_workspaces
from sgl_asap_amd.moe.layer import AsapMoE
from sgl_asap_amd.moe.shared import SharedExpertMLP
from sgl_asap_amd.moe.topk import StandardTopKOutput

pytestmark = pytest.mark.gpu

SHAPE = W.SHAPES["dsv4_zipf"]
N, SHARED_I = 8192, 1536


def subset_against_oracle(w13, w2, x, ids, w, got_bits, keep=4, limit=384):
    """Tokens whose local experts are all among the job's ``keep`` most used local experts
    (spread over the whole job) plus 64 tokens with no local expert, against the oracle run
    with those experts only (renumbered 0..keep-1: a token's pairs, their k order and the
    finalize sum do not depend on the numbering)."""
    lo, nl = SHAPE.local.start, SHAPE.num_local
    rel = ids.numpy().astype(np.int64) - lo
    local = (rel >= 0) & (rel < nl)
    counts = np.bincount(rel[local], minlength=nl)
    chosen = np.argsort(-counts, kind="stable")[:keep]
    table = np.full(nl, -1, dtype=np.int64)
    table[chosen] = np.arange(keep)
    inside = ~(local & (table[np.where(local, rel, 0)] < 0)).any(axis=1)
    has = local.any(axis=1)
    cand = np.nonzero(inside & has)[0]
    assert len(cand) >= 128, len(cand)
    pick = cand[np.linspace(0, len(cand) - 1, min(limit, len(cand))).astype(np.int64)]
    none = np.nonzero(~has)[0][:64]
    sub = np.concatenate([pick, none])
    c13, s13 = F.mx_quantize(w13[torch.from_numpy(chosen)].numpy(), "e2m1")
    c2, s2 = F.mx_quantize(w2[torch.from_numpy(chosen)].numpy(), "e2m1")
    sub_ids = np.where(local[sub], table[np.where(local[sub], rel[sub], 0)], -1).astype(np.int32)
    ref = OX.moe_ffn(x[torch.from_numpy(sub)], sub_ids, w.numpy()[sub].astype(np.float32),
                     F.mx_dequantize(c13, s13, "e2m1"), F.mx_dequantize(c2, s2, "e2m1"), 0, act="mxfp8")
    got = got_bits[sub]
    err = rel_l2(F.bf16_to_f32(got[: len(pick)]), F.bf16_to_f32(ref[: len(pick)]))
    say(f"  {len(pick)} tokens of experts {chosen.tolist()} (counts {counts[chosen].tolist()}), rel_l2 = {err:.2e}")
    assert err <= 1e-2
    assert not got[len(pick):].any()


@pytest.fixture(scope="module")
def workload():
    say("C5 loop workload: packing 64 MXFP4 experts (hidden 4096, inter 2048)")
    gen = W.generator(dev(), 7)
    w13, w2 = W.expert_weights(SHAPE.num_local, SHAPE.hidden, SHAPE.inter, gen, dev())
    experts = {0: AfdExperts(SHAPE.num_experts, SHAPE.top_k, 0, SHAPE.local, pack_mxfp4_experts(w13, w2), n_max=N)}
    w13, w2 = w13.cpu(), w2.cpu()
    shared = SharedExpertMLP.random(SHAPE.hidden, SHARED_I, W.generator(dev(), 8), dev())
    mbs = []
    for m in range(2):
        x, ids, w = W.job(SHAPE, n=N, seed=400 + m, device="cpu")
        mbs.append((x, ids.to(torch.int32), w.to(torch.float32)))
    torch.cuda.synchronize()
    yield experts, (w13, w2), shared, mbs
    del experts
    release_workspaces()  # the shared per-stream workspaces of this size
    torch.cuda.empty_cache()


@pytest.mark.parametrize("act", ["bf16", "mxfp8"])
def test_loop_two_micro_batches_with_shared_expert(workload, act):
    experts, (w13, w2), shared, mbs = workload
    say(f"C5 loop: 2 x {N} tokens, wire {act}, shared expert I={SHARED_I}")
    seen = []

    def recording_shared(x):
        out = shared(x)
        seen.append(out)
        return out

    inputs = [(x.to(dev()), StandardTopKOutput(w.to(dev()), ids.to(dev()))) for x, ids, w in mbs]
    with OneGpuAfd(experts, n_max=N, slots=2, graph_max_tokens=N, act=act) as afd:
        layer = AsapMoE(SHAPE.num_experts, SHAPE.hidden, SHAPE.inter, 0, top_k=SHAPE.top_k)
        outs = [None, None]
        # both micro-batches in flight before either combine, as two-batch overlap runs them
        sent = [layer.dispatcher.dispatch(x, t, micro_batch=m) for m, (x, t) in enumerate(inputs)]
        afd.scheduler.serve_pending()
        for m, (x, _) in enumerate(inputs):
            outs[m] = layer.dispatcher.combine(sent[m], recording_shared(x))
        torch.cuda.synchronize()
        routed = []
        for m in range(2):
            routed.append(bits16(afd.channel.result_view(0, m, N)))
        assert afd.server.stats["jobs"] == 2 and afd.server.stats["lost_messages"] == 0
    for m, (x, ids, w) in enumerate(mbs):
        direct = experts[0](inputs[m][0], inputs[m][1])
        torch.cuda.synchronize()
        assert np.array_equal(routed[m], bits16(direct)), m
        assert np.array_equal(bits16(outs[m]), OX.combine([routed[m]], bits16(seen[m]))), m
        if act == "bf16":  # the same experts and shared weights serve both wire formats
            rows = torch.arange(0, N, 37)
            ref = OX.shared_mlp(x[rows], shared.w_gate.cpu(), shared.w_up.cpu(), shared.w_down.cpu())
            err = rel_l2(F.bf16_to_f32(bits16(seen[m][rows.to(dev())])), F.bf16_to_f32(bits16(ref)))
            say(f"  micro-batch {m}: shared expert rel_l2 = {err:.2e}")
            assert err <= 1e-2
            subset_against_oracle(w13, w2, x, ids, w, routed[m])
