"""GPU: fp8 activations on the wire. The attention side's quantizer (``quant_act`` over
afd_quant_act) is bit-exact with the oracle, the expert call on quantized rows
(afd_moe_ffn_q) equals the call on the bf16 rows bit for bit, and the one-GPU loop carrying
"mxfp8" / "fp8_1x128" activations returns exactly what the expert call returns."""

import numpy as np
import pytest
import torch

from gpu_util import bits16, dev, say, u8
from oracle import formats as F
from sgl_asap_amd import workloads as W
from sgl_asap_amd.loop import OneGpuAfd
from sgl_asap_amd.moe.experts import AfdExperts, pack_fp8_block_experts, pack_mxfp4_experts, quant_act
from sgl_asap_amd.moe.layer import AsapMoE
from sgl_asap_amd.moe.topk import StandardTopKOutput
from sgl_asap_amd.transport import hip

pytestmark = pytest.mark.gpu

H, I, E, K = 256, 128, 16, 4
LOCAL = range(0, 8)
WEIGHTS = {"mxfp8": pack_mxfp4_experts, "fp8_1x128": pack_fp8_block_experts}


def stage_order(s: np.ndarray) -> np.ndarray:
    """Natural MX block order -> the MX GEMM's: block j of each group of 4 at byte
    2(j & 1) | (j >> 1) of the group."""
    j = np.arange(s.shape[1])
    dest = (j & ~3) | (2 * (j & 1)) | ((j >> 1) & 1)
    out = np.empty_like(s)
    out[:, dest] = s
    return out


def bf16_rows(rows, cols, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g) * torch.logspace(-3, 3, cols)[None, :]
    x[0, :] = 0.0
    return x.to(torch.bfloat16)


def x_f32(x):
    return F.bf16_to_f32(x.contiguous().view(torch.int16).numpy().view(np.uint16))


def make_experts(act, n_max, layers=(0,), seed=0):
    gen = W.generator("cpu", seed)
    out = {}
    for layer in layers:
        w13, w2 = W.expert_weights(len(LOCAL), H, I, gen, "cpu")
        out[layer] = AfdExperts(E, K, layer, LOCAL, WEIGHTS[act](w13, w2, device=dev()), n_max=n_max)
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


@pytest.mark.parametrize("act", ["mxfp8", "fp8_1x128"])
@pytest.mark.parametrize("rows,cols", [(1, 256), (37, 512), (300, 4096)])
def test_quant_act_bitexact(act, rows, cols):
    say(f"quant_act {act} rows={rows} cols={cols}")
    x = bf16_rows(rows, cols, seed=rows + cols)
    q, s = quant_act(act, x.to(dev()))
    torch.cuda.synchronize()
    if act == "mxfp8":
        q_ref, s_ref = F.mx_quantize(x_f32(x), "e4m3")
        assert np.array_equal(u8(s), stage_order(s_ref))
    else:
        q_ref, s_ref = F.fp8_group_quantize(x_f32(x))
        assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(u8(q), q_ref)


@pytest.mark.parametrize("act", ["mxfp8", "fp8_1x128"])
def test_forward_q_equals_forward(act):
    say(f"forward_q == forward, {act}")
    experts = make_experts(act, 256)
    layer = experts[0]
    assert layer.act_format == act
    for n, seed in ((1, 1), (77, 2), (256, 3)):
        x, topk = job(n, seed)
        q, s = layer.quant_act(x)
        q2, s2 = quant_act(act, x)  # the attention side's quantizer, without the layer
        out_q = layer.forward_q(q, s, topk)
        torch.cuda.synchronize()
        assert np.array_equal(u8(q), u8(q2)) and np.array_equal(u8(s.view(torch.uint8)), u8(s2.view(torch.uint8)))
        assert np.array_equal(bits16(out_q), direct(experts, 0, x, topk)), n


@pytest.mark.parametrize("act", ["mxfp8", "fp8_1x128"])
@pytest.mark.parametrize("graphs", [0, 64])
def test_loop_fp8_on_the_wire(act, graphs):
    say(f"loop: {act} on the wire, graph_max_tokens={graphs}")
    experts = make_experts(act, 64, layers=(0, 1))
    with OneGpuAfd(experts, n_max=64, act=act, graph_max_tokens=graphs) as afd:
        assert afd.buffer.stage and afd.geometry.act == act
        layers = [AsapMoE(E, H, I, lid, top_k=K) for lid in (0, 1)]
        for i, n in enumerate((1, 17, 64, 40)):
            lid = i % 2
            x, topk = job(n, 50 + i)
            out = layers[lid](x, topk)
            torch.cuda.synchronize()
            assert np.array_equal(bits16(out), direct(experts, lid, x, topk)), (lid, n)
        assert afd.server.stats["jobs"] == 4 and afd.server.stats["lost_messages"] == 0


@pytest.mark.parametrize("act", ["mxfp8", "fp8_1x128"])
@pytest.mark.parametrize("graphs", [0, 64])
def test_grouped_rows_fp8_on_the_wire(act, graphs):
    """Two A ranks of one replica: their rows form one F job (the codes and the scales are
    concatenated row by row); each rank's answer equals the expert call on its own rows."""
    say(f"loop: {act} on the wire, a group of 2 A ranks, graph_max_tokens={graphs}")
    experts = make_experts(act, 64)
    with OneGpuAfd(experts, n_max=64, act=act, group=2, graph_max_tokens=graphs) as afd:
        sends = [torch.cuda.Stream() for _ in range(2)]
        main = torch.cuda.current_stream()
        keep, tickets = [], []
        for r in range(2):
            x, topk = job(9 + 20 * r, 400 + r)
            ids = topk.topk_ids.to(torch.int32).contiguous()
            w = topk.topk_weights.to(torch.float32).contiguous()
            q, s = quant_act(act, x)
            sends[r].wait_stream(main)
            t = afd.channels[r].send(0, 0, q.data_ptr(), ids.data_ptr(), w.data_ptr(), x.shape[0], sends[r],
                                     xs_ptr=s.data_ptr())
            keep.append((x, topk, q, s, ids, w))
            tickets.append(t)
        assert afd.scheduler.serve_pending() == 1
        for r, (t, (x, topk, *_)) in enumerate(zip(tickets, keep)):
            ptr = afd.channels[r].wait(t, main)[0]
            got = torch.empty(x.shape[0], H, dtype=torch.bfloat16, device=dev())
            hip.copy_async(got.data_ptr(), ptr, got.numel() * 2, main.cuda_stream)
            torch.cuda.synchronize()
            assert np.array_equal(bits16(got), direct(experts, 0, x, topk)), r
        assert afd.server.stats["jobs"] == 1


def test_send_checks_the_wire_format():
    say("loop: scales required exactly when fp8 is on the wire")
    experts = make_experts("mxfp8", 64)
    with pytest.raises(ValueError):
        OneGpuAfd(experts, n_max=64, act="fp8_1x128")
    with OneGpuAfd(experts, n_max=64, act="mxfp8") as afd:
        x, topk = job(4, 9)
        ids = topk.topk_ids.to(torch.int32).contiguous()
        w = topk.topk_weights.to(torch.float32).contiguous()
        with pytest.raises(ValueError):
            afd.channel.send(0, 0, x.data_ptr(), ids.data_ptr(), w.data_ptr(), 4, torch.cuda.current_stream())
        assert afd.server.stats["jobs"] == 0
